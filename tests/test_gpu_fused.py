"""GPU parity: fused QK-RMSNorm + RoPE + KV write against the oracle's separate steps
(RmsNorm q/k, RopeHalf q/k, WriteKvCache) in the decoder's decode and prefill layouts."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as orc
from gpu_helpers import down, say, up
from helpers import SplitMix64
from orator_amd import decoder_attn as da

pytestmark = pytest.mark.gpu

EPS, THETA = 1e-6, 1e6


def _oracle(q, k, v, qw, kw, pos):
    """q [T,Hq,Dh], k/v [T,Hkv,Dh] -> normed+roped q, k (reference order)."""
    T, Hq, Dh = q.shape
    Hkv = k.shape[1]
    qn = orc.rms_norm(q.reshape(T * Hq, Dh), qw, EPS).reshape(T, Hq, Dh)
    kn = orc.rms_norm(k.reshape(T * Hkv, Dh), kw, EPS).reshape(T, Hkv, Dh)
    return orc.rope_half(qn, pos, THETA), orc.rope_half(kn, pos, THETA)


def _bf16_close(got, ref):
    """Equal except rare 1-ulp bf16 flips where an fp32 ulp difference crosses a rounding
    midpoint."""
    d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert d.max() <= 1 and np.count_nonzero(d) <= max(4, d.size // 1000), (d.max(), np.count_nonzero(d))


def test_fused_prefill_layout_contiguous():
    r = SplitMix64(31)
    T, Hq, Hkv, Dh, cap, pos0 = 503, 16, 8, 128, 600, 40
    q, k, v = r.normal((T, Hq, Dh)), r.normal((T, Hkv, Dh)), r.normal((T, Hkv, Dh))
    qw, kw = r.normal((Dh,), 0.5) + 1.0, r.normal((Dh,), 0.5) + 1.0
    pos = np.arange(pos0, pos0 + T, dtype=np.int32)
    q_ref, k_ref = _oracle(q, k, v, qw, kw, pos)
    kc_ref = np.zeros((cap, Hkv, Dh), np.uint16)
    vc_ref = np.zeros_like(kc_ref)
    orc.kv_write(k_ref, v, kc_ref, vc_ref, pos0)
    dq, dk, dv = up(q), up(k), up(v)
    dkc, dvc = up(np.zeros_like(kc_ref)), up(np.zeros_like(vc_ref))
    say("fused prefill")
    da.QkNormRopeKvWrite(dq, dk, dv, Hq * Dh, Hkv * Dh, up(qw), up(kw), EPS, up(pos), THETA, T, T,
                         Hq, Hkv, Dh, dkc, dvc, None, 0, 0, cap)
    # unit-scale values: the sum-of-squares order differs from the oracle's, so allow a few
    # fp32 ulps of absolute error
    assert np.max(np.abs(down(dq, q.shape) - q_ref)) < 2e-6
    assert np.max(np.abs(down(dk, k.shape) - k_ref)) < 2e-6
    _bf16_close(down(dkc, kc_ref.shape, np.uint16), kc_ref)
    np.testing.assert_array_equal(down(dvc, vc_ref.shape, np.uint16), vc_ref)


def test_fused_decode_layout_paged_streams():
    """The decode step's fused qkv row [q | k | v] per stream (asr_text_decoder.cu:381-384),
    B = 16 streams at different positions, 16-token pages."""
    r = SplitMix64(32)
    B, Hq, Hkv, Dh, ps, max_pages = 16, 16, 8, 128, 16, 8
    row = (Hq + 2 * Hkv) * Dh
    qkv = r.normal((B, row))
    qw, kw = r.normal((Dh,), 0.5) + 1.0, r.normal((Dh,), 0.5) + 1.0
    pos = np.array(SplitMix64(4).uniform(B) * (max_pages * ps), np.int32)
    n_pages = B * max_pages
    table = np.array(SplitMix64(5).uniform(n_pages).argsort(), np.int32).reshape(B, max_pages)
    q = qkv[:, :Hq * Dh].reshape(B, Hq, Dh)
    k = qkv[:, Hq * Dh:(Hq + Hkv) * Dh].reshape(B, Hkv, Dh)
    v = qkv[:, (Hq + Hkv) * Dh:].reshape(B, Hkv, Dh)
    q_ref, k_ref = _oracle(q, k, v, qw, kw, pos)
    kp_ref = np.zeros((n_pages, ps, Hkv, Dh), np.uint16)
    vp_ref = np.zeros_like(kp_ref)
    for b in range(B):
        orc.kv_write_paged(k_ref[b:b + 1], v[b:b + 1], kp_ref, vp_ref, table[b], ps, int(pos[b]))
    dqkv = up(qkv)
    base = dqkv.ptr
    dkp, dvp = up(np.zeros_like(kp_ref)), up(np.zeros_like(vp_ref))
    say("fused decode paged")
    da.QkNormRopeKvWrite(base, base + Hq * Dh * 4, base + (Hq + Hkv) * Dh * 4, row, row, up(qw),
                         up(kw), EPS, up(pos), THETA, B, 1, Hq, Hkv, Dh, dkp, dvp, up(table),
                         max_pages, ps, n_pages)
    got = down(dqkv, qkv.shape)
    assert np.max(np.abs(got[:, :Hq * Dh].reshape(B, Hq, Dh) - q_ref)) < 2e-6
    assert np.max(np.abs(got[:, Hq * Dh:(Hq + Hkv) * Dh].reshape(B, Hkv, Dh) - k_ref)) < 2e-6
    np.testing.assert_array_equal(got[:, (Hq + Hkv) * Dh:], qkv[:, (Hq + Hkv) * Dh:])  # v untouched
    _bf16_close(down(dkp, kp_ref.shape, np.uint16), kp_ref)
    np.testing.assert_array_equal(down(dvp, vp_ref.shape, np.uint16), vp_ref)


@pytest.mark.parametrize("paged", [False, True])
def test_fused_token_kernel_matches_row_kernel(paged):
    """Prompts (>= 64 tokens) run a workgroup per token, a few tokens a wave per row: the same
    arithmetic per row, so a 96-token call equals three 32-token calls bit for bit."""
    r = SplitMix64(33 + paged)
    T, Hq, Hkv, Dh, pos0, ps = 96, 16, 8, 128, 10, 16
    q, k, v = r.normal((T, Hq, Dh)), r.normal((T, Hkv, Dh)), r.normal((T, Hkv, Dh))
    qw, kw = r.normal((Dh,), 0.5) + 1.0, r.normal((Dh,), 0.5) + 1.0
    pos = np.arange(pos0, pos0 + T, dtype=np.int32)
    cap = 128
    n_pages = cap // ps
    table = np.array(SplitMix64(6).uniform(n_pages).argsort(), np.int32) if paged else None
    shape = (n_pages, ps, Hkv, Dh) if paged else (cap, Hkv, Dh)
    outs = []
    for chunks in ([(0, T)], [(0, 32), (32, 64), (64, 96)]):
        dq, dk = up(q), up(k)
        dkc, dvc = up(np.zeros(shape, np.uint16)), up(np.zeros(shape, np.uint16))
        dt = up(table) if paged else None
        dpos, dv = up(pos), up(v)
        for a, b in chunks:
            n = b - a
            say("fused token/row", paged, a, b)
            da.QkNormRopeKvWrite(dq.ptr + a * Hq * Dh * 4, dk.ptr + a * Hkv * Dh * 4,
                                 dv.ptr + a * Hkv * Dh * 4, Hq * Dh, Hkv * Dh, up(qw), up(kw), EPS,
                                 dpos.ptr + a * 4, THETA, n, n, Hq, Hkv, Dh, dkc, dvc, dt,
                                 n_pages if paged else 0, ps if paged else 0,
                                 n_pages if paged else cap)
        outs.append([down(dq, q.shape), down(dk, k.shape), down(dkc, shape, np.uint16),
                     down(dvc, shape, np.uint16)])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    q_ref, k_ref = _oracle(q, k, v, qw, kw, pos)
    assert np.max(np.abs(outs[0][0] - q_ref)) < 2e-6
    assert np.max(np.abs(outs[0][1] - k_ref)) < 2e-6
