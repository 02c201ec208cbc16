"""GPU parity: fused QK-RMSNorm + RoPE + KV write against the oracle's separate steps
(RmsNorm q/k, RopeHalf q/k, WriteKvCache) in the decoder's decode and prefill layouts."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as orc
import truth64 as t64
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


def _bf16_close(got, ref, abs_tol=2e-6):
    """The cache holds bf16(k) of a k that matches the oracle to abs_tol (fp32 rounding: the
    sum of squares runs in another order), so every element is within one bf16 step
    (2^-7 |k|) plus abs_tol of the oracle's.  Near-zero k (RoPE's n0 c - n1 s cancelling) may
    differ by many bf16 ulps in bits while meeting that; elements differing at all must stay
    rare."""
    g, r = orc.from_bf16(got).astype(np.float64), orc.from_bf16(ref).astype(np.float64)
    d = np.abs(g - r)
    bound = abs_tol + 2.0 ** -7 * np.abs(r)
    assert np.all(d <= bound), (float(np.max(d - bound)), int(np.count_nonzero(d > bound)))
    n = int(np.count_nonzero(got != ref))
    assert n <= max(4, got.size // 1000), n


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


# Positions around 2048 and 4090-4100, where the fp32 RoPE angle (position * inv_freq, up to
# ~4100 rad) is largest: the angle is formed in fp32 exactly as RopeHalf does
# (src/model/asr_ops.cu:102-109) and its cos/sin must still match the oracle's.
HIGH_POS = [2046, 2047, 2048, 2049, 2050, 2063, 2064, 2065,
            4090, 4091, 4093, 4095, 4096, 4097, 4099, 4100]


def _rope_table(n):
    from gpu_helpers import empty
    t = empty((n, 64, 2), np.float32)
    da.RopeTable(t, n, THETA)
    return t


@pytest.mark.parametrize("paged", [False, True])
def test_decode_folded_qknorm_rope_append_high_positions(paged):
    """The decoder's decode-step launch (raw q / k projections in; QK-RMSNorm, RoPE from the
    position's table row, bf16 KV write and split-K attention in one kernel) against the
    oracle's separate reference steps: RmsNorm q/k, RopeHalf q/k, WriteKvCache, decode
    attention.  Paged: B = 16 streams at HIGH_POS; contiguous: one stream per position."""
    import math
    from gpu_helpers import empty
    from helpers import check_fp32
    Hq, Hkv, Dh, ps = 16, 8, 128, 16
    r = SplitMix64(41 + paged)
    qw, kw = r.normal((Dh,), 0.5) + 1.0, r.normal((Dh,), 0.5) + 1.0
    scale = 1.0 / math.sqrt(Dh)
    cap = 4112
    rope = _rope_table(cap)
    dqw, dkw = up(qw), up(kw)
    if paged:
        B = len(HIGH_POS)
        pos = np.array(HIGH_POS, np.int32)
        max_pages = cap // ps
        n_pages = B * max_pages
        table = np.array(r.uniform(n_pages).argsort(), np.int32).reshape(B, max_pages)
        kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
        vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
        q, kn, vn = r.normal((B, Hq, Dh)), r.normal((B, Hkv, Dh)), r.normal((B, Hkv, Dh))
        q_ref, k_ref = _oracle(q, kn, vn, qw, kw, pos)
        kp_ref, vp_ref = kp.copy(), vp.copy()
        for b in range(B):
            orc.kv_write_paged(k_ref[b][None], vn[b][None], kp_ref, vp_ref, table[b], ps,
                               int(pos[b]))
        ref = orc.gqa_decode_paged(q_ref, kp_ref, vp_ref, table, ps, pos, scale, threads=8)
        dk, dv, out = up(kp), up(vp), empty((B, Hq, Dh), np.float32)
        say("decode qknorm paged high positions")
        da.GqaDecodeAttnAppendQkNormPaged(up(q), up(kn), up(vn), dk, dv, up(table), max_pages, ps,
                                          n_pages, up(pos), out, B, Hq, Hkv, Dh, scale, dqw, dkw,
                                          EPS, rope, cap)
        check_fp32(down(out, (B, Hq, Dh)), ref, 1e-4,
                   truth=t64.decode_paged(q_ref, kp_ref, vp_ref, table, ps, pos, scale))
        _bf16_close(down(dk, kp.shape, np.uint16), kp_ref)
        np.testing.assert_array_equal(down(dv, vp.shape, np.uint16), vp_ref)
        return
    kc = orc.to_bf16(r.normal((cap, Hkv, Dh)))
    vc = orc.to_bf16(r.normal((cap, Hkv, Dh)))
    for p in HIGH_POS:
        q, kn, vn = r.normal((1, Hq, Dh)), r.normal((1, Hkv, Dh)), r.normal((1, Hkv, Dh))
        pa = np.array([p], np.int32)
        q_ref, k_ref = _oracle(q, kn, vn, qw, kw, pa)
        kc_ref, vc_ref = kc.copy(), vc.copy()
        orc.kv_write(k_ref, vn, kc_ref, vc_ref, p)
        ref = orc.gqa_decode(q_ref[0], kc_ref, vc_ref, p, scale)
        dk, dv, out = up(kc), up(vc), empty((Hq, Dh), np.float32)
        say("decode qknorm contiguous", p)
        da.GqaDecodeAttnAppendQkNorm(up(q), up(kn), up(vn), dk, dv, out, Hq, Hkv, Dh, up(pa), cap,
                                     scale, dqw, dkw, EPS, rope, cap)
        check_fp32(down(out, (Hq, Dh)), ref, 1e-4,
                   truth=t64.decode(q_ref[0], kc_ref, vc_ref, p, scale))
        _bf16_close(down(dk, kc.shape, np.uint16), kc_ref)
        np.testing.assert_array_equal(down(dv, vc.shape, np.uint16), vc_ref)


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("table", [False, True])
def test_fused_prompt_kernel_high_positions(paged, table):
    """The prompt-path QK-norm/RoPE/KV-write kernel (a workgroup per token) at positions
    2016..2107 and 4040..4167: B = 16 streams of 64 tokens (paged) or one 128-token stream
    at 4040.. (contiguous); RoPE formed per call (fp64 trig of the fp32 angle) or read from
    the decoder's table."""
    Hq, Hkv, Dh, ps, cap = 16, 8, 128, 16, 4224
    r = SplitMix64(51 + 2 * paged + table)
    if paged:
        B, tps = 16, 64
        base = [2016 + 6 * b for b in range(8)] + [4040 + 8 * b for b in range(8)]
        pos = np.concatenate([np.arange(s, s + tps) for s in base]).astype(np.int32)
    else:
        B, tps = 1, 128
        pos = np.arange(4040, 4040 + tps, dtype=np.int32)
    T = B * tps
    q, k, v = r.normal((T, Hq, Dh)), r.normal((T, Hkv, Dh)), r.normal((T, Hkv, Dh))
    qw, kw = r.normal((Dh,), 0.5) + 1.0, r.normal((Dh,), 0.5) + 1.0
    q_ref, k_ref = _oracle(q, k, v, qw, kw, pos)
    max_pages = cap // ps
    if paged:
        n_pages = B * max_pages
        tbl = np.array(r.uniform(n_pages).argsort(), np.int32).reshape(B, max_pages)
        kc_ref = np.zeros((n_pages, ps, Hkv, Dh), np.uint16)
        vc_ref = np.zeros_like(kc_ref)
        for b in range(B):
            sl = slice(b * tps, (b + 1) * tps)
            for t in range(tps):
                orc.kv_write_paged(k_ref[sl][t:t + 1], v[sl][t:t + 1], kc_ref, vc_ref, tbl[b], ps,
                                   int(pos[b * tps + t]))
    else:
        tbl = None
        kc_ref = np.zeros((cap, Hkv, Dh), np.uint16)
        vc_ref = np.zeros_like(kc_ref)
        orc.kv_write(k_ref, v, kc_ref, vc_ref, int(pos[0]))
    dq, dk, dv = up(q), up(k), up(v)
    dkc, dvc = up(np.zeros_like(kc_ref)), up(np.zeros_like(vc_ref))
    args = (Hq * Dh, Hkv * Dh, up(qw), up(kw), EPS, up(pos), THETA)
    tail = (T, tps, Hq, Hkv, Dh, dkc, dvc, up(tbl) if paged else None,
            max_pages if paged else 0, ps if paged else 0, B * max_pages if paged else cap)
    say("fused prompt high positions", paged, table)
    if table:
        da.QkNormRopeKvWriteTable(dq, dk, dv, *args, _rope_table(cap), cap, *tail)
    else:
        da.QkNormRopeKvWrite(dq, dk, dv, *args, *tail)
    assert np.max(np.abs(down(dq, q.shape) - q_ref)) < 2e-6
    assert np.max(np.abs(down(dk, k.shape) - k_ref)) < 2e-6
    _bf16_close(down(dkc, kc_ref.shape, np.uint16), kc_ref)
    np.testing.assert_array_equal(down(dvc, vc_ref.shape, np.uint16), vc_ref)
