"""GPU parity for the asr_ops family: the reference's own fixtures (tests/golden, with the
reference test's tolerances) and the oracle on seeded inputs."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as orc
import truth64 as t64
from gpu_helpers import down, empty, say, up
from helpers import SplitMix64, check_fp32, rel_err
from orator_amd import asr_ops

pytestmark = pytest.mark.gpu


def test_rmsnorm_fixture_and_oracle(golden):
    x, w = golden["rmsnorm_x"], golden["rmsnorm_w"]
    rows, dim = x.shape
    dout = empty(x.shape, np.float32)
    say("rmsnorm fixture")
    asr_ops.RmsNorm(up(x), up(w), dout, rows, dim, 1e-6)
    got = down(dout, x.shape)
    assert np.max(np.abs(got - golden["rmsnorm_out"])) < 1e-4  # test_asr_ops.cc:93
    assert rel_err(got, orc.rms_norm(x, w, 1e-6), 1e-3) < 1e-5


@pytest.mark.parametrize("rows,dim", [(16 * 503, 128), (8, 128), (3, 2048), (5, 130), (4, 512),
                                      (7, 1024), (2, 4096)])
def test_rmsnorm_qk_shapes_in_place(rows, dim):
    r = SplitMix64(rows + dim)
    x, w = r.normal((rows, dim)), r.normal((dim,))
    dx = up(x)
    say("rmsnorm", rows, dim)
    asr_ops.RmsNorm(dx, up(w), dx, rows, dim, 1e-6)  # in place, as the decoder calls it
    assert rel_err(down(dx, x.shape), orc.rms_norm(x, w, 1e-6), 1e-3) < 1e-5


def test_rope_interleaved_fixture(golden):
    x, pos = golden["rope_x"], golden["rope_pos"]
    T, H, Dh = x.shape
    dx = up(x)
    say("rope interleaved fixture")
    asr_ops.RopeInterleaved(dx, up(pos), T, H, Dh, 1e6)
    got = down(dx, x.shape)
    assert np.max(np.abs(got - golden["rope_out"])) < 1e-4  # test_asr_ops.cc:118
    assert np.max(np.abs(got - orc.rope_interleaved(x, pos, 1e6))) < 1e-6


@pytest.mark.parametrize("p0,T,H", [(0, 503, 16), (4096, 3, 8), (100000, 2, 8)])
def test_rope_half_vs_oracle(p0, T, H):
    r = SplitMix64(p0 + T)
    Dh = 128
    x = r.normal((T, H, Dh))
    pos = np.arange(p0, p0 + T, dtype=np.int32)
    dx = up(x)
    say("rope half", p0, T, H)
    asr_ops.RopeHalf(dx, up(pos), T, H, Dh, 1e6)
    got = down(dx, x.shape)
    # same fp32 angle, sin/cos rounded once from fp64: equal up to rare double roundings
    assert np.max(np.abs(got - orc.rope_half(x, pos, 1e6))) < 1e-6


def test_swiglu_fixture(golden):
    g, u = golden["swiglu_gate"], golden["swiglu_up"]
    dout = empty(g.shape, np.float32)
    say("swiglu")
    asr_ops.SwiGLU(up(g), up(u), dout, g.size)
    assert np.max(np.abs(down(dout, g.shape) - golden["swiglu_out"])) < 1e-5  # :141


@pytest.mark.parametrize("n", [1, 3, 4, 1001, 1 << 20])
def test_bf16_casts_bit_exact(n):
    r = SplitMix64(n)
    x = r.normal((n,), 3.0)
    db = empty((n,), np.uint16)
    say("f32_to_bf16", n)
    asr_ops.F32ToBf16(up(x), db, n)
    bits = down(db, (n,), np.uint16)
    np.testing.assert_array_equal(bits, orc.to_bf16(x))
    df = empty((n,), np.float32)
    asr_ops.Bf16ToF32(db, df, n)
    np.testing.assert_array_equal(down(df, (n,)), orc.from_bf16(bits))
    # the same at element offsets 1 and 3 (natural alignment only: the element-access path)
    for off in (1, 3):
        src = up(np.concatenate([np.zeros(off, np.float32), x]))
        d16 = empty((n + off,), np.uint16)
        asr_ops.F32ToBf16(src.ptr + 4 * off, d16.ptr + 2 * off, n)
        got16 = down(d16, (n + off,), np.uint16)[off:]
        np.testing.assert_array_equal(got16, bits)
        d32 = empty((n + off,), np.float32)
        asr_ops.Bf16ToF32(d16.ptr + 2 * off, d32.ptr + 4 * off, n)
        np.testing.assert_array_equal(down(d32, (n + off,))[off:], orc.from_bf16(bits))


def _argmax_gpu(x, b0=-1, b1=-1):
    di = empty((1,), np.int32)
    asr_ops.ArgmaxBanned(up(x), x.size, b0, b1, di)
    return int(down(di, (1,), np.int32)[0])


def test_argmax_banned_random_and_ties():
    r = SplitMix64(77)
    x = r.normal((151936,))
    top = np.argsort(-x)
    say("argmax")
    assert _argmax_gpu(x) == orc.argmax_banned(x) == int(top[0])
    assert _argmax_gpu(x, int(top[0]), int(top[1])) == int(top[2])
    for idx in ([2, 258], [1, 2], [1, 3], [130, 2], [5, 5 + 256 * 7, 99]):
        y = np.zeros(2000, np.float32)
        y[idx] = 5.0
        assert _argmax_gpu(y) == orc.argmax_banned(y), idx


@pytest.mark.parametrize("n", [2049, 4096, 151936])
def test_argmax_two_stage_keeps_the_tie_rule(n):
    """Rows longer than 2048 run the two-stage kernels: planted ties inside one slot across
    stage-1 ranges, across slots in different ranges, bans and an all -inf row give the
    single-pass rule's answers."""
    cases = [[2, 2 + 256 * 7, 2 + 256 * 8], [1, 2 + 256 * 9], [3 + 256 * 8, 1], [130 + 2048, 2],
             [5, 5 + 256 * 7, 99, 99 + 256 * 8], [n - 1, (n - 1) % 256]]
    for idx in cases:
        y = np.zeros(n, np.float32)
        y[[i for i in idx if i < n]] = 5.0
        assert _argmax_gpu(y) == orc.argmax_banned(y), (n, idx)
        assert _argmax_gpu(y, idx[0], idx[1]) == orc.argmax_banned(y, idx[0], idx[1]), (n, idx)
    assert _argmax_gpu(np.full(n, -np.inf, np.float32)) == 0
    x = SplitMix64(n).normal((n,))
    assert _argmax_gpu(x, 7, 9) == orc.argmax_banned(x, 7, 9)


def test_gqa_attention_fixture(golden):
    """The reference's own GQA check: T=24, 16/8 heads, causal, max-abs 5e-4 against torch
    SDPA (test/unit/model/test_asr_ops.cc:145-169)."""
    q, k, v = golden["gqa_q"], golden["gqa_k"], golden["gqa_v"]
    T, Hq, Dh = q.shape
    Hkv = k.shape[1]
    dout = empty(q.shape, np.float32)
    say("gqa_attention fixture")
    asr_ops.GqaAttention(up(q), up(k), up(v), dout, T, Hq, Hkv, Dh, 1.0 / np.sqrt(Dh), True)
    got = down(dout, q.shape)
    assert np.max(np.abs(got - golden["gqa_out"])) < 5e-4
    check_fp32(got, orc.gqa_attention(q, k, v, 1.0 / np.sqrt(Dh), True), 1e-4,
               truth=t64.self_attention(q, k, v, 1.0 / np.sqrt(Dh), True))


@pytest.mark.parametrize("T,Hq,Hkv,Dh,causal", [(1, 16, 8, 128, True), (256, 16, 8, 128, True),
                                               (100, 8, 8, 64, False), (300, 16, 4, 64, True),
                                               (129, 16, 8, 128, False),
                                               # the generic kernel: other power-of-two head
                                               # sizes and group sizes (G = 8, 3, 16)
                                               (64, 16, 2, 32, True), (50, 8, 1, 256, False),
                                               (33, 16, 2, 1024, True), (40, 12, 4, 16, True),
                                               (17, 16, 1, 1, False), (200, 8, 4, 512, True)])
def test_gqa_attention_vs_oracle(T, Hq, Hkv, Dh, causal):
    r = SplitMix64(T * 7 + Hkv)
    q, k, v = r.normal((T, Hq, Dh), 0.3), r.normal((T, Hkv, Dh), 0.3), r.normal((T, Hkv, Dh))
    scale = 1.0 / np.sqrt(Dh)
    dout = empty(q.shape, np.float32)
    say("gqa_attention", T, Hq, Hkv, Dh, causal)
    asr_ops.GqaAttention(up(q), up(k), up(v), dout, T, Hq, Hkv, Dh, scale, causal)
    ref = orc.gqa_attention(q, k, v, scale, causal)
    check_fp32(down(dout, q.shape), ref, 1e-4, truth=t64.self_attention(q, k, v, scale, causal))
