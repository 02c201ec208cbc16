"""GPU parity: MFMA prefill attention against the oracle's GqaCacheAttnKernel restatement.

fp32 mode: max |g - r| / max(|r|, 0.05) <= 1e-4.  bf16 mode: max |g - r| <= 2e-2 on
unit-scale outputs.  Inputs follow BASELINE configs[1]: N(0,1) q/k/v, QK-RMSNorm (unit
gain, eps 1e-6) and RoPE theta 1e6 at the tokens' absolute positions, K/V rounded to bf16
by the KV write."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle_lib as orc
import truth64 as t64
from gpu_helpers import down, empty, say, up
from helpers import SplitMix64, check_fp32, rel_err
from orator_amd import decoder_attn as da

pytestmark = pytest.mark.gpu

FLOOR, TOL32, TOL16 = 0.05, 1e-4, 2e-2


def _layer_inputs(seed, T, pos0, Hq=16, Hkv=8, Dh=128, cap=None):
    """q (normed, roped) for positions pos0..pos0+T-1 and a bf16 cache holding positions
    0..pos0+T-1 (earlier positions = a previous prefill)."""
    r = SplitMix64(seed)
    S = pos0 + T
    cap = cap or S
    ones = np.ones(Dh, np.float32)
    k = orc.rms_norm(r.normal((S * Hkv, Dh)), ones, 1e-6).reshape(S, Hkv, Dh)
    k = orc.rope_half(k, np.arange(S, dtype=np.int32), 1e6)
    v = r.normal((S, Hkv, Dh))
    kc = np.zeros((cap, Hkv, Dh), np.uint16)
    vc = np.zeros_like(kc)
    orc.kv_write(k, v, kc, vc, 0)
    q = orc.rms_norm(r.normal((T * Hq, Dh)), ones, 1e-6).reshape(T, Hq, Dh)
    q = orc.rope_half(q, np.arange(pos0, pos0 + T, dtype=np.int32), 1e6)
    return q, kc, vc


def _run(q, kc, vc, pos0, cap, mode, Hkv, page=None):
    T, Hq, Dh = q.shape
    dout = empty(q.shape, np.float32)
    scale = 1.0 / math.sqrt(Dh)
    dpos = up(np.array([pos0], np.int32))
    if page is None:
        if mode == da.PREFILL_FP32:
            da.GqaCacheAttn(up(q), up(kc), up(vc), dout, T, Hq, Hkv, Dh, dpos, cap, scale)
        else:
            da.GqaCacheAttnEx(up(q), None, up(kc), up(vc), None, 0, 0, dout, T, Hq, Hkv, Dh, dpos,
                              cap, scale, mode)
    else:
        kp, vp, table, ps = page
        da.GqaCacheAttnEx(up(q), None, up(kp), up(vp), up(table), table.size, ps, dout, T, Hq, Hkv,
                          Dh, dpos, cap, scale, mode)
    return down(dout, q.shape)


@pytest.mark.parametrize("mode", [da.PREFILL_FP32, da.PREFILL_BF16])
def test_prefill_config2_shape(mode):
    """T = 503 (128 prompt + 375 audio), pos0 = 0."""
    T, Hq, Hkv, Dh = 503, 16, 8, 128
    q, kc, vc = _layer_inputs(503, T, 0)
    ref = orc.gqa_prefill(q, kc, vc, 0, 1.0 / math.sqrt(Dh), threads=8)
    say("prefill config2", mode)
    got = _run(q, kc, vc, 0, T, mode, Hkv)
    if mode == da.PREFILL_FP32:
        check_fp32(got, ref, TOL32, truth=t64.prefill(q, kc, vc, 0, 1.0 / math.sqrt(Dh)))
    else:
        assert np.max(np.abs(got - ref)) <= TOL16


def test_prefill_streaming_split_equals_full():
    """PrefillAt(0..128) then PrefillAt(128..503) on the same cache gives the full result
    (test/unit/model/test_asr_decoder.cc:76-127)."""
    T, split, Hkv, Dh = 503, 128, 8, 128
    q, kc, vc = _layer_inputs(7, T, 0)
    say("prefill split")
    full = _run(q, kc, vc, 0, T, da.PREFILL_FP32, Hkv)
    a = _run(np.ascontiguousarray(q[:split]), kc, vc, 0, T, da.PREFILL_FP32, Hkv)
    b = _run(np.ascontiguousarray(q[split:]), kc, vc, split, T, da.PREFILL_FP32, Hkv)
    # same rows, same keys, same kernel: identical up to the row's tile grouping
    assert rel_err(np.concatenate([a, b]), full, FLOOR) <= 2e-6


def _check(got, ref, mode, truth=None):
    if mode == da.PREFILL_FP32:
        check_fp32(got, ref, TOL32, truth=truth)
    else:
        assert np.max(np.abs(got - ref)) <= TOL16


MODES = [da.PREFILL_FP32, da.PREFILL_BF16]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("T,pos0,cap", [(1, 0, 64), (1, 700, 1024), (37, 1000, 2048),
                                        (64, 0, 64), (65, 3, 128), (200, 1800, 2048),
                                        (129, 0, 160), (300, 77, 400)])
def test_prefill_offsets_and_ragged(T, pos0, cap, mode):
    Hkv, Dh = 8, 128
    q, kc, vc = _layer_inputs(T + pos0, T, pos0, cap=cap)
    ref = orc.gqa_prefill(q, kc, vc, pos0, 1.0 / math.sqrt(Dh), threads=8)
    say("prefill offsets", T, pos0, cap, mode)
    got = _run(q, kc, vc, pos0, cap, mode, Hkv)
    _check(got, ref, mode, t64.prefill(q, kc, vc, pos0, 1.0 / math.sqrt(Dh)))
    if T == 1 and pos0 == 0:  # one key: the output is v0
        np.testing.assert_allclose(got[0], np.repeat(orc.from_bf16(vc[0]), 2, axis=0), atol=1e-6)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 4)])
def test_prefill_group_variants(Hq, Hkv, mode):
    T, pos0, Dh = 150, 20, 128
    q, kc, vc = _layer_inputs(Hq * 10 + Hkv, T, pos0, Hq=Hq, Hkv=Hkv)
    ref = orc.gqa_prefill(q, kc, vc, pos0, 1.0 / math.sqrt(Dh), threads=8)
    say("prefill groups", Hq, Hkv, mode)
    got = _run(q, kc, vc, pos0, pos0 + T, mode, Hkv)
    _check(got, ref, mode, t64.prefill(q, kc, vc, pos0, 1.0 / math.sqrt(Dh)))


@pytest.mark.parametrize("mode", MODES)
def test_prefill_paged_matches_contiguous(mode):
    T, pos0, Hkv, Dh, ps = 300, 100, 8, 128, 16
    q, kc, vc = _layer_inputs(11, T, pos0, cap=400)
    n_pages = 400 // ps
    perm = np.array(SplitMix64(3).uniform(n_pages).argsort(), np.int32)
    kp = np.empty((n_pages, ps, Hkv, Dh), np.uint16)
    vp = np.empty_like(kp)
    kp[perm] = kc.reshape(n_pages, ps, Hkv, Dh)
    vp[perm] = vc.reshape(n_pages, ps, Hkv, Dh)
    say("prefill paged", mode)
    a = _run(q, kc, vc, pos0, 400, mode, Hkv)
    b = _run(q, kc, vc, pos0, 400, mode, Hkv, page=(kp, vp, perm, ps))
    np.testing.assert_array_equal(a, b)


def _paged_copy(kc, vc, ps, seed):
    cap, Hkv, Dh = kc.shape
    n_pages = cap // ps
    perm = np.array(SplitMix64(seed).uniform(n_pages).argsort(), np.int32)
    kp = np.empty((n_pages, ps, Hkv, Dh), np.uint16)
    vp = np.empty_like(kp)
    kp[perm] = kc.reshape(n_pages, ps, Hkv, Dh)
    vp[perm] = vc.reshape(n_pages, ps, Hkv, Dh)
    return kp, vp, perm


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("ps", [32, 128])
def test_prefill_paged_page_sizes(ps, mode):
    """Pages of 32 and 128 keys through a permuted table: the same bits as the contiguous
    cache, and the oracle's result."""
    T, pos0, Hkv, Dh, cap = 300, 100, 8, 128, 512
    q, kc, vc = _layer_inputs(17 + ps, T, pos0, cap=cap)
    kp, vp, perm = _paged_copy(kc, vc, ps, ps)
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_prefill(q, kc, vc, pos0, scale, threads=8)
    say("prefill paged page size", ps, mode)
    a = _run(q, kc, vc, pos0, cap, mode, Hkv)
    b = _run(q, kc, vc, pos0, cap, mode, Hkv, page=(kp, vp, perm, ps))
    np.testing.assert_array_equal(a, b)
    _check(b, ref, mode, t64.prefill(q, kc, vc, pos0, scale))


@pytest.mark.parametrize("mode", MODES)
def test_prefill_paged_at_the_16k_key_limit(mode):
    """The last 64 prompt rows of a full 16384-key paged cache (the largest a paged cache may
    hold: the kernel's LDS page-row table): queries at 16320..16383 against the oracle, and
    the same bits as the contiguous cache."""
    T, pos0, Hkv, Dh, ps = 64, 16320, 8, 128, 16
    cap = pos0 + T
    q, kc, vc = _layer_inputs(16384, T, pos0, cap=cap)
    kp, vp, perm = _paged_copy(kc, vc, ps, 5)
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_prefill(q, kc, vc, pos0, scale, threads=8)
    say("prefill paged 16k", mode)
    a = _run(q, kc, vc, pos0, cap, mode, Hkv)
    b = _run(q, kc, vc, pos0, cap, mode, Hkv, page=(kp, vp, perm, ps))
    np.testing.assert_array_equal(a, b)
    # outputs over 16K keys are ~0.01: at the 1e-3 floor the fp32 sums' rounding shows, so the
    # device is held to the oracle's own distance from the fp64 value there
    _check(b, ref, mode, t64.prefill(q, kc, vc, pos0, scale))


def test_prefill_bf16_q_input():
    T, Hkv, Dh = 96, 8, 128
    q, kc, vc = _layer_inputs(13, T, 0)
    qb = orc.to_bf16(q)
    ref = orc.gqa_prefill(orc.from_bf16(qb), kc, vc, 0, 1.0 / math.sqrt(Dh), threads=8)
    dout = empty(q.shape, np.float32)
    say("prefill bf16 q")
    da.GqaCacheAttnEx(None, up(qb), up(kc), up(vc), None, 0, 0, dout, T, 16, Hkv, Dh,
                      up(np.array([0], np.int32)), T, 1.0 / math.sqrt(Dh), da.PREFILL_BF16)
    assert np.max(np.abs(down(dout, q.shape) - ref)) <= TOL16


# Long bf16 prompts over a contiguous cache take the stream-K kernel (prefill_attn.hip
# launch_prefill: Tq >= 2048, GQA group 1 or 2): ragged last blocks, offsets into a longer
# cache, capacity past the keys, q given in fp32 (rounded on the device) and in bf16.
SK_CASES = [(2085, 100, 2300, 16, 8), (2048, 1000, 3100, 8, 8), (2111, 0, 2111, 16, 16)]


@pytest.mark.parametrize("T,pos0,cap,Hq,Hkv", SK_CASES)
def test_prefill_stream_k_cases(T, pos0, cap, Hq, Hkv):
    q, kc, vc = _layer_inputs(T + pos0 + Hkv, T, pos0, Hq=Hq, Hkv=Hkv, cap=cap)
    qb = orc.to_bf16(q)
    scale = 1.0 / math.sqrt(128)
    ref = orc.gqa_prefill(orc.from_bf16(qb), kc, vc, pos0, scale, threads=16)
    dpos = up(np.array([pos0], np.int32))
    for q_in in ("fp32", "bf16"):
        say(f"prefill stream-K T={T} pos0={pos0} cap={cap} Hq={Hq} Hkv={Hkv} q={q_in}")
        dout = empty(q.shape, np.float32)
        if q_in == "fp32":
            da.GqaCacheAttnEx(up(q), None, up(kc), up(vc), None, 0, 0, dout, T, Hq, Hkv, 128,
                              dpos, cap, scale, da.PREFILL_BF16)
        else:
            da.GqaCacheAttnEx(None, up(qb), up(kc), up(vc), None, 0, 0, dout, T, Hq, Hkv, 128,
                              dpos, cap, scale, da.PREFILL_BF16)
        err = float(np.max(np.abs(down(dout, q.shape) - ref)))
        print(f"bf16 max |g - r| = {err:.3e}")
        assert err <= TOL16


def test_prefill_stream_k_reference_redo():
    """Scores that grow along the keys by far more than 2^64 (log2 units) past a segment's
    first tile: the stream-K kernel's fixed softmax reference is exceeded and the segment is
    redone with the maxima seen (without the redo the weights overflow to inf).  q = 1 and key j
    = 12 j / T in every dim: score(t, j) = 1536 j / T / sqrt(128), up to 196 in log2 units."""
    T, Hq, Hkv, Dh = 2048, 16, 8, 128
    q = np.ones((T, Hq, Dh), np.float32)
    kc = orc.to_bf16(np.repeat((12.0 * np.arange(T, dtype=np.float32) / T)[:, None, None],
                               Hkv * Dh, axis=1).reshape(T, Hkv, Dh))
    vc = orc.to_bf16(SplitMix64(21).normal((T, Hkv, Dh)))
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_prefill(q, kc, vc, 0, scale, threads=16)
    say("prefill stream-K reference redo")
    got = _run(q, kc, vc, 0, T, da.PREFILL_BF16, Hkv)
    assert np.all(np.isfinite(got))
    err = float(np.max(np.abs(got - ref)))
    print(f"bf16 max |g - r| = {err:.3e}")
    assert err <= TOL16


def _launcher_rw(T, Hq, Hkv, cus=256):
    """The launcher's choice of row waves per workgroup and pairing (prefill_attn.hip
    launch_g), so each case below names the instantiation it runs on a 256-CU MI355X."""
    G = Hq // Hkv
    tw = 32 // G
    blocks4 = -(-T // (4 * tw))
    blocks2 = -(-T // (2 * tw))
    rw = 4 if blocks4 * Hkv >= 2 * cus else (1 if blocks2 * Hkv < cus else 2)
    n_tblocks = -(-T // (rw * tw))
    paired = rw > 1 and n_tblocks * Hkv >= 2 * cus
    return rw, paired


_ORACLE_CACHE: dict = {}


def _large_case(T, Hq, Hkv):
    key = (T, Hq, Hkv)
    if key not in _ORACLE_CACHE:
        _ORACLE_CACHE.clear()  # one shape at a time (the fp64 value of T = 4096 is large)
        q, kc, vc = _layer_inputs(T * 7 + Hq + Hkv, T, 0, Hq=Hq, Hkv=Hkv)
        scale = 1.0 / math.sqrt(128)
        ref = orc.gqa_prefill(q, kc, vc, 0, scale, threads=16)
        _ORACLE_CACHE[key] = (q, kc, vc, ref)
    return _ORACLE_CACHE[key]


# Every instantiation the row-wave launcher takes at long prompts: RW = 2 row waves paired
# (T = 2048, G = 2: the decoder's own 2048-token fp32 prefill kernel), RW = 2 unpaired, RW = 4
# paired (T = 4096), for GQA groups 1, 2 and 4.  In bf16 mode the group 1 and 2 cases run the
# stream-K kernel instead (G = 4 stays on the row-wave kernel).
LARGE = [(2048, 16, 8), (2048, 8, 8), (2048, 16, 16), (2048, 16, 4),
         (4096, 16, 8), (4096, 16, 16), (4096, 16, 4)]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("T,Hq,Hkv", LARGE)
def test_prefill_long_prompt_instantiations(T, Hq, Hkv, mode):
    q, kc, vc, ref = _large_case(T, Hq, Hkv)
    rw, paired = _launcher_rw(T, Hq, Hkv)
    say(f"prefill T={T} Hq={Hq} Hkv={Hkv} mode={mode} (RW={rw}, paired={paired})")
    got = _run(q, kc, vc, 0, T, mode, Hkv)
    truth = t64.prefill(q, kc, vc, 0, 1.0 / math.sqrt(128)) if mode == da.PREFILL_FP32 else None
    if mode == da.PREFILL_FP32:
        check_fp32(got, ref, TOL32, truth=truth)
    else:
        err = float(np.max(np.abs(got - ref)))
        print(f"bf16 max |g - r| = {err:.3e}")
        assert err <= TOL16


def test_prefill_instantiation_table():
    """The cases above reach the instantiations they are named for (host-side rule)."""
    got = {c: _launcher_rw(*c) for c in LARGE}
    assert got[(2048, 16, 8)] == (2, True)
    assert got[(2048, 8, 8)] == (2, False)
    assert got[(2048, 16, 16)] == (2, True)
    assert got[(2048, 16, 4)] == (2, True)
    assert got[(4096, 16, 8)] == (4, True)
    assert got[(4096, 16, 16)] == (4, True)
    assert got[(4096, 16, 4)] == (4, True)
    assert _launcher_rw(503, 16, 8) == (1, False)


@pytest.mark.parametrize("S", [513, 4097])
def test_decode_equals_last_prefill_row(S):
    """A size-independent invariant at the decode target size: decode at position p attends
    the same keys [0, p] as the last row of a causal prefill ending at p, so the two kernels
    (split-K decode, MFMA prefill in fp32 mode) agree to the sum of their tolerances; each is
    also checked against the oracle's decode."""
    T, Hq, Hkv, Dh = 4, 16, 8, 128
    pos0 = S - T
    q, kc, vc = _layer_inputs(S, T, pos0)
    scale = 1.0 / math.sqrt(Dh)
    say("decode vs prefill last row", S)
    pre = _run(q, kc, vc, pos0, S, da.PREFILL_FP32, Hkv)[T - 1]
    dout = empty((Hq, Dh), np.float32)
    da.GqaDecodeAttn(up(np.ascontiguousarray(q[T - 1])), up(kc), up(vc), dout, Hq, Hkv, Dh,
                     up(np.array([S - 1], np.int32)), S, scale)
    dec = down(dout, (Hq, Dh))
    ref = orc.gqa_decode(q[T - 1], kc, vc, S - 1, scale)
    truth = t64.decode(q[T - 1], kc, vc, S - 1, scale)
    check_fp32(dec, ref, TOL32, truth=truth)
    check_fp32(pre, ref, TOL32, truth=truth)
    assert rel_err(pre, dec, FLOOR) <= 2 * TOL32


@pytest.mark.parametrize("T,Hq,Hkv,Dh,pos0", [(37, 12, 4, 80, 5), (20, 8, 1, 256, 0),
                                              (9, 6, 6, 48, 100), (33, 16, 8, 64, 0),
                                              (3, 2, 1, 1024, 7), (5, 3, 3, 1, 2)])
def test_prefill_generic_shapes(T, Hq, Hkv, Dh, pos0):
    """Head sizes and groups the MFMA kernels are not built for (the reference's kernel takes
    any Dh <= 256 and any group): Hq/Hkv 3 and 8, Dh 80 / 256 / 48 / 64 / 1024 / 1, a pos0
    offset -- the generic kernel, fp32 mode, against the oracle at the kernel gate."""
    r = SplitMix64(T * 31 + Dh)
    S = pos0 + T
    kc = orc.to_bf16(r.normal((S, Hkv, Dh)))
    vc = orc.to_bf16(r.normal((S, Hkv, Dh)))
    q = r.normal((T, Hq, Dh))
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_prefill(q, kc, vc, pos0, scale)
    say("prefill generic", T, Hq, Hkv, Dh, pos0)
    got = _run(q, kc, vc, pos0, S, da.PREFILL_FP32, Hkv)
    check_fp32(got, ref, TOL32, truth=t64.prefill(q, kc, vc, pos0, scale))


def test_prefill_generic_paged_and_bf16_mode():
    """The generic kernel through a page table (16-key pages, shuffled) and in bf16 mode with
    a bf16 q (the q_bf16 argument): Hq/Hkv = 3, Dh = 96."""
    T, Hq, Hkv, Dh, pos0, ps = 41, 6, 2, 96, 30, 16
    r = SplitMix64(4242)
    S = pos0 + T
    n_pages = (S + ps - 1) // ps + 2
    table = np.array(r.uniform(n_pages).argsort()[: (S + ps - 1) // ps], np.int32)
    kc = orc.to_bf16(r.normal((S, Hkv, Dh)))
    vc = orc.to_bf16(r.normal((S, Hkv, Dh)))
    kp = np.zeros((n_pages, ps, Hkv, Dh), np.uint16)
    vp = np.zeros_like(kp)
    for j in range(S):
        kp[table[j // ps], j % ps] = kc[j]
        vp[table[j // ps], j % ps] = vc[j]
    q = r.normal((T, Hq, Dh))
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_prefill(q, kc, vc, pos0, scale)
    say("prefill generic paged")
    got = _run(q, kc, vc, pos0, S, da.PREFILL_FP32, Hkv, page=(kp, vp, table, ps))
    check_fp32(got, ref, TOL32, truth=t64.prefill(q, kc, vc, pos0, scale))
    # bf16 mode with q given as bf16 bits: the generic kernel reads the rounded q
    qb = orc.to_bf16(q)
    ref_b = orc.gqa_prefill(orc.from_bf16(qb), kc, vc, pos0, scale)
    dout = empty(q.shape, np.float32)
    say("prefill generic bf16 q")
    da.GqaCacheAttnEx(None, up(qb), up(kc), up(vc), None, 0, 0, dout, T, Hq, Hkv, Dh,
                      up(np.array([pos0], np.int32)), S, scale, da.PREFILL_BF16)
    check_fp32(down(dout, q.shape), ref_b, TOL32,
               truth=t64.prefill(orc.from_bf16(qb), kc, vc, pos0, scale))
