"""GPU parity: split-K decode attention (contiguous and paged) and the KV write against the
oracle.  Bar: fp32 q / bf16 KV / fp32 accumulate, so the fp32-mode tolerance applies:
max |g - r| / max(|r|, 0.05) <= 1e-4 (0.05 = 5% of the unit-scale V), and bit-exact bf16
for the KV write."""
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

FLOOR = 0.05
TOL = 1e-4


def _contig_case(seed, S, cap, Hq=16, Hkv=8, Dh=128):
    r = SplitMix64(seed)
    k, v = r.normal((S, Hkv, Dh)), r.normal((S, Hkv, Dh))
    kc = np.zeros((cap, Hkv, Dh), np.uint16)
    vc = np.zeros_like(kc)
    orc.kv_write(k, v, kc, vc, 0)
    q = r.normal((Hq, Dh))
    return q, kc, vc


@pytest.mark.parametrize("S,cap", [(1, 64), (2, 64), (64, 64), (65, 128), (257, 512),
                                   (513, 2048), (2048, 2048), (3001, 4096), (4097, 4224)])
def test_decode_contiguous_matches_oracle(S, cap):
    Hq, Hkv, Dh = 16, 8, 128
    q, kc, vc = _contig_case(100 + S, S, cap)
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_decode(q, kc, vc, S - 1, scale)
    dq, dk, dv = up(q), up(kc), up(vc)
    dpos = up(np.array([S - 1], np.int32))
    dout = empty((Hq, Dh), np.float32)
    say("decode contiguous", S, cap)
    da.GqaDecodeAttn(dq, dk, dv, dout, Hq, Hkv, Dh, dpos, cap, scale)
    got = down(dout, (Hq, Dh))
    check_fp32(got, ref, TOL, truth=t64.decode(q, kc, vc, S - 1, scale))
    if S == 1:  # a single key: the output is v0 of the group's kv head
        np.testing.assert_allclose(got, np.repeat(orc.from_bf16(vc[0]), 2, axis=0), atol=1e-7)


@pytest.mark.parametrize("Hq,Hkv,Dh", [(8, 8, 128), (16, 4, 128), (8, 4, 64), (4, 4, 64)])
def test_decode_group_and_headdim_variants(Hq, Hkv, Dh):
    S, cap = 777, 1024
    q, kc, vc = _contig_case(7, S, cap, Hq, Hkv, Dh)
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_decode(q, kc, vc, S - 1, scale)
    dout = empty((Hq, Dh), np.float32)
    say("decode variant", Hq, Hkv, Dh)
    da.GqaDecodeAttn(up(q), up(kc), up(vc), dout, Hq, Hkv, Dh, up(np.array([S - 1], np.int32)),
                     cap, scale)
    check_fp32(down(dout, (Hq, Dh)), ref, TOL, truth=t64.decode(q, kc, vc, S - 1, scale))


def test_decode_back_to_back_calls_reuse_combine_state():
    """The split combine's counters must be left at zero: run several positions in a row
    on the same cache and check every result."""
    Hq, Hkv, Dh, cap = 16, 8, 128, 2048
    q, kc, vc = _contig_case(9, cap, cap)
    dq, dk, dv = up(q), up(kc), up(vc)
    dout = empty((Hq, Dh), np.float32)
    for pos in (2047, 100, 1500, 63, 2047):
        say("decode repeat", pos)
        da.GqaDecodeAttn(dq, dk, dv, dout, Hq, Hkv, Dh, up(np.array([pos], np.int32)), cap,
                         0.08838834764831845)
        ref = orc.gqa_decode(q, kc, vc, pos, 0.08838834764831845)
        check_fp32(down(dout, (Hq, Dh)), ref, TOL,
                   truth=t64.decode(q, kc, vc, pos, 0.08838834764831845))


@pytest.mark.parametrize("seq", [
    # (lens, Hq, Hkv, Dh): small grids merge their splits inside the split launch, counting
    # workgroups in per (stream, kv head); every launch must leave its counters at zero for
    # the next one, whatever its shape
    [([4097], 16, 8, 128), ([300, 1, 2500, 129, 4000], 16, 8, 128), ([4097], 16, 8, 128),
     ([2000, 700], 16, 4, 128), ([1500], 8, 8, 64), ([1025] * 3, 16, 8, 128),
     ([4097], 16, 8, 128)],
])
def test_decode_paged_in_launch_merge_back_to_back(seq):
    for i, (lens, Hq, Hkv, Dh) in enumerate(seq):
        ps = 16
        q, kp, vp, table, pos = _paged_case(500 + i, lens, Hq, Hkv, Dh, ps)
        B, max_pages = table.shape
        scale = 1.0 / math.sqrt(Dh)
        ref = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, scale, threads=8)
        dout = empty((B, Hq, Dh), np.float32)
        say("decode in-launch merge", i, lens, Hq, Hkv, Dh)
        da.GqaDecodeAttnPaged(up(q), up(kp), up(vp), up(table), max_pages, ps, up(pos), dout, B,
                              Hq, Hkv, Dh, scale)
        check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
                   truth=t64.decode_paged(q, kp, vp, table, ps, pos, scale))


def test_decode_position_past_capacity_is_clamped():
    Hq, Hkv, Dh, cap = 16, 8, 128, 256
    q, kc, vc = _contig_case(10, cap, cap)
    dout = empty((Hq, Dh), np.float32)
    say("decode clamp")
    da.GqaDecodeAttn(up(q), up(kc), up(vc), dout, Hq, Hkv, Dh, up(np.array([5000], np.int32)), cap,
                     0.1)
    ref = orc.gqa_decode(q, kc, vc, cap - 1, 0.1)
    check_fp32(down(dout, (Hq, Dh)), ref, TOL, truth=t64.decode(q, kc, vc, cap - 1, 0.1))


def _paged_case(seed, lens, Hq=16, Hkv=8, Dh=128, ps=16, spare_pages=3):
    r = SplitMix64(seed)
    B = len(lens)
    max_pages = max((n + ps - 1) // ps for n in lens)
    n_pages = B * max_pages + spare_pages
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    perm = np.array(r.uniform(n_pages).argsort(), np.int32)
    table = perm[:B * max_pages].reshape(B, max_pages).copy()
    q = r.normal((B, Hq, Dh))
    pos = np.array(lens, np.int32) - 1
    return q, kp, vp, table, pos


@pytest.mark.parametrize("lens", [[1], [4097], [1025, 2049, 17, 4097, 640, 1, 3333, 2000],
                                  [4096 + 1] * 16])
def test_decode_paged_ragged_streams(lens):
    Hq, Hkv, Dh, ps = 16, 8, 128, 16
    q, kp, vp, table, pos = _paged_case(sum(lens), lens)
    B, max_pages = table.shape
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, scale, threads=8)
    dout = empty((B, Hq, Dh), np.float32)
    say("decode paged", lens[:4], len(lens))
    da.GqaDecodeAttnPaged(up(q), up(kp), up(vp), up(table), max_pages, ps, up(pos), dout, B, Hq,
                          Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp, vp, table, ps, pos, scale))


@pytest.mark.parametrize("B,Hq,Hkv,Dh", [(16, 16, 8, 128), (32, 16, 8, 128), (16, 8, 8, 64)])
def test_decode_paged_wide_ranges(B, Hq, Hkv, Dh):
    """Many streams over long contexts take the wide split kernel (two 2080-key ranges per
    (stream, kv head) at 16 streams, one whole-context range at 32): ragged lengths around the
    range and chunk edges."""
    base = [2080, 2081, 2079, 4160, 1, 32, 33, 2112, 4097, 3000, 64, 4159, 2, 1500, 4128, 2047]
    lens = (base * 2)[:B]
    ps = 16
    q, kp, vp, table, pos = _paged_case(B * 7 + Dh, lens, Hq=Hq, Hkv=Hkv, Dh=Dh)
    B, max_pages = table.shape
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, scale, threads=8)
    dout = empty((B, Hq, Dh), np.float32)
    say("decode paged wide", B, Hq, Hkv, Dh)
    da.GqaDecodeAttnPaged(up(q), up(kp), up(vp), up(table), max_pages, ps, up(pos), dout, B, Hq,
                          Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp, vp, table, ps, pos, scale))


def test_decode_paged_wide_merge_three_and_four_ranges():
    """Wide-kernel grids of 4 ranges (8 streams) and 3 ranges (12 streams) per (stream, kv
    head), whose last range merges the others' partials inside the launch: streams ending in
    every range (1 .. 4 ranges used), each launch against the oracle, and the first case run
    again after the second (the pair blocks' partial words then hold two earlier launches')
    with bit-identical output."""
    Hq, Hkv, Dh, ps = 16, 8, 128, 16
    cases = [[8200, 6150, 4100, 2050, 1, 8192, 5000, 3000],
             [6000, 1, 1792, 1793, 3584, 3585, 5999, 100, 4000, 2500, 17, 5376]]
    outs = []
    for i, lens in enumerate(cases + cases[:1]):
        q, kp, vp, table, pos = _paged_case(900 + i % 2, lens, Hq, Hkv, Dh, ps)
        B, max_pages = table.shape
        scale = 1.0 / math.sqrt(Dh)
        dout = empty((B, Hq, Dh), np.float32)
        say("decode wide merge", i, B, max_pages * ps)
        da.GqaDecodeAttnPaged(up(q), up(kp), up(vp), up(table), max_pages, ps, up(pos), dout, B,
                              Hq, Hkv, Dh, scale)
        got = down(dout, (B, Hq, Dh))
        outs.append(got)
        if i < 2:
            ref = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, scale, threads=8)
            check_fp32(got, ref, TOL, truth=t64.decode_paged(q, kp, vp, table, ps, pos, scale))
    np.testing.assert_array_equal(outs[2], outs[0])


def test_decode_paged_equals_contiguous_for_identity_table():
    Hq, Hkv, Dh, ps, S = 16, 8, 128, 16, 1000
    q, kc, vc = _contig_case(12, S, 1024)
    table = np.arange(1024 // ps, dtype=np.int32)[None, :]
    dpos = up(np.array([S - 1], np.int32))
    o1, o2 = empty((Hq, Dh), np.float32), empty((Hq, Dh), np.float32)
    dq, dk, dv = up(q), up(kc), up(vc)
    say("decode paged identity")
    da.GqaDecodeAttn(dq, dk, dv, o1, Hq, Hkv, Dh, dpos, 1024, 0.1)
    da.GqaDecodeAttnPaged(dq, dk, dv, up(table), table.shape[1], ps, dpos, o2, 1, Hq, Hkv, Dh, 0.1)
    np.testing.assert_array_equal(down(o1, (Hq, Dh)), down(o2, (Hq, Dh)))


def test_kv_write_bit_exact():
    r = SplitMix64(13)
    Tq, Hkv, Dh, cap, pos0 = 7, 8, 128, 32, 20
    k, v = r.normal((Tq, Hkv, Dh)), r.normal((Tq, Hkv, Dh))
    kc = np.zeros((cap, Hkv, Dh), np.uint16)
    vc = np.zeros_like(kc)
    orc.kv_write(k[:cap - pos0], v[:cap - pos0], kc, vc, pos0)  # rows past capacity dropped
    dkc, dvc = up(np.zeros_like(kc)), up(np.zeros_like(vc))
    say("kv_write")
    da.WriteKvCache(up(k), up(v), dkc, dvc, Tq, Hkv, Dh, up(np.array([pos0], np.int32)), cap)
    np.testing.assert_array_equal(down(dkc, kc.shape, np.uint16), kc)
    np.testing.assert_array_equal(down(dvc, vc.shape, np.uint16), vc)


def test_kv_write_paged_bit_exact():
    r = SplitMix64(14)
    B, Tq, Hkv, Dh, ps, max_pages = 3, 5, 8, 128, 16, 4
    n_pages = B * max_pages
    table = np.array(r.uniform(n_pages).argsort(), np.int32).reshape(B, max_pages)
    pos0 = np.array([0, 14, 59], np.int32)
    k, v = r.normal((B, Tq, Hkv, Dh)), r.normal((B, Tq, Hkv, Dh))
    kp = np.zeros((n_pages, ps, Hkv, Dh), np.uint16)
    vp = np.zeros_like(kp)
    for b in range(B):
        n = min(Tq, max_pages * ps - int(pos0[b]))
        orc.kv_write_paged(k[b, :n], v[b, :n], kp, vp, table[b], ps, int(pos0[b]))
    dkp, dvp = up(np.zeros_like(kp)), up(np.zeros_like(vp))
    say("kv_write_paged")
    da.WriteKvCachePaged(up(k), up(v), dkp, dvp, up(table), max_pages, ps, n_pages, B, Tq, Hkv, Dh,
                         up(pos0))
    np.testing.assert_array_equal(down(dkp, kp.shape, np.uint16), kp)
    np.testing.assert_array_equal(down(dvp, vp.shape, np.uint16), vp)


@pytest.mark.parametrize("ps", [32, 64, 256])
def test_decode_paged_page_sizes(ps):
    """Pages of 32, 64 and 256 keys (every power of two >= 16 is accepted): ragged streams
    through random page tables, against the oracle."""
    Hq, Hkv, Dh = 16, 8, 128
    lens = [17, 1000, 2049, 4097]
    q, kp, vp, table, pos = _paged_case(ps + 5, lens, ps=ps)
    B, max_pages = table.shape
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, scale, threads=8)
    dout = empty((B, Hq, Dh), np.float32)
    say("decode paged page size", ps)
    da.GqaDecodeAttnPaged(up(q), up(kp), up(vp), up(table), max_pages, ps, up(pos), dout, B, Hq,
                          Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp, vp, table, ps, pos, scale))


def test_decode_contiguous_16k_context():
    """A 16384-key context (128 splits, 8 merge batches): against the oracle."""
    Hq, Hkv, Dh, S = 16, 8, 128, 16384
    q, kc, vc = _contig_case(16384, S, S)
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_decode(q, kc, vc, S - 1, scale)
    dout = empty((Hq, Dh), np.float32)
    say("decode 16k")
    da.GqaDecodeAttn(up(q), up(kc), up(vc), dout, Hq, Hkv, Dh, up(np.array([S - 1], np.int32)), S,
                     scale)
    check_fp32(down(dout, (Hq, Dh)), ref, TOL, truth=t64.decode(q, kc, vc, S - 1, scale))


@pytest.mark.parametrize("Hq,Hkv,Dh,S,cap", [(12, 4, 80, 701, 1024), (8, 1, 256, 33, 64),
                                             (3, 3, 1024, 130, 256), (16, 2, 48, 2049, 2100)])
def test_decode_generic_shapes(Hq, Hkv, Dh, S, cap):
    """GqaDecodeAttnKernel takes any Dh and group (blockDim = Dh): the shapes the split-K
    kernels are not built for run on the generic kernel, contiguous cache, against the oracle."""
    q, kc, vc = _contig_case(S * 7 + Dh, S, cap, Hq, Hkv, Dh)
    dout = empty((Hq, Dh), np.float32)
    scale = 1.0 / math.sqrt(Dh)
    say("decode generic", Hq, Hkv, Dh, S)
    da.GqaDecodeAttn(up(q), up(kc), up(vc), dout, Hq, Hkv, Dh, up(np.array([S - 1], np.int32)),
                     cap, scale)
    ref = orc.gqa_decode(q, kc, vc, S - 1, scale)
    check_fp32(down(dout, (Hq, Dh)), ref, TOL, truth=t64.decode(q, kc, vc, S - 1, scale))


def test_decode_paged_generic_shapes():
    """Paged batched decode with group 3 and Dh 72 (generic kernel): ragged streams."""
    Hq, Hkv, Dh, ps = 9, 3, 72, 16
    lens = [1, 16, 17, 500, 1024, 77]
    q, kp, vp, table, pos = _paged_case(77, lens, Hq=Hq, Hkv=Hkv, Dh=Dh, ps=ps)
    B, max_pages = table.shape
    scale = 1.0 / math.sqrt(Dh)
    ref = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, scale, threads=8)
    dout = empty((B, Hq, Dh), np.float32)
    say("decode paged generic")
    da.GqaDecodeAttnPaged(up(q), up(kp), up(vp), up(table), max_pages, ps, up(pos), dout, B, Hq,
                          Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp, vp, table, ps, pos, scale))
