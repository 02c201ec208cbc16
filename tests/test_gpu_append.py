"""GPU parity: decode with the new token appended in the same launch (WriteKvCacheKernel +
GqaDecodeAttnKernel of one decode step, src/model/asr_text_decoder.cu:412-418).

The oracle runs the two reference steps in order: the bf16 KV write of the new rows, then the
decode over pos + 1 keys.  Bar: attention outputs max |g - r| / max(|r|, 0.05) <= 1e-4 (fp32
q, bf16 KV, fp32 accumulation); the written cache rows bit-exact, every other row untouched."""
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

FLOOR, TOL = 0.05, 1e-4


@pytest.mark.parametrize("pos,cap", [(0, 64), (1, 64), (31, 64), (32, 64), (63, 64), (256, 512),
                                     (300, 512), (4096, 4224), (4223, 4224)])
def test_append_contiguous_matches_write_then_decode(pos, cap):
    Hq, Hkv, Dh = 16, 8, 128
    r = SplitMix64(pos * 7 + cap)
    kc = orc.to_bf16(r.normal((cap, Hkv, Dh)))
    vc = orc.to_bf16(r.normal((cap, Hkv, Dh)))
    q, kn, vn = r.normal((Hq, Dh)), r.normal((Hkv, Dh)), r.normal((Hkv, Dh))
    scale = 1.0 / math.sqrt(Dh)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    orc.kv_write(kn[None], vn[None], kc_ref, vc_ref, pos)
    ref = orc.gqa_decode(q, kc_ref, vc_ref, pos, scale)
    dk, dv = up(kc), up(vc)
    dout = empty((Hq, Dh), np.float32)
    say("append contiguous", pos, cap)
    da.GqaDecodeAttnAppend(up(q), up(kn), up(vn), dk, dv, dout, Hq, Hkv, Dh,
                           up(np.array([pos], np.int32)), cap, scale)
    check_fp32(down(dout, (Hq, Dh)), ref, TOL, truth=t64.decode(q, kc_ref, vc_ref, pos, scale))
    np.testing.assert_array_equal(down(dk, kc.shape, np.uint16), kc_ref)
    np.testing.assert_array_equal(down(dv, vc.shape, np.uint16), vc_ref)


def test_append_past_capacity_is_dropped_and_clamped():
    """pos >= capacity: nothing is written and the capacity keys are attended, as the KV
    write (rows past the capacity dropped) followed by the clamped decode."""
    Hq, Hkv, Dh, cap = 16, 8, 128, 96
    r = SplitMix64(5)
    kc = orc.to_bf16(r.normal((cap, Hkv, Dh)))
    vc = orc.to_bf16(r.normal((cap, Hkv, Dh)))
    q, kn, vn = r.normal((Hq, Dh)), r.normal((Hkv, Dh)), r.normal((Hkv, Dh))
    ref = orc.gqa_decode(q, kc, vc, cap - 1, 0.1)
    dk, dv = up(kc), up(vc)
    dout = empty((Hq, Dh), np.float32)
    say("append past capacity")
    da.GqaDecodeAttnAppend(up(q), up(kn), up(vn), dk, dv, dout, Hq, Hkv, Dh,
                           up(np.array([cap + 5], np.int32)), cap, 0.1)
    check_fp32(down(dout, (Hq, Dh)), ref, TOL, truth=t64.decode(q, kc, vc, cap - 1, 0.1))
    np.testing.assert_array_equal(down(dk, kc.shape, np.uint16), kc)
    np.testing.assert_array_equal(down(dv, vc.shape, np.uint16), vc)


@pytest.mark.parametrize("lens", [[1], [1025, 2049, 17, 4097, 640, 1, 3333, 2000],
                                  [4097 + i for i in range(16)]])
def test_append_paged_ragged_streams(lens):
    """lens[b] = keys after the append (pos = lens[b] - 1); random page tables over a pool with
    spare pages."""
    Hq, Hkv, Dh, ps = 16, 8, 128, 16
    r = SplitMix64(sum(lens) + 3)
    B = len(lens)
    max_pages = max((n + ps - 1) // ps for n in lens)
    n_pages = B * max_pages + 3
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    table = np.array(r.uniform(n_pages).argsort(), np.int32)[:B * max_pages].reshape(B, max_pages)
    q, kn, vn = r.normal((B, Hq, Dh)), r.normal((B, Hkv, Dh)), r.normal((B, Hkv, Dh))
    pos = np.array(lens, np.int32) - 1
    scale = 1.0 / math.sqrt(Dh)
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for b in range(B):
        orc.kv_write_paged(kn[b][None], vn[b][None], kp_ref, vp_ref, table[b], ps, int(pos[b]))
    ref = orc.gqa_decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale, threads=8)
    dk, dv = up(kp), up(vp)
    dout = empty((B, Hq, Dh), np.float32)
    say("append paged", lens[:4], B)
    da.GqaDecodeAttnAppendPaged(up(q), up(kn), up(vn), dk, dv, up(table), max_pages, ps, n_pages,
                                up(pos), dout, B, Hq, Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale))
    np.testing.assert_array_equal(down(dk, kp.shape, np.uint16), kp_ref)
    np.testing.assert_array_equal(down(dv, vp.shape, np.uint16), vp_ref)


# The wide split kernel (many streams and long contexts: each (stream, kv head) cut into two
# ranges of 2080 keys at this capacity, 8 waves striding over 32-key chunks): appended keys at
# the range boundary (lens 2080 / 2081: the new key is the last key of range 0 / the only key
# of range 1), at chunk edges (32, 33, 2112), at the capacity (4160), and one-key streams.
WIDE_LENS = [2080, 2081, 2079, 4160, 1, 32, 33, 2112, 4097, 3000, 64, 4159, 2, 1500, 4128, 2047]


@pytest.mark.parametrize("Hq,Hkv,Dh", [(16, 8, 128), (8, 8, 128), (16, 8, 64)])
def test_append_paged_wide_ranges(Hq, Hkv, Dh):
    ps = 16
    lens = WIDE_LENS
    r = SplitMix64(Hq * 100 + Dh)
    B = len(lens)
    max_pages = max((n + ps - 1) // ps for n in lens)
    n_pages = B * max_pages + 2
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    table = np.array(r.uniform(n_pages).argsort(), np.int32)[:B * max_pages].reshape(B, max_pages)
    q, kn, vn = r.normal((B, Hq, Dh)), r.normal((B, Hkv, Dh)), r.normal((B, Hkv, Dh))
    pos = np.array(lens, np.int32) - 1
    scale = 1.0 / math.sqrt(Dh)
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for b in range(B):
        orc.kv_write_paged(kn[b][None], vn[b][None], kp_ref, vp_ref, table[b], ps, int(pos[b]))
    ref = orc.gqa_decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale, threads=8)
    dk, dv = up(kp), up(vp)
    dout = empty((B, Hq, Dh), np.float32)
    say("append paged wide", Hq, Hkv, Dh)
    da.GqaDecodeAttnAppendPaged(up(q), up(kn), up(vn), dk, dv, up(table), max_pages, ps, n_pages,
                                up(pos), dout, B, Hq, Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale))
    np.testing.assert_array_equal(down(dk, kp.shape, np.uint16), kp_ref)
    np.testing.assert_array_equal(down(dv, vp.shape, np.uint16), vp_ref)


def test_append_equals_write_then_decode_on_device():
    """Same inputs through orator_kv_write_paged + orator_gqa_decode_paged: same cache bits,
    outputs equal to fp32 rounding (the appended key is folded in last)."""
    Hq, Hkv, Dh, ps, B, L = 16, 8, 128, 16, 4, 2500
    r = SplitMix64(99)
    max_pages = (L + 1 + ps - 1) // ps
    n_pages = B * max_pages
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    table = np.array(r.uniform(n_pages).argsort(), np.int32).reshape(B, max_pages)
    q, kn, vn = r.normal((B, Hq, Dh)), r.normal((B, Hkv, Dh)), r.normal((B, Hkv, Dh))
    pos = np.array([L, L - 7, 100, 0], np.int32)
    dq, dkn, dvn, dt, dpos = up(q), up(kn), up(vn), up(table), up(pos)
    k1, v1, k2, v2 = up(kp), up(vp), up(kp), up(vp)
    o1, o2 = empty((B, Hq, Dh), np.float32), empty((B, Hq, Dh), np.float32)
    say("append vs two launches")
    da.WriteKvCachePaged(dkn, dvn, k1, v1, dt, max_pages, ps, n_pages, B, 1, Hkv, Dh, dpos)
    da.GqaDecodeAttnPaged(dq, k1, v1, dt, max_pages, ps, dpos, o1, B, Hq, Hkv, Dh, 0.09)
    da.GqaDecodeAttnAppendPaged(dq, dkn, dvn, k2, v2, dt, max_pages, ps, n_pages, dpos, o2, B, Hq,
                                Hkv, Dh, 0.09)
    np.testing.assert_array_equal(down(k1, kp.shape, np.uint16), down(k2, kp.shape, np.uint16))
    np.testing.assert_array_equal(down(v1, vp.shape, np.uint16), down(v2, vp.shape, np.uint16))
    assert rel_err(down(o2, (B, Hq, Dh)), down(o1, (B, Hq, Dh)), FLOOR) <= 2e-6


@pytest.mark.parametrize("bad", ["unmapped", "past_pool"])
def test_append_paged_unmapped_page_is_not_written(bad):
    """The appended position's page-table entry is -1 (unmapped) or names a page past the pool:
    the new row is not written anywhere (every pool byte unchanged), and it is still attended.
    Reference: the row is attended from a spare page the oracle maps in its place."""
    Hq, Hkv, Dh, ps = 16, 8, 128, 16
    r = SplitMix64(7 if bad == "unmapped" else 8)
    # each new row is the first of its page (2, 3, 256, 0): earlier positions stay mapped
    pos = np.array([32, 48, 4096, 0], np.int32)
    B = len(pos)
    max_pages = int(pos.max()) // ps + 1
    n_pages = B * max_pages
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    table = np.array(r.uniform(n_pages).argsort(), np.int32).reshape(B, max_pages)
    bad_entry = -1 if bad == "unmapped" else n_pages + 5
    ref_table = table.copy()
    for b in range(B):
        table[b, pos[b] // ps] = bad_entry
    q, kn, vn = r.normal((B, Hq, Dh)), r.normal((B, Hkv, Dh)), r.normal((B, Hkv, Dh))
    scale = 1.0 / math.sqrt(Dh)
    # oracle: the original (mapped) table; the pages it writes are the ones the device skips
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for b in range(B):
        orc.kv_write_paged(kn[b][None], vn[b][None], kp_ref, vp_ref, ref_table[b], ps, int(pos[b]))
    ref = orc.gqa_decode_paged(q, kp_ref, vp_ref, ref_table, ps, pos, scale, threads=8)
    dk, dv = up(kp), up(vp)
    dout = empty((B, Hq, Dh), np.float32)
    say("append paged, appended page", bad)
    da.GqaDecodeAttnAppendPaged(up(q), up(kn), up(vn), dk, dv, up(table), max_pages, ps, n_pages,
                                up(pos), dout, B, Hq, Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp_ref, vp_ref, ref_table, ps, pos, scale))
    np.testing.assert_array_equal(down(dk, kp.shape, np.uint16), kp)
    np.testing.assert_array_equal(down(dv, vp.shape, np.uint16), vp)


@pytest.mark.parametrize("ps", [32, 128])
def test_append_paged_page_sizes(ps):
    """Pages of 32 and 128 keys: the appended row lands in the right page and offset, and the
    output matches the oracle's write-then-decode."""
    Hq, Hkv, Dh = 16, 8, 128
    lens = [1, ps, ps + 1, 2000, 4097]
    r = SplitMix64(ps + 11)
    B = len(lens)
    max_pages = max((n + ps - 1) // ps for n in lens)
    n_pages = B * max_pages + 2
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    table = np.array(r.uniform(n_pages).argsort(), np.int32)[:B * max_pages].reshape(B, max_pages)
    q, kn, vn = r.normal((B, Hq, Dh)), r.normal((B, Hkv, Dh)), r.normal((B, Hkv, Dh))
    pos = np.array(lens, np.int32) - 1
    scale = 1.0 / math.sqrt(Dh)
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for b in range(B):
        orc.kv_write_paged(kn[b][None], vn[b][None], kp_ref, vp_ref, table[b], ps, int(pos[b]))
    ref = orc.gqa_decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale, threads=8)
    dk, dv = up(kp), up(vp)
    dout = empty((B, Hq, Dh), np.float32)
    say("append paged page size", ps)
    da.GqaDecodeAttnAppendPaged(up(q), up(kn), up(vn), dk, dv, up(table), max_pages, ps, n_pages,
                                up(pos), dout, B, Hq, Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale))
    np.testing.assert_array_equal(down(dk, kp.shape, np.uint16), kp_ref)
    np.testing.assert_array_equal(down(dv, vp.shape, np.uint16), vp_ref)


@pytest.mark.parametrize("Hq,Hkv,Dh", [(12, 4, 96), (8, 1, 256), (6, 6, 40)])
def test_append_paged_generic_shapes(Hq, Hkv, Dh):
    """Head sizes and groups the split-K kernels are not built for (GQA group 3 and 8, Dh 96 /
    256 / 40) on the generic path: attention with the appended key read from the fp32 rows
    (bf16-rounded), then the rows written to the cache; ragged streams, a page beyond the
    pool (not written, still attended as the fused kernels do)."""
    ps = 16
    lens = [1, 300, 1025, 17]
    r = SplitMix64(Hq * 1000 + Dh)
    B = len(lens)
    max_pages = max((n + ps - 1) // ps for n in lens)
    n_pages = B * max_pages + 2
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    table = np.array(r.uniform(n_pages).argsort(), np.int32)[:B * max_pages].reshape(B, max_pages)
    q, kn, vn = r.normal((B, Hq, Dh)), r.normal((B, Hkv, Dh)), r.normal((B, Hkv, Dh))
    pos = np.array(lens, np.int32) - 1
    scale = 1.0 / math.sqrt(Dh)
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for b in range(B):
        orc.kv_write_paged(kn[b][None], vn[b][None], kp_ref, vp_ref, table[b], ps, int(pos[b]))
    ref = orc.gqa_decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale, threads=8)
    dk, dv = up(kp), up(vp)
    dout = empty((B, Hq, Dh), np.float32)
    say("append paged generic", Hq, Hkv, Dh)
    da.GqaDecodeAttnAppendPaged(up(q), up(kn), up(vn), dk, dv, up(table), max_pages, ps, n_pages,
                                up(pos), dout, B, Hq, Hkv, Dh, scale)
    check_fp32(down(dout, (B, Hq, Dh)), ref, TOL,
               truth=t64.decode_paged(q, kp_ref, vp_ref, table, ps, pos, scale))
    np.testing.assert_array_equal(down(dk, kp.shape, np.uint16), kp_ref)
    np.testing.assert_array_equal(down(dv, vp.shape, np.uint16), vp_ref)
    # a new row whose page lies past the pool: attended from the rows, not written
    table2 = table.copy()
    table2[3, (lens[3] - 1) // ps] = n_pages + 5
    kp2 = kp_ref.copy()
    kp2[table[3, (lens[3] - 1) // ps], (lens[3] - 1) % ps] = orc.to_bf16(kn[3])
    vp2 = vp_ref.copy()
    vp2[table[3, (lens[3] - 1) // ps], (lens[3] - 1) % ps] = orc.to_bf16(vn[3])
    ref2 = orc.gqa_decode_paged(q[3:4], kp2, vp2, table[3:4], ps, pos[3:4], scale)
    dk2, dv2 = up(kp_ref), up(vp_ref)
    dout2 = empty((1, Hq, Dh), np.float32)
    say("append paged generic, page past the pool")
    da.GqaDecodeAttnAppendPaged(up(q[3:4]), up(kn[3:4]), up(vn[3:4]), dk2, dv2, up(table2[3:4]),
                                max_pages, ps, n_pages, up(pos[3:4]), dout2, 1, Hq, Hkv, Dh, scale)
    check_fp32(down(dout2, (1, Hq, Dh)), ref2, TOL,
               truth=t64.decode_paged(q[3:4], kp2, vp2, table[3:4], ps, pos[3:4], scale))
    np.testing.assert_array_equal(down(dk2, kp.shape, np.uint16), kp_ref)
