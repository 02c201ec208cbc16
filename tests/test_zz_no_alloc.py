"""GPU: the allocation-free decode entry point (orator_gqa_decode_paged_noalloc, split partials
in a static device array) against orator_gqa_decode_paged on the same inputs, through the C
ABI: three calls in a row, each smaller than the one before, outputs bit-identical (same
kernels, same split plan) and within 1e-4 relative (floor 0.05) of the oracle; the no-alloc entry runs first, on a
fresh stream, and the library's workspace holds exactly the blocks and bytes it held before it
(so it cannot have been served from a block an earlier allocating call left behind); sizes past
the static scratch are rejected on the host with ORATOR_ERR_CAPACITY."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle_lib as orc
from gpu_helpers import down, empty, say, up
from helpers import SplitMix64, rel_err
from orator_amd import _lib
from orator_amd import decoder_attn as da
from orator_amd.runtime import Stream, workspace_stats

pytestmark = pytest.mark.gpu


def _case(seed, lens, Hq=16, Hkv=8, Dh=128, ps=16):
    r = SplitMix64(seed)
    B = len(lens)
    max_pages = max((n + ps - 1) // ps for n in lens)
    n_pages = B * max_pages
    kp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((n_pages, ps, Hkv, Dh)))
    table = np.array(r.uniform(n_pages).argsort(), np.int32).reshape(B, max_pages)
    q = r.normal((B, Hq, Dh))
    pos = np.array(lens, np.int32) - 1
    return q, kp, vp, table, max_pages, ps, pos


def test_noalloc_matches_allocating_entry_twice():
    Hq, Hkv, Dh = 16, 8, 128
    scale = 1.0 / math.sqrt(Dh)
    # second call smaller (fewer streams, shorter contexts): stale partials of the first call
    # stay in the scratch and must not leak into it
    # (the smaller calls are small grids: their splits are merged inside the split launch,
    # with arrival counters in the scratch's last 512 KiB, one per 128-byte line, left at zero
    # by every launch)
    for seed, lens in ((1, [4097 + i for i in range(16)]), (2, [700, 1, 129]), (3, [2000])):
        q, kp, vp, table, max_pages, ps, pos = _case(seed, lens)
        B = len(lens)
        dq, dk, dv, dt, dpos = up(q), up(kp), up(vp), up(table), up(pos)
        o_ref, o_na = empty((B, Hq, Dh), np.float32), empty((B, Hq, Dh), np.float32)
        st = Stream()  # fresh: no workspace block exists for it yet
        say("noalloc first, on a fresh stream", seed, B, max(lens))
        before = workspace_stats()
        da.GqaDecodeAttnPagedNoAlloc(dq, dk, dv, dt, max_pages, ps, dpos, o_na, B, Hq, Hkv, Dh,
                                     scale, st)
        st.synchronize()
        assert workspace_stats() == before, (before, workspace_stats())
        say("paged (allocating) on the same stream", seed)
        da.GqaDecodeAttnPaged(dq, dk, dv, dt, max_pages, ps, dpos, o_ref, B, Hq, Hkv, Dh, scale,
                              st)
        st.synchronize()
        got, ref = down(o_na, (B, Hq, Dh)), down(o_ref, (B, Hq, Dh))
        st.close()
        np.testing.assert_array_equal(got, ref)
        truth = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, scale, threads=8)
        assert rel_err(got, truth, 0.05) <= 1e-4


def test_noalloc_rejects_sizes_past_the_scratch():
    say("noalloc capacity check (host only)")
    # B = 16, Hq = 16, Dh = 128 at 16384 keys needs 17 MB of partials (> 16 MiB): rejected
    # before any launch
    with pytest.raises(_lib.GpuError) as e:
        da.GqaDecodeAttnPagedNoAlloc(None, None, None, 1, 1024, 16, None, None, 16, 16, 8, 128,
                                     0.1)
    assert e.value.code == _lib.ORATOR_ERR_CAPACITY
