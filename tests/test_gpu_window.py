"""GPU parity: the audio tower's windowed self-attention (WindowAttnKernel,
src/model/asr_audio_tower.cu:204-258) against the oracle on the same seeded inputs.
Bar: max |g - r| / max(|r|, 0.05) <= 1e-4 (fp32 throughout)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as orc
import truth64 as t64
from gpu_helpers import down, empty, say, up
from helpers import SplitMix64, check_fp32, rel_err
from orator_amd.audio_attn import WindowAttention

pytestmark = pytest.mark.gpu

FLOOR, TOL = 0.05, 1e-4


def windows(N, width):
    ss, se = np.zeros(N, np.int32), np.zeros(N, np.int32)
    for s0 in range(0, N, width):
        ss[s0:s0 + width], se[s0:s0 + width] = s0, min(N, s0 + width)
    return ss, se


@pytest.mark.parametrize("N,H,Dh,kind", [(1, 16, 64, "full"), (37, 16, 64, "full"),
                                          (390, 16, 64, "full"), (390, 16, 64, "w104"),
                                          (1500, 16, 64, "w104"), (300, 8, 128, "ragged"),
                                          (300, 8, 64, "ragged"), (150, 4, 64, "clamp"),
                                          (257, 16, 64, "empty"),
                                          # head sizes of the generic kernel
                                          (200, 4, 32, "ragged"), (210, 2, 80, "w104")])
def test_window_attention_vs_oracle(N, H, Dh, kind):
    r = SplitMix64(N * 3 + H + Dh)
    q, k, v = r.normal((N, H, Dh)), r.normal((N, H, Dh)), r.normal((N, H, Dh))
    if kind == "full":
        ss, se = np.zeros(N, np.int32), np.full(N, N, np.int32)
    elif kind == "w104":  # the trained windowing: 13 tokens x 8 chunks
        ss, se = windows(N, 104)
    elif kind == "ragged":  # arbitrary per-query ranges
        a = (r.uniform(N) * N).astype(np.int32)
        b = (r.uniform(N) * N).astype(np.int32)
        ss, se = np.minimum(a, b), np.maximum(a, b) + 1
    elif kind == "clamp":  # ranges reaching outside [0, N) are clamped into it
        ss = (r.uniform(N) * 2 * N).astype(np.int32) - N
        se = ss + (r.uniform(N) * 2 * N).astype(np.int32)
    else:  # every 7th query has an empty window
        ss, se = windows(N, 50)
        se[::7] = ss[::7]
    scale = 1.0 / np.sqrt(Dh)
    # the device clamps each range into [0, N) (the reference reads outside it); the oracle
    # gets the clamped ranges
    cs = np.clip(ss, 0, N).astype(np.int32)
    ref = orc.window_attention(q, k, v, cs, np.clip(se, cs, N).astype(np.int32), scale)
    out = empty((N, H, Dh), np.float32)
    say("window attention", N, H, Dh, kind)
    WindowAttention(up(q), up(k), up(v), out, up(ss), up(se), N, H, Dh, scale)
    got = down(out, (N, H, Dh))
    check_fp32(got, ref, TOL,
               truth=t64.attention_ranges(q, k, v, scale, cs, np.clip(se, cs, N)))
    if kind == "empty":
        assert np.all(got[::7] == 0)
