"""GPU parity: the Sortformer decoder's masked self-attention (src/model/sortformer_decoder.cu:
280-298) against the oracle's restatement of the reference decomposition.
Bar: max |g - r| / max(|r|, 0.05) <= 1e-4 (fp32; the reference's __expf and this kernel's
online softmax both sit well inside it)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle_lib as orc
import truth64 as t64
from gpu_helpers import down, empty, say, up
from helpers import SplitMix64, check_fp32, rel_err
from orator_amd.sortformer_attn import MaskedSelfAttention

pytestmark = pytest.mark.gpu

FLOOR, TOL = 0.05, 1e-4


@pytest.mark.parametrize("T,H,Dk,valid", [(1, 8, 24, 1), (7, 8, 24, 7), (65, 8, 24, 50),
                                           (717, 8, 24, 717), (717, 8, 24, 600),
                                           (376, 8, 24, 0), (300, 4, 32, 299),
                                           (200, 8, 64, 1000), (1024, 1, 24, 1000),
                                           (2000, 1, 32, 0)])
def test_masked_mha_vs_oracle(T, H, Dk, valid):
    r = SplitMix64(T * 11 + Dk + valid)
    q, k, v = r.normal((T, H, Dk)), r.normal((T, H, Dk)), r.normal((T, H, Dk))
    scale = 1.0 / math.sqrt(Dk)
    ref = orc.masked_mha(q, k, v, valid, scale)
    out = empty((T, H, Dk), np.float32)
    say("masked mha", T, H, Dk, valid)
    MaskedSelfAttention(up(q), up(k), up(v), out, T, H, Dk, valid, scale)
    truth = (np.broadcast_to(v.astype(np.float64).mean(0), v.shape) if valid <= 0 else
             t64.attention_ranges(q, k, v, scale, 0, min(valid, T)))
    check_fp32(down(out, (T, H, Dk)), ref, TOL, truth=truth)
