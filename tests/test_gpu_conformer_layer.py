"""GPU parity: one FastConformer layer (ConformerLayer::Forward, src/model/conformer_layer.cu:
364-488) against the oracle composition on the same seeded weights and inputs.
Bars (max |g - r| / max(|r|, 0.05)): 2e-4 with the fp32 attention core (every pass fp32, ten
GEMMs in another accumulation order, renormalised by five LayerNorms); 1e-2 with the fused
fp16 core (fp16 operands, ~1e-3 on the core's unit-scale output, carried through linear_out,
the conv module and FFN2 into the final LayerNorm: 7.3e-3 measured at T = 128)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as orc
from conformer_model import conformer_weights
from gpu_helpers import down, say, up
from helpers import SplitMix64, rel_err
from orator_amd.conformer_attn import ConformerLayer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,valid,mode,tol", [(1, 1, 0, 2e-4), (23, 20, 0, 2e-4),
                                               (340, 340, 0, 2e-4), (717, 529, 0, 2e-4),
                                               (717, 529, 1, 1e-2), (128, 100, 1, 1e-2)])
def test_conformer_layer_vs_oracle(T, valid, mode, tol):
    D, H, Dff, K = 512, 8, 2048, 9
    r = SplitMix64(T + 7 * mode)
    W = conformer_weights(r, D, H, Dff, K)
    x = r.normal((T, D))
    pe = orc.build_pos_emb(T, D)
    ref = orc.conformer_layer(x, T, valid, pe, W, H)
    dW = {k: up(v) for k, v in W.items()}
    layer = ConformerLayer(dW, D, H, Dff, K)
    dx = up(x)
    say("conformer layer", T, valid, mode)
    layer.Forward(dx, T, valid, up(pe), attn_mode=mode)
    got = down(dx, (T, D))
    layer.close()
    assert rel_err(got, ref, 0.05) <= tol
