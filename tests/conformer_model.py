"""Seeded synthetic weights of one FastConformer layer for the Conformer tests."""
from __future__ import annotations

import math

import numpy as np

import oracle_lib as orc


def conformer_weights(r, D, H, Dff, K):
    """Random fp32 weights of one ConformerLayer, keyed by OratorConformerWeights field."""
    Dk = D // H
    W = {}
    lin = lambda n_out, n_in: r.normal((n_out, n_in), 1.0 / math.sqrt(n_in))
    for p in ("ff1", "ff2"):
        W[f"norm_{p}_w"], W[f"norm_{p}_b"] = 1 + r.normal(D, 0.1), r.normal(D, 0.1)
        W[f"{p}_w1"], W[f"{p}_b1"] = lin(Dff, D), r.normal(Dff, 0.1)
        W[f"{p}_w2"], W[f"{p}_b2"] = lin(D, Dff), r.normal(D, 0.1)
    for n in ("att", "conv", "out"):
        W[f"norm_{n}_w"], W[f"norm_{n}_b"] = 1 + r.normal(D, 0.1), r.normal(D, 0.1)
    for n in ("q", "k", "v", "out"):
        W[f"{n}_w"], W[f"{n}_b"] = lin(D, D), r.normal(D, 0.1)
    W["pos_w"] = lin(D, D)
    W["pos_bias_u"], W["pos_bias_v"] = r.normal((H, Dk), 0.1), r.normal((H, Dk), 0.1)
    W["pw1_w"], W["pw1_b"] = lin(2 * D, D), r.normal(2 * D, 0.1)
    W["dw_w"], W["dw_b"] = r.normal((D, K), 1.0 / math.sqrt(K)), r.normal(D, 0.1)
    W["bn_w"], W["bn_b"] = 1 + r.normal(D, 0.1), r.normal(D, 0.1)
    W["bn_mean"], W["bn_var"] = r.normal(D, 0.1), (0.5 + r.uniform(D)).astype(np.float32)
    W["pw2_w"], W["pw2_b"] = lin(D, D), r.normal(D, 0.1)
    assert set(W) == set(orc.CONFORMER_FIELDS)
    return {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in W.items()}
