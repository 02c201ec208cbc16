"""Rounding model of the fused fp16 rel-pos core (orator_relpos_attention_fast), for deriving
its parity bars before any device result is seen: the kernel's operand roundings applied to
an fp64 evaluation of the reference formula (src/model/conformer_layer.cu:387-448):
(q + u), (q + v), K, P and V rounded to fp16; scores, softmax and sums in fp64; the softmax
weights rounded to fp16 for the P.V product while the row sum keeps them unrounded.  The
deviation of this model from the fp32 oracle is the error the fp16 operands alone cause."""
from __future__ import annotations

import numpy as np


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def relpos_attention_f16(q, k, v, p, u, vb, valid, scale):
    T, H, Dk = q.shape
    out = np.zeros((T, H, Dk))
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    for h in range(H):
        qu, qv = _f16(q[:, h] + u[h]), _f16(q[:, h] + vb[h])
        kk, vv, pp = _f16(k[:, h]), _f16(v[:, h]), _f16(p[:, h])
        s = (qu @ kk.T + (qv @ pp.T)[i, T - 1 - i + j]) * scale
        if valid <= 0:
            s = np.zeros_like(s)  # every key masked with the same finite value
        else:
            s[:, valid:] = -np.inf
        e = np.exp(s - s.max(1, keepdims=True))
        out[:, h] = (_f16(e) @ vv) / e.sum(1, keepdims=True)
    return out.astype(np.float32)


def conformer_layer_f16_core(x, T, valid, pos_emb, W, H):
    """oracle_lib.conformer_layer with the rel-pos core replaced by the fp16 rounding model."""
    import oracle_lib as orc
    orig = orc.relpos_attention
    orc.relpos_attention = relpos_attention_f16
    try:
        return orc.conformer_layer(x, T, valid, pos_emb, W, H)
    finally:
        orc.relpos_attention = orig
