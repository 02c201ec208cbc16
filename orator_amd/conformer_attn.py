"""The FastConformer layer's relative-position attention core (the block of
ConformerLayer::Forward between linear_q/k/v/pos and linear_out,
src/model/conformer_layer.cu:405-444) and BuildPosEmb (:314-329) over the HIP library."""
from __future__ import annotations

import math

import numpy as np

from ._lib import call
from .runtime import _sh, ptr


def RelPosAttention(q, k, v, p, pos_bias_u, pos_bias_v, out, T: int, H: int, Dk: int,
                    valid_len: int, scale: float | None = None, stream=None) -> None:
    """out [T,H,Dk] = softmax((AC + rel_shift(BD)) * scale, keys >= valid masked) . v."""
    if scale is None:
        scale = 1.0 / math.sqrt(Dk)
    call("orator_relpos_attention", ptr(q), ptr(k), ptr(v), ptr(p), ptr(pos_bias_u),
         ptr(pos_bias_v), ptr(out), T, H, Dk, valid_len, scale, _sh(stream))


def RelPosAttentionFast(q, k, v, p, pos_bias_u, pos_bias_v, out, T: int, H: int, Dk: int,
                        valid_len: int, scale: float | None = None, in_f16: bool | int = True,
                        stream=None) -> None:
    """Fused fp16-MFMA form of RelPosAttention: inputs fp16 bits (in_f16 True or 1), fp32
    (False or 0), or q fp32 with k, v, p fp16 bits (2)."""
    if scale is None:
        scale = 1.0 / math.sqrt(Dk)
    mode = 2 if in_f16 == 2 and not isinstance(in_f16, bool) else int(bool(in_f16))
    call("orator_relpos_attention_fast", ptr(q), ptr(k), ptr(v), ptr(p), ptr(pos_bias_u),
         ptr(pos_bias_v), ptr(out), T, H, Dk, valid_len, scale, mode, _sh(stream))


def BuildPosEmb(T: int, d_model: int) -> np.ndarray:
    """RelPositionalEncoding pos_emb [2T-1, d_model] for positions T-1 .. -(T-1), built on the
    host by the library with the reference's float math (conformer_layer.cu:314-329)."""
    pe = np.empty((max(2 * T - 1, 0), d_model), np.float32)
    call("orator_build_pos_emb", pe.ctypes.data, T, d_model)
    return pe


class ConformerLayer:
    """ConformerLayer (include/model/conformer_layer.h:31-65) over caller-owned fp32 device
    weights: `weights` maps each OratorConformerWeights field name to a device buffer."""

    def __init__(self, weights: dict, d_model: int = 512, n_heads: int = 8, d_ff: int = 2048,
                 conv_kernel: int = 9):
        from ._lib import ConformerWeights
        import ctypes as C
        w = ConformerWeights(*[ptr(weights[name]) for name, _ in ConformerWeights._fields_])
        h = C.c_void_p()
        call("orator_conformer_create", d_model, n_heads, d_ff, conv_kernel, C.byref(w),
             C.byref(h))
        self._h = h
        self._keep = weights
        self.d_model = d_model

    def Forward(self, x, T: int, valid_len: int, pos_emb, stream=None, attn_mode: int = 0):
        """x [T, d_model] device fp32 in place; pos_emb [2T-1, d_model] device fp32."""
        call("orator_conformer_forward", self._h, ptr(x), T, valid_len, ptr(pos_emb), attn_mode,
             _sh(stream))

    @staticmethod
    def BuildPosEmb(T: int, d_model: int):
        return BuildPosEmb(T, d_model)

    def close(self) -> None:
        if self._h:
            from ._lib import lib
            lib().orator_conformer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
