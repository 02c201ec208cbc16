"""The reference's `orator::model::asr_ops` / `asr_gemm` launchers over the HIP library.

Same names, argument order and meaning as include/model/asr_ops.cuh:21-62 and
include/model/asr_gemm.h:23-25.  Arguments are device buffers (DeviceBuffer or int
addresses); `stream` is a runtime.Stream, a raw handle or None (default stream).
Failures raise GpuError, as the reference's launchers throw GpuMemoryException.
"""
from __future__ import annotations

from ._lib import call
from .runtime import _sh, ptr


def RmsNorm(x, weight, out, rows: int, dim: int, eps: float, stream=None) -> None:
    """include/model/asr_ops.cuh:21-25."""
    call("orator_rms_norm", ptr(x), ptr(weight), ptr(out), rows, dim, eps, _sh(stream))


def RopeInterleaved(x, positions, n_tokens: int, n_heads: int, head_dim: int,
                    theta_base: float) -> None:
    """include/model/asr_ops.cuh:27-34 (default stream, in place)."""
    call("orator_rope_interleaved", ptr(x), ptr(positions), n_tokens, n_heads, head_dim,
         theta_base)


def SwiGLU(gate, up, out, n: int, stream=None) -> None:
    """include/model/asr_ops.cuh:36-39."""
    call("orator_swiglu", ptr(gate), ptr(up), ptr(out), n, _sh(stream))


def RopeHalf(x, positions, n_tokens: int, n_heads: int, head_dim: int, theta_base: float,
             stream=None) -> None:
    """include/model/asr_ops.cuh:41-48 (rotate_half, in place)."""
    call("orator_rope_half", ptr(x), ptr(positions), n_tokens, n_heads, head_dim, theta_base,
         _sh(stream))


def GqaAttention(q, k, v, out, T: int, Hq: int, Hkv: int, Dh: int, scale: float,
                 causal: bool) -> None:
    """include/model/asr_ops.cuh:55-56 (fp32 GQA self-attention, default stream)."""
    call("orator_gqa_attention", ptr(q), ptr(k), ptr(v), ptr(out), T, Hq, Hkv, Dh, scale,
         int(bool(causal)))


def ArgmaxBanned(logits, n: int, ban0: int, ban1: int, out_idx, stream=None) -> None:
    """include/model/asr_ops.cuh:58-62."""
    call("orator_argmax_banned", ptr(logits), n, ban0, ban1, ptr(out_idx), _sh(stream))


def F32ToBf16(inp, out, n: int, stream=None) -> None:
    """include/model/asr_gemm.h:24."""
    call("orator_f32_to_bf16", ptr(inp), ptr(out), n, _sh(stream))


def Bf16ToF32(inp, out, n: int, stream=None) -> None:
    """include/model/asr_gemm.h:25."""
    call("orator_bf16_to_f32", ptr(inp), ptr(out), n, _sh(stream))
