"""The reference's `orator::model::asr_gemm` linear layers (include/model/asr_gemm.h:23-41)
over the HIP library: bf16 weights, fp32 accumulation; M == 1 runs a streaming GEMV and
M > 1 an MFMA GEMM.  The casts F32ToBf16 / Bf16ToF32 live in asr_ops."""
from __future__ import annotations

from ._lib import call
from .asr_ops import Bf16ToF32, F32ToBf16  # noqa: F401  (the cast half of asr_gemm.h)
from .runtime import _sh, ptr


def Linear(in_f32, W_bf16, bias, out, M: int, K: int, N: int, act: int, stream=None) -> None:
    """out[M,N] = act(bf16(in)[M,K] . W[N,K]^T + bias); act 0 none, 1 GELU, 2 ReLU."""
    call("orator_linear", ptr(in_f32), ptr(W_bf16), ptr(bias), ptr(out), M, K, N, act,
         _sh(stream))


def LinearPre(in_bf16, W_bf16, bias, out, M: int, K: int, N: int, act: int,
              stream=None) -> None:
    """Linear with an input that is already bf16."""
    call("orator_linear_pre", ptr(in_bf16), ptr(W_bf16), ptr(bias), ptr(out), M, K, N, act,
         _sh(stream))


def LinearPreSwiGLU(in_bf16, W_gateup_bf16, out_bf16, M: int, K: int, I: int,
                    stream=None) -> None:
    """The decoder MLP's gate|up projection, SwiGLU and bf16 cast in one launch:
    out[M,I] (bf16) = bf16(silu(in . W[0:I]^T) * (in . W[I:2I]^T)) (asr_text_decoder.cu:
    547-552); the same values as LinearPre + SwiGLU + F32ToBf16."""
    call("orator_linear_pre_swiglu", ptr(in_bf16), ptr(W_gateup_bf16), ptr(out_bf16), M, K, I,
         _sh(stream))


def Shutdown() -> None:
    """The reference frees its cast scratch here; the library's workspace is released with
    the process, so there is nothing to do."""
