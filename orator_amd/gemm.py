"""The reference's `orator::gemm` launchers (include/model/gemm.cuh:160-268) over the HIP
library: fp32 NT GEMM with fused bias/activation and its strided-batched form."""
from __future__ import annotations

from ._lib import call
from .runtime import _sh, ptr


def LaunchSgemm(inp, W, bias, out, M: int, K: int, N: int, act: int, stream=None) -> None:
    """out[M,N] = act(in[M,K] . W[N,K]^T + bias); act 0 none, 1 SiLU, 2 ReLU, 3 sigmoid."""
    call("orator_sgemm", ptr(inp), ptr(W), ptr(bias), ptr(out), M, K, N, act, _sh(stream))


def LaunchSgemmBatched(inp, W, out, M: int, K: int, N: int, act: int, batch: int,
                       strideIn: int, strideW: int, strideOut: int, stream=None) -> None:
    call("orator_sgemm_batched", ptr(inp), ptr(W), ptr(out), M, K, N, act, batch, strideIn,
         strideW, strideOut, _sh(stream))


def LaunchBf16Gemm(inp_bf16, W_bf16, bias, out, M: int, K: int, N: int, act: int,
                   stream=None) -> None:
    """out[M,N] = act(in[M,K] . W[N,K]^T + bias), bf16 in and W (include/model/gemm.cuh:
    484-501); act 0 none, 1 exact GELU, 2 ReLU."""
    call("orator_bf16_gemm", ptr(inp_bf16), ptr(W_bf16), ptr(bias), ptr(out), M, K, N, act,
         _sh(stream))
