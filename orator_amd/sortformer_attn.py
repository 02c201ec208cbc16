"""The Sortformer decoder's masked multi-head self-attention
(src/model/sortformer_decoder.cu:280-298) over the HIP library."""
from __future__ import annotations

from ._lib import call
from .runtime import _sh, ptr


def MaskedSelfAttention(q, k, v, out, T: int, H: int, Dk: int, valid_len: int, scale: float,
                        stream=None) -> None:
    """q/k/v/out fp32 [T, H, Dk] (Dk 24, 32 or 64); keys >= valid_len are masked (scored
    -1e30 as the reference, so valid_len <= 0 averages every key)."""
    call("orator_masked_mha", ptr(q), ptr(k), ptr(v), ptr(out), T, H, Dk, valid_len, scale,
         _sh(stream))
