"""The audio tower's windowed self-attention (WindowAttnKernel,
src/model/asr_audio_tower.cu:204-258, launched at :573-575) over the HIP library."""
from __future__ import annotations

from ._lib import call
from .runtime import _sh, ptr


def WindowAttention(q, k, v, out, seg_start, seg_end, N: int, H: int, Dh: int, scale: float,
                    stream=None) -> None:
    """q/k/v/out fp32 [N, H, Dh] (Dh <= 1024; 64 and 128 on the fast kernels); query i
    attends keys [seg_start[i], seg_end[i]) given as device int arrays; an empty window gives
    zeros."""
    call("orator_window_attention", ptr(q), ptr(k), ptr(v), ptr(out), ptr(seg_start),
         ptr(seg_end), N, H, Dh, scale, _sh(stream))
