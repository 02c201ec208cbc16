"""The decode-step glue kernels of the ASR text decoder (src/model/asr_text_decoder.cu:30-58):
embedding gather, residual add, token record and position increment."""
from __future__ import annotations

from ._lib import call
from .runtime import _sh, ptr


def EmbedGather(table_bf16, d_token, out, hidden: int, stream=None) -> None:
    """out[:hidden] = table[*d_token] widened to fp32 (EmbedGatherKernel, :38-45)."""
    call("orator_embed_gather", ptr(table_bf16), ptr(d_token), ptr(out), hidden, _sh(stream))


def AddResidual(a, b, n: int, stream=None) -> None:
    """a += b (AddResidualKernel, :30-34)."""
    call("orator_add_residual", ptr(a), ptr(b), n, _sh(stream))


def RecordToken(out, d_count, d_token, capacity: int, stream=None) -> None:
    """out[*d_count] = *d_token (dropped at or past capacity); ++*d_count (:50-55)."""
    call("orator_record_token", ptr(out), ptr(d_count), ptr(d_token), capacity, _sh(stream))


def IncPos(d_pos, stream=None) -> None:
    """++*d_pos (IncPosKernel, :58)."""
    call("orator_inc_pos", ptr(d_pos), _sh(stream))
