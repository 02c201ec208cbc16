"""The text decoder's KV-cache write and attention launchers over the HIP library.

The reference keeps these kernels file-static inside src/model/asr_text_decoder.cu
(WriteKvCacheKernel :62-77, GqaCacheAttnKernel :88-142, GqaDecodeAttnKernel :149-213);
the functions here take the same arguments as those kernels' launches (:412-418,
:534-541), plus the cache capacity the host already knows (AsrTextConfig.max_seq_len).
Paged variants add a page table; with contiguous in-order pages they address exactly the
reference layout [max_seq_len, Hkv, Dh].  As the reference's kernels, the attention
launchers take any head size (up to 1024) and any Hq that is a multiple of Hkv; the
QK-norm-folded forms take Dh 128 and Hq / Hkv in {1, 2, 4}.
"""
from __future__ import annotations

from ._lib import PREFILL_BF16, PREFILL_FP32, call  # noqa: F401
from .runtime import _sh, ptr


def WriteKvCache(k, v, kc, vc, Tq: int, Hkv: int, Dh: int, d_pos0, capacity: int,
                 stream=None) -> None:
    """cache[pos0 + t] = bf16_rne(k/v[t]); pos0 = *d_pos0 on the device."""
    call("orator_kv_write", ptr(k), ptr(v), ptr(kc), ptr(vc), Tq, Hkv, Dh, ptr(d_pos0), capacity,
         _sh(stream))


def WriteKvCachePaged(k, v, kpool, vpool, page_table, max_pages: int, page_size: int,
                      n_pages: int, B: int, Tq: int, Hkv: int, Dh: int, d_pos0,
                      stream=None) -> None:
    call("orator_kv_write_paged", ptr(k), ptr(v), ptr(kpool), ptr(vpool), ptr(page_table),
         max_pages, page_size, n_pages, B, Tq, Hkv, Dh, ptr(d_pos0), _sh(stream))


def GqaDecodeAttn(q, kc, vc, out, Hq: int, Hkv: int, Dh: int, d_pos, capacity: int,
                  scale: float, stream=None) -> None:
    """q [Hq, Dh] attends the S = *d_pos + 1 cached keys."""
    call("orator_gqa_decode", ptr(q), ptr(kc), ptr(vc), ptr(out), Hq, Hkv, Dh, ptr(d_pos),
         capacity, scale, _sh(stream))


def GqaDecodeAttnPaged(q, kpool, vpool, page_table, max_pages: int, page_size: int, d_pos,
                       out, B: int, Hq: int, Hkv: int, Dh: int, scale: float,
                       stream=None) -> None:
    """Stream b's q [Hq, Dh] attends d_pos[b] + 1 keys through page-table row b."""
    call("orator_gqa_decode_paged", ptr(q), ptr(kpool), ptr(vpool), ptr(page_table), max_pages,
         page_size, ptr(d_pos), ptr(out), B, Hq, Hkv, Dh, scale, _sh(stream))


def GqaDecodeAttnPagedNoAlloc(q, kpool, vpool, page_table, max_pages: int, page_size: int,
                              d_pos, out, B: int, Hq: int, Hkv: int, Dh: int, scale: float,
                              stream=None) -> None:
    """GqaDecodeAttnPaged with its split partials in the library's static device scratch:
    allocates nothing (for graph capture / allocation-free loops); overlapping calls on one
    GPU race."""
    call("orator_gqa_decode_paged_noalloc", ptr(q), ptr(kpool), ptr(vpool), ptr(page_table),
         max_pages, page_size, ptr(d_pos), ptr(out), B, Hq, Hkv, Dh, scale, _sh(stream))


def GqaDecodeAttnAppend(q, k_new, v_new, kc, vc, out, Hq: int, Hkv: int, Dh: int, d_pos,
                        capacity: int, scale: float, stream=None) -> None:
    """WriteKvCacheKernel + GqaDecodeAttnKernel of one decode step in one launch: k_new/v_new
    [Hkv, Dh] fp32 are stored at *d_pos and q attends the *d_pos + 1 keys including them."""
    call("orator_gqa_decode_append", ptr(q), ptr(k_new), ptr(v_new), ptr(kc), ptr(vc), ptr(out),
         Hq, Hkv, Dh, ptr(d_pos), capacity, scale, _sh(stream))


def GqaDecodeAttnAppendPaged(q, k_new, v_new, kpool, vpool, page_table, max_pages: int,
                             page_size: int, n_pages: int, d_pos, out, B: int, Hq: int, Hkv: int,
                             Dh: int, scale: float, stream=None) -> None:
    """Batched paged append + decode: stream b stores k_new/v_new[b] at d_pos[b] through
    page-table row b and attends d_pos[b] + 1 keys."""
    call("orator_gqa_decode_append_paged", ptr(q), ptr(k_new), ptr(v_new), ptr(kpool), ptr(vpool),
         ptr(page_table), max_pages, page_size, n_pages, ptr(d_pos), ptr(out), B, Hq, Hkv, Dh,
         scale, _sh(stream))


def GqaCacheAttn(q, kc, vc, out, Tq: int, Hq: int, Hkv: int, Dh: int, d_pos0, capacity: int,
                 scale: float, stream=None) -> None:
    """Prefill: row t of q [Tq, Hq, Dh] (absolute position *d_pos0 + t) attends keys
    [0, pos0 + t]; fp32 mode."""
    call("orator_gqa_prefill", ptr(q), ptr(kc), ptr(vc), ptr(out), Tq, Hq, Hkv, Dh, ptr(d_pos0),
         capacity, scale, _sh(stream))


def GqaCacheAttnEx(q, q_bf16, kpool, vpool, page_table, max_pages: int, page_size: int, out,
                   Tq: int, Hq: int, Hkv: int, Dh: int, d_pos0, capacity: int, scale: float,
                   mode: int = PREFILL_FP32, stream=None) -> None:
    """Prefill with fp32 or bf16 q, contiguous or paged cache, fp32 or bf16 precision mode."""
    call("orator_gqa_prefill_ex", ptr(q), ptr(q_bf16), ptr(kpool), ptr(vpool), ptr(page_table),
         max_pages, page_size, ptr(out), Tq, Hq, Hkv, Dh, ptr(d_pos0), capacity, scale, mode,
         _sh(stream))


def QkNormRopeKvWrite(q, k, v, q_stride: int, kv_stride: int, q_norm, k_norm, eps: float,
                      positions, theta: float, n_tokens: int, tokens_per_stream: int, Hq: int,
                      Hkv: int, Dh: int, kpool, vpool, page_table=None, max_pages: int = 0,
                      page_size: int = 0, capacity: int = 0, stream=None) -> None:
    """RmsNorm(q), RmsNorm(k), RopeHalf(q, k) in place and the bf16 KV write, fused."""
    call("orator_qk_norm_rope_kv_write", ptr(q), ptr(k), ptr(v), q_stride, kv_stride, ptr(q_norm),
         ptr(k_norm), eps, ptr(positions), theta, n_tokens, tokens_per_stream, Hq, Hkv, Dh,
         ptr(kpool), ptr(vpool), ptr(page_table), max_pages, page_size, capacity, _sh(stream))


def RopeTable(out, n_pos: int, theta: float, stream=None) -> None:
    """(cos, sin) of every rotate-half pair (Dh 128) for positions [0, n_pos): [n_pos][64][2]."""
    call("orator_rope_table", ptr(out), n_pos, theta, _sh(stream))


def QkNormRopeKvWriteTable(q, k, v, q_stride: int, kv_stride: int, q_norm, k_norm, eps: float,
                           positions, theta: float, rope, rope_rows: int, n_tokens: int,
                           tokens_per_stream: int, Hq: int, Hkv: int, Dh: int, kpool, vpool,
                           page_table, max_pages: int, page_size: int, capacity: int,
                           stream=None) -> None:
    """QkNormRopeKvWrite with (cos, sin) from a RopeTable of rope_rows positions."""
    call("orator_qk_norm_rope_kv_write_table", ptr(q), ptr(k), ptr(v), q_stride, kv_stride,
         ptr(q_norm), ptr(k_norm), eps, ptr(positions), theta, ptr(rope), rope_rows, n_tokens,
         tokens_per_stream, Hq, Hkv, Dh, ptr(kpool), ptr(vpool), ptr(page_table), max_pages,
         page_size, capacity, _sh(stream))


def GqaDecodeAttnAppendQkNorm(q, k_new, v_new, kc, vc, out, Hq: int, Hkv: int, Dh: int, d_pos,
                              capacity: int, scale: float, q_norm, k_norm, eps: float, rope,
                              rope_rows: int, stream=None) -> None:
    """RmsNorm q/k + RopeHalf q/k + KV write + decode attention of one step, one launch."""
    call("orator_gqa_decode_append_qknorm", ptr(q), ptr(k_new), ptr(v_new), ptr(kc), ptr(vc),
         ptr(out), Hq, Hkv, Dh, ptr(d_pos), capacity, scale, ptr(q_norm), ptr(k_norm), eps,
         ptr(rope), rope_rows, _sh(stream))


def GqaDecodeAttnAppendQkNormPaged(q, k_new, v_new, kpool, vpool, page_table, max_pages: int,
                                   page_size: int, n_pages: int, d_pos, out, B: int, Hq: int,
                                   Hkv: int, Dh: int, scale: float, q_norm, k_norm, eps: float,
                                   rope, rope_rows: int, stream=None) -> None:
    call("orator_gqa_decode_append_qknorm_paged", ptr(q), ptr(k_new), ptr(v_new), ptr(kpool),
         ptr(vpool), ptr(page_table), max_pages, page_size, n_pages, ptr(d_pos), ptr(out), B, Hq,
         Hkv, Dh, scale, ptr(q_norm), ptr(k_norm), eps, ptr(rope), rope_rows, _sh(stream))
