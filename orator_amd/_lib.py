"""Loads liborator_attn.so (the gfx950 HIP library) and declares its C ABI for ctypes.

There is no CPU fallback: if the library was not built, importing the operator modules
raises.  Device pointers are plain ints.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liborator_attn.so"

ORATOR_OK = 0
ORATOR_ERR_INVALID = -1
ORATOR_ERR_UNSUPPORTED = -2
ORATOR_ERR_CAPACITY = -3
ORATOR_ERR_HIP = -4


class GpuError(RuntimeError):
    """A failed launch or HIP call; mirrors the reference's GpuMemoryException
    (src/gpu/memory.cc:14-21), a std::runtime_error."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


_p = C.c_void_p
_i = C.c_int
_l = C.c_long
_f = C.c_float
_sz = C.c_size_t

class DecoderConfig(C.Structure):
    """OratorDecoderConfig (AsrTextConfig, include/model/asr_text_decoder.h:30-42)."""
    _fields_ = [("num_layers", _i), ("hidden_size", _i), ("num_q_heads", _i),
                ("num_kv_heads", _i), ("head_dim", _i), ("intermediate_size", _i),
                ("vocab_size", _i), ("max_seq_len", _i), ("rms_norm_eps", _f),
                ("rope_theta", _f), ("profile", _i)]


class DecoderLayer(C.Structure):
    """OratorDecoderLayer: one layer's device weight pointers (fused qkv and gate|up)."""
    _fields_ = [("in_ln", _p), ("q_norm", _p), ("k_norm", _p), ("post_ln", _p),
                ("qkv_w", _p), ("o_w", _p), ("gateup_w", _p), ("down_w", _p)]


class ConformerWeights(C.Structure):
    """OratorConformerWeights: the 39 fp32 tensors of one ConformerLayer, checkpoint order
    (src/model/conformer_layer.cu:270-308)."""
    _fields_ = [(n, _p) for n in (
        "norm_ff1_w", "norm_ff1_b", "ff1_w1", "ff1_b1", "ff1_w2", "ff1_b2",
        "norm_att_w", "norm_att_b", "q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "out_w", "out_b",
        "pos_w", "pos_bias_u", "pos_bias_v",
        "norm_conv_w", "norm_conv_b", "pw1_w", "pw1_b", "dw_w", "dw_b",
        "bn_w", "bn_b", "bn_mean", "bn_var", "pw2_w", "pw2_b",
        "norm_ff2_w", "norm_ff2_b", "ff2_w1", "ff2_b1", "ff2_w2", "ff2_b2",
        "norm_out_w", "norm_out_b")]


# name -> argument types (all return int status)
SIGNATURES: dict[str, list] = {
    # bf16-weight linear and decode-step glue
    "orator_linear_pre": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "orator_linear_pre_swiglu": [_p, _p, _p, _i, _i, _i, _p],
    "orator_linear": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "orator_bf16_gemm": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "orator_embed_gather": [_p, _p, _p, _i, _p],
    "orator_add_residual": [_p, _p, _l, _p],
    "orator_record_token": [_p, _p, _p, _i, _p],
    "orator_inc_pos": [_p, _p],
    # decoder
    "orator_decoder_create": [C.POINTER(DecoderConfig), _p, _p, _p, C.POINTER(DecoderLayer),
                              C.POINTER(_p)],
    "orator_decoder_destroy": [_p],
    "orator_decoder_prefill_at": [_p, _p, _i, _i, _p],
    "orator_decoder_decode_step": [_p, _p, _i, _p],
    "orator_decoder_decode_step_device": [_p, _p, _i, _p],
    "orator_decoder_argmax_to_device": [_p, _p, _i, _i, _p],
    "orator_decoder_embed": [_p, _i, _p],
    "orator_decoder_reset": [_p],
    "orator_decoder_argmax": [_p, _i, _i, C.POINTER(_i), _p],
    "orator_decoder_logits": [_p, C.POINTER(_p)],
    "orator_decoder_decode_greedy": [_p, _i, _i, _i, _i, _i, _i, _i, C.POINTER(_i),
                                     C.POINTER(_i), _p],
    "orator_decoder_truncate": [_p, _i],
    "orator_decoder_cache_len": [_p, C.POINTER(_i)],
    # runtime
    "orator_version": [],
    "orator_device_count": [C.POINTER(_i)],
    "orator_set_device": [_i],
    "orator_device_name": [C.c_char_p, _i],
    "orator_malloc": [C.POINTER(_p), _sz],
    "orator_free": [_p],
    "orator_memcpy_htod": [_p, _p, _sz],
    "orator_memcpy_dtoh": [_p, _p, _sz],
    "orator_memcpy_dtod": [_p, _p, _sz, _p],
    "orator_memset": [_p, _i, _sz, _p],
    "orator_stream_create": [C.POINTER(_p)],
    "orator_stream_destroy": [_p],
    "orator_stream_synchronize": [_p],
    "orator_device_synchronize": [],
    "orator_event_create": [C.POINTER(_p)],
    "orator_event_destroy": [_p],
    "orator_event_record": [_p, _p],
    "orator_event_elapsed_ms": [C.POINTER(_f), _p, _p],
    "orator_workspace_reserve": [_sz, _p],
    "orator_workspace_stats": [C.POINTER(_sz), C.POINTER(_sz)],
    "orator_time_next_decode": [_p, _p, _p],
    # asr_ops family
    "orator_rms_norm": [_p, _p, _p, _i, _i, _f, _p],
    "orator_rope_interleaved": [_p, _p, _i, _i, _i, _f],
    "orator_swiglu": [_p, _p, _p, _i, _p],
    "orator_rope_half": [_p, _p, _i, _i, _i, _f, _p],
    "orator_argmax_banned": [_p, _i, _i, _i, _p, _p],
    "orator_gqa_attention": [_p, _p, _p, _p, _i, _i, _i, _i, _f, _i],
    "orator_f32_to_bf16": [_p, _p, _l, _p],
    "orator_bf16_to_f32": [_p, _p, _l, _p],
    # decoder KV + attention
    "orator_kv_write": [_p, _p, _p, _p, _i, _i, _i, _p, _i, _p],
    "orator_kv_write_paged": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p, _p],
    "orator_gqa_decode": [_p, _p, _p, _p, _i, _i, _i, _p, _i, _f, _p],
    "orator_gqa_decode_paged": [_p, _p, _p, _p, _i, _i, _p, _p, _i, _i, _i, _i, _f, _p],
    "orator_gqa_decode_paged_noalloc": [_p, _p, _p, _p, _i, _i, _p, _p, _i, _i, _i, _i, _f, _p],
    "orator_decode_read_probe": [_p, _p, _p, _i, _i, _i, _i, _i, _p, _p],
    "orator_gqa_decode_append_qknorm": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _i, _f, _p, _p,
                                        _f, _p, _i, _p],
    "orator_gqa_decode_append_qknorm_paged": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _p, _i, _i,
                                              _i, _i, _f, _p, _p, _f, _p, _i, _p],
    "orator_rope_table": [_p, _i, _f, _p],
    "orator_conformer_create": [_i, _i, _i, _i, C.POINTER(ConformerWeights), C.POINTER(_p)],
    "orator_conformer_destroy": [_p],
    "orator_conformer_forward": [_p, _p, _i, _i, _p, _i, _p],
    "orator_masked_mha": [_p, _p, _p, _p, _i, _i, _i, _i, _f, _p],
    "orator_window_attention": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _f, _p],
    "orator_gqa_decode_append": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _i, _f, _p],
    "orator_gqa_decode_append_paged": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _p, _i, _i, _i,
                                       _i, _f, _p],
    "orator_qk_norm_rope_kv_write": [_p, _p, _p, _l, _l, _p, _p, _f, _p, _f, _i, _i, _i, _i, _i,
                                     _p, _p, _p, _i, _i, _i, _p],
    "orator_qk_norm_rope_kv_write_table": [_p, _p, _p, _l, _l, _p, _p, _f, _p, _f, _p, _i, _i,
                                           _i, _i, _i, _i, _p, _p, _p, _i, _i, _i, _p],
    "orator_sgemm": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "orator_sgemm_batched": [_p, _p, _p, _i, _i, _i, _i, _i, _l, _l, _l, _p],
    "orator_build_pos_emb": [_p, _i, _i],
    "orator_relpos_attention_fast": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _i, _p],
    "orator_relpos_attention": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _p],
    "orator_gqa_prefill": [_p, _p, _p, _p, _i, _i, _i, _i, _p, _i, _f, _p],
    "orator_gqa_prefill_ex": [_p, _p, _p, _p, _p, _i, _i, _p, _i, _i, _i, _i, _p, _i, _f, _i, _p],
}

PREFILL_FP32 = 0
PREFILL_BF16 = 1

_lib = None


def lib() -> C.CDLL:
    """Returns the loaded library, loading it on first use; raises if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m orator_amd.build` "
                "(the HIP path has no CPU fallback)")
        handle = C.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _i
        handle.orator_last_error.argtypes = []
        handle.orator_last_error.restype = C.c_char_p
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != ORATOR_OK:
        msg = lib().orator_last_error().decode(errors="replace")
        raise GpuError(status, msg)


def call(name: str, *args) -> None:
    """Calls an entry point and raises GpuError on a non-zero status."""
    check(getattr(lib(), name)(*args))
