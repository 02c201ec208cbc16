"""The ASR text decoder (AsrTextDecoder, include/model/asr_text_decoder.h:45-112) over the
HIP library: prefill, single-token decode, argmax and greedy decoding with the reference's
stop rules, on caller-owned device weights."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import DecoderConfig, DecoderLayer, call, lib
from .runtime import _sh, ptr

EOS_IDS = (151645, 151643)  # src/model/qwen3_asr.cc:160-161


@dataclass
class AsrTextConfig:
    """AsrTextConfig (include/model/asr_text_decoder.h:30-42) with Qwen3-ASR-1.7B defaults."""
    num_layers: int = 28
    hidden_size: int = 2048
    num_q_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 6144
    vocab_size: int = 151936
    max_seq_len: int = 2048
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    profile: bool = False  # event timing printed to stderr, as the reference's

    def c_struct(self) -> DecoderConfig:
        return DecoderConfig(self.num_layers, self.hidden_size, self.num_q_heads,
                             self.num_kv_heads, self.head_dim, self.intermediate_size,
                             self.vocab_size, self.max_seq_len, self.rms_norm_eps,
                             self.rope_theta, int(self.profile))


def _addr(x):
    """Host numpy arrays pass their data pointer (the library copies with hipMemcpyDefault)."""
    if isinstance(x, np.ndarray):
        assert x.dtype == np.float32 and x.flags.c_contiguous
        return x.ctypes.data
    return ptr(x)


class AsrTextDecoder:
    """layers: one dict per layer with device buffers in_ln, q_norm, k_norm, post_ln (fp32),
    qkv_w, o_w, gateup_w, down_w (bf16, fused layout).  lm_head None = tied to embed."""

    def __init__(self, config: AsrTextConfig, embed, final_norm, lm_head, layers):
        self.config = config
        arr = (DecoderLayer * config.num_layers)()
        for i, L in enumerate(layers):
            arr[i] = DecoderLayer(ptr(L["in_ln"]), ptr(L["q_norm"]), ptr(L["k_norm"]),
                                  ptr(L["post_ln"]), ptr(L["qkv_w"]), ptr(L["o_w"]),
                                  ptr(L["gateup_w"]), ptr(L["down_w"]))
        self._keep = (embed, final_norm, lm_head, layers)
        h = C.c_void_p()
        cfg = config.c_struct()
        call("orator_decoder_create", C.byref(cfg), ptr(embed), ptr(final_norm), ptr(lm_head),
             arr, C.byref(h))
        self._h = h

    def close(self) -> None:
        if self._h:
            lib().orator_decoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    def ResetCache(self) -> None:
        call("orator_decoder_reset", self._h)

    def Embed(self, token_id: int) -> np.ndarray:
        """The token's embedding row [hidden] as host fp32."""
        out = np.empty(self.config.hidden_size, np.float32)
        call("orator_decoder_embed", self._h, token_id, out.ctypes.data)
        return out

    def hidden_size(self) -> int:
        return self.config.hidden_size

    def vocab_size(self) -> int:
        return self.config.vocab_size

    def Prefill(self, embeds, T: int, stream=None) -> None:
        self.PrefillAt(embeds, T, 0, stream)

    def PrefillAt(self, embeds, T: int, pos0: int, stream=None) -> None:
        """embeds: [T, hidden] fp32, a host numpy array or a device buffer."""
        call("orator_decoder_prefill_at", self._h, _addr(embeds), T, pos0, _sh(stream))

    def DecodeStep(self, embed, pos: int, stream=None) -> None:
        """embed: [hidden] fp32, host numpy array or device buffer."""
        call("orator_decoder_decode_step", self._h, _addr(embed), pos, _sh(stream))

    def DecodeStepDevice(self, d_token, pos: int, stream=None) -> None:
        call("orator_decoder_decode_step_device", self._h, ptr(d_token), pos, _sh(stream))

    def ArgmaxToDevice(self, d_out, ban0: int = -1, ban1: int = -1, stream=None) -> None:
        call("orator_decoder_argmax_to_device", self._h, ptr(d_out), ban0, ban1, _sh(stream))

    def CopyLogits(self) -> np.ndarray:
        out = np.empty(self.config.vocab_size, np.float32)
        call("orator_device_synchronize")
        call("orator_memcpy_dtoh", out.ctypes.data, self.logits_ptr(), out.nbytes)
        return out

    def Argmax(self, ban0: int = -1, ban1: int = -1, stream=None) -> int:
        t = C.c_int()
        call("orator_decoder_argmax", self._h, ban0, ban1, C.byref(t), _sh(stream))
        return t.value

    def logits_ptr(self) -> int:
        p = C.c_void_p()
        call("orator_decoder_logits", self._h, C.byref(p))
        return p.value

    def DecodeGreedy(self, start_pos: int, max_new: int, eos0: int, eos1: int,
                     ban_steps: int = 3, batch: int = 32, use_graph: bool = True,
                     stream=None) -> list[int]:
        buf = (C.c_int * max(1, max_new))()
        n = C.c_int()
        call("orator_decoder_decode_greedy", self._h, start_pos, max_new, eos0, eos1, ban_steps,
             batch, int(use_graph), buf, C.byref(n), _sh(stream))
        return list(np.frombuffer(buf, np.int32, n.value)) if n.value else []

    def TruncateCache(self, length: int) -> None:
        call("orator_decoder_truncate", self._h, length)

    def cache_len(self) -> int:
        n = C.c_int()
        call("orator_decoder_cache_len", self._h, C.byref(n))
        return n.value
