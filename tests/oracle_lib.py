"""numpy-facing wrappers over the CPU oracle (oracle/liborator_oracle.so).

Test infrastructure: only tests, __graft_entry__.smoke() and bench.py's cpu_baseline
leg use this module, always as the checker.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "liborator_oracle.so"

_lib = None

_F = C.POINTER(C.c_float)
_D = C.POINTER(C.c_double)
_U16 = C.POINTER(C.c_uint16)
_I = C.POINTER(C.c_int)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
        L = C.CDLL(str(ORACLE_SO))
        i, f, l = C.c_int, C.c_float, C.c_long
        sig = {
            "orc_f32_to_bf16": ([f], C.c_uint16),
            "orc_bf16_to_f32": ([C.c_uint16], f),
            "orc_f32_to_bf16_n": ([_F, _U16, l], None),
            "orc_bf16_to_f32_n": ([_U16, _F, l], None),
            "orc_rms_norm": ([_F, _F, _F, i, i, f], None),
            "orc_rope_inv_freq": ([f, i, i], f),
            "orc_rope_half": ([_F, _I, i, i, i, f], None),
            "orc_rope_interleaved": ([_F, _I, i, i, i, f], None),
            "orc_swiglu": ([_F, _F, _F, i], None),
            "orc_kv_write": ([_F, _F, _U16, _U16, i, i, i, i], None),
            "orc_kv_write_paged": ([_F, _F, _U16, _U16, _I, i, i, i, i, i], None),
            "orc_gqa_prefill": ([_F, _U16, _U16, _F, i, i, i, i, i, f], None),
            "orc_gqa_prefill_paged": ([_F, _U16, _U16, _I, i, _F, i, i, i, i, i, f], None),
            "orc_gqa_prefill_mt": ([_F, _U16, _U16, _F, i, i, i, i, i, f, i], None),
            "orc_gqa_decode": ([_F, _U16, _U16, _F, i, i, i, i, f], None),
            "orc_gqa_decode_paged": ([_F, _U16, _U16, _I, i, i, _I, _F, i, i, i, i, f], None),
            "orc_gqa_decode_paged_mt": ([_F, _U16, _U16, _I, i, i, _I, _F, i, i, i, i, f, i],
                                        None),
            "orc_gqa_attention": ([_F, _F, _F, _F, i, i, i, i, f, i], None),
            "orc_attention_f64": ([_F, _F, _F, _D, i, i, i, i, i, i, C.c_double, i], None),
            "orc_build_pos_emb": ([i, i, _F], None),
            "orc_relpos_attention": ([_F, _F, _F, _F, _F, _F, _F, i, i, i, i, f], None),
            "orc_relpos_attention_f64": ([_F, _F, _F, _F, _F, _F, _D, i, i, i, i, C.c_double],
                                         None),
            "orc_relshift_column": ([i, i, i, _I], i),
            "orc_sgemm": ([_F, _F, _F, _F, i, i, i, i], None),
            "orc_sgemm_batched": ([_F, _F, _F, i, i, i, i, i, l, l, l], None),
            "orc_argmax_banned": ([_F, i, i, i], i),
            "orc_linear_bf16": ([_U16, _U16, _F, _F, i, i, i, i], None),
            "orc_window_attention": ([_F, _F, _F, _F, _I, _I, i, i, i, f], None),
            "orc_masked_mha": ([_F, _F, _F, _F, i, i, i, i, f], None),
            "orc_layer_norm": ([_F, _F, _F, _F, i, i, f], None),
            "orc_glu_mask": ([_F, _F, i, i, i], None),
            "orc_dwconv_bn_silu": ([_F, _F, _F, _F, _F, _F, _F, _F, i, i, i, f], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _d(a):
    assert a.dtype == np.float64 and a.flags.c_contiguous
    return a.ctypes.data_as(_D)


def _u16(a):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(_U16)


def _i(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_I)


def f32c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- bf16 ----
def to_bf16(x) -> np.ndarray:
    x = f32c(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_f(x), _u16(out), x.size)
    return out


def from_bf16(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_to_f32_n(_u16(b), _f(out), b.size)
    return out


# ------------------------------------------------------------ asr_ops ----
def rms_norm(x, w, eps) -> np.ndarray:
    x, w = f32c(x), f32c(w)
    rows, dim = x.shape
    out = np.empty_like(x)
    lib().orc_rms_norm(_f(x), _f(w), _f(out), rows, dim, eps)
    return out


def rope_half(x, pos, base) -> np.ndarray:
    x = f32c(x).copy()
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    T, H, Dh = x.shape
    lib().orc_rope_half(_f(x), _i(pos), T, H, Dh, base)
    return x


def rope_interleaved(x, pos, base) -> np.ndarray:
    x = f32c(x).copy()
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    T, H, Dh = x.shape
    lib().orc_rope_interleaved(_f(x), _i(pos), T, H, Dh, base)
    return x


def swiglu(g, u) -> np.ndarray:
    g, u = f32c(g), f32c(u)
    out = np.empty_like(g)
    lib().orc_swiglu(_f(g), _f(u), _f(out), g.size)
    return out


def argmax_banned(x, ban0=-1, ban1=-1) -> int:
    x = f32c(x)
    return lib().orc_argmax_banned(_f(x), x.size, ban0, ban1)


# --------------------------------------------------------- KV + attention ----
def kv_write(k, v, kc, vc, pos0) -> None:
    """In place into the uint16 caches kc/vc [cap, Hkv, Dh]."""
    k, v = f32c(k), f32c(v)
    Tq, Hkv, Dh = k.shape
    lib().orc_kv_write(_f(k), _f(v), _u16(kc), _u16(vc), Tq, Hkv, Dh, pos0)


def kv_write_paged(k, v, kpool, vpool, page_table_row, page_size, pos0) -> None:
    k, v = f32c(k), f32c(v)
    pt = np.ascontiguousarray(page_table_row, dtype=np.int32)
    Tq, Hkv, Dh = k.shape
    lib().orc_kv_write_paged(_f(k), _f(v), _u16(kpool), _u16(vpool), _i(pt), page_size, Tq, Hkv,
                             Dh, pos0)


def gqa_prefill(q, kc, vc, pos0, scale, threads: int = 1) -> np.ndarray:
    q = f32c(q)
    Tq, Hq, Dh = q.shape
    Hkv = kc.shape[1]
    out = np.empty_like(q)
    if threads > 1:
        lib().orc_gqa_prefill_mt(_f(q), _u16(kc), _u16(vc), _f(out), Tq, Hq, Hkv, Dh, pos0, scale,
                                 threads)
    else:
        lib().orc_gqa_prefill(_f(q), _u16(kc), _u16(vc), _f(out), Tq, Hq, Hkv, Dh, pos0, scale)
    return out


def gqa_prefill_paged(q, kpool, vpool, page_table_row, page_size, pos0, scale) -> np.ndarray:
    q = f32c(q)
    Tq, Hq, Dh = q.shape
    Hkv = kpool.shape[-2]
    pt = np.ascontiguousarray(page_table_row, dtype=np.int32)
    out = np.empty_like(q)
    lib().orc_gqa_prefill_paged(_f(q), _u16(kpool), _u16(vpool), _i(pt), page_size, _f(out), Tq,
                                Hq, Hkv, Dh, pos0, scale)
    return out


def gqa_decode(q, kc, vc, pos, scale) -> np.ndarray:
    q = f32c(q)
    Hq, Dh = q.shape
    Hkv = kc.shape[1]
    out = np.empty_like(q)
    lib().orc_gqa_decode(_f(q), _u16(kc), _u16(vc), _f(out), Hq, Hkv, Dh, pos, scale)
    return out


def gqa_decode_paged(q, kpool, vpool, page_table, page_size, pos, scale,
                     threads: int = 1) -> np.ndarray:
    q = f32c(q)
    B, Hq, Dh = q.shape
    Hkv = kpool.shape[-2]
    pt = np.ascontiguousarray(page_table, dtype=np.int32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    out = np.empty_like(q)
    lib().orc_gqa_decode_paged_mt(_f(q), _u16(kpool), _u16(vpool), _i(pt), pt.shape[1],
                                  page_size, _i(pos), _f(out), B, Hq, Hkv, Dh, scale, threads)
    return out


def gqa_attention(q, k, v, scale, causal) -> np.ndarray:
    q, k, v = f32c(q), f32c(k), f32c(v)
    T, Hq, Dh = q.shape
    Hkv = k.shape[1]
    out = np.empty_like(q)
    lib().orc_gqa_attention(_f(q), _f(k), _f(v), _f(out), T, Hq, Hkv, Dh, scale, int(causal))
    return out


def attention_f64(q, k, v, scale, causal, kv_off=0) -> np.ndarray:
    """fp64 truth; k/v are float arrays [S, Hkv, Dh] (decode bf16 caches with from_bf16)."""
    q, k, v = f32c(q), f32c(k), f32c(v)
    T, Hq, Dh = q.shape
    S, Hkv = k.shape[0], k.shape[1]
    out = np.empty(q.shape, np.float64)
    lib().orc_attention_f64(_f(q), _f(k), _f(v), _d(out), T, S, Hq, Hkv, Dh, kv_off, scale,
                            int(causal))
    return out


# ------------------------------------------------------------ conformer ----
def build_pos_emb(T, d_model) -> np.ndarray:
    pe = np.empty((2 * T - 1, d_model), np.float32)
    lib().orc_build_pos_emb(T, d_model, _f(pe))
    return pe


def relpos_attention(q, k, v, p, u, vb, valid, scale) -> np.ndarray:
    q, k, v, p, u, vb = map(f32c, (q, k, v, p, u, vb))
    T, H, Dk = q.shape
    out = np.empty_like(q)
    lib().orc_relpos_attention(_f(q), _f(k), _f(v), _f(p), _f(u), _f(vb), _f(out), T, H, Dk,
                               valid, scale)
    return out


def relpos_attention_f64(q, k, v, p, u, vb, valid, scale) -> np.ndarray:
    q, k, v, p, u, vb = map(f32c, (q, k, v, p, u, vb))
    T, H, Dk = q.shape
    out = np.empty(q.shape, np.float64)
    lib().orc_relpos_attention_f64(_f(q), _f(k), _f(v), _f(p), _f(u), _f(vb), _d(out), T, H, Dk,
                                   valid, scale)
    return out


def relshift_column(T, i, j):
    row = C.c_int(-1)
    m = lib().orc_relshift_column(T, i, j, C.byref(row))
    return row.value, m


# ----------------------------------------------------------------- gemm ----
def sgemm(inp, W, bias=None, act=0) -> np.ndarray:
    inp, W = f32c(inp), f32c(W)
    M, K = inp.shape
    N = W.shape[0]
    out = np.empty((M, N), np.float32)
    b = f32c(bias) if bias is not None else None
    lib().orc_sgemm(_f(inp), _f(W), _f(b) if b is not None else None, _f(out), M, K, N, act)
    return out


def sgemm_batched(inp, W, act=0) -> np.ndarray:
    inp, W = f32c(inp), f32c(W)
    B, M, K = inp.shape
    N = W.shape[1]
    out = np.empty((B, M, N), np.float32)
    lib().orc_sgemm_batched(_f(inp), _f(W), _f(out), M, K, N, act, B, M * K, N * K, M * N)
    return out


# ------------------------------------------------------- window attention ----
def window_attention(q, k, v, seg_start, seg_end, scale) -> np.ndarray:
    q, k, v = f32c(q), f32c(k), f32c(v)
    N, H, Dh = q.shape
    ss = np.ascontiguousarray(seg_start, dtype=np.int32)
    se = np.ascontiguousarray(seg_end, dtype=np.int32)
    out = np.empty_like(q)
    lib().orc_window_attention(_f(q), _f(k), _f(v), _f(out), _i(ss), _i(se), N, H, Dh, scale)
    return out


def masked_mha(q, k, v, valid, scale) -> np.ndarray:
    q, k, v = f32c(q), f32c(k), f32c(v)
    T, H, Dk = q.shape
    out = np.empty_like(q)
    lib().orc_masked_mha(_f(q), _f(k), _f(v), _f(out), T, H, Dk, valid, scale)
    return out


# -------------------------------------------------------------- Conformer ----
CONFORMER_FIELDS = (
    "norm_ff1_w", "norm_ff1_b", "ff1_w1", "ff1_b1", "ff1_w2", "ff1_b2",
    "norm_att_w", "norm_att_b", "q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "out_w", "out_b",
    "pos_w", "pos_bias_u", "pos_bias_v",
    "norm_conv_w", "norm_conv_b", "pw1_w", "pw1_b", "dw_w", "dw_b",
    "bn_w", "bn_b", "bn_mean", "bn_var", "pw2_w", "pw2_b",
    "norm_ff2_w", "norm_ff2_b", "ff2_w1", "ff2_b1", "ff2_w2", "ff2_b2",
    "norm_out_w", "norm_out_b")


def layer_norm(x, g, b, eps=1e-5) -> np.ndarray:
    x, g, b = f32c(x), f32c(g), f32c(b)
    T, C = x.shape
    out = np.empty_like(x)
    lib().orc_layer_norm(_f(x), _f(g), _f(b), _f(out), T, C, eps)
    return out


def glu_mask(x, valid) -> np.ndarray:
    x = f32c(x)
    T, C2 = x.shape
    out = np.empty((T, C2 // 2), np.float32)
    lib().orc_glu_mask(_f(x), _f(out), T, C2 // 2, valid)
    return out


def dwconv_bn_silu(x, w, bias, mean, var, gamma, beta, eps=1e-5) -> np.ndarray:
    x, w, bias, mean, var, gamma, beta = map(f32c, (x, w, bias, mean, var, gamma, beta))
    T, C = x.shape
    K = w.shape[-1]
    out = np.empty_like(x)
    lib().orc_dwconv_bn_silu(_f(x), _f(w), _f(bias), _f(mean), _f(var), _f(gamma), _f(beta),
                             _f(out), T, C, K, eps)
    return out


def conformer_layer(x, T, valid, pos_emb, W, H, eps=1e-5):
    """ConformerLayer::Forward (src/model/conformer_layer.cu:364-488) on the oracle pieces:
    LaunchLinear = orc_sgemm (act 1 SiLU), the rel-pos core = orc_relpos_attention."""
    x = f32c(x).copy()
    D = x.shape[1]
    Dk = D // H

    def ffn(x, p):
        ln = layer_norm(x, W[f"norm_{p}_w"], W[f"norm_{p}_b"], eps)
        h = sgemm(ln, W[f"{p}_w1"], W[f"{p}_b1"], act=1)
        return x + np.float32(0.5) * sgemm(h, W[f"{p}_w2"], W[f"{p}_b2"])

    x = ffn(x, "ff1")
    ln = layer_norm(x, W["norm_att_w"], W["norm_att_b"], eps)
    q = sgemm(ln, W["q_w"], W["q_b"]).reshape(T, H, Dk)
    k = sgemm(ln, W["k_w"], W["k_b"]).reshape(T, H, Dk)
    v = sgemm(ln, W["v_w"], W["v_b"]).reshape(T, H, Dk)
    p = sgemm(pos_emb, W["pos_w"]).reshape(2 * T - 1, H, Dk)
    ctx = relpos_attention(q, k, v, p, W["pos_bias_u"], W["pos_bias_v"], valid,
                           float(1.0 / np.sqrt(np.float32(Dk))))
    x = x + sgemm(ctx.reshape(T, D), W["out_w"], W["out_b"])
    ln = layer_norm(x, W["norm_conv_w"], W["norm_conv_b"], eps)
    g = glu_mask(sgemm(ln, W["pw1_w"], W["pw1_b"]), valid)
    c = dwconv_bn_silu(g, W["dw_w"], W["dw_b"], W["bn_mean"], W["bn_var"], W["bn_w"],
                       W["bn_b"], eps)
    x = x + sgemm(c, W["pw2_w"], W["pw2_b"])
    x = ffn(x, "ff2")
    return layer_norm(x, W["norm_out_w"], W["norm_out_b"], eps)


# ------------------------------------------------------------- bf16 linear ----
def linear_bf16(inp, W, bias=None, act=0, threads: int = 1) -> np.ndarray:
    """asr_gemm::LinearPre: inp [M,K] and W [N,K] as uint16 bf16 bits; fp32 out [M,N].
    threads > 1 splits the N rows over a thread pool (ctypes drops the GIL)."""
    inp = np.ascontiguousarray(inp, dtype=np.uint16)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    M, K = inp.shape
    N = W.shape[0]
    b = f32c(bias) if bias is not None else None

    def part(n0, n1):
        o = np.empty((M, n1 - n0), np.float32)
        bb = np.ascontiguousarray(b[n0:n1]) if b is not None else None
        lib().orc_linear_bf16(_u16(inp), _u16(W[n0:n1]), _f(bb) if bb is not None else None,
                              _f(o), M, K, n1 - n0, act)
        return o

    if threads <= 1 or N < 2 * threads:
        return part(0, N)
    from concurrent.futures import ThreadPoolExecutor
    cuts = np.linspace(0, N, threads + 1).astype(int)
    with ThreadPoolExecutor(threads) as ex:
        parts = list(ex.map(lambda t: part(cuts[t], cuts[t + 1]), range(threads)))
    return np.concatenate(parts, axis=1)


# ----------------------------------------------------------------- decoder ----
EOS_IDS = (151645, 151643)  # src/model/qwen3_asr.cc:160-161
REPEAT_STOP = 6             # src/model/asr_text_decoder.cu:741-757


class OracleDecoder:
    """AsrTextDecoder restated on the oracle primitives (src/model/asr_text_decoder.cu).

    cfg: dict with num_layers, hidden_size, num_q_heads, num_kv_heads, head_dim,
    intermediate_size, vocab_size, max_seq_len, rms_norm_eps, rope_theta.  Weights are numpy:
    embed / lm_head uint16 [vocab, hidden] (lm_head None = tied), final_norm fp32, and per layer
    in_ln, q_norm, k_norm, post_ln fp32 plus qkv_w, o_w, gateup_w, down_w uint16 (fused)."""

    def __init__(self, cfg, embed, final_norm, lm_head, layers, threads: int = 1):
        self.c = dict(cfg)
        self.embed = embed
        self.final_norm = f32c(final_norm)
        self.lm_head = embed if lm_head is None else lm_head
        self.layers = layers
        self.threads = threads
        c = self.c
        shape = (c["max_seq_len"], c["num_kv_heads"], c["head_dim"])
        self.kc = [np.zeros(shape, np.uint16) for _ in range(c["num_layers"])]
        self.vc = [np.zeros(shape, np.uint16) for _ in range(c["num_layers"])]
        self.cache_len = 0
        self.logits = np.zeros(c["vocab_size"], np.float32)

    def _lin(self, x_bf16, W):
        return linear_bf16(x_bf16, W, None, 0, self.threads)

    def _layer_qkv(self, L, x, pos):
        """RmsNorm -> bf16 -> q, k, v -> QK-RMSNorm -> RopeHalf (:518-535 / :398-411)."""
        c = self.c
        Hq, Hkv, Dh, H = c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["hidden_size"]
        Qd, KVd = Hq * Dh, Hkv * Dh
        T = x.shape[0]
        nb = to_bf16(rms_norm(x, L["in_ln"], c["rms_norm_eps"]))
        q = self._lin(nb, L["qkv_w"][:Qd])
        k = self._lin(nb, L["qkv_w"][Qd:Qd + KVd])
        v = self._lin(nb, L["qkv_w"][Qd + KVd:Qd + 2 * KVd])
        q = rms_norm(q.reshape(T * Hq, Dh), L["q_norm"], c["rms_norm_eps"]).reshape(T, Hq, Dh)
        k = rms_norm(k.reshape(T * Hkv, Dh), L["k_norm"], c["rms_norm_eps"]).reshape(T, Hkv, Dh)
        q = rope_half(q, pos, c["rope_theta"])
        k = rope_half(k, pos, c["rope_theta"])
        assert H == x.shape[1]
        return q, k, v.reshape(T, Hkv, Dh)

    def _layer_tail(self, L, x, attn):
        """o projection + residual, RmsNorm, gate/up, SwiGLU, down + residual (:542-556)."""
        c = self.c
        I, T = c["intermediate_size"], x.shape[0]
        x = x + self._lin(to_bf16(attn.reshape(T, -1)), L["o_w"])
        nb = to_bf16(rms_norm(x, L["post_ln"], c["rms_norm_eps"]))
        gate = self._lin(nb, L["gateup_w"][:I])
        up = self._lin(nb, L["gateup_w"][I:2 * I])
        return x + self._lin(to_bf16(swiglu(gate, up)), L["down_w"])

    def _head(self, last):
        c = self.c
        n = rms_norm(last.reshape(1, -1), self.final_norm, c["rms_norm_eps"])
        self.logits = self._lin(to_bf16(n), self.lm_head)[0]

    def prefill_at(self, embeds, pos0: int) -> None:
        """Forward (:457-583) over T rows at positions pos0.. (causal attention a5)."""
        x = f32c(embeds).copy()
        T = x.shape[0]
        pos = np.arange(pos0, pos0 + T, dtype=np.int32)
        scale = 1.0 / np.sqrt(np.float32(self.c["head_dim"]))
        for li, L in enumerate(self.layers):
            q, k, v = self._layer_qkv(L, x, pos)
            kv_write(k, v, self.kc[li], self.vc[li], pos0)
            attn = gqa_prefill(q, self.kc[li], self.vc[li], pos0, float(scale),
                               threads=self.threads)
            x = self._layer_tail(L, x, attn)
        self.cache_len = pos0 + T
        self._head(x[-1])

    def decode_step(self, embed_row, pos: int) -> None:
        """DecodeForwardOnStream (:360-455): one row at pos, decode attention a6."""
        x = f32c(embed_row).reshape(1, -1).copy()
        scale = 1.0 / np.sqrt(np.float32(self.c["head_dim"]))
        p = np.array([pos], np.int32)
        for li, L in enumerate(self.layers):
            q, k, v = self._layer_qkv(L, x, p)
            kv_write(k, v, self.kc[li], self.vc[li], pos)
            attn = gqa_decode(q[0], self.kc[li], self.vc[li], pos, float(scale))
            x = self._layer_tail(L, x, attn[None])
        self.cache_len = pos + 1
        self._head(x[0])

    def embed_row(self, token: int) -> np.ndarray:
        return from_bf16(self.embed[token])

    def argmax(self, ban0=-1, ban1=-1) -> int:
        return argmax_banned(self.logits, ban0, ban1)

    def decode_greedy(self, start_pos, max_new, eos0, eos1, ban_steps=3, batch=32,
                      use_graph=True, graph_ready=False, choose=None):
        """DecodeGreedy (:698-889).  Token j is the argmax with EOS banned iff j < ban_steps
        (seed :767-770 and body argmax :690 under the schedules' ban flags); body k records
        token k and forwards it at start_pos + k.  The host harvests at batch ends and stops at
        EOS (excluded) or the 6th identical token in a row (included); every body of the last
        batch still ran, so cache_len = start_pos + bodies run.  Returns (tokens, bodies).

        choose(j, logits, ban0, ban1) -> token picks stream token j instead of the banned
        argmax (a checker uses it to follow another implementation through near ties)."""
        if max_new <= 0:
            return [], 0
        if choose is None:
            def choose(_j, _logits, b0, b1):
                return self.argmax(b0, b1)
        cums = greedy_schedule(max_new, ban_steps, batch, use_graph, graph_ready)
        toks = [choose(0, self.logits, *((eos0, eos1) if 0 < ban_steps else (-1, -1)))]
        out, stop_at, bodies = [], None, 0
        for end in cums:
            while bodies < end:  # run body `bodies`
                k = bodies
                self.decode_step(self.embed_row(toks[k]), start_pos + k)
                ban = (eos0, eos1) if (k + 1) < ban_steps else (-1, -1)
                toks.append(choose(k + 1, self.logits, *ban))
                bodies += 1
            for i in range(len(out), end):
                t = toks[i]
                if t in (eos0, eos1):
                    stop_at = i
                    break
                out.append(t)
                if len(out) >= REPEAT_STOP and len(set(out[-REPEAT_STOP:])) == 1:
                    stop_at = i
                    break
            if stop_at is not None:
                break
        self.cache_len = start_pos + bodies
        return out, bodies


class BlasOrderDecoder(OracleDecoder):
    """The oracle's composition with every linear layer a float32 BLAS product (blocked
    summation with FMA: another valid fp32 order) instead of the serial chains; weights
    widened to fp32 once and kept.  Its logits beside the oracle's measure the noise that fp32
    summation order alone causes in this composition (bf16 re-rounding of activations turns
    last-bit differences into whole bf16 steps)."""

    _wide: dict = {}

    def _lin(self, x_bf16, W):
        key = (W.__array_interface__["data"][0], W.shape)
        Wf = self._wide.get(key)
        if Wf is None:
            Wf = self._wide[key] = np.ascontiguousarray(from_bf16(W))
        return np.matmul(from_bf16(x_bf16), Wf.T).astype(np.float32)


class TwinDecoder(OracleDecoder):
    """The oracle (its logits are this object's) with a BlasOrderDecoder shadow stepped on the
    same inputs (`shadow.logits`), so a greedy checker can tell a near tie that summation order
    alone can flip from a real disagreement."""

    def __init__(self, cfg, embed, final_norm, lm_head, layers, threads: int = 1):
        super().__init__(cfg, embed, final_norm, lm_head, layers, threads)
        self.shadow = BlasOrderDecoder(cfg, embed, final_norm, lm_head, layers, threads)

    def prefill_at(self, embeds, pos0: int) -> None:
        super().prefill_at(embeds, pos0)
        self.shadow.prefill_at(embeds, pos0)

    def decode_step(self, embed_row, pos: int) -> None:
        super().decode_step(embed_row, pos)
        self.shadow.decode_step(embed_row, pos)


def greedy_schedule(max_new, ban_steps, batch, use_graph, graph_ready):
    """Cumulative body counts at each host harvest of DecodeGreedy
    (src/model/asr_text_decoder.cu:801-884): the eager loop runs banned bodies one at a time
    then batches (:855-866); the graph path first runs one eager warm-up body when the graphs
    are not captured yet (:802-830), then replays the banned graph up to ban_steps - 1 bodies
    and the unbanned graph in batches (:871-884)."""
    batch = max(1, batch)
    cums, emitted = [], 0
    if not use_graph:
        while emitted < max_new:
            nb = (emitted + 1) < ban_steps
            emitted += 1 if nb else min(batch, max_new - emitted)
            cums.append(emitted)
        return cums
    if not graph_ready:
        emitted = 1
        cums.append(1)
    while emitted < max_new:
        in_ban = (emitted + 1) < ban_steps
        limit = min(ban_steps - 1, max_new) if in_ban else max_new
        emitted += max(1, min(batch, limit - emitted))
        cums.append(emitted)
    return cums
