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
