"""fp64 references of the attention formulas, for judging fp32 results at the reference's error
floor 1e-3 (test/unit/model/test_asr_gemm.cc:368): an output near 1e-3 is a cancellation of
terms ~1000x larger, where any fp32 summation order (the oracle's serial one included) is off
by ~1e-4 relative, so a device result is held to being as close to the exact value as the
oracle is (helpers.check_fp32).  Plain softmax attention in numpy float64 over explicit key
ranges; K/V given as float arrays (bf16 caches decoded exactly)."""
from __future__ import annotations

import numpy as np

import oracle_lib as orc


def attention_ranges(q, k, v, scale, lo, hi):
    """Row r of q [R, Hq, Dh] attends keys [lo[r], hi[r]) of k/v [S, Hkv, Dh] (head h uses kv
    head h // (Hq / Hkv)); an empty range gives 0."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    R, Hq, Dh = q.shape
    S, Hkv = k.shape[0], k.shape[1]
    G = Hq // Hkv
    lo = np.broadcast_to(np.asarray(lo), (R,))
    hi = np.broadcast_to(np.asarray(hi), (R,))
    out = np.zeros((R, Hq, Dh))
    j = np.arange(S)[None, :]
    step = max(1, (1 << 24) // max(S, 1))
    for r0 in range(0, R, step):
        r1 = min(R, r0 + step)
        mask = (j >= lo[r0:r1, None]) & (j < hi[r0:r1, None])
        for h in range(Hq):
            s = (q[r0:r1, h] @ k[:, h // G].T) * scale
            s = np.where(mask, s, -np.inf)
            m = np.max(s, axis=1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0.0)
            e = np.exp(s - m)
            l = e.sum(1, keepdims=True)
            out[r0:r1, h] = np.where(l > 0, (e @ v[:, h // G]) / np.where(l > 0, l, 1.0), 0.0)
    return out


def decode_paged(q, kpool, vpool, page_table, page_size, pos, scale):
    """Stream b of q [B, Hq, Dh] attends pos[b] + 1 keys through page-table row b."""
    q = np.asarray(q)
    B = q.shape[0]
    out = np.zeros(q.shape)
    for b in range(B):
        S = int(pos[b]) + 1
        rows = np.asarray(page_table[b])[np.arange(S) // page_size] * page_size + \
            np.arange(S) % page_size
        kp = orc.from_bf16(kpool.reshape(-1, *kpool.shape[-2:])[rows])
        vp = orc.from_bf16(vpool.reshape(-1, *vpool.shape[-2:])[rows])
        out[b] = attention_ranges(q[b][None], kp, vp, scale, 0, S)[0]
    return out


def decode(q, kc, vc, pos, scale):
    """q [Hq, Dh] attends keys [0, pos] of a contiguous bf16 cache."""
    S = min(int(pos) + 1, kc.shape[0])
    return attention_ranges(np.asarray(q)[None], orc.from_bf16(kc[:S]), orc.from_bf16(vc[:S]),
                            scale, 0, S)[0]


def prefill(q, kc, vc, pos0, scale):
    """Row t of q [T, Hq, Dh] attends keys [0, pos0 + t] of a contiguous bf16 cache."""
    T = q.shape[0]
    S = min(pos0 + T, kc.shape[0])
    return attention_ranges(q, orc.from_bf16(kc[:S]), orc.from_bf16(vc[:S]), scale, 0,
                            np.minimum(pos0 + np.arange(T) + 1, S))


def self_attention(q, k, v, scale, causal):
    T = q.shape[0]
    return attention_ranges(q, k, v, scale, 0, np.arange(T) + 1 if causal else T)
