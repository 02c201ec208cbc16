"""Benchmark of the MI355X attention hot path (one GPU).

Headline workload (the decode target "KV length 4096"):
a 28-layer stack of GQA decode attention, Qwen3-1.7B layer shape (16 q / 8 kv heads,
head_dim 128), B = 16 independent streams, base KV length L = 4096, bf16 KV in 16-token
pages with per-stream page tables.  One step = for each of the 28 layers: append the new
token's K/V to the paged cache and attend S = L + t + 1 keys (orator_gqa_decode_append_paged:
the write and the attention share one launch, followed by the split merge).  Inputs are
synthetic and resident in HBM before timing.

`value` = decode-attention algorithmic bytes / wall time of the K timed steps, where the
bytes per (stream, layer, step) are 2*S*Hkv*Dh*2 (K and V read once) + Hq*Dh*4 (q) +
Hq*Dh*4 (out) + 4 B per page-table entry.  The roofline object divides the bytes of one
decode operation (the split-K kernel and its merge, B = 16 streams of one layer) by the
operation's average duration: the HIP events that bracket the timed region on the launch
stream, over its K * 28 back-to-back operations.  The CPU baseline is the oracle's scalar
decode on the host cores, over a bounded sample of the same workload.

Secondary fields: prefill attention (T = 503, 2048; bf16 and fp32 modes), the 17-layer
Conformer rel-pos stack, the decode sweep, the 28-layer decoder end to end, and `aux`: the
windowed attention, the Sortformer MHA and a whole Conformer layer at their reference shapes.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--only PART]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, published

LAYERS, B, HQ, HKV, DH, L_BASE, PAGE = 28, 16, 16, 8, 128, 4096, 16
# HBM bytes per decode op measured with rocprofv3 --pmc at S = 4097..4105 (FETCH_SIZE x 1.9943
# KiB + WRITE_SIZE KiB, profiles/decode_b16_l4096_hbm_traffic.md) and the algorithmic bytes of
# the same ops, for the traffic / algorithmic ratio
HBM_TRAFFIC_PER_OP = 269.36e6
ALGORITHMIC_AT_TRAFFIC = 269.04e6


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="decoder part: run the greedy steps eagerly (same kernels, no graph "
                         "replay), e.g. for a per-kernel profile")
    ap.add_argument("--only", choices=["decode", "prefill", "conformer", "sweep", "decoder",
                                       "aux", "copy"],
                    default=None,
                    help="run one part (for profiling); prints that part's numbers only")
    return ap.parse_args()


def decode_bytes(S: int, n_pages: int) -> int:
    return 2 * S * HKV * DH * 2 + HQ * DH * 4 * 2 + 4 * n_pages


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def run_decode(steps: int, warmup: int):
    from orator_amd import decoder_attn as da
    from orator_amd._lib import call
    from orator_amd.runtime import DeviceBuffer, Event, Stream, synchronize

    total_tok = L_BASE + warmup + steps + 1
    max_pages = (total_tok + PAGE - 1) // PAGE
    n_pages = B * max_pages
    pool_elems = n_pages * PAGE * HKV * DH
    log(f"decode: {LAYERS} layers x B={B} x L={L_BASE}, {max_pages} pages/stream, "
        f"{2 * LAYERS * pool_elems * 2 / 1e9:.2f} GB of KV")

    rng = np.random.default_rng(1234)
    # One random block, tiled over every pool with device copies: contents do not change
    # the traffic, and host generation of 7.8 GB would dominate the run.
    block = (rng.standard_normal(1 << 22).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    dblock = DeviceBuffer.from_array(block)
    stream = Stream()

    def filled_pool():
        buf = DeviceBuffer(pool_elems * 2)
        off = 0
        while off < buf.nbytes:
            n = min(dblock.nbytes, buf.nbytes - off)
            call("orator_memcpy_dtod", buf.ptr + off, dblock.ptr, n, stream.handle)
            off += n
        return buf

    kpools = [filled_pool() for _ in range(LAYERS)]
    vpools = [filled_pool() for _ in range(LAYERS)]
    stream.synchronize()
    # page tables: a random permutation of the pool per layer
    tables = []
    for _ in range(LAYERS):
        perm = rng.permutation(n_pages).astype(np.int32).reshape(B, max_pages)
        tables.append(DeviceBuffer.from_array(perm))
    n_var = 4
    qs = [DeviceBuffer.from_array(rng.standard_normal((B, HQ, DH)).astype(np.float32))
          for _ in range(n_var)]
    ks = [DeviceBuffer.from_array(rng.standard_normal((B, 1, HKV, DH)).astype(np.float32))
          for _ in range(n_var)]
    vs = [DeviceBuffer.from_array(rng.standard_normal((B, 1, HKV, DH)).astype(np.float32))
          for _ in range(n_var)]
    outs = DeviceBuffer(B * HQ * DH * 4)
    n_all = warmup + steps
    pos_all = (L_BASE + np.arange(n_all, dtype=np.int32))[:, None].repeat(B, 1)
    dpos = DeviceBuffer.from_array(np.ascontiguousarray(pos_all))
    scale = 1.0 / math.sqrt(DH)

    def step(t):
        pos_ptr = dpos.ptr + t * B * 4
        v = t % n_var
        for l in range(LAYERS):
            # KV append of the new token + attention over pos + 1 keys, one launch (+ merge)
            da.GqaDecodeAttnAppendPaged(qs[v], ks[v], vs[v], kpools[l], vpools[l], tables[l],
                                        max_pages, PAGE, n_pages, pos_ptr, outs, B, HQ, HKV, DH,
                                        scale, stream)

    for t in range(warmup):
        step(t)
    stream.synchronize()
    synchronize()

    # ---- whole-job timing: exactly `steps` steps between two device syncs ----
    e0, e1 = Event(), Event()
    t_wall0 = time.perf_counter()
    e0.record(stream)
    for t in range(warmup, warmup + steps):
        step(t)
    e1.record(stream)
    stream.synchronize()
    synchronize()
    wall_s = time.perf_counter() - t_wall0
    gpu_ms = e0.elapsed_ms(e1)
    step_bytes = sum(B * decode_bytes(L_BASE + t + 1, (L_BASE + t + 1 + PAGE - 1) // PAGE)
                     for t in range(warmup, warmup + steps)) * LAYERS
    elapsed_s = max(wall_s, gpu_ms / 1e3)
    value_gbs = step_bytes / elapsed_s / 1e9

    # ---- the decode operation's average duration: the HIP events bracketing the timed
    # region on the launch stream, over its steps * LAYERS back-to-back operations (each the
    # split-K kernel and its merge; nothing else runs on the stream in between) ----
    n_ops = steps * LAYERS
    avg_ms = gpu_ms / n_ops
    op_bytes = step_bytes / n_ops
    achieved = op_bytes / (avg_ms / 1e3) / 1e9

    # ---- the access pattern's streaming ceiling: the same K/V bytes of every layer read by
    # the read probe (the decode grid and loads, no arithmetic, no partials, no merge) ----
    S_last = L_BASE + warmup + steps
    sink = DeviceBuffer(4)
    probe = lambda l: call("orator_decode_read_probe", kpools[l].ptr, vpools[l].ptr,
                           tables[l].ptr, max_pages, PAGE, S_last, B, HKV, sink.ptr,
                           stream.handle)
    for l in range(LAYERS):
        probe(l)
    stream.synchronize()
    p0, p1 = Event(), Event()
    p0.record(stream)
    for r in range(2):
        for l in range(LAYERS):
            probe(l)
    p1.record(stream)
    stream.synchronize()
    probe_us = p0.elapsed_ms(p1) * 1e3 / (2 * LAYERS)
    probe_gbs = B * 2 * S_last * HKV * DH * 2 / (probe_us * 1e-6) / 1e9

    # ---- spot parity of the last launch against the oracle (stream 0..1, layer 27) ----
    parity = spot_check(kpools[-1], vpools[-1], tables[-1], max_pages, qs, outs,
                        L_BASE + warmup + steps - 1, (warmup + steps - 1) % n_var, scale)
    return {
        "gpu_ms": gpu_ms, "wall_s": wall_s, "ms_per_step": elapsed_s * 1e3 / steps,
        "value_gbs": value_gbs, "kernel_avg_us": avg_ms * 1e3,
        "kernel_bytes": op_bytes, "achieved_gbs": achieved,
        "max_pages": max_pages, "parity": parity,
        "read_probe_us": probe_us, "read_probe_gbs": probe_gbs,
    }


def run_prefill(T: int, mode: int, iters: int = 20):
    """Prefill attention over one layer's bf16 cache at pos0 = 0 (BASELINE configs[1] shape
    for T = 503; T = 2048 is the throughput target), rotating over 4 layers' caches.
    Returns the kernel's average time and algorithmic causal TFLOP/s, 4*Hq*Dh*T(T+1)/2."""
    from orator_amd import decoder_attn as da
    from orator_amd.runtime import DeviceBuffer, Event, Stream

    rng = np.random.default_rng(T)
    st = Stream()
    nl = 4
    bits = lambda shape: DeviceBuffer.from_array(
        (rng.standard_normal(shape).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
    kc = [bits((T, HKV, DH)) for _ in range(nl)]
    vc = [bits((T, HKV, DH)) for _ in range(nl)]
    q = DeviceBuffer.from_array(rng.standard_normal((T, HQ, DH)).astype(np.float32))
    qb = bits((T, HQ, DH))
    out = DeviceBuffer(T * HQ * DH * 4)
    pos = DeviceBuffer.from_array(np.zeros(1, np.int32))
    scale = 1.0 / math.sqrt(DH)

    def run(l):
        if mode == da.PREFILL_BF16:
            da.GqaCacheAttnEx(None, qb, kc[l], vc[l], None, 0, 0, out, T, HQ, HKV, DH, pos, T,
                              scale, mode, st)
        else:
            da.GqaCacheAttnEx(q, None, kc[l], vc[l], None, 0, 0, out, T, HQ, HKV, DH, pos, T,
                              scale, mode, st)

    for l in range(nl):
        run(l)
    st.synchronize()
    e0, e1 = Event(), Event()
    e0.record(st)
    for i in range(iters):
        run(i % nl)
    e1.record(st)
    st.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / iters
    flops = 4.0 * HQ * DH * T * (T + 1) / 2
    tf = flops / (us * 1e-6) / 1e12
    return {"T": T, "mode": "bf16" if mode == da.PREFILL_BF16 else "fp32", "us": round(us, 2),
            "tflops": round(tf, 2), "frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4)}


def run_conformer(T: int = 717, layers: int = 17, H: int = 8, Dk: int = 64):
    """17 back-to-back rel-pos MHSA cores, T = 717, fp16 inputs N(0,1),
    non-causal.  Algorithmic flops 6*H*T^2*Dk per layer (AC, the used BD band, PV)."""
    from orator_amd import conformer_attn as ca
    from orator_amd.runtime import DeviceBuffer, Event, Stream

    rng = np.random.default_rng(4)
    st = Stream()
    f16 = lambda shape: DeviceBuffer.from_array(
        rng.standard_normal(shape).astype(np.float16).view(np.uint16))
    f32 = lambda shape: DeviceBuffer.from_array(rng.standard_normal(shape).astype(np.float32))
    P = 2 * T - 1
    ins = [(f16((T, H, Dk)), f16((T, H, Dk)), f16((T, H, Dk)), f16((P, H, Dk))) for _ in range(layers)]
    ins32 = [f32((T, H, Dk)), f32((T, H, Dk)), f32((T, H, Dk)), f32((P, H, Dk))]
    u, vb = f32((H, Dk)), f32((H, Dk))
    out = DeviceBuffer(T * H * Dk * 4)
    scale = 1.0 / math.sqrt(Dk)
    for l in range(layers):
        ca.RelPosAttentionFast(*ins[l], u, vb, out, T, H, Dk, T, scale, True, st)
    ca.RelPosAttention(*ins32, u, vb, out, T, H, Dk, T, scale, st)
    st.synchronize()
    e0, e1, e2 = Event(), Event(), Event()
    reps = 5
    e0.record(st)
    for _ in range(reps):
        for l in range(layers):
            ca.RelPosAttentionFast(*ins[l], u, vb, out, T, H, Dk, T, scale, True, st)
    e1.record(st)
    for _ in range(reps):
        ca.RelPosAttention(*ins32, u, vb, out, T, H, Dk, T, scale, st)
    e2.record(st)
    st.synchronize()
    us_f16 = e0.elapsed_ms(e1) * 1e3 / (reps * layers)
    us_f32 = e1.elapsed_ms(e2) * 1e3 / reps
    flops = 6.0 * H * T * T * Dk
    tf = flops / (us_f16 * 1e-6) / 1e12
    return {"T": T, "layers": layers, "fused_f16_us_per_layer": round(us_f16, 2),
            "fused_f16_tflops": round(tf, 2), "frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
            "stack_ms": round(us_f16 * layers / 1e3, 4),
            "fp32_reference_order_us_per_layer": round(us_f32, 2)}


FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 (the VALU-bound aux kernels are quoted against it)


def run_aux(reps: int = 20):
    """The path's sibling operators at their reference shapes:
    * the audio tower's windowed self-attention (asr_audio_tower.cu:204-258): 390 frames (30 s
      of audio after the CNN), 104-frame windows (:510), 16 heads x Dh 64, fp32;
    * the Sortformer decoder's masked MHA (sortformer_decoder.cu:280-298): T = 717, 8 heads x
      Dk 24 (d_model 192), fp32;
    * one whole FastConformer layer (conformer_layer.cu:364-488): T = 717, d_model 512, 8 heads,
      d_ff 2048, conv kernel 9, both attention modes.
    Algorithmic flops: attention 4*H*Dh*(attended pairs); the layer's GEMMs 2*rows*in*out each
    plus its rel-pos core 6*H*T^2*Dk."""
    from orator_amd import audio_attn, conformer_attn as ca, sortformer_attn
    from orator_amd.runtime import DeviceBuffer, Event, Stream

    rng = np.random.default_rng(9)
    st = Stream()
    f32 = lambda shape, s=1.0: DeviceBuffer.from_array(
        (s * rng.standard_normal(shape)).astype(np.float32))

    def timed(fn):
        fn()
        st.synchronize()
        e0, e1 = Event(), Event()
        e0.record(st)
        for _ in range(reps):
            fn()
        e1.record(st)
        st.synchronize()
        return e0.elapsed_ms(e1) * 1e3 / reps

    out = {}
    # windowed attention
    N, H, Dh, W = 390, 16, 64, 104
    bounds = list(range(0, N, W)) + [N]
    seg_s = np.concatenate([[a] * (b - a) for a, b in zip(bounds[:-1], bounds[1:])]).astype(np.int32)
    seg_e = np.concatenate([[b] * (b - a) for a, b in zip(bounds[:-1], bounds[1:])]).astype(np.int32)
    q, k, v, o = f32((N, H, Dh)), f32((N, H, Dh)), f32((N, H, Dh)), DeviceBuffer(N * H * Dh * 4)
    ds, de = DeviceBuffer.from_array(seg_s), DeviceBuffer.from_array(seg_e)
    us = timed(lambda: audio_attn.WindowAttention(q, k, v, o, ds, de, N, H, Dh, 0.125, st))
    pairs = sum((b - a) ** 2 for a, b in zip(bounds[:-1], bounds[1:]))
    fl = 4.0 * H * Dh * pairs
    out["window_attention"] = {"N": N, "H": H, "Dh": Dh, "window": W, "us": round(us, 2),
                               "tflops": round(fl / us / 1e6, 3),
                               "GBs": round(4 * N * H * Dh * 4 / us / 1e3, 1)}
    # Sortformer masked MHA
    T, H, Dk = 717, 8, 24
    q, k, v, o = f32((T, H, Dk)), f32((T, H, Dk)), f32((T, H, Dk)), DeviceBuffer(T * H * Dk * 4)
    us = timed(lambda: sortformer_attn.MaskedSelfAttention(q, k, v, o, T, H, Dk, T,
                                                          1.0 / math.sqrt(Dk), st))
    fl = 4.0 * H * Dk * T * T
    out["sortformer_mha"] = {"T": T, "H": H, "Dk": Dk, "us": round(us, 2),
                             "tflops": round(fl / us / 1e6, 3),
                             "frac_fp32": round(fl / us / 1e6 / FP32_PEAK_TFLOPS, 4)}
    # whole Conformer layer
    T, D, H, Dff, K = 717, 512, 8, 2048, 9
    lin = lambda n_out, n_in: f32((n_out, n_in), 1.0 / math.sqrt(n_in))
    vec = lambda n, s=0.1: f32((n,), s)
    w = {}
    for p in ("ff1", "ff2"):
        w[f"norm_{p}_w"], w[f"norm_{p}_b"] = vec(D), vec(D)
        w[f"{p}_w1"], w[f"{p}_b1"], w[f"{p}_w2"], w[f"{p}_b2"] = lin(Dff, D), vec(Dff), lin(D, Dff), vec(D)
    for n in ("att", "conv", "out"):
        w[f"norm_{n}_w"], w[f"norm_{n}_b"] = vec(D), vec(D)
    for n in ("q", "k", "v", "out"):
        w[f"{n}_w"], w[f"{n}_b"] = lin(D, D), vec(D)
    w["pos_w"], w["pos_bias_u"], w["pos_bias_v"] = lin(D, D), vec(D), vec(D)
    w["pw1_w"], w["pw1_b"], w["pw2_w"], w["pw2_b"] = lin(2 * D, D), vec(2 * D), lin(D, D), vec(D)
    w["dw_w"], w["dw_b"] = f32((D, K), 1.0 / math.sqrt(K)), vec(D)
    w["bn_w"], w["bn_b"], w["bn_mean"] = vec(D), vec(D), vec(D)
    w["bn_var"] = DeviceBuffer.from_array((0.5 + rng.uniform(size=D)).astype(np.float32))
    layer = ca.ConformerLayer(w, D, H, Dff, K)
    pe = DeviceBuffer.from_array(ca.BuildPosEmb(T, D))
    x = f32((T, D))
    gemm = 2.0 * (T * D * Dff * 4 + T * D * D * 5 + (2 * T - 1) * D * D + T * D * 2 * D)
    att = 6.0 * H * T * T * (D // H)
    for mode, name in ((1, "fused_f16"), (0, "fp32")):
        us = timed(lambda: layer.Forward(x, T, T, pe, st, attn_mode=mode))
        out[f"conformer_layer_{name}"] = {"T": T, "d_model": D, "us": round(us, 2),
                                          "tflops": round((gemm + att) / us / 1e6, 2)}
    layer.close()
    return out


def run_decoder_e2e(T: int = 2048, new: int = 256, use_graph: bool = True):
    """the full synthetic Qwen3-ASR text decoder (28 layers, hidden 2048,
    16/8 heads, head_dim 128, SwiGLU 6144, vocab 151936, lm_head tied to embed as
    asr_text_decoder.cu:255-257), random-init bf16 weights, a 2048-row prefill of N(0, 0.02)
    embeddings, then `new` greedy tokens through DecodeGreedy (graph replay, batch 32).  EOS is
    disabled (ids -1) so the run is not cut short by a random model; the repetition stop of
    the reference stays, and the tokens actually run are reported.  Per-token bytes: every
    weight once (layers + lm_head) plus the K/V rows attended."""
    from orator_amd._lib import call
    from orator_amd.decoder import AsrTextConfig, AsrTextDecoder
    from orator_amd.runtime import DeviceBuffer, synchronize

    cfg = AsrTextConfig(max_seq_len=T + new)
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    Qd, KVd = cfg.num_q_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    rng = np.random.default_rng(77)
    pool_n = 1 << 25
    pool = DeviceBuffer.from_array(
        (rng.standard_normal(pool_n, dtype=np.float32) * np.float32(0.02)).view(np.uint32)
        .__rshift__(16).astype(np.uint16))

    def weight(n):
        # windows of the random pool at random offsets: every matrix differs, no host
        # generation of 3.4 GB
        buf = DeviceBuffer(n * 2)
        off = 0
        while off < n:
            m = min(n - off, pool_n // 2)
            src = int(rng.integers(0, pool_n - m + 1))
            call("orator_memcpy_dtod", buf.ptr + 2 * off, pool.ptr + 2 * src, 2 * m, None)
            off += m
        return buf

    def gain(n):
        return DeviceBuffer.from_array((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))

    embed = weight(V * H)
    final_norm = gain(H)
    layers = [dict(in_ln=gain(H), q_norm=gain(cfg.head_dim), k_norm=gain(cfg.head_dim),
                   post_ln=gain(H), qkv_w=weight((Qd + 2 * KVd) * H), o_w=weight(H * Qd),
                   gateup_w=weight(2 * I * H), down_w=weight(H * I))
              for _ in range(cfg.num_layers)]
    synchronize()
    dec = AsrTextDecoder(cfg, embed, final_norm, None, layers)
    emb = DeviceBuffer.from_array((0.02 * rng.standard_normal((T, H))).astype(np.float32))
    # warm-up: one prefill and a short greedy run (captures the step graphs)
    dec.Prefill(emb, T)
    dec.DecodeGreedy(T, 8, -1, -1, ban_steps=3, batch=32, use_graph=use_graph)
    t0 = time.perf_counter()
    dec.Prefill(emb, T)  # synchronises
    prefill_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    toks = dec.DecodeGreedy(T, new, -1, -1, ban_steps=3, batch=32, use_graph=use_graph)
    decode_s = time.perf_counter() - t0
    bodies = dec.cache_len() - T
    # eager bodies must give the same tokens as the replayed graphs
    dec.Prefill(emb, T)
    n_chk = min(32, len(toks))
    eager = dec.DecodeGreedy(T, n_chk, -1, -1, ban_steps=3, batch=32, use_graph=False)
    layer_w = (Qd + 2 * KVd) * H + H * Qd + 2 * I * H + H * I
    w_bytes = 2 * (cfg.num_layers * layer_w + V * H)
    kv_bytes = np.mean([cfg.num_layers * (T + k + 1) * KVd * 2 * 2 for k in range(bodies)])
    tok_s = bodies / decode_s
    dec.close()
    return {"workload": "configs[4]: 28-layer Qwen3-ASR-shaped decoder, prefill 2048 + "
                        f"{new} greedy tokens, batch 1",
            "prefill_ms": round(prefill_s * 1e3, 2),
            "prefill_tok_s": round(T / prefill_s, 1),
            "decode_tokens": len(toks), "decode_steps_run": int(bodies),
            "decode_tok_s": round(tok_s, 1), "decode_ms_per_token": round(decode_s * 1e3 / bodies, 4),
            "decode_bytes_per_token": int(w_bytes + kv_bytes),
            "decode_achieved_gbs": round((w_bytes + kv_bytes) * tok_s / 1e9, 1),
            "decode_frac_of_hbm_peak": round((w_bytes + kv_bytes) * tok_s / 1e9 / HBM_PEAK_GBS, 4),
            "graph_replay": use_graph,
            "graph_equals_eager_first_tokens": [int(t) for t in eager] == [int(t) for t in toks[:n_chk]]}


def run_copy_bandwidth(nbytes: int = 1 << 30, reps: int = 10):
    """Attainable HBM bandwidth of a plain device copy (hipMemcpyAsync device to device, the
    runtime's copy kernel) of 1 GiB: (read + write bytes) / time, the practical ceiling the
    decode kernel's fraction of the published 8 TB/s should be read against."""
    from orator_amd._lib import call
    from orator_amd.runtime import DeviceBuffer, Event, Stream

    st = Stream()
    src, dst = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    call("orator_memset", src.ptr, 1, nbytes, st.handle)
    call("orator_memcpy_dtod", dst.ptr, src.ptr, nbytes, st.handle)
    st.synchronize()
    e0, e1 = Event(), Event()
    e0.record(st)
    for _ in range(reps):
        call("orator_memcpy_dtod", dst.ptr, src.ptr, nbytes, st.handle)
    e1.record(st)
    st.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / reps
    return {"bytes_copied": nbytes, "us": round(us, 1),
            "GBs_read_plus_write": round(2 * nbytes / (us * 1e-6) / 1e9, 1)}


def run_decode_sweep():
    """BASELINE configs[2] sweep: decode kernel GB/s at L in {1024, 2048, 4096}, B in {1, 16}
    (one launch per layer over 28 layers' paged caches)."""
    from orator_amd import decoder_attn as da
    from orator_amd._lib import call
    from orator_amd.runtime import DeviceBuffer, Event, Stream

    st = Stream()
    rng = np.random.default_rng(9)
    block = (rng.standard_normal(1 << 22).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    dblock = DeviceBuffer.from_array(block)
    res = []
    for B_ in (1, 16):
        for L in (1024, 2048, 4096):
            S = L + 1
            mp = (S + PAGE - 1) // PAGE
            npg = B_ * mp
            elems = npg * PAGE * HKV * DH
            nl = 28
            pools = []
            for _ in range(2 * nl):
                buf = DeviceBuffer(elems * 2)
                off = 0
                while off < buf.nbytes:
                    n = min(dblock.nbytes, buf.nbytes - off)
                    call("orator_memcpy_dtod", buf.ptr + off, dblock.ptr, n, st.handle)
                    off += n
                pools.append(buf)
            tab = DeviceBuffer.from_array(rng.permutation(npg).astype(np.int32).reshape(B_, mp))
            q = DeviceBuffer.from_array(rng.standard_normal((B_, HQ, DH)).astype(np.float32))
            out = DeviceBuffer(B_ * HQ * DH * 4)
            pos = DeviceBuffer.from_array(np.full(B_, S - 1, np.int32))
            run = lambda l: da.GqaDecodeAttnPaged(q, pools[2 * l], pools[2 * l + 1], tab, mp, PAGE,
                                                  pos, out, B_, HQ, HKV, DH, 0.0884, st)
            for l in range(nl):
                run(l)
            st.synchronize()
            e0, e1 = Event(), Event()
            e0.record(st)
            for r in range(3):
                for l in range(nl):
                    run(l)
            e1.record(st)
            st.synchronize()
            us = e0.elapsed_ms(e1) * 1e3 / (3 * nl)
            gbs = B_ * decode_bytes(S, mp) / (us * 1e-6) / 1e9
            res.append({"B": B_, "L": L, "us_per_layer": round(us, 2), "GBs": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "footprint_MB": round(nl * B_ * decode_bytes(S, mp) / 1e6, 1)})
            del pools
    return res


def spot_check(kpool, vpool, table, max_pages, qs, outs, last_pos, var, scale):
    """Recomputes streams 0-1 of the last decode launch with the oracle."""
    try:
        sys.path.insert(0, str(ROOT / "tests"))
        import oracle_lib as orc
        from helpers import rel_err
    except Exception as e:  # the oracle is the checker only
        return {"skipped": str(e)}
    nb = 2
    tab = table.download(np.int32, (B, max_pages))[:nb]
    need = sorted(set(tab[:, : (last_pos + PAGE) // PAGE].ravel().tolist()))
    page_elems = PAGE * HKV * DH
    remap = {p: i for i, p in enumerate(need)}
    kp = np.stack([kpool.download(np.uint16, (page_elems,), p * page_elems * 2) for p in need])
    vp = np.stack([vpool.download(np.uint16, (page_elems,), p * page_elems * 2) for p in need])
    kp = kp.reshape(len(need), PAGE, HKV, DH)
    vp = vp.reshape(len(need), PAGE, HKV, DH)
    t2 = np.vectorize(lambda p: remap.get(int(p), 0))(tab).astype(np.int32)
    q = qs[var].download(np.float32, (B, HQ, DH))[:nb]
    got = outs.download(np.float32, (B, HQ, DH))[:nb]
    ref = orc.gqa_decode_paged(q, kp, vp, t2, PAGE, np.full(nb, last_pos, np.int32), scale,
                               threads=min(8, os.cpu_count() or 1))
    return {"streams": nb, "max_rel_err": rel_err(got, ref, 0.05), "floor": 0.05}


def _cpu_info():
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return cores, model


def _median_rate(fn, units_per_call, seconds, max_calls=400, min_calls=3):
    """Runs fn until `seconds` have passed (at least min_calls); returns (median units/s,
    calls)."""
    rates, t_end = [], time.perf_counter() + seconds
    while len(rates) < max_calls:
        t0 = time.perf_counter()
        fn()
        rates.append(units_per_call / (time.perf_counter() - t0))
        if len(rates) >= min_calls and time.perf_counter() >= t_end:
            break
    return float(np.median(rates)), len(rates)


def cpu_baseline(seconds: float):
    """The oracle (scalar C, -O3, no SIMD intrinsics, no fp contraction) timed on the host cores
    beside the GPU: the headline decode workload (one layer-step of B = 16 paged streams at S =
    4097) on 1 thread and on all cores (<= 16), the median of repeated calls within a bounded
    time each; plus fp32 prefill attention (T = 503 on 1 thread and all cores, T = 2048 on all
    cores) and the fp32 Conformer rel-pos core (T = 717, the reference's decomposition,
    1 thread) at their algorithmic flops."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as orc

    cores, model = _cpu_info()
    threads = max(1, min(16, cores))
    S = L_BASE + 1
    max_pages = (S + PAGE - 1) // PAGE
    n_pages = B * max_pages
    rng = np.random.default_rng(7)
    block = (rng.standard_normal(1 << 22).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    pool_elems = n_pages * PAGE * HKV * DH
    reps = -(-pool_elems // block.size)
    kp = np.tile(block, reps)[:pool_elems].reshape(n_pages, PAGE, HKV, DH)
    vp = np.roll(np.tile(block, reps)[:pool_elems], 12345).reshape(n_pages, PAGE, HKV, DH)
    table = rng.permutation(n_pages).astype(np.int32).reshape(B, max_pages)
    q = rng.standard_normal((B, HQ, DH)).astype(np.float32)
    pos = np.full(B, S - 1, np.int32)
    op_bytes = B * decode_bytes(S, max_pages)
    dec = lambda th: orc.gqa_decode_paged(q, kp, vp, table, PAGE, pos, 1.0 / math.sqrt(DH),
                                          threads=th)
    gbs_1, n_1 = _median_rate(lambda: dec(1), op_bytes / 1e9, 0.25 * seconds)
    gbs_n, n_n = _median_rate(lambda: dec(threads), op_bytes / 1e9, 0.25 * seconds)

    # prefill (fp32 mode, bf16 cache) and the Conformer core
    def prefill_case(T, th):
        qq = rng.standard_normal((T, HQ, DH)).astype(np.float32)
        kc = (rng.standard_normal((T, HKV, DH)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        vc = (rng.standard_normal((T, HKV, DH)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        fl = 4.0 * HQ * DH * T * (T + 1) / 2 / 1e9
        return _median_rate(lambda: orc.gqa_prefill(qq, kc, vc, 0, 1.0 / math.sqrt(DH),
                                                    threads=th), fl, 0.1 * seconds, min_calls=1)
    p503_1, _ = prefill_case(503, 1)
    p503_n, _ = prefill_case(503, threads)
    p2048_n, _ = prefill_case(2048, threads)
    T, H, Dk = 717, 8, 64
    x = lambda shape: rng.standard_normal(shape).astype(np.float32)
    cq, ck, cv, cp, cu, cb = x((T, H, Dk)), x((T, H, Dk)), x((T, H, Dk)), x((2 * T - 1, H, Dk)), \
        x((H, Dk)), x((H, Dk))
    conf_1, _ = _median_rate(lambda: orc.relpos_attention(cq, ck, cv, cp, cu, cb, T, 0.125),
                             6.0 * H * T * T * Dk / 1e9, 0.1 * seconds, min_calls=1)
    return {"value": round(gbs_n, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"median of {n_n} calls of one layer-step of the headline workload (B={B} "
                      f"paged decode at S={S}, {op_bytes / 1e6:.1f} MB) through the oracle's "
                      f"orc_gqa_decode_paged_mt on {threads} threads",
            "single_thread": {"value": round(gbs_1, 3), "unit": "GB/s", "cores": 1,
                              "sample": f"median of {n_1} calls, same layer-step"},
            "prefill_fp32": {"T503_1thread_gflops": round(p503_1, 3),
                             f"T503_{threads}threads_gflops": round(p503_n, 3),
                             f"T2048_{threads}threads_gflops": round(p2048_n, 3),
                             "flops": "4*Hq*Dh*T(T+1)/2 (causal, algorithmic)"},
            "conformer_relpos_fp32": {"T717_1thread_gflops": round(conf_1, 3),
                                      "flops": "6*H*T^2*Dk (algorithmic; the oracle runs the "
                                               "reference decomposition)"},
            "cpu_model": model, "cores_visible": cores}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    from orator_amd.runtime import device_name
    log("device:", device_name())
    if args.only:
        from orator_amd import decoder_attn as da
        part = {"decode": lambda: run_decode(args.steps, args.warmup),
                "prefill": lambda: [run_prefill(503, da.PREFILL_BF16),
                                    run_prefill(2048, da.PREFILL_BF16)],
                "conformer": run_conformer, "sweep": run_decode_sweep,
                "copy": run_copy_bandwidth,
                "decoder": lambda: run_decoder_e2e(use_graph=not args.no_graph),
                "aux": run_aux}[args.only]()
        print(json.dumps({"only": args.only, "result": part}, default=float))
        return
    dec = run_decode(args.steps, args.warmup)
    copy = run_copy_bandwidth()
    log("copy:", copy)
    log(f"decode: {dec['ms_per_step']:.3f} ms/step, {dec['value_gbs']:.1f} GB/s; op "
        f"{dec['kernel_avg_us']:.1f} us avg -> {dec['achieved_gbs']:.1f} GB/s; read probe "
        f"{dec['read_probe_us']:.1f} us ({dec['read_probe_gbs']:.1f} GB/s); parity {dec['parity']}")
    from orator_amd import decoder_attn as da
    pre = [run_prefill(503, da.PREFILL_BF16), run_prefill(503, da.PREFILL_FP32),
           run_prefill(2048, da.PREFILL_BF16), run_prefill(2048, da.PREFILL_FP32)]
    log("prefill:", pre)
    conf = run_conformer()
    log("conformer:", conf)
    sweep = run_decode_sweep()
    log("decode sweep:", sweep)
    e2e = run_decoder_e2e()
    log("decoder e2e:", e2e)
    aux = run_aux()
    log("aux:", aux)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": "GQA decode-attn HBM GB/s (% peak); prefill-attn TFLOP/s (% MFMA peak)",
        "value": round(dec["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode sweep (configs[2]): 28-layer GQA decode, B=16, L=4096, "
                               "16q/8kv heads, Dh=128, bf16 paged KV (16-token pages), fp32 q/acc",
                   "layers": LAYERS, "batch": B, "kv_len": L_BASE, "page_size": PAGE,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(dec["achieved_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec["achieved_gbs"] / HBM_PEAK_GBS, 4),
                     # rocprofv3 FETCH_SIZE x 1.9943 + WRITE_SIZE x 1.0 KiB per decode op
                     # (one launch of the wide split kernel, its ranges merged in the launch)
                     # at this workload, S = 4097..4105.
                     "traffic": HBM_TRAFFIC_PER_OP,
                     "traffic_over_algorithmic": round(HBM_TRAFFIC_PER_OP / ALGORITHMIC_AT_TRAFFIC, 3),
                     "kernel": "decode op = gqa_decode_wide_kernel, one launch (each stream and kv "
                               "head cut into a 2048-key and a 2112-key range, one 8-wave "
                               "workgroup each; the last of the two to finish merges them); "
                               "average over the timed region's back-to-back ops (HIP events "
                               "on its stream)",
                     "kernel_avg_us": round(dec["kernel_avg_us"], 2),
                     "bytes_per_launch": int(dec["kernel_bytes"]),
                     "attainable_copy_gbs": copy["GBs_read_plus_write"],
                     "frac_of_attainable_copy": round(dec["achieved_gbs"] /
                                                      copy["GBs_read_plus_write"], 4),
                     # the same K/V bytes read with the decode kernels' access pattern and
                     # nothing else (orator_decode_read_probe over the 28 layers' pools)
                     "attainable_read_gbs": round(dec["read_probe_gbs"], 1),
                     "read_probe_us": round(dec["read_probe_us"], 2),
                     "frac_of_attainable_read": round(dec["achieved_gbs"] /
                                                      dec["read_probe_gbs"], 4)},
        "cpu_baseline": cpu,
        "parity": dec["parity"],
        "prefill": pre,
        "conformer_relpos": conf,
        "decode_sweep": sweep,
        "decoder_e2e": e2e,
        "aux": aux,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
