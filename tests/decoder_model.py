"""Seeded synthetic decoder weights (random-init, Qwen3-ASR decoder layout) for the decoder
tests: numpy arrays in the fused layout the library and the oracle both take."""
from __future__ import annotations

import numpy as np


SMALL = dict(num_layers=2, hidden_size=512, num_q_heads=4, num_kv_heads=2, head_dim=128,
             intermediate_size=1024, vocab_size=4096, max_seq_len=256, rms_norm_eps=1e-6,
             rope_theta=1e6)

# Qwen3-ASR-1.7B text decoder shapes (include/model/asr_text_decoder.h:30-42), 2 layers.
QWEN_2L = dict(num_layers=2, hidden_size=2048, num_q_heads=16, num_kv_heads=8, head_dim=128,
               intermediate_size=6144, vocab_size=151936, max_seq_len=2048, rms_norm_eps=1e-6,
               rope_theta=1e6)


# the full Qwen3-ASR-1.7B-shaped decoder (28 layers), context for a
# 2048-row prefill plus 256 greedy steps.
QWEN_28L = dict(QWEN_2L, num_layers=28, max_seq_len=2048 + 256)

# The configs[4] greedy-parity run (tests/golden/make_decoder_greedy_golden.py writes its
# oracle tokens; tests/test_gpu_decoder_c5.py replays them): seeds of the weights and of the
# N(0, 0.02) prefill embeddings, lm_head tied to the embedding as in Qwen3-1.7B.  The weight
# seed is one whose greedy stream does not repeat a token 6 times within 256 steps, so the
# reference's repetition stop (asr_text_decoder.cu:741-757) does not end the graph-replayed
# run early (seed 2026 stopped after 26 tokens, 2028 after 73, 2030 after 214).
C5 = dict(weight_seed=2032, embed_seed=2033, prefill=2048, new=256, topk=32)


def c5_inputs():
    """(cfg, weights, prefill embeddings) of the configs[4] greedy-parity run."""
    from helpers import SplitMix64
    cfg = dict(QWEN_28L)
    w = make_weights(cfg, C5["weight_seed"], tied=True)
    emb = SplitMix64(C5["embed_seed"]).normal((C5["prefill"], cfg["hidden_size"]), 0.02)
    return cfg, w, emb


def make_weights(cfg, seed: int, w_scale: float = 0.02, tied: bool = False,
                 layer_scale: float = 1.0):
    """Returns (embed, final_norm, lm_head or None, layers).  Matmul weights are random bf16
    bit patterns: random sign and mantissa, magnitude in [s/8, 2s) around s = w_scale (times
    layer_scale inside the layers), drawn straight as integers because the vocab-sized
    matrices are too large to draw as normals in a test; norm gains 1 + N(0, 0.1).  Both sides
    of every comparison read the same arrays."""
    g = np.random.default_rng(seed)
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    Dh, Hq, Hkv = cfg["head_dim"], cfg["num_q_heads"], cfg["num_kv_heads"]

    def bf(shape, scale):
        bits = g.integers(0, 1 << 16, size=shape, dtype=np.uint16)
        e0 = int(np.floor(np.log2(scale))) + 127
        exp = (np.uint16(e0) - ((bits >> np.uint16(7)) & np.uint16(3))).astype(np.uint16)
        return (bits & np.uint16(0x807F)) | (exp << np.uint16(7))

    def gain(n):
        return (1.0 + 0.1 * g.standard_normal(n)).astype(np.float32)

    embed = bf((V, H), w_scale)
    final_norm = gain(H)
    lm_head = None if tied else bf((V, H), w_scale)
    s = w_scale * layer_scale
    layers = []
    for _ in range(cfg["num_layers"]):
        layers.append(dict(
            in_ln=gain(H), q_norm=gain(Dh), k_norm=gain(Dh), post_ln=gain(H),
            qkv_w=bf(((Hq + 2 * Hkv) * Dh, H), s),
            o_w=bf((H, Hq * Dh), s),
            gateup_w=bf((2 * I, H), s),
            down_w=bf((H, I), s),
        ))
    return embed, final_norm, lm_head, layers
