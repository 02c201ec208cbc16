"""Writes tests/golden/decoder_greedy_c5.npz: the oracle's greedy decode of BASELINE
configs[4] (the 28-layer Qwen3-ASR-shaped decoder, random bf16 weights, 2048-row prefill of
N(0, 0.02) embeddings, 256 greedy steps, EOS off), for tests/test_gpu_decoder_c5.py.

Run (CPU, ~10 min on 8 cores):  python tests/golden/make_decoder_greedy_golden.py

Two CPU restatements run side by side:
  A  OracleDecoder -- the oracle (oracle/orator_oracle.c: every linear output one serial fp32
     chain, k ascending), free-running greedy: its tokens are the expected ids;
  B  the same composition with every linear layer as a float32 BLAS matmul (blocked
     summation with FMA, another valid fp32 order), teacher-forced on A's tokens.
Per step (the prefill logits, then each of the 256 step bodies) the file keeps A's argmax,
A's top-k ids and values, B's values at those ids, B's argmax and max |A logits|: B - A is the
logit noise that fp32 summation order alone causes in this composition (bf16 re-rounding of
activations turns last-bit differences into whole bf16 steps), the yardstick for near ties.
It also keeps every 16th prefill logit of A.  Sources: src/model/asr_text_decoder.cu:360-455
(decode step), :457-617 (prefill), :698-889 (DecodeGreedy)."""
from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

TESTS = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(TESTS))
sys.path.insert(0, str(TESTS.parent))

import decoder_model as dm  # noqa: E402
import oracle_lib as orc  # noqa: E402

OUT = Path(__file__).resolve().parent / "decoder_greedy_c5.npz"


def top(logits, k):
    ids = np.argsort(-logits.astype(np.float64), kind="stable")[:k]
    return ids.astype(np.int32), logits[ids].astype(np.float32)


def main() -> None:
    t0 = time.time()
    cfg, w, emb = dm.c5_inputs()
    T, new, k = dm.C5["prefill"], dm.C5["new"], dm.C5["topk"]
    print(f"weights + embeddings {time.time() - t0:.1f} s", flush=True)
    A = orc.OracleDecoder(cfg, *w, threads=8)
    B = orc.BlasOrderDecoder(cfg, *w, threads=8)
    n = new + 1
    rec = dict(tokens=np.zeros(n, np.int32), top_ids=np.zeros((n, k), np.int32),
               top_a=np.zeros((n, k), np.float32), top_b=np.zeros((n, k), np.float32),
               argmax_b=np.zeros(n, np.int32), maxabs_a=np.zeros(n, np.float32))

    def record(s):
        ids, va = top(A.logits, k)
        rec["top_ids"][s], rec["top_a"][s] = ids, va
        rec["top_b"][s] = B.logits[ids]
        rec["tokens"][s] = orc.argmax_banned(A.logits, -1, -1)
        rec["argmax_b"][s] = orc.argmax_banned(B.logits, -1, -1)
        rec["maxabs_a"][s] = np.max(np.abs(A.logits))
        gap = va[0] - va[1]
        d = np.max(np.abs(rec["top_b"][s] - va))
        print(f"step {s}: token {rec['tokens'][s]} margin {gap:.4e} |B-A|top {d:.2e} "
              f"max|A| {rec['maxabs_a'][s]:.3f} ({time.time() - t0:.0f} s)", flush=True)

    A.prefill_at(emb, 0)
    B.prefill_at(emb, 0)
    prefill_sample = A.logits[::16].copy()
    record(0)
    for s in range(new):
        tok = int(rec["tokens"][s])
        A.decode_step(A.embed_row(tok), T + s)
        B.decode_step(B.embed_row(tok), T + s)
        record(s + 1)
    np.savez_compressed(OUT, prefill_sample=prefill_sample, prefill_stride=np.int32(16),
                        weight_seed=np.int32(dm.C5["weight_seed"]),
                        embed_seed=np.int32(dm.C5["embed_seed"]), prefill=np.int32(T),
                        new=np.int32(new), **rec)
    print(f"wrote {OUT} ({time.time() - t0:.0f} s)")


if __name__ == "__main__":
    main()
