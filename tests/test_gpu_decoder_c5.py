"""GPU parity of BASELINE configs[4]: greedy token ids of the full synthetic decoder (28
layers, hidden 2048, 16/8 heads, SwiGLU 6144, vocab 151936, tied lm_head, random bf16 weights,
2048-row prefill of N(0, 0.02) embeddings, 256 greedy steps, EOS off) against the oracle's
(tests/golden/decoder_greedy_c5.npz, written by tests/golden/make_decoder_greedy_golden.py
from the same seeds; src/model/asr_text_decoder.cu:457-617, :360-455, :698-889).

Near ties.  The composition re-rounds activations to bf16 before every projection, so any
two fp32 restatements that sum in different orders differ by whole bf16 steps and their
logits drift apart.  The golden file measures that drift: a second CPU restatement whose
linear layers are BLAS products (B) is run teacher-forced beside the oracle (A).
  * NOISE = the largest change of A's top-1 - top-2 margin that B's summation order causes at
    any of the 257 steps (0.024 on max |logit| ~ 3.5; B itself picks another token than A at
    5 steps, all with margins below 0.005).  A step is excused only when the oracle's margin
    there is below NOISE, and at an excused step the device's token must still be one of the
    oracle's near-tie candidates: among A's top-32, with A's logit within NOISE of A's top-1;
    every other step must give the oracle's token.
  * TOP_TOL = 1.25 x max |B - A| over A's top-32 logits at every step (max |B - A| = 0.019):
    the device is a third fp32 summation order, held to the second one's deviation.
Checks:
  * teacher-forced: the device decodes the oracle's token stream step by step; its argmax
    (the library's ArgmaxBanned) must be the oracle's token at every non-excused step, a
    near-tie candidate at excused steps, and its logits at the oracle's top-32 ids within
    TOP_TOL of the oracle's;
  * free-running: DecodeGreedy with graph replay must emit exactly the oracle's tokens (the
    reference's 6-repeat stop applied to them); the streams may part only at an excused step
    (after which the inputs differ and nothing more is comparable);
  * the prefill logits (every 16th) within 1e-2 * max |logit|.
Every step's margin is printed."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import decoder_model as dm
from gpu_helpers import say, up
from orator_amd.decoder import AsrTextConfig, AsrTextDecoder

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden" / "decoder_greedy_c5.npz"
LOGIT_TOL = 1e-2


def _expected_emitted(tokens, new):
    """DecodeGreedy's host harvest of a token stream with EOS off: the 6-repeat stop
    (src/model/asr_text_decoder.cu:741-757) emits the 6th and ends."""
    out = []
    for t in tokens[:new]:
        out.append(int(t))
        if len(out) >= 6 and len(set(out[-6:])) == 1:
            break
    return out


def test_c5_greedy_token_ids_match_oracle():
    g = dict(np.load(GOLD))
    T, new = int(g["prefill"]), int(g["new"])
    say("c5: generating weights")
    cfg, w, emb = dm.c5_inputs()
    embed, final_norm, lm_head, layers = w
    say("c5: upload")
    dl = [{k: up(v) for k, v in L.items()} for L in layers]
    dec = AsrTextDecoder(AsrTextConfig(**cfg), up(embed), up(final_norm), None, dl)
    del layers, dl
    gold = g["tokens"]
    margins = (g["top_a"][:, 0] - g["top_a"][:, 1]).astype(np.float64)
    margins_b = (g["top_b"][:, 0] - g["top_b"][:, 1]).astype(np.float64)
    noise = float(np.max(np.abs(margins_b - margins)))
    excused = margins < noise
    top_tol = 1.25 * float(np.max(np.abs(g["top_b"] - g["top_a"])))
    print(f"c5: NOISE {noise:.4e}; TOP_TOL {top_tol:.4e}; oracle steps with margin below NOISE: "
          f"{np.flatnonzero(excused).tolist()}", flush=True)
    print(f"c5: steps where the BLAS-order twin's argmax differs from the oracle's: "
          f"{np.flatnonzero(g['argmax_b'] != gold).tolist()}", flush=True)

    # ---- teacher-forced ----
    say("c5: prefill")
    demb = up(emb)
    dec.Prefill(demb, T)
    logits = dec.CopyLogits()
    stride = int(g["prefill_stride"])
    scale = np.max(np.abs(g["prefill_sample"]))
    d_pre = np.max(np.abs(logits[::stride] - g["prefill_sample"]))
    print(f"c5: prefill logits (every {stride}th): max |g - r| = {d_pre:.3e} "
          f"({d_pre / scale:.2e} of max)", flush=True)
    assert d_pre <= LOGIT_TOL * scale
    dev, dtop = [], []
    for s in range(new + 1):
        if s > 0:
            dec.DecodeStep(dec.Embed(int(gold[s - 1])), T + s - 1)
            logits = dec.CopyLogits()
        dev.append(dec.Argmax())
        dtop.append(float(np.max(np.abs(logits[g["top_ids"][s]] - g["top_a"][s]))))
        if s % 32 == 0:
            say(f"c5: teacher-forced step {s}")
    dev = np.array(dev)
    for s in range(new + 1):
        flag = "" if dev[s] == gold[s] else ("  EXCUSED" if excused[s] else "  MISMATCH")
        print(f"c5 step {s:3d}: oracle {gold[s]:6d} device {dev[s]:6d} margin {margins[s]:.4e} "
              f"|dev-oracle| top-32 {dtop[s]:.2e}{flag}")
    bad = [s for s in range(new + 1) if dev[s] != gold[s] and not excused[s]]
    assert not bad, f"token mismatch at non-excused steps {bad}"
    # at an excused step the device's token is a near-tie candidate of the oracle's
    for s in np.flatnonzero(dev != gold):
        ids = g["top_ids"][s].tolist()
        assert int(dev[s]) in ids, f"step {s}: device token {dev[s]} not in the oracle's top-32"
        gap = float(g["top_a"][s][0] - g["top_a"][s][ids.index(int(dev[s]))])
        print(f"c5 step {s}: device token's oracle logit is {gap:.4e} below the top-1")
        assert gap <= noise, f"step {s}: device token {gap:.4e} below the oracle's top-1"
    print(f"c5: max |dev - oracle| over top-32 logits {max(dtop):.4e} (TOP_TOL {top_tol:.4e}); "
          f"device mismatch steps {np.flatnonzero(dev != gold).tolist()}", flush=True)
    assert max(dtop) <= top_tol

    # ---- free-running greedy with graph replay ----
    say("c5: DecodeGreedy (graph replay)")
    dec.Prefill(demb, T)
    toks = [int(t) for t in dec.DecodeGreedy(T, new, -1, -1, ban_steps=3, batch=32,
                                             use_graph=True)]
    expected = _expected_emitted(gold, new)
    n = min(len(toks), len(expected))
    diff = [i for i in range(n) if toks[i] != expected[i]]
    if diff:
        i = diff[0]
        print(f"c5: greedy parts from the oracle at step {i} (margin {margins[i]:.4e}, excused "
              f"{bool(excused[i])}); {i} tokens identical before it", flush=True)
        assert excused[i], f"greedy stream parts at non-excused step {i}"
    else:
        print(f"c5: greedy emitted {len(toks)} tokens, all identical to the oracle's", flush=True)
        assert toks == expected
    dec.close()
