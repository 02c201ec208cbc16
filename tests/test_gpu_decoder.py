"""GPU parity: the bf16 linear layers, the decode-step glue kernels and the ASR text decoder
(AsrTextDecoder: Prefill/PrefillAt, DecodeStep, TruncateCache, DecodeGreedy) against the oracle.

Bars:
  * linear: |g - r| <= 3e-5 * (sum_k |x_k w_k| + 1) against the fp64 product of the bf16
    operands (fp32 accumulation in another order);
  * glue kernels: bit-exact;
  * decoder logits: max |g - r| <= 1e-2 * max |r| and identical argmax.  The composition
    re-rounds activations to bf16 before every projection, so fp32-level differences move
    elements by whole bf16 steps and the steps cascade: the oracle itself moves by 0.38% of
    max |r| (small config) when its input embeddings move by one fp32 ulp, or when its
    linear layers accumulate in fp64 instead of fp32 (0.40%).  The reference's own bar for
    the same check is max |g - r| <= 2.0 (test/unit/model/test_asr_decoder.cc:66-72);
  * greedy tokens: identical ids and cache length.  The oracle runs with a BLAS-order shadow
    (oracle_lib.TwinDecoder): at every step the shadow's change of the oracle's top-1 - top-2
    margin measures what fp32 summation order alone does to the logits there; NOISE = the
    largest such change over the run.  The device may pick another token than the oracle's
    argmax only where the oracle's margin between the two is below NOISE (the oracle then
    follows the device's token, printed); every other step must give the oracle's token."""
from __future__ import annotations

import math

import numpy as np
import pytest

import decoder_model as dm
import oracle_lib as orc
from gpu_helpers import down, empty, say, up
from helpers import SplitMix64
from orator_amd import asr_gemm, decoder_ops
from orator_amd.decoder import AsrTextConfig, AsrTextDecoder

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-2


# ----------------------------------------------------------------------- linear ----
@pytest.mark.parametrize("M,K,N", [(1, 2048, 4096), (1, 6144, 2048), (1, 512, 37), (1, 8, 5),
                                   (2, 512, 130), (17, 1024, 257), (128, 2048, 128),
                                   (300, 2048, 1024), (503, 2048, 4096)])
@pytest.mark.parametrize("act,with_bias", [(0, False), (1, True), (2, True)])
def test_linear_pre_vs_oracle(M, K, N, act, with_bias):
    r = SplitMix64(M * 7 + K + N + act)
    x = orc.to_bf16(r.normal((M, K)))
    W = orc.to_bf16(r.normal((N, K), 0.05))
    bias = r.normal(N) if with_bias else None
    xd, Wd = orc.from_bf16(x).astype(np.float64), orc.from_bf16(W).astype(np.float64)
    ref = xd @ Wd.T + (bias if with_bias else 0.0)
    ref = {0: ref, 1: 0.5 * ref * (1 + np.vectorize(math.erf)(ref / math.sqrt(2))),
           2: np.maximum(ref, 0)}[act]
    bound = 3e-5 * (np.abs(xd) @ np.abs(Wd).T + 1.0)
    out = empty((M, N), np.float32)
    say("linear_pre", M, K, N, act)
    asr_gemm.LinearPre(up(x), up(W), up(bias) if with_bias else None, out, M, K, N, act)
    got = down(out, (M, N))
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)


@pytest.mark.parametrize("M,K,N", [(2048, 2048, 4096), (2048, 2048, 12288), (2048, 6144, 2048)])
def test_linear_pre_prompt_tiles(M, K, N):
    """The decoder's 2048-token prompt projections (q|k|v 4096, gate|up 12288, down 2048 rows of
    2048 / 6144): the GEMM's full-grid 128 x 128 path, epilogue without bias (the shapes above
    take the 128 x 64, split-K and bias / activation paths), same bound."""
    r = SplitMix64(M + K + N)
    x = orc.to_bf16(r.normal((M, K)))
    W = orc.to_bf16(r.normal((N, K), 0.05))
    xd, Wd = orc.from_bf16(x).astype(np.float64), orc.from_bf16(W).astype(np.float64)
    ref = xd @ Wd.T
    bound = 3e-5 * (np.abs(xd) @ np.abs(Wd).T + 1.0)
    out = empty((M, N), np.float32)
    say("linear_pre prompt", M, K, N)
    asr_gemm.LinearPre(up(x), up(W), None, out, M, K, N, 0)
    got = down(out, (M, N))
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)


def _placed(arr, off):
    """arr on the device `off` elements past a 16-byte aligned allocation (off odd: rows
    start at 2-byte alignment only); returns (buffer, device address)."""
    flat = np.ascontiguousarray(arr).reshape(-1)
    pad = np.zeros(off + flat.size, flat.dtype)
    pad[off:] = flat
    buf = up(pad)
    return buf, buf.ptr + off * flat.itemsize


# Any K and any alignment, as the reference's generic fallback (include/model/gemm.cuh:461-501,
# src/model/asr_gemm.cu:188-214): K = 9 is the audio tower's first conv as a GEMM (Cin 1 x 3 x 3,
# src/model/asr_audio_tower.cu:417-445), K = 13 an odd row, K = 4320 a long one that is a
# multiple of 8 but whose operands are not 16-byte aligned.  M = 1 and M > 1, every entry point.
@pytest.mark.parametrize("M,K,N,off", [(1, 9, 480, 0), (390, 9, 480, 0), (1, 13, 37, 1),
                                       (77, 13, 300, 3), (1, 4320, 480, 1), (200, 4320, 480, 5),
                                       (2048, 9, 128, 0), (5, 1, 7, 0)])
@pytest.mark.parametrize("act,with_bias", [(0, False), (1, True)])
def test_linear_any_k_any_alignment(M, K, N, off, act, with_bias):
    from orator_amd import gemm
    r = SplitMix64(M * 31 + K * 7 + N + off + act)
    x = orc.to_bf16(r.normal((M, K)))
    W = orc.to_bf16(r.normal((N, K), 0.05))
    bias = r.normal(N) if with_bias else None
    xd, Wd = orc.from_bf16(x).astype(np.float64), orc.from_bf16(W).astype(np.float64)
    ref = xd @ Wd.T + (bias if with_bias else 0.0)
    if act == 1:
        ref = 0.5 * ref * (1 + np.vectorize(math.erf)(ref / math.sqrt(2)))
    bound = 3e-5 * (np.abs(xd) @ np.abs(Wd).T + 1.0)
    xb, xp = _placed(x, off)
    wb, wp = _placed(W, off)
    db = up(bias) if with_bias else None
    for name, fn in (("LinearPre", asr_gemm.LinearPre), ("LaunchBf16Gemm", gemm.LaunchBf16Gemm)):
        out = empty((M, N), np.float32)
        say(name, "any K", M, K, N, off, act)
        fn(xp, wp, db, out, M, K, N, act)
        got = down(out, (M, N))
        assert np.all(np.abs(got - ref) <= bound), (name, np.max(np.abs(got - ref) / bound))
    # Linear (fp32 input, cast to bf16 by the library): the same bits as LinearPre on the
    # bf16 rows
    xf = orc.from_bf16(x)
    fb, fp = _placed(xf, off)
    out_f, out_p = empty((M, N), np.float32), empty((M, N), np.float32)
    say("Linear any K", M, K, N, off)
    asr_gemm.Linear(fp, wp, db, out_f, M, K, N, act)
    asr_gemm.LinearPre(xp, wp, db, out_p, M, K, N, act)
    np.testing.assert_array_equal(down(out_f, (M, N)), down(out_p, (M, N)))


@pytest.mark.parametrize("M,K,I,off", [(1, 13, 300, 1), (40, 9, 64, 0), (33, 4320, 100, 3)])
def test_linear_pre_swiglu_any_k(M, K, I, off):
    """The gate|up projection with SwiGLU at any K / alignment: bit-identical to LinearPre +
    SwiGLU + F32ToBf16, as at aligned shapes."""
    from orator_amd import asr_ops
    r = SplitMix64(M + 5 * K + I + off)
    x = orc.to_bf16(r.normal((M, K)))
    W = orc.to_bf16(r.normal((2 * I, K), 0.05))
    xb, xp = _placed(x, off)
    wb, wp = _placed(W, off)
    gu = empty((M, 2 * I), np.float32)
    say("linear_pre_swiglu any K", M, K, I, off)
    asr_gemm.LinearPre(xp, wp, None, gu, M, K, 2 * I, 0)
    g_u = down(gu, (M, 2 * I))
    act = empty((M * I,), np.float32)
    asr_ops.SwiGLU(up(np.ascontiguousarray(g_u[:, :I])), up(np.ascontiguousarray(g_u[:, I:])),
                   act, M * I)
    want = empty((M * I,), np.uint16)
    asr_ops.F32ToBf16(act, want, M * I)
    got = empty((M * I,), np.uint16)
    asr_gemm.LinearPreSwiGLU(xp, wp, got, M, K, I)
    np.testing.assert_array_equal(down(got, (M, I), np.uint16), down(want, (M, I), np.uint16))


@pytest.mark.parametrize("M,K,I", [(2048, 2048, 6144), (503, 2048, 6144), (300, 1024, 6000),
                                   (5, 512, 1000), (1, 512, 300)])
def test_linear_pre_swiglu_equals_three_calls(M, K, I):
    """The gate|up GEMM with SwiGLU + bf16 cast in its epilogue is bit-identical to LinearPre
    on the fused [gate; up] weight, SwiGLU and F32ToBf16 (asr_text_decoder.cu:547-552): the
    fused tile (2048 / 503 rows), a ragged one (300 rows, I = 6000: 64-column tiles cut at
    the edge), the short-grid path (5 rows) and the GEMV path (1 row)."""
    from orator_amd import asr_ops
    r = SplitMix64(M + 3 * K + I)
    x = orc.to_bf16(r.normal((M, K)))
    W = orc.to_bf16(r.normal((2 * I, K), 0.05))
    xd, Wd = up(x), up(W)
    gu = empty((M, 2 * I), np.float32)
    say("linear_pre_swiglu", M, K, I)
    asr_gemm.LinearPre(xd, Wd, None, gu, M, K, 2 * I, 0)
    g_u = down(gu, (M, 2 * I))
    act = empty((M * I,), np.float32)
    asr_ops.SwiGLU(up(np.ascontiguousarray(g_u[:, :I])), up(np.ascontiguousarray(g_u[:, I:])),
                   act, M * I)
    want = empty((M * I,), np.uint16)
    asr_ops.F32ToBf16(act, want, M * I)
    got = empty((M * I,), np.uint16)
    asr_gemm.LinearPreSwiGLU(xd, Wd, got, M, K, I)
    np.testing.assert_array_equal(down(got, (M, I), np.uint16), down(want, (M, I), np.uint16))


@pytest.mark.parametrize("M", [1, 33])
def test_linear_f32_input_casts_rne(M):
    """Linear == F32ToBf16 + LinearPre (the cast is round-to-nearest-even, bit-exact)."""
    K, N = 1024, 300
    r = SplitMix64(M)
    x = r.normal((M, K))
    W = orc.to_bf16(r.normal((N, K), 0.05))
    a, b = empty((M, N), np.float32), empty((M, N), np.float32)
    Wd = up(W)
    say("linear f32", M)
    asr_gemm.Linear(up(x), Wd, None, a, M, K, N, 0)
    asr_gemm.LinearPre(up(orc.to_bf16(x)), Wd, None, b, M, K, N, 0)
    np.testing.assert_array_equal(down(a, (M, N)), down(b, (M, N)))


def test_bf16_gemm_m1_matches_gemv():
    K, N = 2048, 1000
    r = SplitMix64(11)
    x, W = orc.to_bf16(r.normal((1, K))), orc.to_bf16(r.normal((N, K), 0.05))
    a, b = empty((1, N), np.float32), empty((1, N), np.float32)
    say("bf16_gemm M=1")
    xd, Wd = up(x), up(W)
    asr_gemm.LinearPre(xd, Wd, None, a, 1, K, N, 0)
    from orator_amd import gemm
    gemm.LaunchBf16Gemm(xd, Wd, None, b, 1, K, N, 0)
    ga, gb = down(a, (N,)), down(b, (N,))
    ref = orc.linear_bf16(x, W)[0]
    assert np.max(np.abs(ga - ref)) < 1e-3 and np.max(np.abs(gb - ref)) < 1e-3


# ------------------------------------------------------------------ glue kernels ----
def test_glue_kernels_bit_exact():
    r = SplitMix64(5)
    V, H = 64, 2048
    table = orc.to_bf16(r.normal((V, H)))
    tok = up(np.array([37], np.int32))
    out = empty((H,), np.float32)
    say("embed_gather")
    decoder_ops.EmbedGather(up(table), tok, out, H)
    np.testing.assert_array_equal(down(out, (H,)), orc.from_bf16(table[37]))
    a, b = r.normal(1027), r.normal(1027)
    da = up(a)
    decoder_ops.AddResidual(da, up(b), 1027)
    np.testing.assert_array_equal(down(da, (1027,)), a + b)
    rec, cnt, pos = up(np.full(4, -1, np.int32)), up(np.zeros(1, np.int32)), up(np.array([9], np.int32))
    for t in (5, 6, 7, 8, 9):  # the fifth record is past the capacity of 4
        decoder_ops.RecordToken(rec, cnt, up(np.array([t], np.int32)), 4)
        decoder_ops.IncPos(pos)
    np.testing.assert_array_equal(down(rec, (4,), np.int32), [5, 6, 7, 8])
    assert int(down(cnt, (1,), np.int32)[0]) == 5 and int(down(pos, (1,), np.int32)[0]) == 14


# ---------------------------------------------------------------------- decoder ----
def build(cfg, weights):
    embed, final_norm, lm_head, layers = weights
    dl = [{k: up(v) for k, v in L.items()} for L in layers]
    dec = AsrTextDecoder(AsrTextConfig(**cfg), up(embed), up(final_norm),
                         up(lm_head) if lm_head is not None else None, dl)
    return dec


def top2_gap(logits, ban=()):
    x = np.array(logits, np.float64)
    for b in ban:
        if b >= 0:
            x[b] = -np.inf
    s = np.sort(x)
    return s[-1] - s[-2]


def follower(o, got):
    """choose() for TwinDecoder.decode_greedy: the oracle's banned argmax, or the device's
    token where they differ (recorded with the oracle's margin between the two); beside it
    the shadow's change of the oracle's top-1 - top-2 margin at every step (the noise)."""
    near, noise = [], []

    def choose(j, logits, b0, b1):
        best = orc.argmax_banned(logits, b0, b1)
        x = np.array(logits, np.float64)
        for b in (b0, b1):
            if b >= 0:
                x[b] = -np.inf
        i1, i2 = np.argsort(-x, kind="stable")[:2]
        sh = o.shadow.logits.astype(np.float64)
        noise.append(abs((sh[i1] - sh[i2]) - (x[i1] - x[i2])))
        if j < len(got) and int(got[j]) != best:
            t = int(got[j])
            assert t not in (b0, b1), (j, t, "banned id emitted")
            near.append((j, t, best, float(logits[best] - logits[t])))
            return t
        return best
    return choose, near, noise


def greedy_check(o, got, *args, **kw):
    choose, near, noise = follower(o, got)
    want, bodies = o.decode_greedy(*args, **kw, choose=choose)
    bound = max(noise) if noise else 0.0
    print("tokens", got, f"noise {bound:.3e}", "steps that follow the device", near)
    assert [int(t) for t in got] == want
    for j, t, best, gap in near:
        assert gap < bound, (j, t, best, gap, bound)
    return bodies


def check_logits(got, ref, what):
    err = np.max(np.abs(got - ref))
    assert err <= LOGIT_TOL * np.max(np.abs(ref)), (what, err, np.max(np.abs(ref)))
    assert int(np.argmax(got)) == int(np.argmax(ref)), what


@pytest.fixture(scope="module")
def small():
    cfg = dm.SMALL
    w = dm.make_weights(cfg, 21)
    return cfg, w


def test_prefill_logits_and_incremental(small):
    """test/unit/model/test_asr_decoder.cc:50-123 on synthetic weights: Prefill logits and
    argmax vs the oracle, split PrefillAt == one Prefill, TruncateCache + re-prefill."""
    cfg, w = small
    T = 97
    emb = SplitMix64(7).normal((T, cfg["hidden_size"]), 0.02)
    o = orc.OracleDecoder(cfg, *w, threads=8)
    o.prefill_at(emb, 0)
    say("decoder prefill", T)
    dec = build(cfg, w)
    dec.ResetCache()
    dec.Prefill(emb, T)
    assert dec.cache_len() == T
    full = dec.CopyLogits()
    check_logits(full, o.logits, "prefill")
    assert dec.Argmax() == o.argmax()
    split = T // 2
    dec.ResetCache()
    dec.PrefillAt(emb[:split], split, 0)
    dec.PrefillAt(up(emb[split:]), T - split, split)  # device embeddings too
    assert dec.cache_len() == T
    inc = dec.CopyLogits()
    assert dec.Argmax() == int(np.argmax(full))
    assert np.max(np.abs(inc - full)) <= LOGIT_TOL * np.max(np.abs(full))
    dec.TruncateCache(split)
    assert dec.cache_len() == split
    dec.PrefillAt(emb[split:], T - split, split)
    assert dec.Argmax() == int(np.argmax(full))
    dec.close()


def test_decode_steps_teacher_forced(small):
    """DecodeStep / DecodeStepDevice + Argmax logits vs the oracle, the oracle's tokens fed."""
    cfg, w = small
    T = 40
    emb = SplitMix64(8).normal((T, cfg["hidden_size"]), 0.02)
    o = orc.OracleDecoder(cfg, *w, threads=8)
    o.prefill_at(emb, 0)
    dec = build(cfg, w)
    say("decoder decode steps")
    dec.Prefill(emb, T)
    tok = o.argmax()
    dtok = up(np.array([tok], np.int32))
    for step in range(12):
        pos = T + step
        o.decode_step(o.embed_row(tok), pos)
        if step % 2:
            dec.DecodeStep(dec.Embed(tok), pos)
        else:
            dec.DecodeStepDevice(dtok, pos)
        assert dec.cache_len() == pos + 1
        check_logits(dec.CopyLogits(), o.logits, f"step {step}")
        tok = o.argmax()
        dec.ArgmaxToDevice(dtok)
        assert int(down(dtok, (1,), np.int32)[0]) == tok
    dec.close()


@pytest.mark.parametrize("use_graph", [False, True])
@pytest.mark.parametrize("batch", [1, 4, 32])
def test_decode_greedy_tokens(small, use_graph, batch):
    """DecodeGreedy token ids and cache length identical to the oracle's greedy loop, across
    two calls (the second replays already-captured graphs), with EOS ids that do and do not
    occur."""
    cfg, w = small
    T = 64
    emb = SplitMix64(9).normal((T, cfg["hidden_size"]), 0.02)
    o = orc.TwinDecoder(cfg, *w, threads=8)
    o.prefill_at(emb, 0)
    free_run, _ = orc.OracleDecoder(cfg, *w, threads=8), None
    free_run.prefill_at(emb, 0)
    stream, _ = free_run.decode_greedy(T, 30, -5, -5, ban_steps=0, batch=30, use_graph=False)
    # an EOS id that the free run emits at index 9 (first occurrence) and one it never emits
    eos0 = stream[9] if stream[9] not in stream[:9] else -7
    eos1 = next(t for t in range(cfg["vocab_size"]) if t not in stream)
    dec = build(cfg, w)
    say("decoder greedy", use_graph, batch)
    dec.Prefill(emb, T)
    got = dec.DecodeGreedy(T, 30, eos0, eos1, ban_steps=3, batch=batch, use_graph=use_graph)
    bodies = greedy_check(o, got, T, 30, eos0, eos1, 3, batch, use_graph, graph_ready=False)
    assert dec.cache_len() == T + bodies
    # second call continues from the cache end: prefill 5 more rows then greedy again
    more = SplitMix64(10).normal((5, cfg["hidden_size"]), 0.02)
    p0 = o.cache_len
    o.prefill_at(more, p0)
    dec.PrefillAt(more, 5, p0)
    check_logits(dec.CopyLogits(), o.logits, "prefill after greedy")
    got2 = dec.DecodeGreedy(p0 + 5, 20, eos0, eos1, ban_steps=3, batch=batch,
                            use_graph=use_graph)
    bodies2 = greedy_check(o, got2, p0 + 5, 20, eos0, eos1, 3, batch, use_graph,
                           graph_ready=use_graph)
    assert dec.cache_len() == p0 + 5 + bodies2
    dec.close()


def test_decode_greedy_repetition_stop():
    """Tied embeddings and tiny layer weights make the model repeat its input token: the
    greedy loop stops after the 6th identical token (included)."""
    cfg = dict(dm.SMALL, num_layers=1)
    w = dm.make_weights(cfg, 31, tied=True, layer_scale=0.01)
    T = 16
    emb = SplitMix64(12).normal((T, cfg["hidden_size"]), 0.02)
    o = orc.TwinDecoder(cfg, *w)
    o.prefill_at(emb, 0)
    dec = build(cfg, w)
    say("decoder repetition stop")
    dec.Prefill(emb, T)
    got = dec.DecodeGreedy(T, 40, -3, -4, ban_steps=3, batch=4, use_graph=True)
    bodies = greedy_check(o, got, T, 40, -3, -4, 3, 4, True, graph_ready=False)
    assert len(got) < 40 and len(set(got[-6:])) == 1
    assert dec.cache_len() == T + bodies
    dec.close()


def test_decoder_qwen_shapes():
    """The real layer shapes (hidden 2048, 16/8 heads, MLP 6144, vocab 151936) on 2 layers:
    prefill logits, then greedy tokens eager and graph-replayed."""
    cfg = dm.QWEN_2L
    w = dm.make_weights(cfg, 41, tied=True)  # lm_head tied to embed (asr_text_decoder.cu:255-257)
    T = 128
    emb = SplitMix64(13).normal((T, cfg["hidden_size"]), 0.02)
    o = orc.TwinDecoder(cfg, *w, threads=16)
    o.prefill_at(emb, 0)
    dec = build(cfg, w)
    say("decoder qwen shapes prefill", T)
    dec.Prefill(emb, T)
    check_logits(dec.CopyLogits(), o.logits, "qwen prefill")
    print("top-2 gap at the seed", top2_gap(o.logits, orc.EOS_IDS))
    got = dec.DecodeGreedy(T, 8, *orc.EOS_IDS, ban_steps=3, batch=4, use_graph=True)
    greedy_check(o, got, T, 8, *orc.EOS_IDS, 3, 4, True, graph_ready=False)
    dec.Prefill(emb, T)
    got_eager = dec.DecodeGreedy(T, 8, *orc.EOS_IDS, ban_steps=3, batch=4, use_graph=False)
    assert got_eager == got  # same device arithmetic, eager or replayed
    dec.close()
