"""Pins the CPU oracle (oracle/orator_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something that does not restate its own code:
the reference's fixture recipe replayed with torch (tests/golden), torch library
routines (SDPA, bf16 casts), fp64 closed forms, and invariants a wrong sign / index /
transposition would break.  CPU only.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle_lib as orc
from helpers import SplitMix64, rel_err

# torch (CPU) is a library oracle here.  It is imported lazily so that collecting this
# module in a GPU run never loads torch's own HIP runtime next to the product library.

def _torch():
    import torch as _t
    import torch.nn.functional as _F
    return _t, _F

# ------------------------------------------------------------------------ bf16 ----


def test_bf16_known_answers():
    cases = {
        1.0: 0x3F80,
        -2.0: 0xC000,
        # halfway cases round to even
        float(np.frombuffer(np.uint32(0x3F808000).tobytes(), np.float32)[0]): 0x3F80,
        float(np.frombuffer(np.uint32(0x3F818000).tobytes(), np.float32)[0]): 0x3F82,
        # just above halfway rounds up
        float(np.frombuffer(np.uint32(0x3F808001).tobytes(), np.float32)[0]): 0x3F81,
        0.0: 0x0000,
        float("inf"): 0x7F80,
    }
    for x, bits in cases.items():
        assert orc.lib().orc_f32_to_bf16(x) == bits, (x, hex(bits))
    assert orc.lib().orc_bf16_to_f32(0x3F80) == 1.0


def test_bf16_matches_torch_rne():
    torch, F = _torch()
    r = SplitMix64(11)
    x = np.concatenate([
        r.normal((4096,)),
        r.normal((1024,), 1e-30),   # subnormal range of fp32 -> bf16
        r.normal((1024,), 1e30),
        np.array([65504.0, -3.3895314e38, 1e-45], np.float32),
    ]).astype(np.float32)
    ours = orc.to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    back = orc.from_bf16(ours)
    np.testing.assert_array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# --------------------------------------------------------------------- RMSNorm ----


def test_rmsnorm_reference_fixture(golden):
    out = orc.rms_norm(golden["rmsnorm_x"], golden["rmsnorm_w"], 1e-6)
    assert np.max(np.abs(out - golden["rmsnorm_out"])) < 1e-4  # test_asr_ops.cc:93
    assert np.max(np.abs(out - golden["rmsnorm_out"])) < 2e-6


def test_rmsnorm_invariants():
    r = SplitMix64(12)
    x = r.normal((16, 128))
    w = r.normal((128,))
    y = orc.rms_norm(x, w, 1e-6)
    # closed form in fp64
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)
    assert rel_err(y, ref * w, 0.05) < 5e-5
    # scale invariance (eps negligible)
    np.testing.assert_allclose(orc.rms_norm(8.0 * x, w, 1e-12), orc.rms_norm(x, w, 1e-12),
                               rtol=2e-6, atol=1e-7)
    # constant row c: y = w * sign(c) / sqrt(1 + eps / c^2)
    c = np.full((2, 128), [[0.5], [-3.0]], np.float32)
    yc = orc.rms_norm(c, w, 1e-6)
    expect = w[None, :] * np.sign(c) / np.sqrt(1.0 + 1e-6 / c.astype(np.float64) ** 2)
    np.testing.assert_allclose(yc, expect, rtol=2e-7, atol=0)


# ------------------------------------------------------------------------ RoPE ----


def test_rope_interleaved_reference_fixture(golden):
    out = orc.rope_interleaved(golden["rope_x"], golden["rope_pos"], 1e6)
    assert np.max(np.abs(out - golden["rope_out"])) < 1e-4  # test_asr_ops.cc:118
    assert np.max(np.abs(out - golden["rope_out"])) < 2e-6


def _hf_rotate_half(x, pos, base, Dh):
    """HF Qwen3 rotary: x*cos + rotate_half(x)*sin, angle formed as fp32 pos*inv_freq
    (the reference's fp32 angle), cos/sin and the rest in fp64."""
    torch, F = _torch()
    i = torch.arange(Dh // 2, dtype=torch.float64)
    inv = torch.pow(torch.tensor(base, dtype=torch.float64), -2.0 * i / Dh).float()
    ang = (torch.from_numpy(pos).float()[:, None] * inv[None, :]).double()
    emb = torch.cat([ang, ang], dim=-1)[:, None, :]
    xt = torch.from_numpy(x).double()
    x1, x2 = xt[..., : Dh // 2], xt[..., Dh // 2:]
    rot = torch.cat([-x2, x1], dim=-1)
    return (xt * emb.cos() + rot * emb.sin()).numpy()


@pytest.mark.parametrize("p0", [0, 500, 4090])
def test_rope_half_matches_hf_formula(p0):
    r = SplitMix64(13 + p0)
    T, H, Dh = 6, 3, 128
    x = r.normal((T, H, Dh))
    pos = np.arange(p0, p0 + T, dtype=np.int32)
    ours = orc.rope_half(x, pos, 1e6)
    ref = _hf_rotate_half(x, pos, 1e6, Dh)
    assert np.max(np.abs(ours - ref)) < 3e-6


def test_rope_half_invariants():
    r = SplitMix64(14)
    T, H, Dh = 8, 2, 128
    x = r.normal((T, H, Dh))
    # position 0 is the identity
    np.testing.assert_array_equal(orc.rope_half(x, np.zeros(T, np.int32), 1e6), x)
    pos = np.arange(T, dtype=np.int32) * 37
    y = orc.rope_half(x, pos, 1e6).astype(np.float64)
    xd = x.astype(np.float64)
    # each (j, j+64) pair keeps its norm
    n_in = xd[..., :64] ** 2 + xd[..., 64:] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)
    # q.k depends on the position difference only
    q, k = r.normal((1, 1, Dh)), r.normal((1, 1, Dh))
    d1 = float((orc.rope_half(q, np.array([10], np.int32), 1e6) *
                orc.rope_half(k, np.array([7], np.int32), 1e6)).sum())
    d2 = float((orc.rope_half(q, np.array([110], np.int32), 1e6) *
                orc.rope_half(k, np.array([107], np.int32), 1e6)).sum())
    assert abs(d1 - d2) < 1e-4 * max(1.0, abs(d1))


# ---------------------------------------------------------------------- SwiGLU ----


def test_swiglu_reference_fixture(golden):
    out = orc.swiglu(golden["swiglu_gate"], golden["swiglu_up"])
    assert np.max(np.abs(out - golden["swiglu_out"])) < 1e-5  # test_asr_ops.cc:141


# ----------------------------------------------------------------- GQA (fp32) ----


def test_gqa_attention_reference_fixture(golden):
    T, Dh = 24, 128
    out = orc.gqa_attention(golden["gqa_q"], golden["gqa_k"], golden["gqa_v"],
                            1.0 / math.sqrt(Dh), True)
    assert np.max(np.abs(out - golden["gqa_out"])) < 5e-4  # test_asr_ops.cc:167
    assert np.max(np.abs(out - golden["gqa_out"])) < 2e-6
    truth = orc.attention_f64(golden["gqa_q"], golden["gqa_k"], golden["gqa_v"],
                              1.0 / math.sqrt(Dh), True)
    assert rel_err(out, truth, 0.05) < 5e-5


@pytest.mark.parametrize("T,Hq,Hkv,Dh,causal", [(20, 16, 2, 32, True), (9, 12, 4, 256, False),
                                               (5, 8, 1, 1024, True)])
def test_gqa_attention_any_head_size_vs_sdpa(T, Hq, Hkv, Dh, causal):
    """GqaAttention accepts any power-of-two Dh <= 1024 and any Hq multiple of Hkv
    (src/model/asr_ops.cu:252-295): the oracle against torch SDPA in fp64 with K/V heads
    repeat-interleaved (the recipe of tools/dump/dump_asr_ops.py:101-108)."""
    torch, F = _torch()
    r = SplitMix64(T * Dh + Hq)
    q, k, v = r.normal((T, Hq, Dh), 0.3), r.normal((T, Hkv, Dh), 0.3), r.normal((T, Hkv, Dh))
    scale = 1.0 / math.sqrt(Dh)
    out = orc.gqa_attention(q, k, v, scale, causal)
    G = Hq // Hkv
    qt = torch.from_numpy(q).double().permute(1, 0, 2)
    kt = torch.from_numpy(k).double().permute(1, 0, 2).repeat_interleave(G, 0)
    vt = torch.from_numpy(v).double().permute(1, 0, 2).repeat_interleave(G, 0)
    ref = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal, scale=scale)
    assert rel_err(out, ref.permute(1, 0, 2).numpy(), 0.05) < 5e-6


def test_gqa_attention_noncausal_vs_sdpa():
    torch, F = _torch()
    r = SplitMix64(15)
    T, Hq, Hkv, Dh = 19, 4, 2, 64
    q, k, v = r.normal((T, Hq, Dh)), r.normal((T, Hkv, Dh)), r.normal((T, Hkv, Dh))
    out = orc.gqa_attention(q, k, v, 0.125, False)
    qt = torch.from_numpy(q).double().permute(1, 0, 2)
    kt = torch.from_numpy(k).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
    vt = torch.from_numpy(v).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
    ref = F.scaled_dot_product_attention(qt, kt, vt, scale=0.125).permute(1, 0, 2).numpy()
    assert rel_err(out, ref, 0.05) < 5e-5


# ----------------------------------------------------------- KV cache + a5/a6 ----


def _cache(r, S, Hkv, Dh, cap=None):
    cap = cap or S
    k, v = r.normal((S, Hkv, Dh)), r.normal((S, Hkv, Dh))
    kc = np.zeros((cap, Hkv, Dh), np.uint16)
    vc = np.zeros((cap, Hkv, Dh), np.uint16)
    orc.kv_write(k, v, kc, vc, 0)
    return k, v, kc, vc


def test_kv_write_bit_exact_and_offset():
    torch, F = _torch()
    r = SplitMix64(16)
    k, v = r.normal((5, 8, 128)), r.normal((5, 8, 128))
    kc = np.zeros((20, 8, 128), np.uint16)
    vc = np.zeros((20, 8, 128), np.uint16)
    orc.kv_write(k, v, kc, vc, 7)
    tk = torch.from_numpy(k).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    tv = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(kc[7:12], tk)
    np.testing.assert_array_equal(vc[7:12], tv)
    assert not kc[:7].any() and not kc[12:].any()


def test_kv_write_paged_identity_and_permuted():
    r = SplitMix64(17)
    S, Hkv, Dh, ps = 64, 2, 64, 16
    k, v = r.normal((S, Hkv, Dh)), r.normal((S, Hkv, Dh))
    kc = np.zeros((S, Hkv, Dh), np.uint16)
    vc = np.zeros_like(kc)
    orc.kv_write(k, v, kc, vc, 0)
    kp = np.zeros((S // ps, ps, Hkv, Dh), np.uint16)
    vp = np.zeros_like(kp)
    orc.kv_write_paged(k, v, kp, vp, np.arange(S // ps), ps, 0)
    np.testing.assert_array_equal(kp.reshape(S, Hkv, Dh), kc)
    perm = np.array([2, 0, 3, 1], np.int32)
    kp2 = np.zeros_like(kp)
    vp2 = np.zeros_like(vp)
    orc.kv_write_paged(k, v, kp2, vp2, perm, ps, 0)
    for i, p in enumerate(perm):
        np.testing.assert_array_equal(kp2[p], kc[i * ps:(i + 1) * ps])
        np.testing.assert_array_equal(vp2[p], vc[i * ps:(i + 1) * ps])


def _sdpa_cache(q, kc, vc, pos0, scale):
    """torch SDPA (fp64) over the bf16-decoded cache; query row t sees keys [0, pos0+t]."""
    torch, F = _torch()
    Tq, Hq, Dh = q.shape
    Hkv = kc.shape[1]
    S = pos0 + Tq
    kf = torch.from_numpy(orc.from_bf16(kc[:S])).double().permute(1, 0, 2)
    vf = torch.from_numpy(orc.from_bf16(vc[:S])).double().permute(1, 0, 2)
    kf = kf.repeat_interleave(Hq // Hkv, 0)
    vf = vf.repeat_interleave(Hq // Hkv, 0)
    qt = torch.from_numpy(q).double().permute(1, 0, 2)
    mask = torch.arange(S)[None, :] <= (pos0 + torch.arange(Tq))[:, None]
    out = F.scaled_dot_product_attention(qt, kf, vf, attn_mask=mask, scale=scale)
    return out.permute(1, 0, 2).numpy()


@pytest.mark.parametrize("pos0,Tq", [(0, 37), (29, 11)])
def test_prefill_vs_sdpa(pos0, Tq):
    r = SplitMix64(18 + pos0)
    Hq, Hkv, Dh = 16, 8, 128
    _, _, kc, vc = _cache(r, pos0 + Tq, Hkv, Dh)
    q = r.normal((Tq, Hq, Dh))
    scale = 1.0 / math.sqrt(Dh)
    out = orc.gqa_prefill(q, kc, vc, pos0, scale)
    assert rel_err(out, _sdpa_cache(q, kc, vc, pos0, scale), 0.05) < 5e-5


def test_prefill_special_cases():
    r = SplitMix64(19)
    Hq, Hkv, Dh = 4, 2, 64
    # S = 1: the output is v0 exactly
    _, _, kc, vc = _cache(r, 1, Hkv, Dh)
    q = r.normal((1, Hq, Dh))
    out = orc.gqa_prefill(q, kc, vc, 0, 0.125)
    expect = np.repeat(orc.from_bf16(vc[0]), Hq // Hkv, axis=0)
    np.testing.assert_array_equal(out[0], expect)
    # identical keys: uniform weights, output = mean(V) over the attended rows
    S = 9
    kc = np.repeat(kc[:1], S, axis=0)
    vc = orc.to_bf16(r.normal((S, Hkv, Dh)))
    q = r.normal((1, Hq, Dh))
    out = orc.gqa_prefill(q, kc, vc, S - 1, 0.125)
    mean = orc.from_bf16(vc).astype(np.float64).mean(0)
    np.testing.assert_allclose(out[0], np.repeat(mean, Hq // Hkv, axis=0), rtol=0, atol=2e-6)


def test_split_prefill_equivalence():
    r = SplitMix64(20)
    T, split, Hq, Hkv, Dh = 40, 13, 16, 8, 128
    _, _, kc, vc = _cache(r, T, Hkv, Dh)
    q = r.normal((T, Hq, Dh))
    full = orc.gqa_prefill(q, kc, vc, 0, 0.088)
    a = orc.gqa_prefill(q[:split], kc, vc, 0, 0.088)
    b = orc.gqa_prefill(q[split:], kc, vc, split, 0.088)
    np.testing.assert_array_equal(np.concatenate([a, b]), full)
    mt = orc.gqa_prefill(q, kc, vc, 0, 0.088, threads=3)
    np.testing.assert_array_equal(mt, full)


def test_decode_is_last_prefill_row_and_fp64():
    r = SplitMix64(21)
    S, Hq, Hkv, Dh = 513, 16, 8, 128
    _, _, kc, vc = _cache(r, S, Hkv, Dh)
    q = r.normal((Hq, Dh))
    scale = 1.0 / math.sqrt(Dh)
    dec = orc.gqa_decode(q, kc, vc, S - 1, scale)
    pre = orc.gqa_prefill(q[None], kc, vc, S - 1, scale)[0]
    assert rel_err(dec, pre, 0.05) < 5e-5
    truth = orc.attention_f64(q[None], orc.from_bf16(kc), orc.from_bf16(vc), scale, True,
                              kv_off=S - 1)[0]
    assert rel_err(dec, truth, 0.05) < 5e-5


def test_decode_paged_permutation_invariance():
    r = SplitMix64(22)
    B, Hq, Hkv, Dh, ps, npages = 2, 8, 4, 64, 16, 12
    pos = np.array([150, 77], np.int32)
    kp = orc.to_bf16(r.normal((npages * B, ps, Hkv, Dh)))
    vp = orc.to_bf16(r.normal((npages * B, ps, Hkv, Dh)))
    table = np.arange(B * npages, dtype=np.int32).reshape(B, npages)
    q = r.normal((B, Hq, Dh))
    base = orc.gqa_decode_paged(q, kp, vp, table, ps, pos, 0.125)
    # contiguous view of stream 0 = pages 0..npages-1 in order
    c0 = orc.gqa_decode(q[0], kp[:npages].reshape(-1, Hkv, Dh), vp[:npages].reshape(-1, Hkv, Dh),
                        int(pos[0]), 0.125)
    np.testing.assert_array_equal(base[0], c0)
    # move the pages of both streams somewhere else and permute the table alike
    perm = np.array(SplitMix64(5).uniform(B * npages).argsort(), np.int32)
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[perm] = kp
    vp2[perm] = vp
    out = orc.gqa_decode_paged(q, kp2, vp2, perm[table], ps, pos, 0.125)
    np.testing.assert_array_equal(out, base)
    mt = orc.gqa_decode_paged(q, kp2, vp2, perm[table], ps, pos, 0.125, threads=4)
    np.testing.assert_array_equal(mt, base)


# ---------------------------------------------------------------- Conformer ----


def test_relshift_closed_form():
    for T in (1, 2, 3, 7, 717):
        idx = range(T) if T < 100 else range(0, T, 37)
        for i in idx:
            for j in idx:
                row, m = orc.relshift_column(T, i, j)
                assert (row, m) == (i, T - 1 - i + j), (T, i, j)


def test_pos_emb_closed_form():
    T, D = 23, 512
    pe = orc.build_pos_emb(T, D).astype(np.float64)
    pos = (T - 1 - np.arange(2 * T - 1))[:, None].astype(np.float64)
    div = np.exp(-math.log(10000.0) * np.arange(0, D, 2) / D)[None, :]
    np.testing.assert_allclose(pe[:, 0::2], np.sin(pos * div), atol=2e-5)
    np.testing.assert_allclose(pe[:, 1::2], np.cos(pos * div), atol=2e-5)


def _relpos_inputs(r, T, H, Dk):
    return (r.normal((T, H, Dk)), r.normal((T, H, Dk)), r.normal((T, H, Dk)),
            r.normal((2 * T - 1, H, Dk)), r.normal((H, Dk), 0.3), r.normal((H, Dk), 0.3))


@pytest.mark.parametrize("T,valid", [(31, 31), (40, 29)])
def test_relpos_vs_closed_form_fp64(T, valid):
    r = SplitMix64(23 + T)
    H, Dk = 4, 64
    q, k, v, p, u, vb = _relpos_inputs(r, T, H, Dk)
    out = orc.relpos_attention(q, k, v, p, u, vb, valid, 0.125)
    truth = orc.relpos_attention_f64(q, k, v, p, u, vb, valid, 0.125)
    assert rel_err(out, truth, 0.05) < 5e-5


def test_relpos_reduces_to_mha_and_masks_keys():
    torch, F = _torch()
    r = SplitMix64(24)
    T, H, Dk = 33, 2, 64
    q, k, v, p, u, vb = _relpos_inputs(r, T, H, Dk)
    z = np.zeros_like
    out = orc.relpos_attention(q, k, v, z(p), z(u), z(vb), T, 0.125)
    qt, kt, vt = (torch.from_numpy(a).double().permute(1, 0, 2) for a in (q, k, v))
    ref = F.scaled_dot_product_attention(qt, kt, vt, scale=0.125).permute(1, 0, 2).numpy()
    assert rel_err(out, ref, 0.05) < 5e-5
    valid = 20
    a = orc.relpos_attention(q, k, v, p, u, vb, valid, 0.125)
    k2, v2 = k.copy(), v.copy()
    k2[valid:] = r.normal(k2[valid:].shape)
    v2[valid:] = r.normal(v2[valid:].shape)
    b = orc.relpos_attention(q, k2, v2, p, u, vb, valid, 0.125)
    np.testing.assert_array_equal(a, b)
    # valid = 0: the finite -1e30 mask makes every score equal, so each row is mean(V)
    # (src/model/conformer_layer.cu:140-143)
    none = orc.relpos_attention(q, k, v, p, u, vb, 0, 0.125)
    np.testing.assert_allclose(none, np.broadcast_to(v.astype(np.float64).mean(0), v.shape),
                               atol=1e-6)


# ------------------------------------------------------------------ SGEMM ----


@pytest.mark.parametrize("rows,inner,cols,batch", [(13, 64, 13, 8), (14, 64, 14, 8)])
def test_sgemm_batched_reference_pattern(rows, inner, cols, batch):
    # test/unit/model/test_gemm_batched.cu:12-61: index%17/17 and index%13/13 inputs
    a = (np.arange(batch * rows * inner) % 17 / 17.0).astype(np.float32).reshape(batch, rows, inner)
    w = (np.arange(batch * cols * inner) % 13 / 13.0).astype(np.float32).reshape(batch, cols, inner)
    out = orc.sgemm_batched(a, w)
    ref = np.einsum("bmk,bnk->bmn", a.astype(np.float64), w.astype(np.float64))
    assert np.max(np.abs(out - ref)) < 1e-4


def test_sgemm_bias_act():
    r = SplitMix64(25)
    a, w, bias = r.normal((7, 48)), r.normal((9, 48)), r.normal((9,))
    pre = a.astype(np.float64) @ w.astype(np.float64).T + bias
    acts = {0: pre, 1: pre / (1 + np.exp(-pre)), 2: np.maximum(pre, 0), 3: 1 / (1 + np.exp(-pre))}
    for act, ref in acts.items():
        assert rel_err(orc.sgemm(a, w, bias, act), ref, 0.05) < 5e-5, act


# ----------------------------------------------------------------- argmax ----


def test_argmax_banned_matches_numpy():
    r = SplitMix64(26)
    x = r.normal((151936,))
    top = np.argsort(-x)
    assert orc.argmax_banned(x) == int(top[0])
    assert orc.argmax_banned(x, int(top[0])) == int(top[1])
    assert orc.argmax_banned(x, int(top[1]), int(top[0])) == int(top[2])


def test_argmax_tie_rule():
    """Hand-worked cases of the 256-slot scan + halving tree (src/model/asr_ops.cu:306-322):
    at level s slot t takes slot t+s only when strictly greater."""
    n = 1000
    x = np.zeros(n, np.float32)
    # tie inside one slot (2 and 258 are both slot 2): the strict '>' scan keeps 2
    x[[2, 258]] = 5.0
    assert orc.argmax_banned(x) == 2
    # tie between slot 1 (index 1) and slot 2 (index 2): at s=2 slot 0 takes slot 2
    # (5 > 0); at s=1 slot 1 (5) is not > slot 0 (5) -> 2, although index 1 is lower
    x[:] = 0
    x[[1, 2]] = 5.0
    assert orc.argmax_banned(x) == 2
    assert int(np.argmax(x)) == 1  # what a first-index argmax would say
    # tie between slot 1 (index 1) and slot 3 (index 3): at s=2 slot 1 keeps 1 against
    # slot 3; at s=1 slot 0 (value 0) takes slot 1 -> 1
    x[:] = 0
    x[[1, 3]] = 5.0
    assert orc.argmax_banned(x) == 1
    # slot 130 meets slot 2 at level 128 and loses the tie -> 2
    x[:] = 0
    x[[130, 2]] = 5.0
    assert orc.argmax_banned(x) == 2
    # everything -inf: no slot ever updates, the reference returns index 0
    assert orc.argmax_banned(np.full(4, -np.inf, np.float32)) == 0


def test_host_build_pos_emb_matches_oracle():
    """orator_amd.conformer_attn.BuildPosEmb (host, like the reference's) vs the oracle."""
    from orator_amd.conformer_attn import BuildPosEmb
    for T, D in ((1, 512), (23, 512), (717, 512), (5, 7)):
        np.testing.assert_array_equal(BuildPosEmb(T, D), orc.build_pos_emb(T, D))


# ---------------------------------------------------------------- bf16 linear ----


@pytest.mark.parametrize("M,K,N", [(1, 512, 37), (5, 1024, 64), (3, 2048, 9)])
def test_linear_bf16_vs_fp64(M, K, N):
    """asr_gemm::LinearPre on bf16 bits: fp64 matmul of the decoded operands, then bias and
    the activation formulas (GELU from math.erf)."""
    r = SplitMix64(M * K + N)
    x, W = orc.to_bf16(r.normal((M, K))), orc.to_bf16(r.normal((N, K), 0.05))
    bias = r.normal(N)
    ref = orc.from_bf16(x).astype(np.float64) @ orc.from_bf16(W).astype(np.float64).T + bias
    scale = np.abs(orc.from_bf16(x)).astype(np.float64) @ np.abs(orc.from_bf16(W)).T
    for act, f in [(0, lambda v: v), (1, lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2)))),
                   (2, lambda v: max(v, 0.0))]:
        got = orc.linear_bf16(x, W, bias, act)
        want = np.vectorize(f)(ref)
        assert np.max(np.abs(got - want) / (scale + 1.0)) < 1e-5, act
    # no bias, threaded split over N is the same computation
    np.testing.assert_array_equal(orc.linear_bf16(x, W, None, 0, threads=4),
                                  orc.linear_bf16(x, W, None, 0))


@pytest.mark.parametrize("M,K,N", [(1, 300, 37), (6, 257, 9), (9, 64, 5)])
def test_linear_bf16_blocking_keeps_the_serial_chain(M, K, N):
    """orc_linear_bf16 runs outputs side by side; each output must still be the reference's
    serial fp32 chain acc += x[k] * w[k] (mul then add, k ascending), bit for bit."""
    r = SplitMix64(M + 7 * K + N)
    x, W = orc.to_bf16(r.normal((M, K))), orc.to_bf16(r.normal((N, K), 0.05))
    got = orc.linear_bf16(x, W)
    xf, wf = orc.from_bf16(x), orc.from_bf16(W)
    want = np.zeros((M, N), np.float32)
    for k in range(K):  # numpy float32 ops round exactly as the C chain does
        want = want + (xf[:, k][:, None] * wf[:, k][None, :])
    np.testing.assert_array_equal(got, want)


# -------------------------------------------------------------------- decoder ----


def _fake_decoder(script, alt):
    """A decoder whose argmax follows `script` (token k of the stream), answering `alt[k]`
    when the scripted token is banned: isolates the greedy loop's host rules."""
    d = orc.OracleDecoder.__new__(orc.OracleDecoder)
    d.step = 0
    d.steps_run = []
    d.logits = None

    def decode_step(_row, pos):
        d.steps_run.append(pos)
        d.step += 1

    def argmax(b0=-1, b1=-1):
        t = script[d.step]
        return alt[d.step] if t in (b0, b1) else t

    d.decode_step = decode_step
    d.argmax = argmax
    d.embed_row = lambda t: None
    return d


def test_greedy_schedule_known_answers():
    """Batch boundaries of DecodeGreedy (src/model/asr_text_decoder.cu:801-884), worked by
    hand for ban_steps 3, batch 4, max_new 10."""
    assert orc.greedy_schedule(10, 3, 4, False, False) == [1, 2, 6, 10]
    assert orc.greedy_schedule(10, 3, 4, True, False) == [1, 2, 6, 10]
    assert orc.greedy_schedule(10, 3, 4, True, True) == [2, 6, 10]
    assert orc.greedy_schedule(10, 0, 4, True, True) == [4, 8, 10]
    assert orc.greedy_schedule(10, 0, 4, False, False) == [4, 8, 10]
    assert orc.greedy_schedule(1, 3, 4, True, False) == [1]
    assert orc.greedy_schedule(2, 5, 32, True, True) == [2]


def test_greedy_stop_rules():
    E0, E1 = 900, 901
    # EOS at stream index 4 is not emitted; the batch [2, 6) ran to its end
    d = _fake_decoder([5, 6, 7, 8, E0, 3, 3, 3, 3, 3, 3], [0] * 11)
    out, bodies = d.decode_greedy(100, 10, E0, E1, ban_steps=3, batch=4, use_graph=False)
    assert out == [5, 6, 7, 8] and bodies == 6 and d.cache_len == 106
    assert d.steps_run == list(range(100, 106))
    # six identical tokens in a row: the sixth is emitted
    d = _fake_decoder([1, 2, 9, 9, 9, 9, 9, 9, 9, 9, 9, 9, 9], [0] * 13)
    out, bodies = d.decode_greedy(0, 12, E0, E1, ban_steps=0, batch=32, use_graph=False)
    assert out == [1, 2, 9, 9, 9, 9, 9, 9] and bodies == 12
    # EOS banned for stream tokens 0..ban_steps-1 (the seed included), allowed after
    d = _fake_decoder([E1, E0, E0, E1, 4], [11, 12, 13, 14, 15])
    out, bodies = d.decode_greedy(0, 4, E0, E1, ban_steps=3, batch=1, use_graph=True)
    assert out == [11, 12, 13] and bodies == 4
    # no stop: max_new tokens
    d = _fake_decoder(list(range(20)), [0] * 20)
    out, bodies = d.decode_greedy(7, 9, E0, E1, ban_steps=3, batch=4, use_graph=True,
                                  graph_ready=True)
    assert out == list(range(9)) and bodies == 9 and d.cache_len == 16


def _small_decoder(seed=1, **kw):
    import decoder_model as dm
    cfg = dict(dm.SMALL, num_layers=1, max_seq_len=64)
    return cfg, orc.OracleDecoder(cfg, *dm.make_weights(cfg, seed, **kw))


def test_decoder_split_prefill_and_decode_step_equivalence():
    """The reference's T010 check (test/unit/model/test_asr_decoder.cc:76-123) on the
    oracle: PrefillAt in two parts == one Prefill; TruncateCache + re-prefill; and a decode
    step == the last row of a prefill one token longer."""
    cfg, d = _small_decoder()
    r = SplitMix64(3)
    emb = r.normal((21, cfg["hidden_size"]), 0.02)
    d.prefill_at(emb, 0)
    full = d.logits.copy()
    d.prefill_at(emb[:9], 0)
    d.prefill_at(emb[9:], 9)
    assert d.cache_len == 21
    assert rel_err(d.logits, full, 0.05) < 1e-5
    d.cache_len = 9
    d.prefill_at(emb[9:], 9)
    assert rel_err(d.logits, full, 0.05) < 1e-5
    d.prefill_at(emb[:20], 0)
    d.decode_step(emb[20], 20)
    assert d.cache_len == 21
    assert rel_err(d.logits, full, 0.05) < 1e-5


def test_twin_decoder_keeps_the_oracle_and_shadows_it():
    """The greedy checkers' TwinDecoder: its own logits are the oracle's bit for bit, and its
    BLAS-order shadow differs from them only by fp32 summation order (within the decoder
    logit bar, 1e-2 of max |logit|, and not identical: the orders do differ)."""
    import decoder_model as dm
    cfg = dict(dm.SMALL, num_layers=1, max_seq_len=64)
    w = dm.make_weights(cfg, 5)
    a, t = orc.OracleDecoder(cfg, *w), orc.TwinDecoder(cfg, *w)
    emb = SplitMix64(6).normal((11, cfg["hidden_size"]), 0.02)
    for d in (a, t):
        d.prefill_at(emb[:10], 0)
        d.decode_step(emb[10], 10)
    np.testing.assert_array_equal(t.logits, a.logits)
    gap = np.max(np.abs(t.shadow.logits - a.logits))
    assert 0 < gap <= 1e-2 * np.max(np.abs(a.logits)), gap


def test_decoder_zero_layers_is_embedding_head():
    """Zero projection weights leave the residual stream at the input: logits =
    lm_head . bf16(RmsNorm(x) * final_norm), checked with fp64 numpy."""
    cfg, d = _small_decoder(seed=2)
    for L in d.layers:
        for k in ("qkv_w", "o_w", "gateup_w", "down_w"):
            L[k] = np.zeros_like(L[k])
    x = SplitMix64(4).normal((5, cfg["hidden_size"]), 0.02)
    d.prefill_at(x, 0)
    last = x[-1].astype(np.float64)
    n = last / np.sqrt(np.mean(last * last) + cfg["rms_norm_eps"]) * d.final_norm
    want = orc.from_bf16(d.lm_head).astype(np.float64) @ orc.from_bf16(orc.to_bf16(n))
    assert np.max(np.abs(d.logits - want)) < 1e-4 * np.max(np.abs(want))


# ------------------------------------------------------------- window attention ----


def _windows(N, width):
    """Consecutive windows of `width` (the last one ragged), as the audio tower's
    cu_seqlens segments (src/model/asr_audio_tower.cu:509-533)."""
    ss, se = np.zeros(N, np.int32), np.zeros(N, np.int32)
    for s0 in range(0, N, width):
        ss[s0:s0 + width], se[s0:s0 + width] = s0, min(N, s0 + width)
    return ss, se


def test_window_attention_full_is_noncausal_gqa_and_fp64():
    r = SplitMix64(61)
    N, H, Dh = 45, 4, 64
    q, k, v = r.normal((N, H, Dh)), r.normal((N, H, Dh)), r.normal((N, H, Dh))
    ss, se = np.zeros(N, np.int32), np.full(N, N, np.int32)
    got = orc.window_attention(q, k, v, ss, se, 0.125)
    assert rel_err(got, orc.gqa_attention(q, k, v, 0.125, False), 0.05) < 1e-6
    assert rel_err(got, orc.attention_f64(q, k, v, 0.125, False), 0.05) < 1e-5


def test_window_attention_block_diagonal_and_empty():
    """Windows of 13 (ragged last) equal attention within each segment; an empty window
    (seg_start == seg_end) gives zeros."""
    r = SplitMix64(62)
    N, H, Dh = 40, 2, 64
    q, k, v = r.normal((N, H, Dh)), r.normal((N, H, Dh)), r.normal((N, H, Dh))
    ss, se = _windows(N, 13)
    se[5] = ss[5]
    got = orc.window_attention(q, k, v, ss, se, 0.2)
    for s0 in range(0, N, 13):
        s1 = min(N, s0 + 13)
        want = orc.attention_f64(q[s0:s1], k[s0:s1], v[s0:s1], 0.2, False)
        rows = [i for i in range(s0, s1) if i != 5]
        assert rel_err(got[rows], want[[i - s0 for i in rows]], 0.05) < 1e-5
    assert np.all(got[5] == 0)


# ------------------------------------------------------------------ masked MHA ----


@pytest.mark.parametrize("valid", [41, 25, 0])
def test_masked_mha_vs_sdpa_and_relpos(valid):
    """The Sortformer decomposition against torch SDPA with a key mask (fp64), against the
    rel-pos oracle with u = v = 0 and P = 0 (the same softmax over AC), and valid_len 0 giving
    the mean of V (every score -1e30, uniform softmax)."""
    torch, F = _torch()
    r = SplitMix64(70 + valid)
    T, H, Dk = 41, 8, 24
    q, k, v = r.normal((T, H, Dk)), r.normal((T, H, Dk)), r.normal((T, H, Dk))
    scale = 1.0 / math.sqrt(Dk)
    got = orc.masked_mha(q, k, v, valid, scale)
    if valid == 0:
        want = np.broadcast_to(v.astype(np.float64).mean(axis=0), v.shape)
        assert rel_err(got, want, 0.05) < 1e-5
        return
    qt, kt, vt = (torch.from_numpy(a).double().permute(1, 0, 2) for a in (q, k, v))
    mask = torch.zeros(T, T, dtype=torch.bool)
    mask[:, :valid] = True
    ref = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    assert rel_err(got, ref.permute(1, 0, 2).numpy(), 0.05) < 1e-5
    z = np.zeros
    rp = orc.relpos_attention(q, k, v, z((2 * T - 1, H, Dk), np.float32), z((H, Dk), np.float32),
                              z((H, Dk), np.float32), valid, scale)
    assert rel_err(got, rp, 0.05) < 1e-5


# ------------------------------------------------------------ Conformer layer ----


from conformer_model import conformer_weights as _conformer_weights  # noqa: E402


def test_conformer_passes_vs_torch():
    torch, F = _torch()
    r = SplitMix64(80)
    T, C, K = 19, 24, 9
    x = r.normal((T, C))
    g, b = 1 + r.normal(C, 0.1), r.normal(C, 0.1)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    want = F.layer_norm(t(x), (C,), t(g), t(b), eps=1e-5).numpy()
    assert rel_err(orc.layer_norm(x, g, b), want, 0.05) < 1e-5
    x2 = r.normal((T, 2 * C))
    want = F.glu(t(x2), dim=-1).numpy()
    want[13:] = 0
    assert rel_err(orc.glu_mask(x2, 13), want, 0.05) < 1e-6
    w, bias = r.normal((C, K), 0.3), r.normal(C, 0.1)
    mean, var = r.normal(C, 0.1), (0.5 + r.uniform(C)).astype(np.float32)
    conv = F.conv1d(t(x).T[None], t(w)[:, None, :], t(bias), padding=(K - 1) // 2, groups=C)
    y = F.silu(F.batch_norm(conv, t(mean), t(var), t(g), t(b), training=False, eps=1e-5))
    got = orc.dwconv_bn_silu(x, w, bias, mean, var, g, b)
    assert rel_err(got, y[0].T.numpy(), 0.05) < 1e-5


def test_conformer_layer_vs_torch_composition():
    """The composed layer against the same steps written with torch routines in fp64 (the
    rel-pos core from the fp64 oracle), so a wrong residual weight, norm or order fails."""
    torch, F = _torch()
    r = SplitMix64(81)
    T, D, H, Dff, K, valid = 21, 32, 2, 64, 9, 17
    W = _conformer_weights(r, D, H, Dff, K)
    x = r.normal((T, D))
    pe = orc.build_pos_emb(T, D)
    got = orc.conformer_layer(x, T, valid, pe, W, H)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    Tw = {k: t(v) for k, v in W.items()}
    X = t(x)
    ln = lambda z, n: F.layer_norm(z, (D,), Tw[f"norm_{n}_w"], Tw[f"norm_{n}_b"], eps=1e-5)
    ffn = lambda z, p: F.linear(F.silu(F.linear(ln(z, p), Tw[f"{p}_w1"], Tw[f"{p}_b1"])),
                                Tw[f"{p}_w2"], Tw[f"{p}_b2"])
    X = X + 0.5 * ffn(X, "ff1")
    a = ln(X, "att")
    q, k, v = (F.linear(a, Tw[f"{n}_w"], Tw[f"{n}_b"]).numpy().reshape(T, H, D // H)
               for n in ("q", "k", "v"))
    p = F.linear(t(pe), Tw["pos_w"]).numpy().reshape(2 * T - 1, H, D // H)
    ctx = orc.relpos_attention_f64(q, k, v, p, W["pos_bias_u"], W["pos_bias_v"], valid,
                                   1.0 / math.sqrt(D // H))
    X = X + F.linear(t(ctx).reshape(T, D), Tw["out_w"], Tw["out_b"])
    c = F.glu(F.linear(ln(X, "conv"), Tw["pw1_w"], Tw["pw1_b"]), dim=-1)
    c[valid:] = 0
    c = F.conv1d(c.T[None], Tw["dw_w"][:, None, :], Tw["dw_b"], padding=(K - 1) // 2, groups=D)
    c = F.silu(F.batch_norm(c, Tw["bn_mean"], Tw["bn_var"], Tw["bn_w"], Tw["bn_b"],
                            training=False, eps=1e-5))[0].T
    X = X + F.linear(c, Tw["pw2_w"], Tw["pw2_b"])
    X = X + 0.5 * ffn(X, "ff2")
    want = ln(X, "out").numpy()
    assert rel_err(got, want, 0.05) < 1e-4


# ------------------------------------------ decoder composition vs transformers Qwen3 ----
class _SwapGateUp(orc.OracleDecoder):
    def _layer_tail(self, L, x, attn):
        I = self.c["intermediate_size"]
        L = dict(L, gateup_w=np.concatenate([L["gateup_w"][I:], L["gateup_w"][:I]]))
        return super()._layer_tail(L, x, attn)


class _SwapLayerNorms(orc.OracleDecoder):
    def _layer_qkv(self, L, x, pos):
        return super()._layer_qkv(dict(L, in_ln=L["post_ln"], post_ln=L["in_ln"]), x, pos)

    def _layer_tail(self, L, x, attn):
        return super()._layer_tail(dict(L, in_ln=L["post_ln"], post_ln=L["in_ln"]), x, attn)


class _SwapQkNorms(orc.OracleDecoder):
    def _layer_qkv(self, L, x, pos):
        return super()._layer_qkv(dict(L, q_norm=L["k_norm"], k_norm=L["q_norm"]), x, pos)


class _NormedResidual(orc.OracleDecoder):
    """Adds the MLP to the normed stream instead of the residual stream."""
    def _layer_tail(self, L, x, attn):
        c = self.c
        T, I = x.shape[0], c["intermediate_size"]
        x = x + self._lin(orc.to_bf16(attn.reshape(T, -1)), L["o_w"])
        n = orc.rms_norm(x, L["post_ln"], c["rms_norm_eps"])
        nb = orc.to_bf16(n)
        gate, up = self._lin(nb, L["gateup_w"][:I]), self._lin(nb, L["gateup_w"][I:])
        return n + self._lin(orc.to_bf16(orc.swiglu(gate, up)), L["down_w"])


HF_BAR = 1e-2  # max |oracle - HF| / max |HF| on the logits


@pytest.mark.parametrize("tied", [False, True])
def test_decoder_composition_matches_transformers_qwen3(tied):
    """OracleDecoder (the decoder composition every a8/a9/a15 GPU result is checked against)
    against an independent restatement: transformers' Qwen3ForCausalLM in fp32 with the same
    bf16-valued weights (q/k/v and gate/up split out of the fused layout as
    src/model/asr_text_decoder.cu:283-306 fuses them), rope_theta 1e6, eps 1e-6, eager
    attention, and the reference's bf16 roundings as hooks (every projection input, the K/V
    cache rows).  Both sides round to bf16 at the same points, so what remains is fp32
    summation order re-rounded to bf16 (a whole bf16 step on the ~1 % of K/V elements whose
    two fp32 values straddle a rounding boundary), 0.25-0.35 % of max |logit| here.  Bar:
    1 %.  Composition mistakes land far outside it (each is checked): gate/up swapped ~18 %,
    in/post layer norms swapped ~27 %, q/k norms swapped ~5.6 %, MLP added to the normed
    stream ~80 %.  Prefill (last row) and one decode step."""
    import decoder_model as dm
    import hf_qwen3 as hq

    cfg = dict(dm.SMALL)
    w = dm.make_weights(cfg, 5, tied=tied)
    T, tok = 40, 123
    emb = SplitMix64(9).normal((T, cfg["hidden_size"]), 0.02)
    model, ctx = hq.build(cfg, w)

    def run(cls):
        d = cls(cfg, *w)
        d.prefill_at(emb, 0)
        lp = d.logits.copy()
        d.decode_step(d.embed_row(tok), T)
        return lp, d.logits.copy(), d.embed_row(tok)

    lp, ld, row = run(orc.OracleDecoder)
    ref = hq.logits(model, ctx, np.concatenate([emb, row[None]]))
    err_p = np.max(np.abs(lp - ref[T - 1])) / np.max(np.abs(ref[T - 1]))
    err_d = np.max(np.abs(ld - ref[T])) / np.max(np.abs(ref[T]))
    print(f"oracle vs HF Qwen3: prefill {err_p:.2e}, decode {err_d:.2e} of max|logit|")
    assert err_p <= HF_BAR and err_d <= HF_BAR
    assert int(np.argmax(lp)) == int(np.argmax(ref[T - 1]))
    for cls in (_SwapGateUp, _SwapLayerNorms, _SwapQkNorms, _NormedResidual):
        mp, _, _ = run(cls)
        err = np.max(np.abs(mp - ref[T - 1])) / np.max(np.abs(ref[T - 1]))
        assert err > 4 * HF_BAR, (cls.__name__, err)
