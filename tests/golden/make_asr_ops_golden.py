"""Regenerates tests/golden/asr_ops_golden.npz: the reference's asr_ops fixtures.

The reference validates RMSNorm, interleaved RoPE, SwiGLU and causal GQA against torch
outputs stored under models/reference/asr_ops (test/unit/model/test_asr_ops.cc:20-23,
73-169).  Those files are not in the reference tree, but their recipe is: the inputs are
numpy default_rng(seed).random() draws mapped to [-1, 1) with seeds 1..4, and the
outputs are torch fp32 formulas (tools/dump/dump_asr_ops.py:36-110).  This script
replays that recipe on the CPU (torch fp32 on "cpu" instead of "cuda") and stores
inputs and outputs.  The C++ test's tolerances travel with the fixture: RMSNorm 1e-4,
RoPE 1e-4, SwiGLU 1e-5, GQA 5e-4 max-abs (test_asr_ops.cc:93,118,141,167).

Run:  python tests/golden/make_asr_ops_golden.py
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
OUT = HERE / "asr_ops_golden.npz"
MANIFEST = HERE / "asr_ops_golden.sha256.json"


def uniform(seed: int):
    g = np.random.default_rng(seed)
    return lambda *shape: (g.random(shape, dtype=np.float64).astype(np.float32) * 2.0 - 1.0)


def rmsnorm():
    rows, dim, eps = 8, 2048, 1e-6
    r = uniform(1)
    x = r(rows, dim)
    w = (0.5 + 0.5 * r(dim)).astype(np.float32)
    xt, wt = torch.from_numpy(x), torch.from_numpy(w)
    y = (xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + eps)) * wt
    return {"rmsnorm_x": x, "rmsnorm_w": w, "rmsnorm_out": y.numpy()}


def rope():
    T, H, Dh, base = 12, 16, 128, 1_000_000.0
    r = uniform(2)
    x = r(T, H, Dh)
    pos = np.arange(T, dtype=np.int32)
    xt = torch.from_numpy(x)
    i = torch.arange(Dh // 2, dtype=torch.float32)
    inv_freq = base ** (-2.0 * i / Dh)
    angle = torch.from_numpy(pos).to(torch.float32)[:, None] * inv_freq[None, :]
    cos, sin = angle.cos()[:, None, :], angle.sin()[:, None, :]
    x1, x2 = xt[..., 0::2], xt[..., 1::2]
    out = torch.empty_like(xt)
    out[..., 0::2] = x1 * cos - x2 * sin
    out[..., 1::2] = x1 * sin + x2 * cos
    return {"rope_x": x, "rope_pos": pos, "rope_out": out.numpy()}


def swiglu():
    n = 8 * 6144
    r = uniform(3)
    g = (3.0 * r(n)).astype(np.float32)
    u = r(n)
    o = F.silu(torch.from_numpy(g)) * torch.from_numpy(u)
    return {"swiglu_gate": g, "swiglu_up": u, "swiglu_out": o.numpy()}


def gqa():
    T, Hq, Hkv, Dh = 24, 16, 8, 128
    scale = 1.0 / np.sqrt(Dh)
    r = uniform(4)
    q = (0.3 * r(T, Hq, Dh)).astype(np.float32)
    k = (0.3 * r(T, Hkv, Dh)).astype(np.float32)
    v = r(T, Hkv, Dh)
    qt = torch.from_numpy(q).permute(1, 0, 2).unsqueeze(0)
    kt = torch.from_numpy(k).permute(1, 0, 2).unsqueeze(0).repeat_interleave(Hq // Hkv, dim=1)
    vt = torch.from_numpy(v).permute(1, 0, 2).unsqueeze(0).repeat_interleave(Hq // Hkv, dim=1)
    out = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=float(scale))
    out = out.squeeze(0).permute(1, 0, 2).contiguous()
    return {"gqa_q": q, "gqa_k": k, "gqa_v": v, "gqa_out": out.numpy()}


def main() -> None:
    torch.manual_seed(0)
    data = {}
    for fn in (rmsnorm, rope, swiglu, gqa):
        data.update(fn())
    np.savez_compressed(OUT, **data)
    manifest = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()
                for k, v in sorted(data.items())}
    manifest["_torch"] = torch.__version__
    MANIFEST.write_text(json.dumps(manifest, indent=1) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
