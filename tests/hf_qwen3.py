"""An independent CPU restatement of the text decoder for pinning the oracle's composition:
transformers' Qwen3ForCausalLM (the upstream model the reference loads its weights from,
src/model/asr_text_decoder.cu:283-306 reads the same q/k/v/o, gate/up/down and norm tensors),
built in fp32 from the same bf16-valued weights, with the reference's bf16 roundings added as
hooks: every projection's input (asr_gemm::Linear/LinearPre cast, asr_text_decoder.cu:400-440,
:518-556) and the K/V cache rows (WriteKvCacheKernel stores bf16 after QK-norm + RoPE,
:60-77)."""
from __future__ import annotations

import contextlib

import numpy as np


def _bf16(t):
    import torch
    return t.to(torch.bfloat16).to(torch.float32)


def build(cfg, weights, bf16_hooks: bool = True, swap_gate_up: bool = False):
    """weights = (embed, final_norm, lm_head or None, layers) in the library's fused layout
    (decoder_model.make_weights).  Returns (model, ctx): run the model inside `with ctx():`."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from transformers.models.qwen3 import modeling_qwen3 as mq

    import oracle_lib as orc

    embed, final_norm, lm_head, layers = weights
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    Hq, Hkv, Dh = cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    Qd, KVd = Hq * Dh, Hkv * Dh
    hc = Qwen3Config(vocab_size=cfg["vocab_size"], hidden_size=H, intermediate_size=I,
                     num_hidden_layers=cfg["num_layers"], num_attention_heads=Hq,
                     num_key_value_heads=Hkv, head_dim=Dh,
                     max_position_embeddings=cfg["max_seq_len"],
                     rms_norm_eps=cfg["rms_norm_eps"],
                     rope_parameters={"rope_type": "default", "rope_theta": cfg["rope_theta"]},
                     tie_word_embeddings=lm_head is None, attention_bias=False)
    hc._attn_implementation = "eager"
    model = Qwen3ForCausalLM(hc).to(torch.float32).eval()

    def t(a):
        a = orc.from_bf16(a) if a.dtype == np.uint16 else np.asarray(a, np.float32)
        return torch.from_numpy(np.ascontiguousarray(a))

    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(t(embed))
        model.model.norm.weight.copy_(t(final_norm))
        if lm_head is not None:
            model.lm_head.weight.copy_(t(lm_head))
        for L, hl in zip(layers, model.model.layers):
            a, m = hl.self_attn, hl.mlp
            hl.input_layernorm.weight.copy_(t(L["in_ln"]))
            hl.post_attention_layernorm.weight.copy_(t(L["post_ln"]))
            a.q_norm.weight.copy_(t(L["q_norm"]))
            a.k_norm.weight.copy_(t(L["k_norm"]))
            a.q_proj.weight.copy_(t(L["qkv_w"][:Qd]))
            a.k_proj.weight.copy_(t(L["qkv_w"][Qd:Qd + KVd]))
            a.v_proj.weight.copy_(t(L["qkv_w"][Qd + KVd:]))
            a.o_proj.weight.copy_(t(L["o_w"]))
            g, u = t(L["gateup_w"][:I]), t(L["gateup_w"][I:])
            if swap_gate_up:
                g, u = u, g
            m.gate_proj.weight.copy_(g)
            m.up_proj.weight.copy_(u)
            m.down_proj.weight.copy_(t(L["down_w"]))
    if lm_head is None:
        model.tie_weights()

    @contextlib.contextmanager
    def ctx():
        handles = []
        orig = mq.apply_rotary_pos_emb
        if bf16_hooks:
            for mod in model.modules():
                if isinstance(mod, torch.nn.Linear):
                    handles.append(mod.register_forward_pre_hook(lambda _m, a: (_bf16(a[0]),)))
            for hl in model.model.layers:
                handles.append(hl.self_attn.v_proj.register_forward_hook(
                    lambda _m, _a, out: _bf16(out)))

            def rope_then_bf16_k(q, k, cos, sin, *a, **kw):
                qe, ke = orig(q, k, cos, sin, *a, **kw)
                return qe, _bf16(ke)
            mq.apply_rotary_pos_emb = rope_then_bf16_k
        try:
            with torch.no_grad():
                yield
        finally:
            mq.apply_rotary_pos_emb = orig
            for h in handles:
                h.remove()

    return model, ctx


def logits(model, ctx, embeds) -> np.ndarray:
    """Logits of every row of a causal forward over embeds [T, hidden] at positions 0..T-1."""
    import torch
    with ctx():
        x = torch.from_numpy(np.ascontiguousarray(embeds, np.float32))[None]
        pos = torch.arange(x.shape[1])[None]
        out = model(inputs_embeds=x, position_ids=pos, use_cache=False)
    return out.logits[0].numpy()
