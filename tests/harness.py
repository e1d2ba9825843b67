"""Shared test helpers: oracle models → the reference's shared-weight /
adapter / meta dicts, GPU activation stores, and error metrics.

Test infrastructure (imports the oracle); used by tests/, smoke() and the
bench's CPU-baseline leg only."""

from __future__ import annotations

import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for _p in (ROOT, os.path.join(ROOT, "deltaserve-vllm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

from oracle import dsb_oracle as O  # noqa: E402

LORA_KEY = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
            "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
            "down": "mlp.down_proj"}


def tiny_meta(family="llama3", L=2, D=256, Hq=2, Hkv=1, I=512, V=1000, r=8, theta=5e5,
              eps=1e-5, scaling=2.0, rope_scaling=None, lr=1e-4, s_max=512, tie=False):
    return dict(family=family, num_hidden_layers=L, hidden_size=D, num_attention_heads=Hq,
                num_key_value_heads=Hkv, head_dim=128, intermediate_size=I, vocab_size=V,
                lora_rank=r, rope_theta=theta, rms_norm_eps=eps, lora_scaling=scaling,
                rope_scaling=rope_scaling, learning_rate=lr, weight_decay=0.0, gamma=1.0,
                max_saved_finetuning_tokens=s_max, tie_word_embeddings=tie)


def peft_key(i, proj, ab):
    return f"base_model.model.model.layers.{i}.{LORA_KEY[proj]}.lora_{ab}.weight"


def shared_from_model(model: O.Model, device="cuda"):
    """(base, ft, meta) exactly as the reference's worker shares them: fused
    bf16 qkv_proj / gate_up_proj, PEFT-keyed fp32 LoRA factors."""
    bf = lambda t: t.to(device=device, dtype=torch.bfloat16).contiguous()  # noqa: E731
    base = {"model.norm.weight": bf(model.norm_w), "model.embed_tokens.weight": bf(model.embed)}
    meta = dict(model.meta)
    if model.meta.get("tie_word_embeddings"):
        meta["lm_head_key"] = "model.embed_tokens.weight"
    else:
        base["lm_head.weight"] = bf(model.lm_w)
        meta["lm_head_key"] = "lm_head.weight"
    meta["norm_weight_key"] = "model.norm.weight"
    ft = {}
    for i, lw in enumerate(model.layers):
        p = f"model.layers.{i}."
        base[p + "self_attn.qkv_proj.weight"] = bf(torch.cat([lw["q"], lw["k"], lw["v"]], 0))
        base[p + "self_attn.o_proj.weight"] = bf(lw["o"])
        base[p + "mlp.gate_up_proj.weight"] = bf(torch.cat([lw["gate"], lw["up"]], 0))
        base[p + "mlp.down_proj.weight"] = bf(lw["down"])
        base[p + "input_layernorm.weight"] = bf(lw["in_ln"])
        base[p + "post_attention_layernorm.weight"] = bf(lw["post_ln"])
        if "q_norm" in lw:
            base[p + "self_attn.q_norm.weight"] = bf(lw["q_norm"])
            base[p + "self_attn.k_norm.weight"] = bf(lw["k_norm"])
        for proj in O.PROJS:
            if proj + "A" in lw:
                ft[peft_key(i, proj, "A")] = lw[proj + "A"].clone()
                ft[peft_key(i, proj, "B")] = lw[proj + "B"].clone()
    return base, ft, meta


def gpu_activations(acts, s_max, device="cuda"):
    """The reference's activation store layout: [s_max + 1, D] bf16 buffers
    (rows past n zero) and int64 ids [s_max]."""
    n, D = acts["final_in"].shape

    def buf(t):
        b = torch.zeros(s_max + 1, D, dtype=torch.bfloat16, device=device)
        b[:n] = t.to(device=device, dtype=torch.bfloat16)
        return b

    ids = torch.zeros(s_max, dtype=torch.int64, device=device)
    ids[:n] = acts["concat_input_ids"].to(device)
    return {"layer_in": [buf(t) for t in acts["layer_in"]], "final_in": buf(acts["final_in"]),
            "concat_input_ids": ids}


def bf16_round_acts(acts):
    """The activations as the GPU sees them (bf16 values), in fp32."""
    return {"layer_in": [t.to(torch.bfloat16).float() for t in acts["layer_in"]],
            "final_in": acts["final_in"].to(torch.bfloat16).float(),
            "concat_input_ids": acts["concat_input_ids"]}


def build_service(model: O.Model, family="llama3", device="cuda"):
    from deltaserve_amd.bwd_services.registry import get_service

    base, ft, meta = shared_from_model(model, device)
    svc = get_service(family)(0)
    svc.shared = {"base": base, "ft": ft, "meta": meta}
    err = svc._on_weights_shared()
    if err:
        raise RuntimeError(err)
    return svc


def max_rel(got, ref):
    """bwd_harness.Checker metric: max|got − ref| / (max|ref| + 1e-8)."""
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    return ((got - ref).abs().max() / (ref.abs().max() + 1e-8)).item()


def cosine(got, ref):
    got, ref = got.detach().float().cpu().flatten(), ref.detach().float().cpu().flatten()
    return torch.nn.functional.cosine_similarity(got, ref, dim=0).item()
