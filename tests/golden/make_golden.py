"""Write the golden fixtures under tests/golden/ from transformers (run on CPU).

    python tests/golden/make_golden.py

Fixtures (data only, no code):
  rope_llama3.json       inverse frequencies and cos/sin at fixed positions
                         from transformers' RoPE initialisers (default, linear,
                         llama3 at the C5 settings).
  cycle_{family}.safetensors
                         one LoRA-SFT cycle of a tiny model computed by
                         transformers' LlamaForCausalLM / Qwen3ForCausalLM with
                         the LoRA delta W + s·B·A applied through
                         torch.func.functional_call and differentiated by
                         autograd: loss, n_valid, the unclipped gradient of
                         every LoRA factor, the token ids and sequence
                         lengths. The model itself is regenerated from
                         (meta, seed) by the oracle's make_model; a checksum of
                         its weights is stored to detect generator drift.

The reference (deltaserve-plugin) is not imported: transformers computes the
same model (tests/bwd_harness.py:160-258 of the reference builds its expected
values the same way, by autograd of a functional forward).
"""

from __future__ import annotations

import json
import os
import sys

import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from harness import O, tiny_meta  # noqa: E402

HF_PROJ = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
           "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
           "down": "mlp.down_proj"}

CYCLES = {
    "llama3": dict(meta=dict(family="llama3", L=2, D=128, Hq=2, Hkv=1, I=160, V=211, r=8,
                             theta=5e5, eps=1e-5, s_max=512,
                             rope_scaling={"rope_type": "llama3", "factor": 8.0,
                                           "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                           "original_max_position_embeddings": 64.0}),
                   seed=11, seq_lens=[37, 1, 90, 16]),
    "qwen3": dict(meta=dict(family="qwen3", L=2, D=128, Hq=4, Hkv=2, I=192, V=197, r=8,
                            theta=1e6, eps=1e-6, s_max=512, tie=True),
                  seed=12, seq_lens=[70, 2, 55]),
}
WSTD, BSTD, JITTER = 0.08, 0.05, 0.2


def weight_checksum(model) -> float:
    tot = model.embed.double().abs().sum() + model.norm_w.double().sum()
    for lw in model.layers:
        for k in sorted(lw):
            tot = tot + lw[k].double().abs().sum()
    return float(tot)


def build_model(spec):
    m = spec["meta"]
    meta = tiny_meta(family=m["family"], L=m["L"], D=m["D"], Hq=m["Hq"], Hkv=m["Hkv"], I=m["I"],
                     V=m["V"], r=m["r"], theta=m["theta"], eps=m["eps"],
                     rope_scaling=m.get("rope_scaling"), s_max=m["s_max"],
                     tie=m.get("tie", False))
    return O.make_model(meta, seed=spec["seed"], w_std=WSTD, b_std=BSTD, norm_jitter=JITTER)


def _hf(model):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    m = model.meta
    rp = {"rope_type": "default", "rope_theta": m["rope_theta"]}
    rp.update(m.get("rope_scaling") or {})
    qwen = m["family"] == "qwen3"
    cfg = (Qwen3Config if qwen else LlamaConfig)(
        hidden_size=m["hidden_size"], intermediate_size=m["intermediate_size"],
        num_hidden_layers=m["num_hidden_layers"], num_attention_heads=m["num_attention_heads"],
        num_key_value_heads=m["num_key_value_heads"], head_dim=128,
        vocab_size=m["vocab_size"], rms_norm_eps=m["rms_norm_eps"], rope_parameters=rp,
        max_position_embeddings=131072, tie_word_embeddings=bool(m.get("tie_word_embeddings")),
        attention_bias=False)
    cfg._attn_implementation = "sdpa"
    hf = (Qwen3ForCausalLM if qwen else LlamaForCausalLM)(cfg).eval()
    with torch.no_grad():
        hf.model.embed_tokens.weight.copy_(model.embed)
        hf.model.norm.weight.copy_(model.norm_w)
        if not m.get("tie_word_embeddings"):
            hf.lm_head.weight.copy_(model.lm_w)
        for i, lw in enumerate(model.layers):
            layer = hf.model.layers[i]
            for p, name in HF_PROJ.items():
                layer.get_submodule(name).weight.copy_(lw[p])
            layer.input_layernorm.weight.copy_(lw["in_ln"])
            layer.post_attention_layernorm.weight.copy_(lw["post_ln"])
            if qwen:
                layer.self_attn.q_norm.weight.copy_(lw["q_norm"])
                layer.self_attn.k_norm.weight.copy_(lw["k_norm"])
    return hf


def hf_cycle(model, ids, seq_lens):
    from torch.func import functional_call

    hf = _hf(model)
    s = model.meta["lora_scaling"]
    leaves, over = {}, {}
    for i, lw in enumerate(model.layers):
        for p, name in HF_PROJ.items():
            A = lw[p + "A"].clone().requires_grad_(True)
            B = lw[p + "B"].clone().requires_grad_(True)
            leaves[f"{i}.{p}A"], leaves[f"{i}.{p}B"] = A, B
            full = f"model.layers.{i}.{name}.weight"
            over[full] = hf.get_parameter(full) + s * B @ A
    tot, cnt, st = 0.0, 0, 0
    for L in seq_lens:
        logits = functional_call(hf, over, (ids[st:st + L][None],),
                                 {"position_ids": torch.arange(L)[None]}).logits[0]
        if L >= 2:
            tot = tot + F.cross_entropy(logits[:-1], ids[st + 1:st + L], reduction="sum")
            cnt += L - 1
        st += L
    loss = tot / cnt
    loss.backward()
    return float(loss.detach()), cnt, {k: t.grad.detach().clone() for k, t in leaves.items()}


def cycle_ids(spec):
    n = sum(spec["seq_lens"])
    g = torch.Generator().manual_seed(spec["seed"] + 100)
    return torch.randint(0, spec["meta"]["V"], (n,), generator=g)


def write_cycles():
    from safetensors.torch import save_file

    for fam, spec in CYCLES.items():
        model = build_model(spec)
        ids = cycle_ids(spec)
        loss, nv, grads = hf_cycle(model, ids, spec["seq_lens"])
        tensors = {f"grad.{k}": v.contiguous() for k, v in grads.items()}
        tensors["ids"] = ids.to(torch.int64)
        tensors["seq_lens"] = torch.tensor(spec["seq_lens"], dtype=torch.int64)
        meta = {"spec": json.dumps(spec), "loss": repr(loss), "n_valid": str(nv),
                "weight_checksum": repr(weight_checksum(model)),
                "init": json.dumps({"w_std": WSTD, "b_std": BSTD, "norm_jitter": JITTER})}
        save_file(tensors, os.path.join(HERE, f"cycle_{fam}.safetensors"), metadata=meta)
        print(f"cycle_{fam}: loss={loss:.6f} n_valid={nv} tensors={len(tensors)}")


def write_rope():
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    positions = [0, 1, 7, 100, 1023, 4097, 8191, 16383]
    cases = [("default_5e5", 5e5, None), ("default_1e6", 1e6, None),
             ("linear_4", 1e4, {"rope_type": "linear", "factor": 4.0}),
             ("llama3_c5", 5e5, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                 "high_freq_factor": 4.0,
                                 "original_max_position_embeddings": 8192})]
    out = {"positions": positions, "head_dim": 128, "cases": []}
    for name, theta, rs in cases:
        rp = {"rope_type": "default", "rope_theta": theta}
        rp.update(rs or {})
        cfg = LlamaConfig(hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
                          head_dim=128, intermediate_size=512, num_hidden_layers=1,
                          vocab_size=64, rope_parameters=rp, max_position_embeddings=131072)
        if rs is None:
            inv, _ = LlamaRotaryEmbedding.compute_default_rope_parameters(cfg)
        else:
            inv, _ = ROPE_INIT_FUNCTIONS[rs["rope_type"]](cfg)
        emb = LlamaRotaryEmbedding(cfg)
        cos, sin = emb(torch.zeros(1, len(positions), 128), torch.tensor([positions]))
        out["cases"].append({"name": name, "theta": theta, "rope_scaling": rs,
                             "inv_freq": inv.tolist(), "cos": cos[0, :, :64].tolist(),
                             "sin": sin[0, :, :64].tolist()})
    with open(os.path.join(HERE, "rope_llama3.json"), "w") as f:
        json.dump(out, f)
    print("rope_llama3.json:", [c["name"] for c in out["cases"]])


if __name__ == "__main__":
    torch.set_num_threads(8)
    write_rope()
    write_cycles()
