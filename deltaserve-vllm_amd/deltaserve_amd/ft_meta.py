"""The backward ``meta`` contract (ft_meta.py:24-213 of the reference): RoPE
base and scaling read from an HF config, α/r from the adapter config, and the
dict the worker ships to the backward child."""

from __future__ import annotations

import json
import os
from typing import Any

SUPPORTED_ROPE_TYPES = ("default", "linear", "llama3")
_DEFAULT_ROPE_THETA = 10000.0


def rope_theta_of(hf_config: Any) -> float:
    rp = getattr(hf_config, "rope_parameters", None)
    if isinstance(rp, dict) and rp.get("rope_theta") is not None:
        return float(rp["rope_theta"])
    theta = getattr(hf_config, "rope_theta", None)
    return float(theta) if theta is not None else _DEFAULT_ROPE_THETA


def rope_scaling_of(hf_config: Any) -> dict | None:
    """Normalised RoPE scaling, None for plain RoPE; ValueError for variants
    the backward cannot reproduce (partial rotary, mrope, yarn, …)."""
    rp = getattr(hf_config, "rope_parameters", None)
    if not isinstance(rp, dict) or not rp:
        rp = getattr(hf_config, "rope_scaling", None)
    rp = dict(rp) if isinstance(rp, dict) else {}
    rtype = rp.get("rope_type") or rp.get("type") or "default"
    if rtype == "su":
        rtype = "longrope"
    partial = rp.get("partial_rotary_factor", getattr(hf_config, "partial_rotary_factor", 1.0))
    if partial is not None and float(partial) != 1.0:
        raise ValueError(f"[deltaserve] partial_rotary_factor={partial} is not supported")
    if "mrope_section" in rp:
        raise ValueError("[deltaserve] multimodal RoPE (mrope_section) is not supported")
    if rtype not in SUPPORTED_ROPE_TYPES:
        raise ValueError(f"[deltaserve] RoPE type {rtype!r} is not supported by the "
                         f"finetuning backward (supported: {', '.join(SUPPORTED_ROPE_TYPES)})")
    if rtype == "default":
        return None
    need = {"linear": ("factor",),
            "llama3": ("factor", "low_freq_factor", "high_freq_factor",
                       "original_max_position_embeddings")}[rtype]
    missing = [k for k in need if rp.get(k) is None]
    if missing:
        raise ValueError(f"[deltaserve] RoPE type {rtype!r} config lacks {missing}")
    return {"rope_type": rtype, **{k: float(rp[k]) for k in need}}


def read_lora_scaling(adapter_path: str | None) -> float:
    if not adapter_path:
        return 1.0
    cfg_path = os.path.join(adapter_path, "adapter_config.json")
    if not os.path.exists(cfg_path):
        return 1.0
    with open(cfg_path) as f:
        acfg = json.load(f)
    r = float(acfg.get("r", 1) or 1)
    return float(acfg.get("lora_alpha", r)) / r


def build_backward_meta(hf_config: Any, ft_cfg: Any, *, lm_head_key: str | None,
                        embed_weight_key: str | None, has_final_norm: bool,
                        lora_scaling: float, tp_size: int = 1, tp_rank: int = 0) -> dict:
    num_heads = int(hf_config.num_attention_heads)
    head_dim = int(getattr(hf_config, "head_dim", None) or hf_config.hidden_size // num_heads)
    g = lambda name, default=None: getattr(ft_cfg, name, default)  # noqa: E731
    return {
        "lm_head_key": lm_head_key,
        "vocab_size": int(hf_config.vocab_size),
        "logit_scale": float(getattr(hf_config, "logit_scale", 1.0) or 1.0),
        "rms_norm_eps": float(getattr(hf_config, "rms_norm_eps", 1e-5) or 1e-5),
        "norm_weight_key": "model.norm.weight" if has_final_norm else None,
        "embed_weight_key": embed_weight_key,
        "hidden_size": int(hf_config.hidden_size),
        "num_hidden_layers": int(hf_config.num_hidden_layers),
        "num_attention_heads": num_heads,
        "num_key_value_heads": int(getattr(hf_config, "num_key_value_heads", num_heads)),
        "head_dim": head_dim,
        "intermediate_size": int(hf_config.intermediate_size),
        "rope_theta": rope_theta_of(hf_config),
        "rope_scaling": rope_scaling_of(hf_config),
        "lora_scaling": float(lora_scaling),
        "learning_rate": float(g("learning_rate", 1e-4)),
        "finetuning_lora_path": g("finetuning_lora_path"),
        "metrics": bool(g("metrics_dir")),
        "adapter_save_path": g("adapter_save_path"),
        "adapter_save_every_backwards": int(g("adapter_save_every_backwards", 0) or 0),
        "adapter_save_every_epoch": bool(g("adapter_save_every_epoch", False)),
        "adapter_save_keep_last": int(g("adapter_save_keep_last", 0) or 0),
        "weight_decay": float(g("weight_decay", 0.0)),
        "gamma": float(g("gamma", 1.0)),
        "backward_fp32": bool(g("backward_fp32", False)),
        "backward_hip_graph": bool(g("backward_cuda_graph", True)),
        "max_saved_finetuning_tokens": int(g("max_saved_finetuning_tokens", 256)),
        "backward_max_seqs": int(g("backward_max_seqs", 0) or 0),
        "save_attn_qkv": bool(g("save_attn_qkv", False)),
        "save_attn_ctx": bool(g("save_attn_ctx", False)),
        "save_resid_mid": bool(g("save_resid_mid", False)),
        "tp_size": int(tp_size),
        "tp_rank": int(tp_rank),
    }
