"""The record a model family hands to the trainer.

Mirrors ``deltaserve-plugin/deltaserve/bwd_services/common/family.py``: which
frozen base weights a layer needs and which projections carry LoRA. The layer
math itself is not Python here: ``dsb_family`` selects the kernel sequence
(Qwen3 adds the per-head q/k RMSNorm) inside libdsb.
"""

from __future__ import annotations

from dataclasses import dataclass, field

# The LoRA-trained projections, in libdsb's DSB_PROJ_* order. The reference
# trains q/k/v/o only (family.py:20); this build also trains gate/up/down when
# the adapter carries them.
LORA_PROJS = ("q", "k", "v", "o", "gate", "up", "down")

# Per-layer frozen base weights, keyed by role -> name under model.layers.{i}.
# (family.py:27-34; vLLM's fused qkv_proj / gate_up_proj are bound as-is).
BASE_LAYER_WEIGHTS: dict[str, str] = {
    "qkv": "self_attn.qkv_proj.weight",
    "o": "self_attn.o_proj.weight",
    "gate_up": "mlp.gate_up_proj.weight",
    "down": "mlp.down_proj.weight",
    "in_ln": "input_layernorm.weight",
    "post_ln": "post_attention_layernorm.weight",
}


@dataclass(frozen=True)
class Family:
    name: str
    archs: tuple[str, ...]
    dsb_family: int
    layer_weights: dict[str, str] = field(default_factory=lambda: dict(BASE_LAYER_WEIGHTS))
    supports_saved_qkv: bool = True
    saved_qkv_pre_transform: bool = False
