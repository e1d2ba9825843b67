"""Qwen3 family (bwd_services/qwen3.py of the reference): Llama-3's layer plus
per-head q/k RMSNorm before RoPE (DSB_FAMILY_QWEN3 in libdsb)."""

from deltaserve_amd._lib import FAMILY_QWEN3
from deltaserve_amd.bwd_services.common.family import BASE_LAYER_WEIGHTS, Family
from deltaserve_amd.bwd_services.common.trainer import LoraSftTrainerService

QWEN3 = Family(
    name="qwen3", archs=("Qwen3ForCausalLM", "qwen3"), dsb_family=FAMILY_QWEN3,
    layer_weights={**BASE_LAYER_WEIGHTS, "q_norm": "self_attn.q_norm.weight",
                   "k_norm": "self_attn.k_norm.weight"},
    saved_qkv_pre_transform=True)


class Qwen3BackwardService(LoraSftTrainerService):
    """The Qwen3 backward child."""

    family = QWEN3
