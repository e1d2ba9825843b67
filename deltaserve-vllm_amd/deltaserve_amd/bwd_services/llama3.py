"""Llama-3 family (bwd_services/llama3.py:386-400 of the reference): the
decoder-layer recompute + backward runs in libdsb (DSB_FAMILY_LLAMA3)."""

from deltaserve_amd._lib import FAMILY_LLAMA3
from deltaserve_amd.bwd_services.common.family import Family
from deltaserve_amd.bwd_services.common.trainer import LoraSftTrainerService

LLAMA3 = Family(name="llama3", archs=("LlamaForCausalLM", "llama3", "llama"),
                dsb_family=FAMILY_LLAMA3)


class Llama3BackwardService(LoraSftTrainerService):
    """The Llama-3 backward child."""

    family = LLAMA3
