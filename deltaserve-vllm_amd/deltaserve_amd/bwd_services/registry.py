"""Model architecture → backward service (bwd_services/registry.py:15-49 of
the reference). A drop-in deployment points the reference's ``_SERVICES``
entries at these ``module:Class`` strings."""

from __future__ import annotations

import importlib

_SERVICES: dict[str, str] = {
    "LlamaForCausalLM": "deltaserve_amd.bwd_services.llama3:Llama3BackwardService",
    "llama3": "deltaserve_amd.bwd_services.llama3:Llama3BackwardService",
    "llama": "deltaserve_amd.bwd_services.llama3:Llama3BackwardService",
    "Qwen3ForCausalLM": "deltaserve_amd.bwd_services.qwen3:Qwen3BackwardService",
    "qwen3": "deltaserve_amd.bwd_services.qwen3:Qwen3BackwardService",
    "ipc": "deltaserve_amd.bwd_services.base:BackwardService",
}


def supported_names() -> list[str]:
    return sorted(_SERVICES)


def get_service(name: str):
    """The BackwardService subclass for an architecture string; raises
    ``NotImplementedError`` listing what is supported otherwise."""
    target = _SERVICES.get(name)
    if target is None:
        raise NotImplementedError(
            f"[deltaserve] no backward service for {name!r}; supported: "
            f"{', '.join(supported_names())}")
    module_name, _, class_name = target.partition(":")
    return getattr(importlib.import_module(module_name), class_name)


def get_family(name: str):
    try:
        return getattr(get_service(name), "family", None)
    except NotImplementedError:
        return None
