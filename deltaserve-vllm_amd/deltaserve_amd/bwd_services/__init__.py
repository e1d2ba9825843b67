"""Per-model backward (SFT) services, selected by HF architecture string."""
from deltaserve_amd.bwd_services.base import BackwardService, service_main
from deltaserve_amd.bwd_services.registry import get_family, get_service, supported_names

__all__ = ["BackwardService", "get_family", "get_service", "service_main", "supported_names"]
