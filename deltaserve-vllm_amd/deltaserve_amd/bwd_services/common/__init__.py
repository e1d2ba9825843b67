"""Family-agnostic pieces of the backward services: the ``Family`` record and
``LoraSftTrainerService`` (which drives libdsb). Mirrors the role of the
reference's ``bwd_services/common`` package; the per-op math lives in the HIP
kernels instead of Python modules."""
