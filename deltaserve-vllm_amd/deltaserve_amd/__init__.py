"""MI355X-native DeltaServe LoRA-SFT backward (the ``deltaserve`` backward child).

``bwd_services`` mirrors the reference's backward-service surface
(``deltaserve-plugin/deltaserve/bwd_services``); the arithmetic runs in
``libdsb.so`` (hand-written gfx950 HIP kernels behind the C-ABI of
``include/dsb.h``), loaded through ``_lib``.
"""

import os
import sys

_CHILD = False


def mark_backward_process() -> None:
    """Tag this process as the backward child (log colour), as the reference's
    ``deltaserve.mark_backward_process`` does (deltaserve/__init__.py:13-44)."""
    global _CHILD
    _CHILD = True


def dprint(*args, **kwargs) -> None:
    """Coloured print: green in the parent, purple in the backward child."""
    colour = "\033[95m" if _CHILD else "\033[92m"
    end = "\033[0m"
    if os.environ.get("NO_COLOR") or not sys.stdout.isatty():
        colour = end = ""
    print(colour + " ".join(str(a) for a in args) + end, **kwargs, flush=True)
