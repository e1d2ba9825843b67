"""Content fingerprints the parent and the backward child compare.

The reference's parent (``deltaserve-plugin/deltaserve/backward_process.py:44-141``)
hashes its own view of the shared weights and activation buffers and asks the
child for the same report (``share_weights`` with ``print_hash``,
``hash_activations``, ``checksum``). Matching values prove that the child maps
the very bytes the serving side wrote (zero-copy IPC), which is this design's
stand-in for a race detector on the handoff. The values are therefore a wire
contract: the digest (SHA-1 of the fp32 bytes, first 16 hex digits), which
tensors are picked and the report labels are the parent's.
"""

from __future__ import annotations

import hashlib
import re

import torch

from deltaserve_amd import dprint

_LAYER_NO = re.compile(r"layers?\.(\d+)\.")


def tensor_digest(t: torch.Tensor) -> str:
    """16-hex-digit SHA-1 of the tensor's values as fp32, whatever its dtype
    (backward_process.py:44-47)."""
    data = t.detach().to("cpu", torch.float32).contiguous().numpy()
    return hashlib.sha1(data.tobytes()).hexdigest()[:16]


def _layer_extremes(state: dict, need: tuple, skip: tuple = ()):
    """(layer, key, tensor) of the lowest and of the highest numbered layer
    among keys holding every ``need`` substring and no ``skip`` one."""
    picked = []
    for key, t in state.items():
        if any(s not in key for s in need) or any(s in key for s in skip):
            continue
        m = _LAYER_NO.search(key)
        if m is not None:
            picked.append((int(m.group(1)), key, t))
    if not picked:
        return None
    picked.sort(key=lambda e: e[0])
    return picked[0], picked[-1]


def weight_hash_report(base: dict, ft: dict) -> dict:
    """First/last-layer FFN ``fc1`` base weight and first/last-layer q_proj
    LoRA-A (backward_process.py:68-90): label -> (layer, key, digest)."""
    out: dict = {}
    picks = (("base_ffn_fc1", base, ("fc1", "weight"), ("lora", "bias")),
             ("ft_q_loraA", ft, ("q_proj", "lora_A"), ()))
    for label, state, need, skip in picks:
        ends = _layer_extremes(state or {}, need, skip)
        if ends is None:
            continue
        for tag, (layer, key, t) in zip(("first", "last"), ends):
            out[f"{label}_{tag}"] = (layer, key, tensor_digest(t))
    return out


def activation_hash_report(buffers: dict, n: int) -> dict:
    """Digests of the first ``n`` rows of the captured buffers
    (backward_process.py:93-111): first and last layer of each per-layer
    list, and each single buffer."""
    out: dict = {}
    if n <= 0 or not buffers:
        return out
    for name in ("layer_in", "mlp_gate_up"):
        per_layer = buffers.get(name) or []
        if per_layer:
            out[f"{name}_first"] = tensor_digest(per_layer[0][:n])
            out[f"{name}_last"] = tensor_digest(per_layer[-1][:n])
    for name in ("final_in", "final_hidden", "concat_input_ids"):
        t = buffers.get(name)
        if t is not None:
            out[name] = tensor_digest(t[:n])
    return out


def print_hash_report(report: dict, who: str) -> None:
    for label, value in report.items():
        if isinstance(value, tuple):
            layer, key, digest = value
            dprint(f"[hash:{who}] {label:>20s}  L{layer:<2d} {digest}  ({key})")
        else:
            dprint(f"[hash:{who}] {label:>20s}  {value}")


def checksum(state: dict) -> float:
    """fp64 sum of every value of every tensor (backward_process.py:122-127)."""
    return float(sum(float(t.detach().double().sum()) for t in state.values()))


def weights_summary(base: dict, ft: dict) -> dict:
    """Counts and the adapter checksum sent with a hashed ``weights_received``
    (backward_process.py:130-141)."""
    return {"base_num": len(base),
            "base_numel": int(sum(t.numel() for t in base.values())),
            "ft_num": len(ft),
            "ft_numel": int(sum(t.numel() for t in ft.values())),
            "ft_checksum": checksum(ft)}
