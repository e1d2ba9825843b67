"""ctypes binding of ``libdsb.so`` (the C-ABI declared in ``include/dsb.h``).

The library is built in-tree by ``make -C deltaserve-vllm_amd/csrc`` (or
``__graft_entry__.build()``) into ``deltaserve_amd/_lib/libdsb.so``. There is
no fallback: every entry point raises when the library is missing, so a
backward never silently runs anything but the HIP path.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32,
                    c_int64, c_uint32, c_void_p)

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
# DSB_LIB overrides the library file (e.g. a build kept elsewhere for an A/B
# timing); the in-tree build is the default.
LIB_PATH = os.environ.get("DSB_LIB") or os.path.join(LIB_DIR, "libdsb.so")

ABI_VERSION = 5
FAMILY_LLAMA3, FAMILY_QWEN3 = 0, 1
ROPE_DEFAULT, ROPE_LINEAR, ROPE_LLAMA3 = 0, 1, 2
PROJS = ("q", "k", "v", "o", "gate", "up", "down")
PROJ_INDEX = {p: i for i, p in enumerate(PROJS)}
FLAG_GRAPH, FLAG_NO_CLIP, FLAG_KTIMING, FLAG_SERIAL_LAYERS = 1, 2, 4, 8
DT_BF16, DT_F16, DT_F32 = 0, 1, 2


class DsbDesc(Structure):
    _fields_ = [
        ("abi_version", c_int32), ("family", c_int32),
        ("n_layers", c_int32), ("hidden", c_int32), ("n_heads", c_int32),
        ("n_kv_heads", c_int32), ("head_dim", c_int32), ("intermediate", c_int32),
        ("vocab", c_int32), ("lora_rank", c_int32),
        ("lora_scaling", c_float), ("rms_eps", c_float), ("rope_theta", c_float),
        ("rope_type", c_int32), ("rope_factor", c_float),
        ("rope_low_freq_factor", c_float), ("rope_high_freq_factor", c_float),
        ("rope_orig_max_pos", c_float),
        ("s_max", c_int32), ("max_seqs", c_int32),
        ("beta1", c_float), ("beta2", c_float), ("adam_eps", c_float),
        ("weight_decay", c_float), ("max_grad_norm", c_float),
        ("flags", c_uint32),
        ("vocab_chunk", c_int32), ("gemm_tile", c_int32),
    ]


class DsbLayerWeights(Structure):
    _fields_ = [(k, c_void_p) for k in
                ("qkv", "o", "gate_up", "down", "in_ln", "post_ln", "q_norm", "k_norm")]


class DsbLoraTensors(Structure):
    _fields_ = [("A", c_void_p), ("B", c_void_p), ("gA", c_void_p), ("gB", c_void_p)]


class DsbActivations(Structure):
    _fields_ = [("layer_in", POINTER(c_void_p)), ("final_in", c_void_p),
                ("input_ids", c_void_p), ("ld", c_int64),
                ("mlp_gate_up", POINTER(c_void_p)), ("ld_gate_up", c_int64),
                ("attn_q", POINTER(c_void_p)), ("attn_k", POINTER(c_void_p)),
                ("attn_v", POINTER(c_void_p)), ("ld_q", c_int64), ("ld_k", c_int64),
                ("ld_v", c_int64), ("attn_ctx", POINTER(c_void_p)), ("ld_ctx", c_int64),
                ("resid_mid", POINTER(c_void_p)), ("ld_resid_mid", c_int64)]


class DsbDualPass(Structure):
    _fields_ = [("G", c_void_p), ("ldg", c_int64), ("Z", c_void_p), ("ldz", c_int64),
                ("BT", c_void_p), ("ldbt", c_int64), ("C", c_int32), ("scale", c_float),
                ("gZ", c_void_p), ("ldgz", c_int64), ("gB", c_void_p),
                ("transpose_out", c_int32)]


class DsbCycleInfo(Structure):
    _fields_ = [("gpu_ms", c_float), ("graph", c_int32), ("n_valid", c_int32)]


# name -> (restype, argtypes)
_SIGS = {
    "dsb_create": (c_int, [POINTER(DsbDesc), POINTER(c_void_p)]),
    "dsb_destroy": (None, [c_void_p]),
    "dsb_last_error": (c_char_p, [c_void_p]),
    "dsb_bind_weights": (c_int, [c_void_p, c_int, POINTER(DsbLayerWeights)]),
    "dsb_bind_head": (c_int, [c_void_p, c_void_p, c_void_p]),
    "dsb_bind_lora": (c_int, [c_void_p, c_int, c_int, POINTER(DsbLoraTensors)]),
    "dsb_bind_activations": (c_int, [c_void_p, POINTER(DsbActivations)]),
    "dsb_step": (c_int, [c_void_p, POINTER(c_int32), c_int, c_int, c_float, c_int64,
                         c_void_p, POINTER(c_float), POINTER(c_int),
                         POINTER(DsbCycleInfo)]),
    "dsb_num_segments": (c_int, [c_void_p]),
    "dsb_step_begin": (c_int, [c_void_p, POINTER(c_int32), c_int, c_int, c_float, c_int64,
                               c_void_p]),
    "dsb_step_segment": (c_int, [c_void_p, c_int, c_int]),
    "dsb_step_end": (c_int, [c_void_p, c_void_p, POINTER(c_float), POINTER(c_int),
                             POINTER(DsbCycleInfo)]),
    "dsb_bind_served": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int64, c_void_p, c_int64]),
    "dsb_publish": (c_int, [c_void_p, c_void_p]),
    "dsb_capture_index": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "dsb_save_rows": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int, c_void_p,
                              c_void_p, c_int, c_int, c_void_p, c_int64, c_int64, c_void_p]),
    "dsb_save_ids": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int, c_void_p, c_int64,
                             c_void_p]),
    "dsb_reset_optimizer": (c_int, [c_void_p, c_float]),
    "dsb_kernel_stats": (c_int, [c_void_p, c_int, c_char_p, c_int, POINTER(c_int64),
                                 POINTER(c_double), POINTER(c_double), POINTER(c_double)]),
    "dsb_kernel_stats_reset": (c_int, [c_void_p]),
    "dsb_set_kernel_timing": (c_int, [c_void_p, c_int]),
    "dsb_pack": (c_int, [POINTER(c_int32), c_int, c_int, POINTER(c_int32),
                         POINTER(c_int32)]),
    "dsb_rope_inv_freq": (c_int, [c_int, c_float, c_int, c_float, c_float, c_float,
                                  c_float, POINTER(c_float)]),
    "dsb_op_gemm": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                            c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p,
                            c_int64, c_int, c_int, c_void_p, c_int64, c_int, c_int,
                            c_void_p]),
    "dsb_op_gemm_glu": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_int64,
                                c_void_p, c_int64, c_void_p]),
    "dsb_op_rmsnorm": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int,
                               c_int, c_float, c_void_p]),
    "dsb_op_rmsnorm_bwd": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_int64, c_void_p,
                                   c_void_p, c_int64, c_void_p, c_int64, c_int, c_int,
                                   c_float, c_void_p]),
    "dsb_op_rope_table": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p,
                                  c_void_p]),
    "dsb_op_rope": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int,
                            c_int, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p]),
    "dsb_op_rope_bwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float,
                                c_void_p]),
    "dsb_op_attn_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                c_void_p, c_int64, c_void_p, c_void_p, POINTER(c_int32),
                                c_int, c_int, c_int, c_int, c_void_p]),
    "dsb_op_attn_bwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
                                c_void_p, c_int64, c_void_p, c_int64, POINTER(c_int32),
                                c_int, c_int, c_int, c_int, c_void_p]),
    "dsb_op_head": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, POINTER(c_int32), c_int,
                            c_int, c_int, c_int, c_int, c_void_p, POINTER(c_float),
                            POINTER(c_int), c_void_p]),
    "dsb_op_lora_tn": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int, c_int, c_int,
                               c_float, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "dsb_op_lora_skinny": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int, c_int, c_int,
                                   c_void_p, c_int64, c_void_p]),
    "dsb_op_lora_dual": (c_int, [POINTER(DsbDualPass), c_int, c_int, c_int, c_int, c_void_p]),
    "dsb_op_lora_dual_noalloc": (c_int, [POINTER(DsbDualPass), c_int, c_int, c_int, c_int,
                                         c_void_p]),
    "dsb_op_clip_adamw": (c_int, [POINTER(c_void_p), POINTER(c_void_p), POINTER(c_void_p),
                                  POINTER(c_void_p), POINTER(c_int32), POINTER(c_int32),
                                  c_int, c_int, c_float, c_float, c_float, c_float, c_float,
                                  c_int64, c_float, c_int, c_void_p]),
}

EXPORTED = tuple(_SIGS)

_lib = None


class DsbError(RuntimeError):
    """A libdsb call returned non-zero (message from dsb_last_error)."""


def load(path: str | None = None):
    """Load libdsb.so once; raises ``DsbError`` if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise DsbError(
            f"libdsb.so not found at {p}; build it with "
            "`make -C deltaserve-vllm_amd/csrc` or __graft_entry__.build()")
    lib = ctypes.CDLL(p)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error(handle=None) -> str:
    msg = load().dsb_last_error(handle)
    return msg.decode(errors="replace") if msg else "unknown error"


def check(rc: int, handle=None, what: str = "libdsb") -> None:
    if rc != 0:
        raise DsbError(f"{what}: {last_error(handle)}")


def i32_array(values):
    vals = [int(v) for v in values]
    return (c_int32 * max(len(vals), 1))(*vals)


def kernel_stats(handle) -> list[dict]:
    """Per-kernel-class timing table of a handle created with FLAG_KTIMING."""
    lib = load()
    n = lib.dsb_kernel_stats(handle, -1, None, 0, None, None, None, None)
    if n < 0:
        raise DsbError(last_error(handle))
    out = []
    for i in range(n):
        name = ctypes.create_string_buffer(128)
        calls, ms, fl, by = c_int64(), c_double(), c_double(), c_double()
        if lib.dsb_kernel_stats(handle, i, name, 128, ctypes.byref(calls), ctypes.byref(ms),
                                ctypes.byref(fl), ctypes.byref(by)) < 0:
            raise DsbError(last_error(handle))
        out.append({"name": name.value.decode(), "calls": calls.value, "ms": ms.value,
                    "flops": fl.value, "bytes": by.value})
    return out
