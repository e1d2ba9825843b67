"""The C-ABI boundary without a GPU: libdsb.so loads, exports every function
include/dsb.h declares, the ctypes mirror in deltaserve_amd._lib matches the
header's struct layouts (checked against gcc's own offsetof/sizeof), and the
host-only entry points (integer packing, RoPE frequencies) agree with the
oracle bit for bit. No device compute is called here."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from harness import O, ROOT

HEADER = os.path.join(ROOT, "include", "dsb.h")


def _lib():
    from deltaserve_amd import _lib as L

    if not os.path.exists(L.LIB_PATH):
        subprocess.run(["make", "-C", os.path.join(ROOT, "deltaserve-vllm_amd", "csrc"), "-j8"],
                       check=True, capture_output=True, timeout=1200)
    return L, L.load()


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|void|const char\s*\*)\s*(dsb_\w+)\s*\(", text,
                                 flags=re.M)))


def test_header_declares_the_entry_points():
    names = _declared()
    for core in ("dsb_create", "dsb_destroy", "dsb_last_error", "dsb_bind_weights",
                 "dsb_bind_head", "dsb_bind_lora", "dsb_bind_activations", "dsb_step"):
        assert core in names


def test_library_exports_every_declared_symbol():
    L, lib = _lib()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    # The ctypes signature table covers exactly the declared functions.
    assert sorted(L.EXPORTED) == _declared()


def test_struct_layout_matches_header(tmp_path):
    L, _ = _lib()
    structs = {"dsb_desc": L.DsbDesc, "dsb_layer_weights": L.DsbLayerWeights,
               "dsb_lora_tensors": L.DsbLoraTensors, "dsb_activations": L.DsbActivations,
               "dsb_cycle_info": L.DsbCycleInfo, "dsb_dual_pass": L.DsbDualPass}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "dsb.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} . %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER),
                    str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True,
                               text=True).stdout.splitlines():
        s, f, v = line.split()
        got[(s, f)] = int(v)
    for cname, cls in structs.items():
        assert got[(cname, ".")] == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert got[(cname, f)] == getattr(cls, f).offset, (cname, f)


def test_create_rejects_bad_descriptors():
    """Argument checks of dsb_create run before any device call."""
    L, lib = _lib()

    def desc(**kw):
        d = L.DsbDesc(abi_version=L.ABI_VERSION, family=0, n_layers=1, hidden=256, n_heads=2,
                      n_kv_heads=1, head_dim=128, intermediate=512, vocab=1000, lora_rank=16,
                      lora_scaling=2.0, rms_eps=1e-5, rope_theta=5e5, s_max=64, max_seqs=64)
        for k, v in kw.items():
            setattr(d, k, v)
        return d

    h = ctypes.c_void_p()
    for bad in (dict(abi_version=1), dict(head_dim=96), dict(head_dim=32), dict(lora_rank=0),
                dict(lora_rank=72),
                dict(vocab_chunk=300), dict(vocab_chunk=-256), dict(gemm_tile=96),
                dict(n_heads=3), dict(s_max=0)):
        assert lib.dsb_create(ctypes.byref(desc(**bad)), ctypes.byref(h)) != 0, bad
        assert L.last_error()


def test_abi_version_constant():
    L, _ = _lib()
    m = re.search(r"#define DSB_ABI_VERSION (\d+)", open(HEADER).read())
    assert m and int(m.group(1)) == L.ABI_VERSION


@pytest.mark.parametrize("seq_lens", [[1], [2], [5, 0, 3, 1, 7], [64, 1, 2, 0, 33],
                                      [512] * 16, list(range(0, 40))])
def test_host_pack_bit_exact_vs_oracle(seq_lens):
    from deltaserve_amd import ops

    pos, pred, nv = ops.pack(seq_lens)
    _, opos, rows, _, onv = O.pack(seq_lens)
    assert pos == opos and nv == onv
    n = sum(seq_lens)
    exp = [0] * n
    for r in rows:
        exp[r] = 1
    assert pred == exp


def test_host_pack_rejects_bad_input():
    L, lib = _lib()
    arr = L.i32_array([3, -1])
    out = (ctypes.c_int32 * 4)()
    assert lib.dsb_pack(arr, 2, 2, out, out) < 0
    assert lib.dsb_pack(L.i32_array([3, 2]), 2, 4, out, out) < 0  # lengths do not sum to n


@pytest.mark.parametrize("theta,rs", [
    (5e5, None), (1e6, None), (1e4, {"rope_type": "linear", "factor": 4.0}),
    (5e5, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
           "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})])
def test_host_rope_inv_freq_vs_oracle(theta, rs):
    from deltaserve_amd import ops

    got = ops.rope_inv_freq(128, theta, rs)
    ref = O.rope_inv_freq(128, theta, rs)
    assert ((got - ref).abs() / ref).max().item() < 2e-6


def test_unsupported_rope_type_is_an_error():
    from deltaserve_amd import ops

    with pytest.raises(NotImplementedError):
        ops.rope_inv_freq(128, 1e4, {"rope_type": "yarn", "factor": 4.0})


def test_product_ops_refuse_cpu_tensors():
    """No CPU fallback: the torch front end rejects host tensors outright."""
    from deltaserve_amd import ops

    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.rmsnorm(x, torch.ones(8, dtype=torch.bfloat16), 1e-5)
    with pytest.raises(ValueError):
        ops.gemm_nt(x, x)


@pytest.mark.parametrize("max_saved", [1, 7, 16, 257])
def test_host_capture_index_bit_exact_vs_oracle(max_saved):
    """dsb_capture_index (arm_op_step's index build) against the oracle, over
    every offset / count at the buffer's edges, with interleaved positions."""
    from deltaserve_amd import capture

    g = torch.Generator().manual_seed(max_saved)
    offsets = sorted({0, 1, max_saved // 2, max_saved - 1, max_saved, max_saved + 3})
    counts = sorted({0, 1, max_saved // 3, max_saved - 1, max_saved, max_saved + 5})
    for off in offsets:
        for nft in counts:
            pos = torch.randperm(4 * max_saved + 8, generator=g)[:nft]
            src, dst, n = capture.capture_index(pos, nft, off, max_saved)
            osrc, odst, on = O.capture_index(pos.tolist(), nft, off, max_saved)
            assert n == on and torch.equal(src, osrc) and torch.equal(dst, odst), (off, nft)


def test_capture_entry_points_reject_bad_input():
    from deltaserve_amd import capture

    L, lib = _lib()
    with pytest.raises(ValueError):
        capture.capture_index([1, 2], 3, 0, 8)  # fewer positions than rows
    src = (ctypes.c_int64 * 4)()
    assert lib.dsb_capture_index(None, 0, 0, 0, src, src) < 0  # empty buffer
    assert lib.dsb_capture_index(None, 0, -1, 4, src, src) < 0  # negative offset
    assert lib.dsb_capture_index(None, 2, 0, 4, src, src) < 0  # rows without positions
    # argument checks run before any device work
    assert lib.dsb_save_rows(None, 8, None, 0, 4, 0, src, src, 4, 8, src, 8, 5, None) < 0
    assert lib.dsb_save_rows(src, 8, None, 0, 4, 7, src, src, 4, 8, src, 8, 5, None) < 0
    assert lib.dsb_save_rows(src, 4, None, 0, 4, 0, src, src, 4, 8, src, 8, 5, None) < 0
    assert lib.dsb_save_ids(None, 4, src, src, 4, src, 4, None) < 0
    with pytest.raises(ValueError):  # host tensors: no fallback
        x = torch.zeros(4, 8, dtype=torch.bfloat16)
        i = torch.zeros(4, dtype=torch.int64)
        capture.save_rows(x, None, torch.zeros(5, 8, dtype=torch.bfloat16), i, i)


def test_noalloc_dual_rejects_oversized_requests():
    """The argument and size checks of dsb_op_lora_dual_noalloc run before any
    device call: a request whose partial sums exceed the 64 MiB scratch array
    fails with a message."""
    L, lib = _lib()
    fake = 1 << 20  # aligned stand-in addresses; never dereferenced
    p = L.DsbDualPass(fake, 20480, fake, 32, fake, 20480, 20480, 1.0, fake, 32, fake, 1)
    rc = lib.dsb_op_lora_dual_noalloc(ctypes.byref(p), 1, 100000, 100000, 32, None)
    assert rc != 0 and "64 MiB" in L.last_error()
    bad = L.DsbDualPass(fake, 20480, fake, 32, fake, 20480, 20480, 1.0, fake, 32, fake, 1)
    assert lib.dsb_op_lora_dual_noalloc(ctypes.byref(bad), 1, 10, 10, 24, None) != 0  # rank 24
