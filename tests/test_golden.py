"""The committed golden fixtures (tests/golden/, written by make_golden.py from
transformers) against the oracle on the CPU and against libdsb on the GPU."""

from __future__ import annotations

import json
import os

import pytest
import torch

from harness import O, bf16_round_acts, build_service, cosine, gpu_activations, max_rel

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load_cycle(family):
    from safetensors import safe_open

    import golden.make_golden as G

    path = os.path.join(GOLDEN, f"cycle_{family}.safetensors")
    with safe_open(path, "pt") as f:
        md = f.metadata()
        t = {k: f.get_tensor(k) for k in f.keys()}
    spec = json.loads(md["spec"])
    model = G.build_model(spec)
    assert abs(G.weight_checksum(model) - float(md["weight_checksum"])) < 1e-6 * abs(
        float(md["weight_checksum"])), "make_model no longer regenerates the fixture's weights"
    grads = {}
    for k, v in t.items():
        if k.startswith("grad."):
            i, key = k[5:].split(".")
            grads.setdefault(int(i), {})[key] = v
    return (model, t["ids"], t["seq_lens"].tolist(), float(md["loss"]), int(md["n_valid"]),
            grads)


def _clipped(grads_layer):
    keys = sorted(grads_layer)
    norm = torch.sqrt(sum((grads_layer[k].double() ** 2).sum() for k in keys))
    coef = min(1.0, 1.0 / (float(norm) + 1e-6))
    return {k: grads_layer[k] * coef for k in keys}


def test_rope_fixture_vs_oracle():
    d = json.load(open(os.path.join(GOLDEN, "rope_llama3.json")))
    for c in d["cases"]:
        rs = c["rope_scaling"]
        inv = O.rope_inv_freq(d["head_dim"], c["theta"], rs)
        ref = torch.tensor(c["inv_freq"])
        assert ((inv - ref).abs() / ref).max() < 1e-6, c["name"]
        cos, sin = O.rope_cos_sin(d["positions"], d["head_dim"], c["theta"], rs)
        assert (cos - torch.tensor(c["cos"])).abs().max() < 2e-6, c["name"]
        assert (sin - torch.tensor(c["sin"])).abs().max() < 2e-6, c["name"]


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_cycle_fixture_vs_oracle(family):
    model, ids, seq_lens, loss, nv, grads = _load_cycle(family)
    acts = O.forward_capture(model, ids, seq_lens)
    got_loss, got_nv, got = O.process_backward(model, acts, seq_lens, sum(seq_lens), lr=1e-4,
                                               step=1, clip=False, update=False)
    assert got_nv == nv
    assert abs(got_loss - loss) < 1e-5 * loss
    for i, gl in grads.items():
        for k, g in gl.items():
            assert max_rel(got[i][k], g) < 2e-4, (i, k)


@pytest.mark.gpu
def test_rope_fixture_vs_hip():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from deltaserve_amd import ops

    d = json.load(open(os.path.join(GOLDEN, "rope_llama3.json")))
    pos = torch.tensor(d["positions"], dtype=torch.int32, device="cuda")
    for c in d["cases"]:
        inv = ops.rope_inv_freq(d["head_dim"], c["theta"], c["rope_scaling"])
        assert ((inv - torch.tensor(c["inv_freq"])).abs() / torch.tensor(c["inv_freq"])).max() < 2e-6
        cos, sin = ops.rope_cos_sin(pos, inv.cuda())
        # sin/cos of angles up to ~1.6e4 rad in fp32: |Δ| bounded by the angle's rounding
        assert (cos.cpu() - torch.tensor(c["cos"])).abs().max() < 2e-3, c["name"]
        assert (sin.cpu() - torch.tensor(c["sin"])).abs().max() < 2e-3, c["name"]


@pytest.mark.gpu
@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_cycle_fixture_vs_hip(family):
    """libdsb's cycle (bf16 operands, fp32 accumulation) against transformers'
    fp32 autograd: loss 1e-3 relative, clipped LoRA grads 2e-2 max-rel and
    cosine >= 0.999, n_valid exact."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    model, ids, seq_lens, loss, nv, grads = _load_cycle(family)
    n = sum(seq_lens)
    acts = bf16_round_acts(O.forward_capture(model, ids, seq_lens))
    svc = build_service(model, family)
    try:
        got_loss, got_nv = svc.process_backward(gpu_activations(acts, 512), seq_lens, n, epoch=0)
        assert got_nv == nv
        assert abs(got_loss - loss) / loss < 1e-3, (got_loss, loss)
        for i, gl in grads.items():
            for k, g in _clipped(gl).items():
                got = svc.lora[i][k[:-1]][k[-1]].grad
                assert max_rel(got, g) < 2e-2 and cosine(got, g) > 0.999, (i, k, max_rel(got, g))
    finally:
        svc.close()
