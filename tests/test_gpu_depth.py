"""Parity at full depth: the whole C3 (Llama-3-8B architecture, 32 layers,
8192 tokens, r=16) and C4 (Qwen3-14B architecture, 40 layers, 8192 tokens,
r=32) cycles against the fp32 oracle on float32 device tensors.

The layer-plus-head slices of test_gpu_configs.py show each kernel at the
real widths; these show that the errors do not grow past the bars when the
residual-stream gradient runs through every layer (it is carried in fp32
across layers; the GEMM operands are its bf16 copies). Two cycles each, with
the AdamW-updated masters checked as in the slices (sign-ambiguous elements
only may miss the direct 2e-2 bar). The oracle's fp32 model, activations and
the bf16 copies fit the 288 GB of one MI355X at both sizes.
"""

import pytest
import torch

from harness import assert_north_star, config_meta, cycle_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_full_depth_cycle(name):
    from deltaserve_amd.configs import CONFIGS

    meta, lens = config_meta(name, L=CONFIGS[name]["L"])
    print(f"[depth] {name}: {meta['num_hidden_layers']} layers, {sum(lens)} tokens", flush=True)
    worst = cycle_parity(meta, lens, w_std=0.02, b_std=0.01, norm_jitter=0.0,
                         ref_device="cuda")
    print(f"[depth] {name}: loss rel {worst['loss']:.2e}  grad max-rel {worst['grad']:.2e}  "
          f"cos {worst['cos']:.6f}  master max-rel {worst['w']:.2e} "
          f"({worst['w_off']} of {worst['w_numel']} elements off the 2e-2 bar, "
          f"{worst['w_unexplained']} not sign-ambiguous; vs own-grad AdamW "
          f"{worst['w_own']:.1e})  worst at {worst.get('where')}", flush=True)
    assert_north_star(worst, direct_masters=False)
    assert worst["graph"]
