"""Parity of the production path at the BASELINE configurations.

Each case runs LoraSftTrainerService.process_backward (libdsb, one captured
hipGraph) at a BASELINE configuration's real widths — hidden size, heads,
intermediate size, vocabulary, LoRA rank, family (q/k-norm, tied head), RoPE
(llama3 scaling at C5) and the config's own seed-0 packing — and compares it
with the oracle's process_backward over two cycles (gradients of both and the
AdamW-updated masters). C1 runs its whole 28-layer model; C2–C5 run one
decoder layer plus the full LM head, which exercises every kernel
configuration the full model uses (256-wide tiles, the batched rank-16/32
LoRA passes, every vocab chunk of the streamed LM head, 8192-token sequences
at C5). The oracle runs on float32 device tensors (torch's fp32 products, TF32
off) as the fp32 reference of these shapes; the CPU pins of
tests/test_oracle_pins.py cover the same functions.

Bars: loss 1e-3 relative; LoRA grads 2e-2
max-relative with cosine >= 0.999; n_valid exact; updated masters equal to
the reference AdamW step of the cycle's own gradients, and every master
element further than 2e-2 from the fp32 run's explained by a reference
gradient within the measured error of zero (harness.unexplained_master_misses).
"""

import pytest
import torch

from harness import assert_north_star, config_meta, cycle_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _report(name, worst):
    print(f"[configs] {name}: loss rel {worst['loss']:.2e}  grad max-rel {worst['grad']:.2e}  "
          f"cos {worst['cos']:.6f}  master max-rel {worst['w']:.2e} (vs own-grad AdamW "
          f"{worst['w_own']:.1e}; {worst['w_off']} of {worst['w_numel']} elements off the "
          f"2e-2 bar, {worst['w_unexplained']} not sign-ambiguous)  worst at "
          f"{worst.get('where')}", flush=True)


def test_c1_full_model():
    """C1: Qwen3-0.6B architecture, r=8, 4 sequences in [32, 256], all 28 layers."""
    meta, lens = config_meta("c1", L=28)
    worst = cycle_parity(meta, lens, w_std=0.02, b_std=0.01, norm_jitter=0.0,
                         ref_device="cuda")
    _report("c1", worst)
    assert_north_star(worst, direct_masters=False)


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5", "c4s"])
def test_config_layer_and_head(name):
    """One decoder layer + the full LM head at the config's widths and packing.
    C2 keeps spare capacity (s_max > n, as the serving store does); C3-C5 run
    with s_max = n like bench.py. C4s is the reference's 256-token Qwen3-14B
    serving size: its products take the paths chosen for a single 256-row
    block (128x128 split-K tiles, 256-wide tiles at small M, the skinny LoRA
    pass split over K = 5120, the dK/dV q-head split with 5 q-heads per kv
    head, 128-wide LM-head tiles)."""
    meta, lens = config_meta(name, L=1, s_max=None)
    if name == "c2":
        meta["max_saved_finetuning_tokens"] = sum(lens) + 333
    worst = cycle_parity(meta, lens, w_std=0.02, b_std=0.01, norm_jitter=0.0,
                         ref_device="cuda")
    _report(name, worst)
    assert_north_star(worst, direct_masters=False)
    assert worst["graph"]


def test_llama32_1b_full_model():
    """The reference's end-to-end adapter model, Llama-3.2-1B (head_dim 64,
    32 q-heads over 8 kv heads, tied head, llama3 RoPE scaling, r = 8): all 16
    layers at 2048 tokens in 8 sequences."""
    meta, lens = config_meta("llama32-1b", L=16)
    worst = cycle_parity(meta, lens, w_std=0.02, b_std=0.01, norm_jitter=0.0,
                         ref_device="cuda")
    _report("llama32-1b", worst)
    assert_north_star(worst, direct_masters=False)
    assert worst["graph"]


def test_c4_spare_capacity_tail_split():
    """C4 widths with s_max = 9900 > n = 8192: the products' grids are sized
    for 39 row blocks, so qkv (1092 tiles) and o, gctx, gxn1, gxn2 and the
    head's dH (780 tiles each) leave partly filled last rounds that split K,
    while row blocks past the live rows exit early and the tail reduction
    skips them."""
    meta, lens = config_meta("c4", L=1, s_max=None)
    meta["max_saved_finetuning_tokens"] = 9900
    worst = cycle_parity(meta, lens, w_std=0.02, b_std=0.01, norm_jitter=0.0,
                         ref_device="cuda")
    _report("c4 spare capacity", worst)
    assert_north_star(worst, direct_masters=False)


def test_c3_saved_gate_up():
    """C3 widths with the mlp_gate_up save point bound: the cycle takes gate
    and up from the store instead of recomputing them (llama3.py:63-72)."""
    meta, lens = config_meta("c3", L=1)
    worst = cycle_parity(meta, lens, w_std=0.02, b_std=0.01, norm_jitter=0.0,
                         ref_device="cuda", save_gate_up=True)
    _report("c3 saved gate_up", worst)
    assert_north_star(worst, direct_masters=False)


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_all_save_points(name):
    """Every save point of the store bound at the config's widths: gate‖up,
    q/k/v (Llama-3 post-RoPE, Qwen3 pre-norm), the attention context and the
    post-attention residual, so the layer recompute is the input RMSNorm,
    the LoRA Z passes and the attention forward (trainer.py:532-552)."""
    meta, lens = config_meta(name, L=1)
    worst = cycle_parity(meta, lens, w_std=0.02, b_std=0.01, norm_jitter=0.0,
                         ref_device="cuda", save_gate_up=True,
                         saves=("attn_qkv", "attn_ctx", "resid_mid"))
    _report(f"{name} all save points", worst)
    assert_north_star(worst, direct_masters=False)
