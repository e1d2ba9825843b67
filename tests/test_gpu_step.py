"""Whole-cycle parity: LoraSftTrainerService.process_backward on libdsb (one
captured hipGraph) against the oracle's process_backward on identical
seeded inputs.

Bar: loss within 1e-3 relative; every LoRA gradient
and updated master within 2e-2 max-relative error with cosine >= 0.999
against the fp32 oracle; n_valid exact.
"""

import pytest
import torch

from harness import (O, assert_north_star, bf16_round_acts, build_service, cosine, cycle_parity,
                     gpu_activations, max_rel, tiny_meta)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _run(meta, seq_lens, projs=O.PROJS, steps=2, seed=0, w_std=0.05, b_std=0.02, **kw):
    return cycle_parity(meta, seq_lens, projs=projs, steps=steps, seed=seed, w_std=w_std,
                        b_std=b_std, **kw)


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_cycle_parity_7proj(family):
    meta = tiny_meta(family=family, L=2)
    worst = _run(meta, [37, 128, 1, 200, 64])
    assert_north_star(worst)


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_cycle_parity_head_dim_64(family):
    """head_dim 64 (Llama-3.2-1B's): RoPE over 32-wide halves, the q/k norm
    over 64 dims (Qwen3), attention on heads zero-padded to 128 with scale
    1/8, and the qkv / o widths of 64-dim heads; GQA group of 4."""
    meta = tiny_meta(family=family, L=2, D=512, Hq=8, Hkv=2, Hd=64, I=768)
    worst = _run(meta, [37, 128, 1, 200, 64])
    assert_north_star(worst)


def test_cycle_parity_qkvo_only_llama3_rope_scaling():
    """The reference's own configuration: LoRA on q/k/v/o only, llama3 RoPE."""
    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
          "high_freq_factor": 4.0, "original_max_position_embeddings": 256.0}
    meta = tiny_meta(L=2, rope_scaling=sc, Hq=4, Hkv=2, D=512, I=768)
    worst = _run(meta, [300, 170], projs=("q", "k", "v", "o"))
    assert_north_star(worst)


def test_cycle_varying_n_reuses_graph():
    """One captured graph serves cycles of different n and packing."""
    meta = tiny_meta(L=1, s_max=512)
    model = O.make_model(meta, seed=3, w_std=0.05, b_std=0.02)
    svc = build_service(model, "llama3")
    V = meta["vocab_size"]
    for seq_lens in ([100, 20], [7], [250, 250, 3]):
        n = sum(seq_lens)
        ids = torch.randint(0, V, (n,), generator=torch.Generator().manual_seed(n))
        acts = bf16_round_acts(O.forward_capture(model, ids, seq_lens))
        ref = O.Model(meta=model.meta, layers=[{k: v.clone() for k, v in lw.items()}
                                               for lw in model.layers],
                      lm_w=model.lm_w, norm_w=model.norm_w, embed=model.embed)
        # align the reference masters with the service's current masters
        for i, lw in enumerate(ref.layers):
            for proj in O.PROJS:
                for ab in "AB":
                    lw[proj + ab] = svc.lora[i][proj][ab].detach().cpu().clone()
        loss, nv = svc.process_backward(gpu_activations(acts, 512), seq_lens, n, epoch=0)
        rloss, rnv, rgrads = O.process_backward(ref, acts, seq_lens, n, lr=0.0, step=1, update=False)
        assert nv == rnv and abs(loss - rloss) / rloss < 1e-3
        assert svc.last_cycle_info["graph"]
        for key, g in rgrads[0].items():
            assert max_rel(svc.lora[0][key[:-1]][key[-1]].grad, g) < 2e-2
    svc.close()


@pytest.mark.parametrize("family,r", [("llama3", 16), ("qwen3", 32), ("llama3", 64)])
def test_cycle_parity_production_kernels(family, r):
    """The kernel configurations of the BASELINE runs on a small model: rank
    16/32 (the fused grad_Z + grad_B passes, q/k/v batched in one launch;
    rank 64 takes the separate skinny + TN kernels), 256×256 product tiles
    forced, the LM head streamed in four vocab chunks, and spare capacity
    (n < s_max)."""
    meta = tiny_meta(family=family, L=2, D=512, Hq=4, Hkv=2, I=768, V=1000, r=r,
                     scaling=2.0, s_max=900, vocab_chunk=256, gemm_tile=256)
    worst = _run(meta, [37, 128, 1, 200, 64, 300])
    assert_north_star(worst)


@pytest.mark.parametrize("family,r", [("llama3", 4), ("qwen3", 12), ("llama3", 20),
                                      ("qwen3", 1)])
def test_cycle_parity_rank_not_a_multiple_of_8(family, r):
    """Ranks the reference takes that are not multiples of 8 (ops.py:115-146 is
    rank-agnostic): the kernels run at r rounded up to 8 with zero rows in the
    bf16 A operands and zero columns in B, so the padding adds nothing; the
    gradients and the AdamW step cover the adapter's own r rows and columns
    (12 runs at 16 on the fused grad_Z + grad_B passes; 20 runs at 24 and 4
    and 1 at 8 on the separate skinny + TN kernels)."""
    meta = tiny_meta(family=family, L=2, D=512, Hq=4, Hkv=2, I=768, V=1000, r=r,
                     scaling=2.0, s_max=900)
    worst = _run(meta, [37, 128, 1, 200, 64, 300])
    assert_north_star(worst)


@pytest.mark.parametrize("projs", [("q", "v"), ("k", "o", "up", "down"), ("gate",)])
def test_cycle_parity_partial_lora_groups(projs):
    """Any subset of the seven projections may carry LoRA (the reference's
    ld.get(proj) may be None, trainer.py:457-460): unbound members of the
    q/k/v and gate/up groups stay frozen."""
    meta = tiny_meta(L=2, r=16, D=512, Hq=4, Hkv=2, I=768)
    worst = _run(meta, [37, 128, 1, 200, 64], projs=projs)
    assert_north_star(worst)


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_cycle_parity_saved_gate_up(family):
    """The mlp_gate_up save point (accumulate.py:174, :210-212): gate and up
    come from the store, no gate_up recompute (llama3.py:63-72)."""
    meta = tiny_meta(family=family, L=2, r=16)
    worst = _run(meta, [37, 128, 1, 200, 64], save_gate_up=True)
    assert_north_star(worst)


def test_saved_gate_up_matches_recompute():
    """Saved-shortcut == recompute (the reference's test_llama3_backward.py:
    140-149): with the store holding the forward's own gate‖up, a cycle gives
    the gradients of the recompute cycle (up to the bf16 rounding of the
    stored values)."""
    meta = tiny_meta(L=2, r=16)
    model = O.make_model(meta, seed=4, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    seq = [37, 128, 1, 200, 64]
    n = sum(seq)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(9))
    acts = bf16_round_acts(O.forward_capture(model, ids, seq, save_gate_up=True))
    plain = {k: v for k, v in acts.items() if k != "mlp_gate_up"}
    a = build_service(model, "llama3")
    b = build_service(model, "llama3")
    try:
        la, na = a.process_backward(gpu_activations(plain, 512), seq, n, epoch=0)
        lb, nb = b.process_backward(gpu_activations(acts, 512), seq, n, epoch=0)
        assert na == nb and abs(la - lb) / la < 1e-3
        for i, d in a.lora.items():
            for p, dd in d.items():
                for ab in "AB":
                    ga, gb = dd[ab].grad, b.lora[i][p][ab].grad
                    assert max_rel(gb, ga) < 2e-2 and cosine(gb, ga) > 0.999, (i, p, ab)
    finally:
        a.close()
        b.close()


SAVE_CASES = [("attn_qkv",), ("attn_ctx",), ("resid_mid",), ("attn_qkv", "attn_ctx", "resid_mid")]


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
@pytest.mark.parametrize("saves", SAVE_CASES, ids=["+".join(c) for c in SAVE_CASES])
def test_cycle_parity_saved_points(family, saves):
    """The optional save points (trainer.py:532-552; llama3.py:62-142,
    qwen3.py:68-130): saved q/k/v skip the Q/K/V projection (and Llama-3's
    RoPE), the saved post-attention residual skips the O projection, the
    saved context feeds the O projection. Against the oracle fed the same
    saved values, at the north-star bars, with the 256-wide tiles and batched
    LoRA passes of the production shapes."""
    meta = tiny_meta(family=family, L=2, D=512, Hq=4, Hkv=2, I=768, r=16, s_max=700)
    worst = _run(meta, [37, 128, 1, 200, 64], saves=saves, save_gate_up=True)
    assert_north_star(worst)


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_saved_points_match_recompute(family):
    """Saved-shortcut == recompute (test_llama3_backward_graph.py:271-311):
    with the store holding the forward's own q/k/v, context and residual
    mid-point, a cycle gives the recompute cycle's gradients up to the bf16
    rounding of the stored values; without the worker's save_attn_qkv /
    save_resid_mid meta keys those buffers are not read at all (the cycle is
    bit-identical to the recompute cycle)."""
    meta = tiny_meta(family=family, L=2, r=16)
    model = O.make_model(meta, seed=4, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    seq = [37, 128, 1, 200, 64]
    n = sum(seq)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(9))
    acts = bf16_round_acts(O.forward_capture(model, ids, seq, save_attn_qkv=True,
                                             save_resid_mid=True))
    plain = {k: v for k, v in acts.items() if k in ("layer_in", "final_in", "concat_input_ids")}
    a = build_service(model, "llama3" if family == "llama3" else "qwen3")
    b = build_service(model, "llama3" if family == "llama3" else "qwen3")
    c = build_service(model, "llama3" if family == "llama3" else "qwen3")
    b.shared["meta"].update(save_attn_qkv=True, save_resid_mid=True)
    try:
        la, na = a.process_backward(gpu_activations(plain, 512), seq, n, epoch=0)
        lb, nb = b.process_backward(gpu_activations(acts, 512), seq, n, epoch=0)
        lc, nc = c.process_backward(gpu_activations(acts, 512), seq, n, epoch=0)
        assert b.saved_points == ["attn_kh", "attn_qh", "attn_vh", "resid_mid"]
        assert c.saved_points == []
        assert na == nb == nc and abs(la - lb) / la < 1e-3 and la == lc
        for i, d in a.lora.items():
            for p, dd in d.items():
                for ab in "AB":
                    ga, gb, gc = dd[ab].grad, b.lora[i][p][ab].grad, c.lora[i][p][ab].grad
                    assert max_rel(gb, ga) < 2e-2 and cosine(gb, ga) > 0.999, (i, p, ab)
                    assert torch.equal(gc, ga), (i, p, ab)
    finally:
        a.close()
        b.close()
        c.close()


def test_cycle_many_short_sequences():
    """A packing of many short samples (more than the attention grid of the
    first capture holds): the cycle captures a graph for the larger tile
    capacity and stays exact; zero-length samples are dropped."""
    meta = tiny_meta(L=1, r=16, s_max=1024)
    g = torch.Generator().manual_seed(11)
    seq = torch.randint(1, 4, (400,), generator=g).tolist()
    seq[5] = 0
    seq = seq[:1000]
    n = sum(seq)
    assert n <= 1024
    model = O.make_model(meta, seed=6, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    svc = build_service(model, "llama3")
    try:
        for lens in ([120, 300, 7], seq):
            m = sum(lens)
            ids = torch.randint(0, meta["vocab_size"], (m,), generator=torch.Generator().manual_seed(m))
            acts = bf16_round_acts(O.forward_capture(model, ids, [x for x in lens if x > 0]))
            ref = O.Model(meta=model.meta, layers=[{k: v.clone() for k, v in lw.items()}
                                                   for lw in model.layers],
                          lm_w=model.lm_w, norm_w=model.norm_w, embed=model.embed)
            for i, lw in enumerate(ref.layers):
                for proj in O.PROJS:
                    for ab in "AB":
                        lw[proj + ab] = svc.lora[i][proj][ab].detach().cpu().clone()
            loss, nv = svc.process_backward(gpu_activations(acts, 1024), lens, m, epoch=0)
            rl, rnv, rg = O.process_backward(ref, acts, [x for x in lens if x > 0], m, lr=0.0,
                                             step=1, update=False)
            assert nv == rnv and abs(loss - rl) / rl < 1e-3
            assert svc.last_cycle_info["graph"]
            for key, gr in rg[0].items():
                got = svc.lora[0][key[:-1]][key[-1]].grad
                assert max_rel(got, gr) < 2e-2 and cosine(got, gr) > 0.999, key
    finally:
        svc.close()
