"""Pins for the CPU oracle (oracle/dsb_oracle.py). CPU only.

Every oracle function is checked against something that does not restate
its formula: a library implementation (transformers' Llama / Qwen3 modules
and RoPE initialisers, torch's SDPA, cross-entropy, AdamW and
clip_grad_norm_), autograd of an independent forward, float64 finite
differences, or brute force over integers. Each ``check_*`` raises
AssertionError on a mismatch. The negative controls at the end plant a
plausible mistake in an oracle function (on the CPU, via a wrapped copy) and
show that the same check catches it.

Reference behaviour each pin stands for (paths under
``deltaserve-plugin/deltaserve/``):
  pack              trainer.py:510-518, head.py:63-72
  rope_*            ops.py:26-81 (transformers substitutes for vLLM get_rope,
                    as tests/test_rope_scaling.py:95-103 does)
  rmsnorm*          ops.py:84-100
  proj*             ops.py:103-146
  attn_*            attention.py:20-112
  layer_*           llama3.py:62-219, qwen3.py:68-204, ffn.py:18-48
  head_backward     head.py:42-100
  clip_, adamw_     trainer.py:252-256, :624-636, :668 (torch AdamW / clip)
  process_backward  trainer.py:503-678 vs transformers *ForCausalLM autograd
  capture_index     accumulate.py:325-343 (brute-force set semantics, and the
                    cases of tests/test_ft_save_op.py:230-262)
  save_rows_        ft_save_op.py:72-89 (per-row loop with an independent
                    round-to-nearest-even bf16, and the expectations of
                    tests/test_ft_save_op.py:40-90)
"""

from __future__ import annotations

import math
import random

import pytest
import torch
import torch.nn.functional as F

from harness import O, tiny_meta

torch.set_num_threads(min(8, torch.get_num_threads()))


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


# --------------------------------------------------------------------------- #
# a18: integer packing — brute force per token
# --------------------------------------------------------------------------- #

def check_pack(pack, seq_lens):
    b_start, positions, rows, tgt, n_valid = pack(seq_lens)
    n = sum(seq_lens)
    owner = []  # sample index of every token row, by enumeration
    for i, L in enumerate(seq_lens):
        owner.extend([i] * L)
    assert len(positions) == n
    exp_rows = [t for t in range(n) if t + 1 < n and owner[t + 1] == owner[t]]
    for t in range(n):
        first = min(u for u in range(n) if owner[u] == owner[t])
        assert positions[t] == t - first
    assert rows == exp_rows and tgt == [t + 1 for t in exp_rows]
    assert n_valid == len(exp_rows) == sum(max(L - 1, 0) for L in seq_lens)
    assert b_start == [sum(seq_lens[:i]) for i in range(len(seq_lens))]


@pytest.mark.parametrize("seq_lens", [[], [0], [1], [2], [1, 1, 1], [5, 0, 3, 1, 7],
                                      [64, 1, 2, 0, 33]])
def test_pack_edge_cases(seq_lens):
    check_pack(O.pack, seq_lens)


def test_pack_random():
    rng = random.Random(7)
    for _ in range(20):
        check_pack(O.pack, [rng.choice([0, 1, 2, rng.randint(3, 40)])
                            for _ in range(rng.randint(1, 12))])


# --------------------------------------------------------------------------- #
# a1, a2: RoPE
# --------------------------------------------------------------------------- #

ROPE_CASES = [
    (5e5, None),
    (1e6, None),
    (1e4, {"rope_type": "linear", "factor": 4.0}),
    (5e5, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
           "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}),
    (5e5, {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
           "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}),
]


def _hf_config(theta, rope_scaling, head_dim=128, max_pos=131072):
    from transformers import LlamaConfig

    rp = {"rope_type": "default", "rope_theta": theta}
    if rope_scaling:
        rp.update(rope_scaling)
    return LlamaConfig(hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
                       head_dim=head_dim, intermediate_size=512, num_hidden_layers=1,
                       vocab_size=64, rope_parameters=rp, max_position_embeddings=max_pos)


def _hf_inv_freq(theta, rope_scaling):
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    cfg = _hf_config(theta, rope_scaling)
    rtype = (rope_scaling or {}).get("rope_type", "default")
    if rtype == "default":
        inv, _ = LlamaRotaryEmbedding.compute_default_rope_parameters(cfg)
    else:
        inv, _ = ROPE_INIT_FUNCTIONS[rtype](cfg)
    return inv


def check_rope_inv_freq(fn, theta, rope_scaling):
    got = fn(128, theta, rope_scaling)
    ref = _hf_inv_freq(theta, rope_scaling)
    assert _rel(got, ref) < 1e-6, (theta, rope_scaling, _rel(got, ref))


@pytest.mark.parametrize("theta,rs", ROPE_CASES)
def test_rope_inv_freq_vs_transformers(theta, rs):
    check_rope_inv_freq(O.rope_inv_freq, theta, rs)


@pytest.mark.parametrize("theta,rs", ROPE_CASES[::3])
def test_rope_cos_sin_vs_transformers(theta, rs):
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    pos = [0, 1, 2, 63, 511, 4095, 8191, 3]
    emb = LlamaRotaryEmbedding(_hf_config(theta, rs))
    x = torch.zeros(1, len(pos), 128)
    hc, hs = emb(x, torch.tensor([pos]))
    c, s = O.rope_cos_sin(pos, 128, theta, rs)
    assert (hc[0, :, :64] - c).abs().max() < 2e-6 and (hc[0, :, 64:] - c).abs().max() < 2e-6
    assert (hs[0, :, :64] - s).abs().max() < 2e-6


def test_apply_rope_vs_transformers():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(1)
    n, H = 19, 3
    q = torch.randn(n, H, 128, generator=g)
    pos = list(range(11)) + list(range(8))
    c, s = O.rope_cos_sin(pos, 128, 5e5)
    cc, ss = torch.cat([c, c], -1)[None], torch.cat([s, s], -1)[None]
    hq, _ = apply_rotary_pos_emb(q.transpose(0, 1)[None], q.transpose(0, 1)[None], cc, ss)
    assert _rel(O.apply_rope(q, c, s), hq[0].transpose(0, 1)) < 1e-6


def check_rope_backward(rope_backward, seed=2):
    """rope_backward is the adjoint (and, the rotation being orthogonal, the
    inverse) of apply_rope: <R x, g> = <x, Rᵀ g> and Rᵀ R x = x."""
    g = torch.Generator().manual_seed(seed)
    n, H = 13, 2
    x = torch.randn(n, H, 128, generator=g, dtype=torch.float64)
    gy = torch.randn(n, H, 128, generator=g, dtype=torch.float64)
    ang = torch.outer(torch.arange(n, dtype=torch.float64), O.rope_inv_freq(128, 1e4).double())
    c, s = ang.cos(), ang.sin()  # float64, so cos² + sin² = 1 to 1e-16
    lhs = (O.apply_rope(x, c, s) * gy).sum()
    rhs = (x * rope_backward(gy, c, s)).sum()
    assert abs(lhs - rhs) < 1e-9 * (abs(lhs) + 1), (lhs, rhs)
    assert _rel(rope_backward(O.apply_rope(x, c, s), c, s), x) < 1e-12


def test_rope_backward_adjoint():
    check_rope_backward(O.rope_backward)


# --------------------------------------------------------------------------- #
# a3: RMSNorm
# --------------------------------------------------------------------------- #

def test_rmsnorm_vs_transformers():
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 96, generator=g) * 3
    w = torch.rand(96, generator=g) + 0.5
    m = LlamaRMSNorm(96, eps=1e-5)
    m.weight.data.copy_(w)
    assert _rel(O.rmsnorm(x, w, 1e-5), m(x)) < 1e-6


def check_rmsnorm_backward(rmsnorm_backward, seed=4):
    """Central finite differences of <rmsnorm(x)·w, gy> in float64."""
    g = torch.Generator().manual_seed(seed)
    n, D, eps, h = 3, 8, 1e-5, 1e-6
    x = torch.randn(n, D, generator=g, dtype=torch.float64)
    w = torch.rand(D, generator=g, dtype=torch.float64) + 0.5
    gy = torch.randn(n, D, generator=g, dtype=torch.float64)
    fd = torch.zeros_like(x)
    for i in range(n):
        for j in range(D):
            e = torch.zeros_like(x)
            e[i, j] = h
            fd[i, j] = ((O.rmsnorm(x + e, w, eps) * gy).sum()
                        - (O.rmsnorm(x - e, w, eps) * gy).sum()) / (2 * h)
    got = rmsnorm_backward(x, gy, w, eps)
    assert _rel(got, fd) < 1e-7, _rel(got, fd)


def test_rmsnorm_backward_finite_differences():
    check_rmsnorm_backward(O.rmsnorm_backward)


# --------------------------------------------------------------------------- #
# a4: LoRA projection
# --------------------------------------------------------------------------- #

def test_proj_backward_vs_autograd():
    g = torch.Generator().manual_seed(5)
    n, din, dout, r, s = 9, 24, 20, 4, 2.0
    x = torch.randn(n, din, generator=g, dtype=torch.float64, requires_grad=True)
    W = torch.randn(dout, din, generator=g, dtype=torch.float64)
    A = torch.randn(r, din, generator=g, dtype=torch.float64, requires_grad=True)
    B = torch.randn(dout, r, generator=g, dtype=torch.float64, requires_grad=True)
    gy = torch.randn(n, dout, generator=g, dtype=torch.float64)
    # Independent forward: the merged weight W + s·B·A (what PEFT's merge does).
    (x @ (W + s * B @ A).t() * gy).sum().backward()
    gx, gA, gB = O.proj_backward(x.detach(), gy, W, A.detach(), B.detach(), s)
    for got, ref in ((gx, x.grad), (gA, A.grad), (gB, B.grad)):
        assert _rel(got, ref) < 1e-12
    assert _rel(O.proj(x.detach(), W, A.detach(), B.detach(), s),
                x.detach() @ (W + s * B @ A.detach()).t()) < 1e-12


# --------------------------------------------------------------------------- #
# a5, a6: attention vs SDPA (causal, GQA) + autograd
# --------------------------------------------------------------------------- #

def _sdpa_packed(qh, kh, vh, seq_lens):
    outs, st = [], 0
    for L in seq_lens:
        q = qh[st:st + L].transpose(0, 1)[None]
        k = kh[st:st + L].transpose(0, 1)[None]
        v = vh[st:st + L].transpose(0, 1)[None]
        if L:
            outs.append(F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                       enable_gqa=True)[0].transpose(0, 1))
        st += L
    return torch.cat(outs, 0).reshape(qh.shape[0], -1)


def check_attention(attn_forward, attn_backward, Hq=4, Hkv=2, seq_lens=(5, 1, 17, 9)):
    seq_lens = list(seq_lens)
    g = torch.Generator().manual_seed(6)
    n = sum(seq_lens)
    b_start, *_ = O.pack(seq_lens)
    qh = torch.randn(n, Hq, 128, generator=g, dtype=torch.float64, requires_grad=True)
    kh = torch.randn(n, Hkv, 128, generator=g, dtype=torch.float64, requires_grad=True)
    vh = torch.randn(n, Hkv, 128, generator=g, dtype=torch.float64, requires_grad=True)
    gctx = torch.randn(n, Hq * 128, generator=g, dtype=torch.float64)
    ref = _sdpa_packed(qh, kh, vh, seq_lens)
    (ref * gctx).sum().backward()
    got = attn_forward(qh.detach(), kh.detach(), vh.detach(), seq_lens, b_start, Hq, Hkv)
    assert _rel(got, ref) < 1e-10, _rel(got, ref)
    gq, gk, gv = attn_backward(qh.detach(), kh.detach(), vh.detach(), gctx, seq_lens, b_start,
                               Hq, Hkv)
    for a, b in ((gq, qh.grad), (gk, kh.grad), (gv, vh.grad)):
        assert _rel(a, b) < 1e-10, _rel(a, b)


def test_attention_vs_sdpa():
    check_attention(O.attn_forward, O.attn_backward)


def test_attention_vs_sdpa_mha_and_group8():
    check_attention(O.attn_forward, O.attn_backward, Hq=2, Hkv=2, seq_lens=(3, 12))
    check_attention(O.attn_forward, O.attn_backward, Hq=8, Hkv=1, seq_lens=(20, 2))


# --------------------------------------------------------------------------- #
# a7, a9, a10: one decoder layer vs transformers' module + autograd
# --------------------------------------------------------------------------- #

HF_PROJ = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
           "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
           "down": "mlp.down_proj"}


def _hf_cfg_from_meta(meta):
    from transformers import LlamaConfig, Qwen3Config

    rp = {"rope_type": "default", "rope_theta": meta["rope_theta"]}
    if meta.get("rope_scaling"):
        rp.update(meta["rope_scaling"])
    cls = Qwen3Config if meta["family"] == "qwen3" else LlamaConfig
    cfg = cls(hidden_size=meta["hidden_size"], intermediate_size=meta["intermediate_size"],
              num_hidden_layers=meta["num_hidden_layers"],
              num_attention_heads=meta["num_attention_heads"],
              num_key_value_heads=meta["num_key_value_heads"], head_dim=meta["head_dim"],
              vocab_size=meta["vocab_size"], rms_norm_eps=meta["rms_norm_eps"],
              rope_parameters=rp, max_position_embeddings=131072,
              tie_word_embeddings=bool(meta.get("tie_word_embeddings")),
              attention_bias=False)
    cfg._attn_implementation = "sdpa"
    return cfg


def _load_layer(mod, lw):
    with torch.no_grad():
        for p, name in HF_PROJ.items():
            mod.get_submodule(name).weight.copy_(lw[p])
        mod.input_layernorm.weight.copy_(lw["in_ln"])
        mod.post_attention_layernorm.weight.copy_(lw["post_ln"])
        if "q_norm" in lw:
            mod.self_attn.q_norm.weight.copy_(lw["q_norm"])
            mod.self_attn.k_norm.weight.copy_(lw["k_norm"])


def _lora_params(mod, lw, s, prefix=""):
    """Functional-call parameter overrides W + s·B·A (differentiable in A, B)."""
    leaves, over = {}, {}
    for p, name in HF_PROJ.items():
        if p + "A" not in lw:
            continue
        A = lw[p + "A"].clone().requires_grad_(True)
        B = lw[p + "B"].clone().requires_grad_(True)
        leaves[p + "A"], leaves[p + "B"] = A, B
        over[prefix + name + ".weight"] = mod.get_submodule(prefix + name).weight + s * B @ A
    return leaves, over


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_layer_vs_transformers(family):
    from torch.func import functional_call
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaRotaryEmbedding
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer

    meta = tiny_meta(family=family, L=1, D=128, Hq=4, Hkv=2, I=192, r=4,
                     eps=1e-6 if family == "qwen3" else 1e-5)
    model = O.make_model(meta, seed=3, w_std=0.05, b_std=0.05, norm_jitter=0.3)
    lw, s = model.layers[0], meta["lora_scaling"]
    cfg = _hf_cfg_from_meta(meta)
    mod = (Qwen3DecoderLayer if family == "qwen3" else LlamaDecoderLayer)(cfg, 0)
    _load_layer(mod, lw)
    rot = LlamaRotaryEmbedding(cfg)
    seq_lens = [7, 1, 12]
    n = sum(seq_lens)
    b_start, positions, *_ = O.pack(seq_lens)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(n, 128, generator=g).requires_grad_(True)
    gout = torch.randn(n, 128, generator=g)
    leaves, over = _lora_params(mod, lw, s)
    outs = []
    for st, L in zip(b_start, seq_lens):
        xs = x[st:st + L][None]
        pe = rot(xs, torch.arange(L)[None])
        outs.append(functional_call(mod, over, (xs,), {"position_embeddings": pe})[0])
    y_ref = torch.cat(outs, 0)
    (y_ref * gout).sum().backward()

    cos, sin = O.rope_cos_sin(positions, 128, meta["rope_theta"])
    dims = (4, 2, 128)
    qk = family == "qwen3"
    cache = O.layer_forward(x.detach(), lw, s, cos, sin, seq_lens, b_start, dims,
                            meta["rms_norm_eps"], qk)
    assert _rel(O.layer_output(cache, lw, s), y_ref) < 1e-5
    gx, grads = O.layer_backward(gout, cache, lw, s, cos, sin, seq_lens, b_start, dims,
                                 meta["rms_norm_eps"], qk)
    assert _rel(gx, x.grad) < 1e-4, _rel(gx, x.grad)
    assert sorted(grads) == sorted(leaves)
    for k, leaf in leaves.items():
        assert _rel(grads[k], leaf.grad) < 1e-4, (k, _rel(grads[k], leaf.grad))


# --------------------------------------------------------------------------- #
# a8: LM head cross-entropy
# --------------------------------------------------------------------------- #

def check_head(head_backward, seq_lens=(6, 1, 9, 0, 2)):
    seq_lens = list(seq_lens)
    g = torch.Generator().manual_seed(10)
    n, D, V, eps = sum(seq_lens), 64, 97, 1e-5
    x = torch.randn(n, D, generator=g, dtype=torch.float64, requires_grad=True)
    W = torch.randn(V, D, generator=g, dtype=torch.float64) * 0.3
    nw = torch.rand(D, generator=g, dtype=torch.float64) + 0.5
    ids = torch.randint(0, V, (n,), generator=g)
    # Independent forward: per-sample next-token CE, summed, / predicting rows.
    normed = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * nw
    tot, cnt, st = 0.0, 0, 0
    for L in seq_lens:
        if L >= 2:
            logits = normed[st:st + L - 1] @ W.t()
            tot = tot + F.cross_entropy(logits, ids[st + 1:st + L], reduction="sum")
            cnt += L - 1
        st += L
    (tot / cnt).backward()
    loss, nv, gx = head_backward(x.detach(), W, nw, eps, ids, seq_lens)
    assert nv == cnt
    assert abs(loss - (tot / cnt).item()) < 1e-10 * abs(loss)
    assert _rel(gx, x.grad) < 1e-10, _rel(gx, x.grad)


def test_head_vs_cross_entropy():
    check_head(O.head_backward)


def test_head_no_predicting_rows():
    x = torch.randn(3, 16)
    loss, nv, gx = O.head_backward(x, torch.randn(11, 16), torch.ones(16), 1e-5,
                                   torch.zeros(3, dtype=torch.long), [1, 1, 1])
    assert loss == 0.0 and nv == 0 and not gx.any()


def test_head_loss_at_init_near_log_vocab():
    """With tiny logits the CE is ≈ ln V (closed form of the uniform softmax)."""
    g = torch.Generator().manual_seed(11)
    V = 1000
    x = torch.randn(40, 32, generator=g)
    W = torch.randn(V, 32, generator=g) * 1e-4
    loss, _, _ = O.head_backward(x, W, torch.ones(32), 1e-5,
                                 torch.randint(0, V, (40,), generator=g), [20, 20])
    assert abs(loss - math.log(V)) < 1e-3


# --------------------------------------------------------------------------- #
# a13: clip + AdamW vs torch
# --------------------------------------------------------------------------- #

@pytest.mark.parametrize("scale", [10.0, 1e-3])
def test_clip_vs_torch(scale):
    g = torch.Generator().manual_seed(12)
    gs = [torch.randn(5, 7, generator=g) * scale, torch.randn(13, generator=g) * scale]
    ps = [torch.nn.Parameter(torch.zeros_like(t)) for t in gs]
    for p, t in zip(ps, gs):
        p.grad = t.clone()
    tn = torch.nn.utils.clip_grad_norm_(ps, 1.0)
    mine = [t.clone() for t in gs]
    on = O.clip_(mine, 1.0)
    assert abs(on.item() - tn.item()) < 1e-5 * tn.item()
    for a, p in zip(mine, ps):
        assert _rel(a, p.grad) < 1e-6


def check_adamw(adamw, wd=0.05, steps=5):
    g = torch.Generator().manual_seed(13)
    w0 = torch.randn(33, generator=g)
    p = torch.nn.Parameter(w0.clone())
    opt = torch.optim.AdamW([p], lr=3e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd,
                            foreach=False, fused=False)
    w, m, v = w0.clone(), torch.zeros(33), torch.zeros(33)
    for step in range(1, steps + 1):
        gr = torch.randn(33, generator=g)
        p.grad = gr.clone()
        opt.step()
        adamw(w, gr, m, v, step, 3e-3, wd=wd)
        assert _rel(w, p.detach()) < 1e-6, (step, _rel(w, p.detach()))


def test_adamw_vs_torch():
    check_adamw(O.adamw_)


def test_adamw_step1_closed_form():
    """Step 1: ΔW = −lr·g/(|g| + eps) − lr·wd·W."""
    w0 = torch.tensor([1.0, -2.0, 0.5, 3.0])
    gr = torch.tensor([0.3, -1e-3, 0.0, 2.0])
    lr, wd = 1e-2, 0.1
    w, m, v = w0.clone(), torch.zeros(4), torch.zeros(4)
    O.adamw_(w, gr, m, v, 1, lr, wd=wd)
    exp = w0 * (1 - lr * wd) - lr * gr / (gr.abs() + 1e-8)
    assert _rel(w, exp) < 1e-6


# --------------------------------------------------------------------------- #
# a12: the whole cycle vs transformers *ForCausalLM with LoRA, autograd
# --------------------------------------------------------------------------- #

def _hf_model(model):
    from transformers import LlamaForCausalLM, Qwen3ForCausalLM

    meta = model.meta
    cfg = _hf_cfg_from_meta(meta)
    hf = (Qwen3ForCausalLM if meta["family"] == "qwen3" else LlamaForCausalLM)(cfg).eval()
    with torch.no_grad():
        hf.model.embed_tokens.weight.copy_(model.embed)
        hf.model.norm.weight.copy_(model.norm_w)
        if not meta.get("tie_word_embeddings"):
            hf.lm_head.weight.copy_(model.lm_w)
        for i, lw in enumerate(model.layers):
            _load_layer(hf.model.layers[i], lw)
    return hf


def check_cycle(process_backward, family, rope_scaling=None, projs=O.PROJS):
    from torch.func import functional_call

    meta = tiny_meta(family=family, L=2, D=128, Hq=2, Hkv=1, I=160, V=211, r=4,
                     rope_scaling=rope_scaling, tie=family == "qwen3",
                     eps=1e-6 if family == "qwen3" else 1e-5)
    model = O.make_model(meta, seed=5, projs=projs, w_std=0.08, b_std=0.05, norm_jitter=0.2)
    hf = _hf_model(model)
    seq_lens = [9, 1, 14, 5]
    n = sum(seq_lens)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(4))
    s = meta["lora_scaling"]
    leaves, over = {}, {}
    for i, lw in enumerate(model.layers):
        lv, ov = _lora_params(hf, lw, s, prefix=f"model.layers.{i}.")
        leaves.update({(i, k): t for k, t in lv.items()})
        over.update(ov)
    tot, cnt, st, hidden = 0.0, 0, 0, []
    for L in seq_lens:
        out = functional_call(hf, over, (ids[st:st + L][None],),
                              {"position_ids": torch.arange(L)[None],
                               "output_hidden_states": True})
        hidden.append(out.hidden_states)
        if L >= 2:
            tot = tot + F.cross_entropy(out.logits[0, :-1], ids[st + 1:st + L], reduction="sum")
            cnt += L - 1
        st += L
    (tot / cnt).backward()

    acts = O.forward_capture(model, ids, seq_lens)
    for li in range(len(model.layers)):
        hf_in = torch.cat([h[li][0] for h in hidden], 0)
        assert _rel(acts["layer_in"][li], hf_in) < 1e-5, li
    loss, nv, grads = process_backward(model, acts, seq_lens, n, lr=1e-4, step=1, clip=False,
                                       update=False)
    assert nv == cnt
    assert abs(loss - (tot / cnt).item()) < 1e-5 * abs(loss), (loss, (tot / cnt).item())
    for (i, k), leaf in leaves.items():
        assert _rel(grads[i][k], leaf.grad) < 2e-4, (i, k, _rel(grads[i][k], leaf.grad))


def test_cycle_vs_transformers_llama3():
    check_cycle(O.process_backward, "llama3")


def test_cycle_vs_transformers_llama3_rope_scaling_qkvo():
    check_cycle(O.process_backward, "llama3",
                rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                              "high_freq_factor": 4.0, "original_max_position_embeddings": 8},
                projs=("q", "k", "v", "o"))


def test_cycle_vs_transformers_qwen3_tied():
    check_cycle(O.process_backward, "qwen3")


def check_saved_gate_up(capture=O.forward_capture):
    """Saved shortcut == recompute (the reference's test_llama3_backward.py:
    140-149): the cycle fed the forward's own gate‖up through the
    mlp_gate_up save point gives the recompute cycle's loss and gradients
    (the recompute path is pinned to transformers above)."""
    meta = tiny_meta(L=2, D=128, Hq=2, Hkv=1, I=160, V=97, r=4)
    model = O.make_model(meta, seed=12, w_std=0.08, b_std=0.05)
    seq_lens = [6, 11]
    ids = torch.randint(0, 97, (17,), generator=torch.Generator().manual_seed(3))
    acts = capture(model, ids, seq_lens, save_gate_up=True)
    plain = {k: v for k, v in acts.items() if k != "mlp_gate_up"}
    l1, n1, g1 = O.process_backward(model, plain, seq_lens, 17, lr=0.0, step=1, update=False)
    l2, n2, g2 = O.process_backward(model, acts, seq_lens, 17, lr=0.0, step=1, update=False)
    assert n1 == n2 and abs(l1 - l2) < 1e-6 * abs(l1)
    for a, b in zip(g1, g2):
        for k in a:
            assert _rel(b[k], a[k]) < 1e-5, k


def test_saved_gate_up_equals_recompute():
    check_saved_gate_up()


def check_saved_points(family, capture=O.forward_capture):
    """The other save points (trainer.py:532-552, llama3.py:62-142,
    qwen3.py:68-130): the cycle fed the forward's own q/k/v (Llama-3 after
    RoPE, Qwen3 before its q/k-norm), attention context and post-attention
    residual — each alone and all together — gives the recompute cycle's loss
    and gradients. The meta keys gate q/k/v and resid_mid as the trainer
    does: without them the buffers are ignored."""
    meta = tiny_meta(family=family, L=2, D=128, Hq=2, Hkv=1, I=160, V=97, r=4)
    model = O.make_model(meta, seed=13, w_std=0.08, b_std=0.05, norm_jitter=0.2)
    seq_lens = [6, 11]
    ids = torch.randint(0, 97, (17,), generator=torch.Generator().manual_seed(4))
    acts = capture(model, ids, seq_lens, save_attn_qkv=True, save_attn_ctx=True,
                   save_resid_mid=True)
    base_keys = ("layer_in", "final_in", "concat_input_ids")
    plain = {k: acts[k] for k in base_keys}
    l1, n1, g1 = O.process_backward(model, plain, seq_lens, 17, lr=0.0, step=1, update=False)
    cases = [(("attn_qh", "attn_kh", "attn_vh"), {"save_attn_qkv": True}),
             (("attn_ctx",), {}), (("resid_mid",), {"save_resid_mid": True}),
             (("attn_qh", "attn_kh", "attn_vh", "attn_ctx", "resid_mid"),
              {"save_attn_qkv": True, "save_resid_mid": True})]
    for keys, flags in cases:
        model.meta.update(flags)
        try:
            a = dict(plain, **{k: acts[k] for k in keys})
            l2, n2, g2 = O.process_backward(model, a, seq_lens, 17, lr=0.0, step=1, update=False)
        finally:
            for f in flags:
                model.meta.pop(f)
        assert n1 == n2 and abs(l1 - l2) < 1e-6 * abs(l1), keys
        for x, y in zip(g1, g2):
            for k in x:
                assert _rel(y[k], x[k]) < 1e-5, (keys, k)


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_saved_points_equal_recompute(family):
    check_saved_points(family)


def test_saved_qkv_ignored_without_the_meta_flag():
    """trainer.py:539-544: q/k/v buffers are read only with save_attn_qkv on;
    corrupted buffers then change nothing."""
    meta = tiny_meta(L=1, D=128, Hq=2, Hkv=1, I=160, V=97, r=4)
    model = O.make_model(meta, seed=14, w_std=0.08, b_std=0.05)
    seq_lens = [9]
    ids = torch.randint(0, 97, (9,), generator=torch.Generator().manual_seed(5))
    acts = O.forward_capture(model, ids, seq_lens, save_attn_qkv=True, save_resid_mid=True)
    junk = dict(acts, attn_qh=[t * 0 + 3 for t in acts["attn_qh"]],
                resid_mid=[t * 0 - 1 for t in acts["resid_mid"]])
    la, _, ga = O.process_backward(model, acts, seq_lens, 9, lr=0.0, step=1, update=False)
    lb, _, gb = O.process_backward(model, junk, seq_lens, 9, lr=0.0, step=1, update=False)
    assert la == lb and all(torch.equal(x[k], y[k]) for x, y in zip(ga, gb) for k in x)


def _bad_capture_qk_before_rope(model, ids, seq_lens, **kw):  # Llama-3 q/k saved pre-RoPE
    acts = O.forward_capture(model, ids, seq_lens, **kw)
    m = model.meta
    _, positions, *_ = O.pack(seq_lens)
    cos, sin = O.rope_cos_sin(positions, m["head_dim"], m["rope_theta"])
    n = len(positions)
    for key, H in (("attn_qh", m["num_attention_heads"]), ("attn_kh", m["num_key_value_heads"])):
        acts[key] = [O.rope_backward(t.reshape(n, H, -1), cos, sin).reshape(n, -1)
                     for t in acts[key]]
    return acts


def _bad_capture_resid(model, ids, seq_lens, **kw):  # resid_mid without the residual x
    acts = O.forward_capture(model, ids, seq_lens, **kw)
    acts["resid_mid"] = [r - x for r, x in zip(acts["resid_mid"], acts["layer_in"])]
    return acts


def _bad_capture_gate_up(model, ids, seq_lens, save_gate_up=False):  # halves stored up‖gate
    acts = O.forward_capture(model, ids, seq_lens, save_gate_up=save_gate_up)
    I = acts["mlp_gate_up"][0].shape[1] // 2
    acts["mlp_gate_up"] = [torch.cat([t[:, I:], t[:, :I]], 1) for t in acts["mlp_gate_up"]]
    return acts


def test_cycle_clip_and_update_compose():
    """process_backward(clip, update) == unclipped grads → per-layer
    clip_grad_norm_ → torch AdamW, on the same model."""
    meta = tiny_meta(L=2, D=128, Hq=2, Hkv=1, I=160, V=97, r=4)
    model = O.make_model(meta, seed=8, w_std=0.08, b_std=0.05)
    seq_lens = [6, 11]
    ids = torch.randint(0, 97, (17,), generator=torch.Generator().manual_seed(2))
    acts = O.forward_capture(model, ids, seq_lens)
    _, _, raw = O.process_backward(model, acts, seq_lens, 17, lr=1e-2, step=1, clip=False,
                                   update=False)
    params = {}
    for i, gr in enumerate(raw):
        ps = []
        for k in sorted(gr):
            p = torch.nn.Parameter(model.layers[i][k].clone())
            p.grad = gr[k].clone()
            ps.append(p)
            params[(i, k)] = p
        torch.nn.utils.clip_grad_norm_(ps, 1.0)
    opt = torch.optim.AdamW(list(params.values()), lr=1e-2, weight_decay=0.0, foreach=False)
    opt.step()
    _, _, clipped = O.process_backward(model, acts, seq_lens, 17, lr=1e-2, step=1)
    for (i, k), p in params.items():
        assert _rel(clipped[i][k], p.grad) < 1e-5
        assert _rel(model.layers[i][k], p.detach()) < 1e-5


# --------------------------------------------------------------------------- #
# Forward-side capture
# --------------------------------------------------------------------------- #

def check_capture_index(fn, M=9):
    """Against the set definition: the non-scratch (src, dst) pairs are exactly
    {(positions[i], offset + i) : i < num_ft, offset + i < M}, every other
    slot gathers row 0 into row M, and the count is the number of such i."""
    rng = random.Random(11)
    for offset in range(0, M + 2):
        for num_ft in range(0, M + 2):
            pos = [rng.randrange(0, 40) for _ in range(num_ft)]
            src, dst, n = fn(pos, num_ft, offset, M)
            want = {(pos[i], offset + i) for i in range(num_ft) if offset + i < M}
            got = {(int(a), int(b)) for a, b in zip(src, dst) if int(b) != M}
            assert got == want, (offset, num_ft)
            assert n == len(want)
            assert all(int(a) == 0 for a, b in zip(src, dst) if int(b) == M)
            assert len(src) == len(dst) == M
    # tests/test_ft_save_op.py:230 and :252 (S_MAX 16): rows 4..8, then 9..10
    src, dst, n = fn([2, 9, 10, 17, 23], 5, 4, 16)
    assert n == 5 and dst[:5].tolist() == [4, 5, 6, 7, 8] and src[:5].tolist() == [2, 9, 10, 17, 23]
    src, dst, n = fn([0, 5], 2, 9, 16)
    assert n == 2 and dst[:2].tolist() == [9, 10] and (dst[2:] == 16).all()


def _bf16_rne(a):
    """float32 -> bf16 round-to-nearest-even on the bit pattern (numpy)."""
    import numpy as np
    b = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (b >> 16) | 0x40, r)
    return torch.from_numpy((r.astype(np.uint32) << 16).view(np.float32).copy())


def check_save_rows(fn):
    """Per row and element: buf[dst[i]] = rne_bf16(x[src[i]] + r[src[i]]) with
    the add done in x's dtype; rows no slot names keep their contents; the
    cases of the reference's own capture test (test_ft_save_op.py:59-75)."""
    import numpy as np
    g = torch.Generator().manual_seed(4)
    M, W, T = 16, 8, 32
    for xdt in (torch.bfloat16, torch.float16, torch.float32):
        x = (torch.randn(T, W, generator=g) * 3).to(xdt)
        r = (torch.randn(T, W, generator=g) * 3).to(xdt)
        for rr in (r, None):
            buf = torch.full((M + 1, W), 5.0, dtype=torch.bfloat16)
            pos = [3, 7, 20, 31, 0]
            src, dst, n = O.capture_index(pos, len(pos), 9, M)
            fn(x, rr, buf, src, dst)
            for i in range(M):
                if i < 9 or i >= 9 + n:
                    assert (buf[i] == 5.0).all(), (xdt, i)
            for i in range(n):
                xs = x[pos[i]].numpy() if xdt != torch.bfloat16 else x[pos[i]].float().numpy()
                if rr is None:
                    v = np.asarray(xs, dtype=np.float32)
                elif xdt == torch.float32:
                    v = xs.astype(np.float32) + r[pos[i]].numpy()
                elif xdt == torch.float16:
                    v = (xs.astype(np.float16) + r[pos[i]].numpy().astype(np.float16)).astype(np.float32)
                else:  # bf16 add: exact float sum rounded once to bf16
                    v = _bf16_rne(xs + r[pos[i]].float().numpy()).numpy()
                assert torch.equal(buf[9 + i].float(), _bf16_rne(v)), (xdt, rr is None, i)
    # test_ft_save_op.py:59-66: positions 3, 7, 20 -> rows 5..7, others untouched
    x = torch.randn(32, 8, generator=g).to(torch.bfloat16)
    r = torch.randn(32, 8, generator=g).to(torch.bfloat16)
    buf = torch.zeros(17, 8, dtype=torch.bfloat16)
    src = torch.tensor([3, 7, 20] + [0] * 13)
    dst = torch.tensor([5, 6, 7] + [16] * 13)
    fn(x, r, buf, src, dst)
    assert torch.equal(buf[5:8], (x[[3, 7, 20]].float() + r[[3, 7, 20]].float()).to(torch.bfloat16))
    assert buf[:5].abs().sum() == 0 and buf[8:16].abs().sum() == 0


def test_capture_index():
    check_capture_index(O.capture_index)


def test_save_rows():
    check_save_rows(O.save_rows_)


# --------------------------------------------------------------------------- #
# Negative controls: each check must reject a planted mistake.
# --------------------------------------------------------------------------- #

def _bad_pack(seq_lens):
    b, pos, rows, tgt, nv = O.pack(seq_lens)
    return b, pos, rows + [sum(seq_lens) - 1] if rows else rows, tgt, nv  # predicts last row


def _bad_inv_freq(hd, theta, rs):  # llama3 band blend with low/high swapped
    if rs and rs.get("rope_type") == "llama3":
        rs = dict(rs, low_freq_factor=rs["high_freq_factor"], high_freq_factor=rs["low_freq_factor"])
    return O.rope_inv_freq(hd, theta, rs)


def _bad_rope_backward(g, c, s):  # sign of the sine term flipped (= applying R, not Rᵀ)
    return O.rope_backward(g, c, -s)


def _bad_rmsnorm_backward(x, gy, w, eps):  # projection term dropped
    return gy * w * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def _bad_attn_fwd(qh, kh, vh, seq_lens, b_start, Hq, Hkv):  # q-head h → kv-head h % Hkv
    perm = torch.arange(Hq).view(Hkv, Hq // Hkv).t().reshape(-1)
    out = O.attn_forward(qh[:, perm], kh, vh, seq_lens, b_start, Hq, Hkv)
    inv = torch.argsort(perm)
    return out.view(-1, Hq, 128)[:, inv].reshape(out.shape)


def _bad_head(x, W, nw, eps, ids, seq_lens):  # targets off by one (predicts itself)
    return O.head_backward(x, W, nw, eps, torch.roll(ids, 1), seq_lens)


def _bad_adamw(w, g, m, v, step, lr, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.0):
    O.adamw_(w, g, m, v, 10 ** 6, lr, beta1, beta2, eps, wd)  # bias correction dropped


def _bad_cycle(model, acts, seq_lens, n, **kw):  # per-layer gradient scaled by LoRA s twice
    loss, nv, grads = O.process_backward(model, acts, seq_lens, n, **kw)
    for gr in grads:
        for k in gr:
            if k.endswith("B"):
                gr[k] = gr[k] * model.meta["lora_scaling"]
    return loss, nv, grads


def _bad_capture_index(pos, num_ft, offset, M):  # n not clipped at the buffer end
    src, dst, n = O.capture_index(pos, num_ft, 0, M + num_ft)
    src, dst = src[:M], dst[:M]
    dst = torch.where(dst < M + num_ft, dst + offset, torch.full_like(dst, M))
    return src, dst, min(num_ft, M)


def _bad_save_rows(x, r, buf, src, dst):  # residual added after the bf16 cast
    rows = x.index_select(0, src).to(buf.dtype)
    if r is not None:
        rows = rows + r.index_select(0, src).to(buf.dtype)
    buf.index_copy_(0, dst, rows)
    return buf


PLANTED = {
    "capture_index_clip": lambda: check_capture_index(_bad_capture_index),
    "save_rows_cast_order": lambda: check_save_rows(_bad_save_rows),
    "pack": lambda: check_pack(_bad_pack, [3, 4]),
    "rope_inv_freq": lambda: check_rope_inv_freq(_bad_inv_freq, *ROPE_CASES[3]),
    "rope_backward": lambda: check_rope_backward(_bad_rope_backward),
    "rmsnorm_backward": lambda: check_rmsnorm_backward(_bad_rmsnorm_backward),
    "attention_gqa": lambda: check_attention(_bad_attn_fwd, O.attn_backward),
    "head_targets": lambda: check_head(_bad_head),
    "adamw_bias_correction": lambda: check_adamw(_bad_adamw),
    "cycle_lora_scale": lambda: check_cycle(_bad_cycle, "llama3", projs=("q", "v")),
    "saved_gate_up_order": lambda: check_saved_gate_up(_bad_capture_gate_up),
    "saved_qk_rope_side": lambda: check_saved_points("llama3", _bad_capture_qk_before_rope),
    "saved_resid_mid_residual": lambda: check_saved_points("qwen3", _bad_capture_resid),
}


@pytest.mark.parametrize("name", sorted(PLANTED))
def test_planted_mistake_is_caught(name):
    with pytest.raises(AssertionError):
        PLANTED[name]()
