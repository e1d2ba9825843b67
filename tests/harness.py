"""Shared test helpers: oracle models → the reference's shared-weight /
adapter / meta dicts, GPU activation stores, and error metrics.

Test infrastructure (imports the oracle); used by tests/, smoke() and the
bench's CPU-baseline leg only."""

from __future__ import annotations

import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for _p in (ROOT, os.path.join(ROOT, "deltaserve-vllm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

from oracle import dsb_oracle as O  # noqa: E402

LORA_KEY = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
            "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
            "down": "mlp.down_proj"}


def tiny_meta(family="llama3", L=2, D=256, Hq=2, Hkv=1, I=512, V=1000, r=8, theta=5e5,
              eps=1e-5, scaling=2.0, rope_scaling=None, lr=1e-4, s_max=512, tie=False,
              vocab_chunk=0, gemm_tile=0, Hd=128):
    """Model dims + the backward meta keys the trainer reads; ``vocab_chunk``
    and ``gemm_tile`` are the libdsb tuning keys (0: defaults)."""
    m = dict(family=family, num_hidden_layers=L, hidden_size=D, num_attention_heads=Hq,
             num_key_value_heads=Hkv, head_dim=Hd, intermediate_size=I, vocab_size=V,
             lora_rank=r, rope_theta=theta, rms_norm_eps=eps, lora_scaling=scaling,
             rope_scaling=rope_scaling, learning_rate=lr, weight_decay=0.0, gamma=1.0,
             max_saved_finetuning_tokens=s_max, tie_word_embeddings=tie)
    if vocab_chunk:
        m["backward_vocab_chunk"] = vocab_chunk
    if gemm_tile:
        m["backward_gemm_tile"] = gemm_tile
    return m


def config_meta(name, L=1, s_max=None):
    """The dims of BASELINE config ``name`` (deltaserve_amd.configs) with L
    layers: the 'one decoder layer + full head at the real widths' slice."""
    from deltaserve_amd.configs import CONFIGS, draw_lengths

    c = CONFIGS[name]
    lens = draw_lengths(c["nseq"], c["lo"], c["hi"], c["total"], seed=0)
    m = tiny_meta(family=c["family"], L=L, D=c["D"], Hq=c["Hq"], Hkv=c["Hkv"], I=c["I"],
                  Hd=c.get("Hd", 128), V=c["V"], r=c["r"], theta=c["theta"], eps=c["eps"],
                  scaling=c["alpha"] / c["r"], rope_scaling=c["rope_scaling"],
                  s_max=s_max or sum(lens), tie=c["tie"])
    return m, lens


def peft_key(i, proj, ab):
    return f"base_model.model.model.layers.{i}.{LORA_KEY[proj]}.lora_{ab}.weight"


def shared_from_model(model: O.Model, device="cuda"):
    """(base, ft, meta) exactly as the reference's worker shares them: fused
    bf16 qkv_proj / gate_up_proj, PEFT-keyed fp32 LoRA factors."""
    bf = lambda t: t.to(device=device, dtype=torch.bfloat16).contiguous()  # noqa: E731
    base = {"model.norm.weight": bf(model.norm_w), "model.embed_tokens.weight": bf(model.embed)}
    meta = dict(model.meta)
    if model.meta.get("tie_word_embeddings"):
        meta["lm_head_key"] = "model.embed_tokens.weight"
    else:
        base["lm_head.weight"] = bf(model.lm_w)
        meta["lm_head_key"] = "lm_head.weight"
    meta["norm_weight_key"] = "model.norm.weight"
    ft = {}
    for i, lw in enumerate(model.layers):
        p = f"model.layers.{i}."
        base[p + "self_attn.qkv_proj.weight"] = bf(torch.cat([lw["q"], lw["k"], lw["v"]], 0))
        base[p + "self_attn.o_proj.weight"] = bf(lw["o"])
        base[p + "mlp.gate_up_proj.weight"] = bf(torch.cat([lw["gate"], lw["up"]], 0))
        base[p + "mlp.down_proj.weight"] = bf(lw["down"])
        base[p + "input_layernorm.weight"] = bf(lw["in_ln"])
        base[p + "post_attention_layernorm.weight"] = bf(lw["post_ln"])
        if "q_norm" in lw:
            base[p + "self_attn.q_norm.weight"] = bf(lw["q_norm"])
            base[p + "self_attn.k_norm.weight"] = bf(lw["k_norm"])
        for proj in O.PROJS:
            if proj + "A" in lw:
                ft[peft_key(i, proj, "A")] = lw[proj + "A"].clone()
                ft[peft_key(i, proj, "B")] = lw[proj + "B"].clone()
    return base, ft, meta


def gpu_activations(acts, s_max, device="cuda"):
    """The reference's activation store layout: [s_max + 1, D] bf16 buffers
    (rows past n zero) and int64 ids [s_max]."""
    n, D = acts["final_in"].shape

    def buf(t):
        b = torch.zeros(s_max + 1, D, dtype=torch.bfloat16, device=device)
        b[:n] = t.to(device=device, dtype=torch.bfloat16)
        return b

    ids = torch.zeros(s_max, dtype=torch.int64, device=device)
    ids[:n] = acts["concat_input_ids"].to(device)
    out = {"layer_in": [buf(t) for t in acts["layer_in"]], "final_in": buf(acts["final_in"]),
           "concat_input_ids": ids}

    def wbuf(t):
        b = torch.zeros(s_max + 1, t.shape[1], dtype=torch.bfloat16, device=device)
        b[:n] = t.to(device=device, dtype=torch.bfloat16)
        return b

    for key in SAVE_POINTS:
        if key in acts:
            out[key] = [wbuf(t) for t in acts[key]]
    return out


# the optional per-layer save points of the activation store (accumulate.py:208-235)
SAVE_POINTS = ("mlp_gate_up", "attn_qh", "attn_kh", "attn_vh", "attn_ctx", "resid_mid")


def bf16_round_acts(acts):
    """The activations as the GPU sees them (bf16 values), in fp32."""
    out = {"layer_in": [t.to(torch.bfloat16).float() for t in acts["layer_in"]],
           "final_in": acts["final_in"].to(torch.bfloat16).float(),
           "concat_input_ids": acts["concat_input_ids"]}
    for key in SAVE_POINTS:
        if key in acts:
            out[key] = [t.to(torch.bfloat16).float() for t in acts[key]]
    return out


def clone_model(model):
    """An independent copy of the oracle model's trainable state (frozen
    weights shared), for a reference run that steps its own masters."""
    return O.Model(meta=model.meta, layers=[{k: v.clone() for k, v in lw.items()}
                                            for lw in model.layers],
                   lm_w=model.lm_w, norm_w=model.norm_w, embed=model.embed)


def fp32_reference_mode():
    """torch's fp32 GEMMs without reduced-precision shortcuts (the oracle as
    the fp32 reference on device tensors)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")


def build_service(model: O.Model, family="llama3", device="cuda", meta_extra=None):
    from deltaserve_amd.bwd_services.registry import get_service

    base, ft, meta = shared_from_model(model, device)
    if meta_extra:
        meta = dict(meta, **meta_extra)
    svc = get_service(family)(0)
    svc.shared = {"base": base, "ft": ft, "meta": meta}
    err = svc._on_weights_shared()
    if err:
        raise RuntimeError(err)
    return svc


def max_rel(got, ref):
    """bwd_harness.Checker metric: max|got − ref| / (max|ref| + 1e-8); +inf
    when either side holds a non-finite value (so no comparison passes it)."""
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    if not (torch.isfinite(got).all() and torch.isfinite(ref).all()):
        return float("inf")
    return ((got - ref).abs().max() / (ref.abs().max() + 1e-8)).item()


def cosine(got, ref):
    """Cosine similarity in float64 (fp32 sums over millions of elements drift
    past 1); -inf when either side holds a non-finite value."""
    got, ref = got.detach().double().cpu().flatten(), ref.detach().double().cpu().flatten()
    if not (torch.isfinite(got).all() and torch.isfinite(ref).all()):
        return float("-inf")
    return torch.nn.functional.cosine_similarity(got, ref, dim=0).item()


def unexplained_master_misses(w_got, w_ref, steps, bar=2e-2):
    """The updated masters' direct bar, made checkable at the BASELINE widths.

    Elements of the master ``w_got`` further than ``bar``·max|w_ref| from the
    fp32 run's ``w_ref`` are allowed only where the fp32 reference gradient
    lay within the measured gradient error of zero at some step: there the
    two runs' gradients can have opposite signs, and AdamW's first steps move
    a weight by about lr·sign(g) whatever |g| is, so no gradient accuracy
    keeps the masters together. ``steps`` holds (our gradient, reference
    gradient) per cycle; the measured error of a step is the tensor's max
    |g_got − g_ref| there. Returns (elements off the bar, of them not
    explained by such a gradient)."""
    w_got, w_ref = w_got.detach().float().cpu(), w_ref.detach().float().cpu()
    off = (w_got - w_ref).abs() > bar * w_ref.abs().max()
    if not bool(off.any()):
        return 0, 0
    ambiguous = torch.zeros_like(off)
    for g_got, g_ref in steps:
        g_got, g_ref = g_got.detach().float().cpu(), g_ref.detach().float().cpu()
        ambiguous |= g_ref.abs() <= (g_got - g_ref).abs().max()
    return int(off.sum()), int((off & ~ambiguous).sum())


def cycle_parity(meta, seq_lens, projs=O.PROJS, steps=2, seed=0, w_std=0.05, b_std=0.02,
                 norm_jitter=0.2, ref_device="cpu", save_gate_up=False, saves=()):
    """Runs ``steps`` cycles of LoraSftTrainerService.process_backward (libdsb,
    one hipGraph) and of the oracle's process_backward on the same seeded
    model and activations; returns the worst gradient / master max-relative
    errors, the worst gradient cosine and the loss relative errors. The
    oracle runs on ``ref_device`` (CPU, or fp32 device tensors for the
    BASELINE-width slices)."""
    if ref_device != "cpu":
        fp32_reference_mode()
    # ``saves``: the other save points ("attn_qkv", "attn_ctx", "resid_mid"),
    # with the meta keys the worker sets when it captures them
    meta = dict(meta, **{"save_" + name: True for name in saves
                         if name in ("attn_qkv", "resid_mid")})
    model = O.make_model(meta, seed=seed, projs=projs, w_std=w_std, b_std=b_std,
                         norm_jitter=norm_jitter, device=ref_device)
    n = sum(seq_lens)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(seed + 1))
    acts = bf16_round_acts(O.forward_capture(
        model, ids.to(ref_device), seq_lens, save_gate_up=save_gate_up,
        **{"save_" + name: True for name in saves}))
    svc = build_service(model, meta["family"])
    gacts = gpu_activations(acts, meta["max_saved_finetuning_tokens"])
    ref = clone_model(model)
    # the masters stepped by the reference AdamW formula from libdsb's own
    # clipped gradients: isolates the optimizer step from gradient rounding
    own = clone_model(model)
    worst = {"grad": 0.0, "w": 0.0, "w_own": 0.0, "cos": 1.0, "loss": 0.0, "n_valid_ok": True,
             "graph": True, "w_off": 0, "w_unexplained": 0, "w_numel": 0}
    history = {}  # (layer, key) -> [(our grad, reference grad) per step], on the host
    wd = float(meta.get("weight_decay", 0.0))
    try:
        for step in range(1, steps + 1):
            loss, nv = svc.process_backward(gacts, seq_lens, n, epoch=0)
            rloss, rnv, rgrads = O.process_backward(ref, acts, seq_lens, n,
                                                    lr=meta["learning_rate"], step=step)
            worst["n_valid_ok"] &= nv == rnv
            worst["graph"] &= bool(svc.last_cycle_info["graph"])
            lr_ = abs(loss - rloss) / abs(rloss)
            worst["loss"] = max(worst["loss"], lr_ if lr_ == lr_ else float("inf"))
            for i, gr in enumerate(rgrads):
                for key, g in gr.items():
                    proj, ab = key[:-1], key[-1]
                    got = svc.lora[i][proj][ab].grad
                    history.setdefault((i, key), []).append((got.detach().float().cpu(),
                                                             g.detach().float().cpu()))
                    mr, c = max_rel(got, g), cosine(got, g)
                    if mr > worst["grad"] or c < worst["cos"]:
                        worst["where"] = f"step {step} layer {i} {key}: max-rel {mr:.3e} cos {c:.6f}"
                    worst["grad"] = max(worst["grad"], mr)
                    worst["cos"] = min(worst["cos"], c)
                    worst["w"] = max(worst["w"], max_rel(svc.lora[i][proj][ab],
                                                         ref.layers[i][key]))
                    st = own.opt_state.setdefault((i, key), (torch.zeros_like(g),
                                                             torch.zeros_like(g)))
                    O.adamw_(own.layers[i][key], got.detach().to(g.device).float(), st[0], st[1],
                             step, meta["learning_rate"], wd=wd)
                    worst["w_own"] = max(worst["w_own"], max_rel(svc.lora[i][proj][ab],
                                                                 own.layers[i][key]))
        for (i, key), hist in history.items():
            off, bad = unexplained_master_misses(svc.lora[i][key[:-1]][key[-1]],
                                                 ref.layers[i][key], hist)
            worst["w_off"] += off
            worst["w_unexplained"] += bad
            worst["w_numel"] += hist[0][1].numel()
    finally:
        svc.close()
    return worst


def assert_north_star(worst, direct_masters=True):
    """BASELINE bars: loss 1e-3 relative; LoRA grads 2e-2 max-relative with
    cosine >= 0.999 against the fp32 reference; n_valid exact; the updated
    masters equal the reference AdamW step of libdsb's own clipped gradients
    (1e-5) and, with ``direct_masters``, the fp32 reference's masters within
    2e-2 max-relative; without it, every master element outside that bar must
    be explained by a sign-ambiguous reference gradient
    (``unexplained_master_misses``).

    The direct master bar is left out at the BASELINE widths: in its first
    steps AdamW moves every element by about lr·sign(g), so an element whose
    fp32 gradient lies within bf16 rounding of zero moves the other way in a
    bf16 run, by up to 2·lr per step whatever the gradient accuracy; against
    down_proj's A (bounded by 1/sqrt(intermediate), 0.0076 at C4) two such
    steps are already 5% of the tensor's largest element."""
    assert worst["n_valid_ok"], worst
    assert worst["loss"] < 1e-3, worst
    assert worst["grad"] < 2e-2 and worst["cos"] > 0.999, worst
    assert worst["w_own"] < 1e-5, worst
    if direct_masters:
        assert worst["w"] < 2e-2, worst
    else:
        assert worst["w_unexplained"] == 0, worst
