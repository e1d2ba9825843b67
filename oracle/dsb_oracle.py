"""CPU oracle: a float32 PyTorch restatement of DeltaServe's LoRA-SFT backward.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this module, and only as
the checker / the timed CPU baseline. The product path (libdsb.so and
``deltaserve_amd``) never calls it.

Each function restates the reference's algorithm (paths relative to the
reference checkout, under ``deltaserve-plugin/deltaserve/``) in float32. The
functions follow the device of their inputs: the pins and the small parity
cases run them on CPU tensors; the BASELINE-width slices of the GPU tests run
the same functions on float32 device tensors (torch's fp32 kernels, TF32 off)
as the fp32 reference of those shapes. The reference trains LoRA on q/k/v/o only
(``bwd_services/common/family.py:20``); this oracle extends the same
``proj``/``proj_backward`` rule to gate/up/down, which is what the MI355X
build trains. How each function is pinned independently of this file is
listed in ``tests/test_oracle_pins.py``; every function here has a pin.

Model representation (``Model``): ``meta`` dims, per-layer ``lw`` dicts with
frozen weights ``q,k,v,o,gate,up,down,in_ln,post_ln`` (+ ``q_norm,k_norm``
for Qwen3) and fp32 LoRA factors ``{p}A`` [r,in], ``{p}B`` [out,r] for the
projections present, plus ``lm_w`` [V,D], ``norm_w`` [D], ``embed`` [V,D].
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

PROJS = ("q", "k", "v", "o", "gate", "up", "down")


# --------------------------------------------------------------------------- #
# Integer packing (bwd_services/common/trainer.py:510-518, common/head.py:63-72)
# --------------------------------------------------------------------------- #

def pack(seq_lens):
    """``(b_start, positions, rows, tgt_index, n_valid)`` for a packed cycle.

    b_start: exclusive prefix sum (trainer.py:510-514); positions:
    cat(arange(L_i)) (trainer.py:516-518); rows: predicting rows
    st..st+L-2 of every sample with L >= 2, targets at rows+1 (head.py:63-72).
    """
    b_start, acc = [], 0
    for s in seq_lens:
        b_start.append(acc)
        acc += int(s)
    positions = [p for s in seq_lens for p in range(int(s))]
    rows, tgt = [], []
    for st, ln in zip(b_start, seq_lens):
        if ln < 2:
            continue
        rows.extend(range(st, st + ln - 1))
        tgt.extend(range(st + 1, st + ln))
    return b_start, positions, rows, tgt, len(rows)


# --------------------------------------------------------------------------- #
# Forward-side capture (accumulate.py:325-343, ft_save_op.py:72-89)
# --------------------------------------------------------------------------- #

def capture_index(positions, num_ft: int, offset: int, max_saved: int):
    """``arm_op_step``'s index pair (accumulate.py:332-340): the first
    n = min(num_ft, max_saved - offset) slots gather ``positions[:n]`` into
    buffer rows offset..offset+n-1; the rest gather row 0 into the scratch row
    ``max_saved``. Returns (src, dst) int64 [max_saved] and max(n, 0)."""
    n = min(int(num_ft), max_saved - int(offset))
    src = torch.zeros(max_saved, dtype=torch.int64)
    dst = torch.full((max_saved,), max_saved, dtype=torch.int64)
    if n > 0:
        src[:n] = torch.as_tensor(list(positions)[:n], dtype=torch.int64)
        dst[:n] = torch.arange(offset, offset + n, dtype=torch.int64)
    return src, dst, max(n, 0)


def save_rows_(x, r, buf, src, dst):
    """The save op on CPU tensors (ft_save_op.py:84-89): rows of ``x`` (+ ``r``,
    added in x's dtype) at ``src``, cast to the buffer's dtype, copied into
    ``buf`` at ``dst``. In place; the scratch row receives whatever the
    unused slots gather."""
    rows = x.index_select(0, src)
    if r is not None:
        rows = rows + r.index_select(0, src)
    buf.index_copy_(0, dst, rows.to(buf.dtype))
    return buf


# --------------------------------------------------------------------------- #
# common/ops.py
# --------------------------------------------------------------------------- #

def rope_inv_freq(head_dim: int, theta: float, rope_scaling: dict | None = None):
    """ops.py:26-57 — inverse frequencies with default / linear / llama3 scaling."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    rtype = (rope_scaling or {}).get("rope_type", "default")
    if rtype in (None, "default"):
        return inv
    if rtype == "linear":
        return inv / float(rope_scaling["factor"])
    if rtype == "llama3":
        factor = float(rope_scaling["factor"])
        low = float(rope_scaling["low_freq_factor"])
        high = float(rope_scaling["high_freq_factor"])
        orig = float(rope_scaling["original_max_position_embeddings"])
        low_wavelen, high_wavelen = orig / low, orig / high
        wavelen = 2 * math.pi / inv
        smooth = ((orig / wavelen - low) / (high - low)) if low != high else 0
        return torch.where(wavelen < high_wavelen, inv,
                           torch.where(wavelen > low_wavelen, inv / factor,
                                       (1 - smooth) * inv / factor + smooth * inv))
    raise NotImplementedError(f"RoPE type {rtype!r}")


def rope_cos_sin(positions, head_dim, theta, rope_scaling=None, device=None):
    """ops.py:60-65 — (cos, sin) [n, head_dim/2] fp32."""
    pos = torch.as_tensor(positions, dtype=torch.float32, device=device)
    freqs = torch.outer(pos, rope_inv_freq(head_dim, theta, rope_scaling).to(pos.device))
    return freqs.cos(), freqs.sin()


def apply_rope(xh, cos, sin):
    """ops.py:68-73 — NeoX rotate-half on [n, H, Hd]."""
    h = xh.shape[-1] // 2
    x1, x2 = xh[..., :h], xh[..., h:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def rope_backward(g, cos, sin):
    """ops.py:76-81 — transpose of the rotation."""
    h = g.shape[-1] // 2
    g1, g2 = g[..., :h], g[..., h:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([g1 * c + g2 * s, -g1 * s + g2 * c], dim=-1)


def rmsnorm(x, w, eps):
    """ops.py:84-88."""
    inv = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return (x * inv) * w


def rmsnorm_backward(x, gy, w, eps):
    """ops.py:91-100 — exact gradient of rmsnorm(x)·w wrt x."""
    inv = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    xhat = x * inv
    gx = gy * w
    dot = (gx * xhat).sum(-1, keepdim=True)
    return (gx - xhat * dot / x.shape[-1]) * inv


def proj(x, W, A, B, s):
    """ops.py:103-112 — y = x Wᵀ + s (x Aᵀ) Bᵀ (A None → frozen projection)."""
    y = x @ W.t()
    if A is not None:
        y = y + s * ((x @ A.t()) @ B.t())
    return y


def proj_backward(x, gy, W, A, B, s):
    """ops.py:115-146 — (grad_x, grad_A, grad_B)."""
    gx = gy @ W
    gA = gB = None
    if A is not None:
        Z = x @ A.t()
        gZ = s * (gy @ B)
        gA = gZ.t() @ x
        gB = s * (gy.t() @ Z)
        gx = gx + gZ @ A
    return gx, gA, gB


# --------------------------------------------------------------------------- #
# common/attention.py
# --------------------------------------------------------------------------- #

def _causal_mask(L, device=None):
    return torch.triu(torch.ones(L, L, dtype=torch.bool, device=device), 1)


def attn_forward(qh, kh, vh, seq_lens, b_start, Hq, Hkv):
    """attention.py:20-45 — per-sample causal GQA, fp32; returns ctx [n, Hq*Hd]."""
    Hd = qh.shape[-1]
    scale = 1.0 / math.sqrt(Hd)
    rep = Hq // Hkv
    out = []
    for st, ln in zip(b_start, seq_lens):
        q = qh[st:st + ln].transpose(0, 1)
        k = kh[st:st + ln].transpose(0, 1).repeat_interleave(rep, 0)
        v = vh[st:st + ln].transpose(0, 1).repeat_interleave(rep, 0)
        sc = (q @ k.transpose(-1, -2)) * scale
        sc = sc.masked_fill(_causal_mask(ln, qh.device), -1e9)
        p = torch.softmax(sc, dim=-1)
        out.append((p @ v).transpose(0, 1))
    n = qh.shape[0]
    return torch.cat(out, 0).reshape(n, Hq * Hd)


def attn_backward(qh, kh, vh, gctx, seq_lens, b_start, Hq, Hkv):
    """attention.py:48-112 — (grad_qh, grad_kh, grad_vh) in [n, H, Hd]."""
    n, _, Hd = qh.shape
    scale = 1.0 / math.sqrt(Hd)
    rep = Hq // Hkv
    gq = torch.zeros_like(qh)
    gk = torch.zeros_like(kh)
    gv = torch.zeros_like(vh)
    g_all = gctx.reshape(n, Hq, Hd)
    for st, ln in zip(b_start, seq_lens):
        q = qh[st:st + ln].transpose(0, 1)
        k = kh[st:st + ln].transpose(0, 1).repeat_interleave(rep, 0)
        v = vh[st:st + ln].transpose(0, 1).repeat_interleave(rep, 0)
        mask = _causal_mask(ln, qh.device)
        p = torch.softmax(((q @ k.transpose(-1, -2)) * scale).masked_fill(mask, -1e9), dim=-1)
        g = g_all[st:st + ln].transpose(0, 1)
        dp = g @ v.transpose(-1, -2)
        dv = p.transpose(-1, -2) @ g
        ds = (p * (dp - (dp * p).sum(-1, keepdim=True))).masked_fill(mask, 0.0)
        dq = (ds @ k) * scale
        dk = (ds.transpose(-1, -2) @ q) * scale
        gq[st:st + ln] = dq.transpose(0, 1)
        gk[st:st + ln] = dk.view(Hkv, rep, ln, Hd).sum(1).transpose(0, 1)
        gv[st:st + ln] = dv.view(Hkv, rep, ln, Hd).sum(1).transpose(0, 1)
    return gq, gk, gv


# --------------------------------------------------------------------------- #
# Decoder layer: llama3.py:62-219 and qwen3.py:68-204 (+ FFN LoRA)
# --------------------------------------------------------------------------- #

def _lora(lw, p):
    return lw.get(p + "A"), lw.get(p + "B")


def layer_forward(x, lw, s, cos, sin, seq_lens, b_start, dims, eps, qk_norm=False,
                  saved_gate_up=None, saved_qkv=None, saved_ctx=None, saved_resid_mid=None):
    """llama3.py:62-146 / qwen3.py:68-130 with ffn.py:18-26 (gate/up LoRA added).
    ``saved_gate_up`` [n, 2I] (gate first): the captured pre-activations,
    used instead of the gate/up recompute (ffn.py:21-24, llama3.py:142).
    ``saved_qkv`` = (q, k, v) flat [n, q|kv]: skips the Q/K/V projections;
    Llama-3 takes q/k as saved after RoPE (llama3.py:120-126), Qwen3 before
    its q/k-norm, re-applying norm and RoPE (qwen3.py:90-96).
    ``saved_ctx`` [n, q]: the attention context, used instead of the attention
    forward (llama3.py:128-132). ``saved_resid_mid`` [n, D]: the
    post-attention residual, used instead of the O projection and residual
    add (llama3.py:134-141)."""
    Hq, Hkv, Hd = dims
    n = x.shape[0]
    xn1 = rmsnorm(x, lw["in_ln"], eps)
    if saved_qkv is not None:
        q, k, v = saved_qkv
    else:
        q = proj(xn1, lw["q"], *_lora(lw, "q"), s)
        k = proj(xn1, lw["k"], *_lora(lw, "k"), s)
        v = proj(xn1, lw["v"], *_lora(lw, "v"), s)
    q_pre, k_pre = q.reshape(n, Hq, Hd), k.reshape(n, Hkv, Hd)
    if qk_norm:
        qh = apply_rope(rmsnorm(q_pre, lw["q_norm"], eps), cos, sin)
        kh = apply_rope(rmsnorm(k_pre, lw["k_norm"], eps), cos, sin)
    elif saved_qkv is not None:
        qh, kh = q_pre, k_pre  # Llama-3 saves them after RoPE
        q_pre = k_pre = None
    else:
        qh, kh = apply_rope(q_pre, cos, sin), apply_rope(k_pre, cos, sin)
    vh = v.reshape(n, Hkv, Hd)
    if saved_ctx is not None:
        ctx = saved_ctx.reshape(n, Hq * Hd)
    else:
        ctx = attn_forward(qh, kh, vh, seq_lens, b_start, Hq, Hkv)
    if saved_resid_mid is not None:
        resid_mid = saved_resid_mid
    else:
        resid_mid = x + proj(ctx, lw["o"], *_lora(lw, "o"), s)
    xn2 = rmsnorm(resid_mid, lw["post_ln"], eps)
    if saved_gate_up is not None:
        inter = saved_gate_up.shape[-1] // 2
        gate, up = saved_gate_up[:, :inter], saved_gate_up[:, inter:]
    else:
        gate = proj(xn2, lw["gate"], *_lora(lw, "gate"), s)
        up = proj(xn2, lw["up"], *_lora(lw, "up"), s)
    return {"x": x, "xn1": xn1, "q_pre": q_pre, "k_pre": k_pre, "qh": qh, "kh": kh,
            "vh": vh, "ctx": ctx, "resid_mid": resid_mid, "xn2": xn2,
            "gate": gate, "up": up}


def layer_output(cache, lw, s):
    """The frozen-or-LoRA down projection + residual (tests/bwd_harness.py:147-150)."""
    h = F.silu(cache["gate"]) * cache["up"]
    return cache["resid_mid"] + proj(h, lw["down"], *_lora(lw, "down"), s)


def ffn_backward(gout, cache, lw, s, eps):
    """ffn.py:29-48 with LoRA on gate/up/down. Returns (grad_resid_mid, grads)."""
    gate, up = cache["gate"], cache["up"]
    sig = torch.sigmoid(gate)
    silu = gate * sig
    dsilu = sig * (1.0 + gate * (1.0 - sig))
    h = silu * up
    gh, gA_d, gB_d = proj_backward(h, gout, lw["down"], *_lora(lw, "down"), s)
    gu = gh * silu
    gg = gh * up * dsilu
    gx_g, gA_g, gB_g = proj_backward(cache["xn2"], gg, lw["gate"], *_lora(lw, "gate"), s)
    gx_u, gA_u, gB_u = proj_backward(cache["xn2"], gu, lw["up"], *_lora(lw, "up"), s)
    grm = rmsnorm_backward(cache["resid_mid"], gx_g + gx_u, lw["post_ln"], eps) + gout
    return grm, {"gateA": gA_g, "gateB": gB_g, "upA": gA_u, "upB": gB_u,
                 "downA": gA_d, "downB": gB_d}


def layer_backward(gout, cache, lw, s, cos, sin, seq_lens, b_start, dims, eps, qk_norm=False):
    """llama3.py:149-219 / qwen3.py:147-204 (+ FFN LoRA). Returns (grad_x, grads)."""
    Hq, Hkv, Hd = dims
    n = gout.shape[0]
    grm, grads = ffn_backward(gout, cache, lw, s, eps)
    gctx, grads["oA"], grads["oB"] = proj_backward(cache["ctx"], grm, lw["o"],
                                                   *_lora(lw, "o"), s)
    gqh, gkh, gvh = attn_backward(cache["qh"], cache["kh"], cache["vh"], gctx,
                                  seq_lens, b_start, Hq, Hkv)
    gq = rope_backward(gqh, cos, sin)
    gk = rope_backward(gkh, cos, sin)
    if qk_norm:
        gq = rmsnorm_backward(cache["q_pre"], gq, lw["q_norm"], eps)
        gk = rmsnorm_backward(cache["k_pre"], gk, lw["k_norm"], eps)
    xn1 = cache["xn1"]
    gx_q, grads["qA"], grads["qB"] = proj_backward(xn1, gq.reshape(n, Hq * Hd), lw["q"],
                                                   *_lora(lw, "q"), s)
    gx_k, grads["kA"], grads["kB"] = proj_backward(xn1, gk.reshape(n, Hkv * Hd), lw["k"],
                                                   *_lora(lw, "k"), s)
    gx_v, grads["vA"], grads["vB"] = proj_backward(xn1, gvh.reshape(n, Hkv * Hd), lw["v"],
                                                   *_lora(lw, "v"), s)
    gx = rmsnorm_backward(cache["x"], gx_q + gx_k + gx_v, lw["in_ln"], eps) + grm
    return gx, {k: v for k, v in grads.items() if v is not None}


# --------------------------------------------------------------------------- #
# common/head.py
# --------------------------------------------------------------------------- #

def head_backward(final_in, lm_w, norm_w, eps, ids, seq_lens):
    """head.py:42-100 — (loss, n_valid, grad_final_in)."""
    b_start, _, rows, tgt, n_valid = pack(seq_lens)
    n = final_in.shape[0]
    if n_valid == 0:
        return 0.0, 0, torch.zeros_like(final_in)
    dev = final_in.device
    rows = torch.as_tensor(rows, dtype=torch.long, device=dev)
    tgt = torch.as_tensor(tgt, dtype=torch.long, device=dev)
    normed = rmsnorm(final_in, norm_w, eps)
    h = normed[rows]
    t = ids.to(dev)[tgt].long()
    logits = h @ lm_w.t()
    loss = F.cross_entropy(logits, t, reduction="sum")
    p = torch.softmax(logits, dim=-1)
    del logits
    p[torch.arange(n_valid, device=dev), t] -= 1.0
    p /= n_valid
    gn = torch.zeros(n, final_in.shape[1], dtype=final_in.dtype, device=dev)
    gn[rows] = p @ lm_w
    return float(loss.item() / n_valid), n_valid, rmsnorm_backward(final_in, gn, norm_w, eps)


# --------------------------------------------------------------------------- #
# Optimizer: trainer.py:252-256, :624-636, :668 (torch AdamW + clip_grad_norm_)
# --------------------------------------------------------------------------- #

def clip_(grads, max_norm=1.0):
    """clip_grad_norm_ semantics (tp.py:249-258): scale in place, return the norm."""
    total = torch.sqrt(sum((g.double() ** 2).sum() for g in grads)).float()
    coef = torch.clamp(max_norm / (total + 1e-6), max=1.0)
    for g in grads:
        g.mul_(coef)
    return total


def adamw_(w, g, m, v, step, lr, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.0):
    """Decoupled-weight-decay Adam (torch.optim.AdamW), in place on w, m, v."""
    w.mul_(1 - lr * wd)
    m.mul_(beta1).add_(g, alpha=1 - beta1)
    v.mul_(beta2).addcmul_(g, g, value=1 - beta2)
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    denom = v.sqrt() / math.sqrt(bc2) + eps
    w.addcdiv_(m, denom, value=-lr / bc1)


# --------------------------------------------------------------------------- #
# The cycle: trainer.py:503-678
# --------------------------------------------------------------------------- #

@dataclass
class Model:
    meta: dict
    layers: list
    lm_w: torch.Tensor
    norm_w: torch.Tensor
    embed: torch.Tensor
    opt_state: dict = field(default_factory=dict)

    @property
    def dims(self):
        m = self.meta
        return (m["num_attention_heads"], m["num_key_value_heads"], m["head_dim"])

    @property
    def qk_norm(self):
        return self.meta.get("family", "llama3") == "qwen3"


def forward_capture(model: Model, ids, seq_lens, save_gate_up=False, save_attn_qkv=False,
                    save_attn_ctx=False, save_resid_mid=False):
    """Full forward → the activation dict process_backward consumes
    (tests/bwd_harness.py:242-258): layer_in[i], final_in, concat_input_ids,
    and with ``save_gate_up`` the per-layer gate‖up projection outputs of the
    ``mlp_gate_up`` save point (accumulate.py:134-135, :174). The other save
    points (accumulate.py:213-235): ``attn_qh/kh/vh`` flat [n, q|kv] — q/k
    after RoPE for Llama-3 (the attention call's inputs), before the q/k-norm
    for Qwen3 (``Family.saved_qkv_pre_transform``, family.py:75-84) —,
    ``attn_ctx`` [n, q] and ``resid_mid`` [n, D]."""
    m = model.meta
    b_start, positions, *_ = pack(seq_lens)
    dev = model.embed.device
    cos, sin = rope_cos_sin(positions, m["head_dim"], m["rope_theta"], m.get("rope_scaling"),
                            device=dev)
    s, eps = m["lora_scaling"], m["rms_norm_eps"]
    x = model.embed[ids.to(dev).long()]
    n = x.shape[0]
    saved = {k: [] for k in ("mlp_gate_up", "attn_qh", "attn_kh", "attn_vh", "attn_ctx",
                             "resid_mid")}
    layer_in = []
    for lw in model.layers:
        layer_in.append(x)
        c = layer_forward(x, lw, s, cos, sin, seq_lens, b_start, model.dims, eps, model.qk_norm)
        saved["mlp_gate_up"].append(torch.cat([c["gate"], c["up"]], dim=1))
        q, k = (c["q_pre"], c["k_pre"]) if model.qk_norm else (c["qh"], c["kh"])
        saved["attn_qh"].append(q.reshape(n, -1))
        saved["attn_kh"].append(k.reshape(n, -1))
        saved["attn_vh"].append(c["vh"].reshape(n, -1))
        saved["attn_ctx"].append(c["ctx"])
        saved["resid_mid"].append(c["resid_mid"])
        x = layer_output(c, lw, s)
    out = {"layer_in": layer_in, "final_in": x, "concat_input_ids": ids}
    keep = {"mlp_gate_up": save_gate_up, "attn_qh": save_attn_qkv, "attn_kh": save_attn_qkv,
            "attn_vh": save_attn_qkv, "attn_ctx": save_attn_ctx, "resid_mid": save_resid_mid}
    out.update({k: v for k, v in saved.items() if keep[k]})
    return out


def process_backward(model: Model, activations, seq_lens, n, lr, step, clip=True,
                     update=True, max_norm=1.0):
    """trainer.py:503-678: head → reversed layer loop → per-layer clip → AdamW.

    Returns ``(loss, n_valid, grads)`` with grads[i][key] the clipped fp32
    gradient of layer i's LoRA factor ``key`` (``qA``, ``qB``, …). When
    ``update`` the masters in ``model.layers`` are stepped in place."""
    m = model.meta
    seq_lens = [int(x) for x in seq_lens]
    b_start, positions, *_ = pack(seq_lens)
    dev = activations["final_in"].device
    cos, sin = rope_cos_sin(positions, m["head_dim"], m["rope_theta"], m.get("rope_scaling"),
                            device=dev)
    s, eps = m["lora_scaling"], m["rms_norm_eps"]
    ids = activations["concat_input_ids"][:n]
    saved_gu = activations.get("mlp_gate_up")
    # the optional save points, gated as the trainer gates them
    # (trainer.py:160-177, :532-552): q/k/v and resid_mid only when the meta
    # says the worker saves them, the context whenever it is there
    qkv_on = bool(m.get("save_attn_qkv")) and all(
        activations.get(k) is not None for k in ("attn_qh", "attn_kh", "attn_vh"))
    ctx_all = activations.get("attn_ctx")
    rm_all = activations.get("resid_mid") if m.get("save_resid_mid") else None
    loss, n_valid, g = head_backward(activations["final_in"][:n].float(), model.lm_w,
                                     model.norm_w, eps, ids, seq_lens)
    grads = [None] * len(model.layers)
    for i in reversed(range(len(model.layers))):
        lw = model.layers[i]
        x = activations["layer_in"][i][:n].float()
        gu = None if saved_gu is None else saved_gu[i][:n].float()
        sq = None
        if qkv_on:
            sq = tuple(activations[k][i][:n].float() for k in ("attn_qh", "attn_kh", "attn_vh"))
        c = layer_forward(x, lw, s, cos, sin, seq_lens, b_start, model.dims, eps, model.qk_norm,
                          saved_gate_up=gu, saved_qkv=sq,
                          saved_ctx=None if ctx_all is None else ctx_all[i][:n].float(),
                          saved_resid_mid=None if rm_all is None else rm_all[i][:n].float())
        g, gr = layer_backward(g, c, lw, s, cos, sin, seq_lens, b_start, model.dims, eps,
                               model.qk_norm)
        if clip and gr:
            clip_([gr[k] for k in sorted(gr)], max_norm)
        grads[i] = gr
    if update:
        wd = float(m.get("weight_decay", 0.0))
        for i, lw in enumerate(model.layers):
            for key, gk in grads[i].items():
                st = model.opt_state.setdefault((i, key), (torch.zeros_like(gk),
                                                           torch.zeros_like(gk)))
                adamw_(lw[key], gk, st[0], st[1], step, lr, wd=wd)
    return loss, n_valid, grads


# --------------------------------------------------------------------------- #
# Synthetic models (seeded per tensor name; BASELINE configs' init rules)
# --------------------------------------------------------------------------- #

def _gen(seed, name, device="cpu"):
    g = torch.Generator(device=device)
    g.manual_seed((hash_name(name) + 1000003 * int(seed)) % (2 ** 63 - 1))
    return g


def hash_name(name: str) -> int:
    """Stable 64-bit FNV-1a of a tensor name (Python's hash() is salted)."""
    h = 0xcbf29ce484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001b3) % (1 << 64)
    return h


def make_model(meta: dict, seed: int = 0, projs=PROJS, w_std=0.02, b_std=0.01,
               norm_jitter=0.0, bf16_round=True, device="cpu") -> Model:
    """Random-init model of the given dims: linear weights N(0, w_std), norms 1
    (+ optional |N(0, jitter)|), LoRA A kaiming-uniform(a=√5) = U(±1/√in),
    B N(0, b_std). ``bf16_round`` rounds frozen weights to bf16 values (what
    the GPU sees), so the fp32 oracle and the bf16 path share inputs.
    ``device`` is where the tensors are drawn (each device's generator gives
    its own seeded values) and kept."""
    D, Hq, Hkv, Hd = meta["hidden_size"], meta["num_attention_heads"], \
        meta["num_key_value_heads"], meta["head_dim"]
    I, V, r, L = meta["intermediate_size"], meta["vocab_size"], meta["lora_rank"], \
        meta["num_hidden_layers"]
    q, kv = Hq * Hd, Hkv * Hd

    def rnd(name, *shape, std):
        t = torch.randn(*shape, generator=_gen(seed, name, device), device=device) * std
        return t.to(torch.bfloat16).float() if bf16_round else t

    def norm(name, n):
        t = torch.ones(n, device=device)
        if norm_jitter:
            t = t + torch.randn(n, generator=_gen(seed, name, device), device=device).abs() \
                * norm_jitter
        return t.to(torch.bfloat16).float() if bf16_round else t

    shapes = {"q": (q, D), "k": (kv, D), "v": (kv, D), "o": (D, q),
              "gate": (I, D), "up": (I, D), "down": (D, I)}
    layers = []
    for i in range(L):
        p = f"layers.{i}."
        lw = {k: rnd(p + k, *sh, std=w_std) for k, sh in shapes.items()}
        lw["in_ln"] = norm(p + "in_ln", D)
        lw["post_ln"] = norm(p + "post_ln", D)
        if meta.get("family") == "qwen3":
            lw["q_norm"] = norm(p + "q_norm", Hd)
            lw["k_norm"] = norm(p + "k_norm", Hd)
        for pr in projs:
            out, inp = shapes[pr]
            bound = 1.0 / math.sqrt(inp)
            lw[pr + "A"] = (torch.rand(r, inp, generator=_gen(seed, p + pr + "A", device),
                                       device=device) * 2 - 1) * bound
            lw[pr + "B"] = torch.randn(out, r, generator=_gen(seed, p + pr + "B", device),
                                       device=device) * b_std
        layers.append(lw)
    embed = rnd("embed", V, D, std=w_std)
    lm_w = embed if meta.get("tie_word_embeddings") else rnd("lm_head", V, D, std=w_std)
    return Model(meta=dict(meta), layers=layers, lm_w=lm_w, norm_w=norm("norm", D),
                 embed=embed)
