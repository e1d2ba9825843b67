"""Torch-tensor front end of libdsb's single-op entry points.

Each function mirrors one op of the reference's ``bwd_services/common``
modules (cited per function; paths under ``deltaserve-plugin/deltaserve/``)
and runs the HIP kernel on the current torch stream. Inputs are bf16 CUDA
tensors with a contiguous last dimension (row strides are passed through);
nothing here falls back to a PyTorch implementation.
"""

from __future__ import annotations

import ctypes
from ctypes import byref, c_float, c_int, c_int32, c_void_p

import torch

from . import _lib as L

BF16 = torch.bfloat16


def _stream():
    return c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return None if t is None else c_void_p(t.data_ptr())


def _ld(t):
    assert t.stride(-1) == 1, "last dimension must be contiguous"
    return t.stride(0) if t.dim() > 1 else t.shape[0]


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("deltaserve_amd ops take CUDA (HIP) tensors")


# ---------------------------------------------------------------- integer packing

def pack(seq_lens):
    """trainer.py:510-518, head.py:63-72 via libdsb: (positions, pred, n_valid)."""
    lib = L.load()
    n = int(sum(int(s) for s in seq_lens))
    arr = L.i32_array(seq_lens)
    pos = (c_int32 * max(n, 1))()
    pred = (c_int32 * max(n, 1))()
    nv = lib.dsb_pack(arr, len(seq_lens), n, pos, pred)
    if nv < 0:
        raise ValueError("seq_lens must be non-negative")
    return list(pos)[:n], list(pred)[:n], nv


def rope_inv_freq(head_dim, theta, rope_scaling=None):
    """ops.py:26-57 via libdsb (host), as a CPU float32 tensor."""
    lib = L.load()
    rs = rope_scaling or {}
    rtype = rs.get("rope_type", "default") or "default"
    code = {"default": L.ROPE_DEFAULT, "linear": L.ROPE_LINEAR, "llama3": L.ROPE_LLAMA3}.get(rtype)
    if code is None:
        raise NotImplementedError(f"RoPE type {rtype!r} is not supported")
    out = (c_float * (head_dim // 2))()
    L.check(lib.dsb_rope_inv_freq(head_dim, float(theta), code, float(rs.get("factor", 1.0)),
                                  float(rs.get("low_freq_factor", 1.0)),
                                  float(rs.get("high_freq_factor", 1.0)),
                                  float(rs.get("original_max_position_embeddings", 1.0)), out))
    return torch.tensor(list(out), dtype=torch.float32)


# ---------------------------------------------------------------- dense products

def gemm_nt(A, B, A2=None, B2=None, out_dtype=BF16, R=None, out=None, accumulate=False, cfg=-1,
            b_kn=False):
    """C = A·Bᵀ (+ A2·B2ᵀ) (+ R) — the projection products of ops.py:103-146.
    b_kn: B [K1, N] and B2 [K2, N] (C = A·B + A2·B2, the backward's dY·W with W
    in its own layout)."""
    _dev(A, B, A2, B2, R)
    M, K1 = A.shape
    N = B.shape[1] if b_kn else B.shape[0]
    K2 = 0 if A2 is None else A2.shape[1]
    f32 = out_dtype == torch.float32
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype, device=A.device)
    L.check(L.load().dsb_op_gemm(_p(A), _ld(A), _p(B), _ld(B), _p(A2), 0 if A2 is None else _ld(A2),
                                 _p(B2), 0 if B2 is None else _ld(B2), M, N, K1, K2, _p(out),
                                 _ld(out), int(f32), int(accumulate), _p(R),
                                 0 if R is None else _ld(R), int(bool(b_kn)), int(cfg),
                                 _stream()),
            what="dsb_op_gemm")
    return out


def gemm_glu(A, B, A2=None, B2=None, with_h=True):
    """Gate‖up product with the SwiGLU forward fused (ffn.py:25-26, silu as
    ffn.py:40-41): returns (GU [M, 2I] = bf16(A·Bᵀ (+ A2·B2ᵀ)) with B = gate
    rows then up rows, H [M, I] = bf16(silu(gate)·up) or None)."""
    _dev(A, B, A2, B2)
    M, K1 = A.shape
    I = B.shape[0] // 2
    K2 = 0 if A2 is None else A2.shape[1]
    GU = torch.empty(M, 2 * I, dtype=BF16, device=A.device)
    H = torch.empty(M, I, dtype=BF16, device=A.device) if with_h else None
    L.check(L.load().dsb_op_gemm_glu(_p(A), _ld(A), _p(B), _ld(B), _p(A2),
                                     0 if A2 is None else _ld(A2), _p(B2),
                                     0 if B2 is None else _ld(B2), M, I, K1, K2, _p(GU), _ld(GU),
                                     _p(H), 0 if H is None else _ld(H), _stream()),
            what="dsb_op_gemm_glu")
    return GU, H


# ---------------------------------------------------------------- norms / rope

def rmsnorm(x, w, eps):
    """ops.py:84-88 (bf16 in/out, fp32 internals)."""
    _dev(x, w)
    y = torch.empty(x.shape, dtype=BF16, device=x.device)
    L.check(L.load().dsb_op_rmsnorm(_p(x), _ld(x), _p(w), _p(y), _ld(y), x.shape[0], x.shape[1],
                                    float(eps), _stream()), what="dsb_op_rmsnorm")
    return y


def rmsnorm_backward(x, g, w, eps, resid=None):
    """ops.py:91-100 (+ bf16 residual add, llama3.py:205); bf16 out."""
    _dev(x, g, w, resid)
    out = torch.empty(x.shape, dtype=BF16, device=x.device)
    L.check(L.load().dsb_op_rmsnorm_bwd(_p(x), _ld(x), _p(g), int(g.dtype == torch.float32),
                                        _ld(g), _p(w), _p(resid), 0 if resid is None else _ld(resid),
                                        _p(out), _ld(out), x.shape[0], x.shape[1], float(eps),
                                        _stream()), what="dsb_op_rmsnorm_bwd")
    return out


def rope_cos_sin(positions, inv_freq):
    """ops.py:60-65: cos, sin [n, Hd/2] fp32 from int32 positions (CUDA)."""
    _dev(positions, inv_freq)
    n, half = positions.shape[0], inv_freq.shape[0]
    c = torch.empty(n, half, dtype=torch.float32, device=positions.device)
    s = torch.empty_like(c)
    L.check(L.load().dsb_op_rope_table(_p(positions), n, _p(inv_freq), half, _p(c), _p(s),
                                       _stream()), what="dsb_op_rope_table")
    return c, s


def apply_rope(qkv_pre, Hq, Hkv, cos, sin, q_norm=None, k_norm=None, eps=1e-6):
    """ops.py:68-73 (+ qwen3.py:96-107): rotated [q | k] of a [n, q+2kv] row block
    (head_dim = 2·cos.shape[1]: 128 or 64)."""
    _dev(qkv_pre, cos, sin)
    n, hd = qkv_pre.shape[0], 2 * cos.shape[1]
    out = torch.empty(n, (Hq + Hkv) * hd, dtype=BF16, device=qkv_pre.device)
    L.check(L.load().dsb_op_rope(_p(qkv_pre), _ld(qkv_pre), _p(out), _ld(out), _p(cos), _p(sin),
                                 n, Hq, Hkv, hd, _p(q_norm), _p(k_norm), float(eps), _stream()),
            what="dsb_op_rope")
    return out


def rope_backward_(g, qkv_pre, Hq, Hkv, cos, sin, q_norm=None, k_norm=None, eps=1e-6):
    """ops.py:76-81 (+ qwen3.py:133-144), in place on g's [q | k] columns."""
    _dev(g, qkv_pre, cos, sin)
    L.check(L.load().dsb_op_rope_bwd(_p(g), _ld(g), _p(qkv_pre), _ld(qkv_pre), _p(cos), _p(sin),
                                     g.shape[0], Hq, Hkv, 2 * cos.shape[1], _p(q_norm),
                                     _p(k_norm), float(eps), _stream()), what="dsb_op_rope_bwd")
    return g


# ---------------------------------------------------------------- attention

def attn_forward(q, k, v, seq_lens, Hq, Hkv, head_dim=None):
    """attention.py:20-45 over packed rows: (ctx bf16, o32 fp32, lse [Hq, n] log2);
    head_dim (128 or 64) defaults to q's width over Hq."""
    _dev(q, k, v)
    n = q.shape[0]
    hd = head_dim or q.shape[1] // Hq
    ctx = torch.empty(n, Hq * hd, dtype=BF16, device=q.device)
    o32 = torch.empty(n, Hq * hd, dtype=torch.float32, device=q.device)
    lse = torch.empty(Hq, max(n, 1), dtype=torch.float32, device=q.device)
    L.check(L.load().dsb_op_attn_fwd(_p(q), _ld(q), _p(k), _ld(k), _p(v), _ld(v), _p(ctx),
                                     _ld(ctx), _p(o32), _p(lse), L.i32_array(seq_lens),
                                     len(seq_lens), Hq, Hkv, hd, _stream()),
            what="dsb_op_attn_fwd")
    return ctx, o32, lse


def attn_backward(q, k, v, o32, lse, dout, seq_lens, Hq, Hkv, head_dim=None):
    """attention.py:48-112: (dq, dk, dv) bf16 in [n, H*head_dim]."""
    _dev(q, k, v, o32, lse, dout)
    n = q.shape[0]
    hd = head_dim or q.shape[1] // Hq
    dq = torch.empty(n, Hq * hd, dtype=BF16, device=q.device)
    dk = torch.empty(n, Hkv * hd, dtype=BF16, device=q.device)
    dv = torch.empty(n, Hkv * hd, dtype=BF16, device=q.device)
    L.check(L.load().dsb_op_attn_bwd(_p(q), _ld(q), _p(k), _ld(k), _p(v), _ld(v), _p(o32),
                                     _p(lse), _p(dout), _ld(dout), _p(dq), _ld(dq), _p(dk),
                                     _ld(dk), _p(dv), _ld(dv), L.i32_array(seq_lens),
                                     len(seq_lens), Hq, Hkv, hd, _stream()),
            what="dsb_op_attn_bwd")
    return dq, dk, dv


# ---------------------------------------------------------------- head

def head_backward(normed, lm_w, ids, seq_lens, vocab_chunk=0):
    """head.py:42-100 from the normed rows: (loss, n_valid, dH fp32 [n, D]),
    streaming the vocabulary in chunks of ``vocab_chunk`` columns (0: 16384)."""
    _dev(normed, lm_w, ids)
    n, D = normed.shape
    V = lm_w.shape[0]
    dH = torch.empty(n, D, dtype=torch.float32, device=normed.device)
    loss = c_float(0.0)
    nv = c_int(0)
    L.check(L.load().dsb_op_head(_p(normed), _ld(normed), _p(lm_w), _p(ids), L.i32_array(seq_lens),
                                 len(seq_lens), n, D, V, int(vocab_chunk), _p(dH), byref(loss),
                                 byref(nv), _stream()),
            what="dsb_op_head")
    return loss.value, nv.value, dH


# ---------------------------------------------------------------- LoRA grads / optimizer

def lora_tn(P, X, rg, transpose_out, outs, scale=1.0):
    """ops.py:143-144: scale · Pᵀ·X over rows (grad_A, or grad_B when
    transpose_out); P bf16 [n, R]."""
    _dev(P, X, *outs)
    n, R = P.shape
    C = X.shape[1]
    o = list(outs) + [None] * (3 - len(outs))
    L.check(L.load().dsb_op_lora_tn(_p(P), _ld(P), _p(X), _ld(X), n, R, C, float(scale), _p(o[0]),
                                    _p(o[1]), _p(o[2]), rg, int(transpose_out), _stream()),
            what="dsb_op_lora_tn")
    return outs


def lora_skinny(X, B):
    """ops.py:141-142: bf16(X·Bᵀ) for a rank-r factor B [R, K]."""
    _dev(X, B)
    n, K = X.shape
    R = B.shape[0]
    Z = torch.empty(n, R, dtype=BF16, device=X.device)
    L.check(L.load().dsb_op_lora_skinny(_p(X), _ld(X), _p(B), _ld(B), n, R, K, _p(Z), _ld(Z),
                                        _stream()), what="dsb_op_lora_skinny")
    return Z


def _dual_passes(passes):
    arr = (L.DsbDualPass * len(passes))()
    for i, (G, Z, BT, gZ, gB, scale, tr) in enumerate(passes):
        _dev(G, Z, BT, gZ, gB)
        arr[i] = L.DsbDualPass(G.data_ptr(), _ld(G), Z.data_ptr(), _ld(Z), BT.data_ptr(), _ld(BT),
                               G.shape[1], float(scale), gZ.data_ptr(), _ld(gZ), gB.data_ptr(),
                               int(tr))
    return arr


def lora_dual_batch(passes, n, n_alloc=None, entry="dsb_op_lora_dual"):
    """One launch over 1-3 passes ``(G, Z, BT, gZ_out, gB_out, scale,
    transpose_out)`` of the same rank over the first ``n`` rows (the row
    count read from device memory, partials laid out for ``n_alloc``): per
    pass gZ_out[:n] = bf16(G·BTᵀ) and gB_out = scale·Gᵀ·Z (ops.py:142, :144)."""
    r = passes[0][2].shape[0]
    arr = _dual_passes(passes)
    L.check(getattr(L.load(), entry)(arr, len(passes), int(n), int(n_alloc or n), int(r),
                                     _stream()), what=entry)


def lora_dual(G, Z, BT, scale=1.0, transpose_out=True):
    """ops.py:142 and :144 from one pass over G [n, C]: returns
    (bf16(G·BTᵀ) [n, r], scale·Gᵀ·Z fp32 [C, r] (or [r, C])) for BT = (s·B)ᵀ
    [r, C]; with G = xin, BT = A, Z = grad_Z it gives Z and grad_A."""
    n, C = G.shape
    r = BT.shape[0]
    gZ = torch.empty(n, r, dtype=BF16, device=G.device)
    shape = (C, r) if transpose_out else (r, C)
    gB = torch.empty(*shape, dtype=torch.float32, device=G.device)
    lora_dual_batch([(G, Z, BT, gZ, gB, scale, transpose_out)], n)
    return gZ, gB


def clip_adamw_(ws, gs, ms, vs, groups, lr, step, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.0,
                max_norm=1.0, clip=True):
    """trainer.py:624-636 + :668 over fp32 CUDA tensors (in place)."""
    _dev(*ws, *gs, *ms, *vs)
    k = len(ws)
    arr = lambda ts: (c_void_p * k)(*[t.data_ptr() for t in ts])  # noqa: E731
    L.check(L.load().dsb_op_clip_adamw(arr(ws), arr(gs), arr(ms), arr(vs),
                                       L.i32_array([t.numel() for t in ws]), L.i32_array(groups),
                                       k, max(groups) + 1, float(lr), float(beta1), float(beta2),
                                       float(eps), float(wd), int(step), float(max_norm),
                                       int(clip), _stream()), what="dsb_op_clip_adamw")
