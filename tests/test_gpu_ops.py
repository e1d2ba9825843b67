"""Per-kernel parity of libdsb's HIP kernels against the CPU oracle.

Every case calls the C-ABI single-op entry points (deltaserve_amd.ops) on a
seeded input and compares with the oracle's restatement of the reference op
(oracle/dsb_oracle.py) on the same bf16-valued inputs in fp32. Tolerances are
stated per test: fp32 outputs ~1e-4 relative (summation order), bf16 outputs
a few bf16 ulps (2^-8 relative), attention/head outputs that pass P or dS
through bf16 MFMA operands 2e-2 max-relative.
"""

import math

import pytest
import torch

from harness import O, cosine, max_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _bf(t):
    return t.to(torch.bfloat16)


def _rnd(*shape, seed=0, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * std


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from deltaserve_amd import _lib as L
    L.load()


def _b_operand(B, kn):
    """B as the product reads it: [N, K], or the [K, N] layout of a weight
    read in place by the backward (b_kn)."""
    if B is None:
        return None
    return (B.t().contiguous() if kn else B).to(DEV)


@pytest.mark.parametrize("kn", [False, True])
@pytest.mark.parametrize("cfg", [0, 1, 2, -2])
@pytest.mark.parametrize("M,N,K,K2", [(300, 520, 264, 24), (64, 64, 64, 0), (513, 260, 1024, 16),
                                      (1, 8, 8, 8), (513, 264, 1024, 16), (200, 1024, 4096, 64),
                                      (1, 8, 512, 8)])
def test_gemm_nt(cfg, M, N, K, K2, kn):
    """cfg -2 splits K (the last three shapes: 4, 8 and 2 K slices, the
    slices crossing into the second K segment) and sums the fp32 partials.
    kn: B and B2 stored [K, N] (N a multiple of 8 there)."""
    from deltaserve_amd import ops
    if kn and N % 8:
        pytest.skip("a [K, N] B needs N a multiple of 8 (test_gemm_kn_refuses_ragged_n)")
    A = _bf(_rnd(M, K, seed=1))
    B = _bf(_rnd(N, K, seed=2))
    A2 = _bf(_rnd(M, K2, seed=3)) if K2 else None
    B2 = _bf(_rnd(N, K2, seed=4)) if K2 else None
    ref = A.float() @ B.float().t()
    if K2:
        ref += A2.float() @ B2.float().t()
    dA, dA2 = A.to(DEV), None if A2 is None else A2.to(DEV)
    dB, dB2 = _b_operand(B, kn), _b_operand(B2, kn)
    c32 = ops.gemm_nt(dA, dB, dA2, dB2, out_dtype=torch.float32, cfg=cfg, b_kn=kn)
    assert max_rel(c32, ref) < 1e-5
    R = _bf(_rnd(M, N, seed=5))
    c16 = ops.gemm_nt(dA, dB, dA2, dB2, R=R.to(DEV), cfg=cfg, b_kn=kn)
    assert max_rel(c16, ref + R.float()) < 8e-3
    # accumulate into an fp32 output
    acc = c32.clone()
    ops.gemm_nt(dA, dB, out_dtype=torch.float32, out=acc, accumulate=True, cfg=cfg, b_kn=kn)
    assert max_rel(acc, ref + A.float() @ B.float().t()) < 1e-5


@pytest.mark.parametrize("M,N,K,K2", [(8192, 4096, 4096, 48), (8100, 1024, 4104, 16),
                                      (300, 5000, 14336, 16)])
def test_gemm_kn_equals_nt(M, N, K, K2):
    """The [K, N] operand path gives the [N, K] path's product bit for bit:
    the same MFMA fragments in the same order, only the B staging differs
    (cycle-sized shapes: 256-wide tiles with ragged M and K, a LoRA segment,
    N not a multiple of the tile)."""
    from deltaserve_amd import ops
    A = _bf(_rnd(M, K, seed=21)).to(DEV)
    B = _bf(_rnd(N, K, seed=22))
    A2 = _bf(_rnd(M, K2, seed=23)).to(DEV)
    B2 = _bf(_rnd(N, K2, seed=24))
    nt = ops.gemm_nt(A, B.to(DEV), A2, B2.to(DEV), out_dtype=torch.float32)
    kn = ops.gemm_nt(A, _b_operand(B, True), A2, _b_operand(B2, True), out_dtype=torch.float32,
                     b_kn=True)
    assert torch.equal(nt, kn)


def test_gemm_kn_refuses_ragged_n():
    from deltaserve_amd import _lib as L
    from deltaserve_amd import ops
    A = torch.zeros(16, 64, dtype=torch.bfloat16, device=DEV)
    B = torch.zeros(64, 264, dtype=torch.bfloat16, device=DEV)[:, :260]  # N = 260, ld 264
    with pytest.raises(L.DsbError, match="multiple of 8"):
        ops.gemm_nt(A, B, b_kn=True)


@pytest.mark.parametrize("kn", [False, True])
@pytest.mark.parametrize("M,N,K,K2", [(4352, 4104, 2048, 0), (4400, 3840, 2048, 64)])
def test_gemm_nt_tail_split(M, N, K, K2, kn):
    """cfg -3: the tiles past the last full round of the CUs (289 tiles: 33
    of them; 270 tiles: 14, with a ragged last row block and the LoRA K
    segment in the second slice) split K in two and reduce their tile
    partials, as the cycle does for products whose tiles leave a partly
    filled last round."""
    from deltaserve_amd import ops
    A = _bf(_rnd(M, K, seed=11))
    B = _bf(_rnd(N, K, seed=12))
    A2 = _bf(_rnd(M, K2, seed=13)) if K2 else None
    B2 = _bf(_rnd(N, K2, seed=14)) if K2 else None
    ref = A.float() @ B.float().t()
    if K2:
        ref += A2.float() @ B2.float().t()
    dA, dB = A.to(DEV), _b_operand(B, kn)
    dA2 = None if A2 is None else A2.to(DEV)
    dB2 = _b_operand(B2, kn)
    c32 = ops.gemm_nt(dA, dB, dA2, dB2, out_dtype=torch.float32, cfg=-3, b_kn=kn)
    assert max_rel(c32, ref) < 1e-5
    # the plain launch gives the same product
    c32p = ops.gemm_nt(dA, dB, dA2, dB2, out_dtype=torch.float32, cfg=0, b_kn=kn)
    assert max_rel(c32, c32p.cpu()) < 1e-5
    R = _bf(_rnd(M, N, seed=15))
    c16 = ops.gemm_nt(dA, dB, dA2, dB2, R=R.to(DEV), cfg=-3, b_kn=kn)
    assert max_rel(c16, ref + R.float()) < 8e-3
    acc = c32.clone()
    ops.gemm_nt(dA, dB, out_dtype=torch.float32, out=acc, accumulate=True, cfg=-3, b_kn=kn)
    assert max_rel(acc, ref + A.float() @ B.float().t()) < 1e-5


def test_gemm_strided_views():
    """Row strides and column offsets (the fused qkv / gate_up slices)."""
    from deltaserve_amd import ops
    big = _bf(_rnd(200, 96, seed=7)).to(DEV)
    A = big[:, 32:96]          # ld 96
    B = _bf(_rnd(40, 64, seed=8)).to(DEV)
    out = ops.gemm_nt(A, B, out_dtype=torch.float32)
    assert max_rel(out, A.float().cpu() @ B.float().cpu().t()) < 1e-5


@pytest.mark.parametrize("M,I,K,K2", [(700, 512, 256, 16), (8192, 1536, 512, 32),
                                      (333, 192, 128, 0), (64, 128, 1024, 48),
                                      (200, 8192, 256, 16)])
def test_gemm_glu(M, I, K, K2):
    """Gate‖up with the SwiGLU forward in the epilogue (256- and 128-wide tiles;
    the last shape is one row block with 64 column tiles, which takes the
    256-wide tile as serving-size cycles do): GU against an fp32 product, H
    exactly silu(gate)·up of the returned halves."""
    from deltaserve_amd import ops
    A = _bf(_rnd(M, K, seed=21))
    B = _bf(_rnd(2 * I, K, seed=22))
    A2 = _bf(_rnd(M, K2, seed=23)) if K2 else None
    B2 = _bf(_rnd(2 * I, K2, seed=24)) if K2 else None
    ref = A.float() @ B.float().t()
    if K2:
        ref += A2.float() @ B2.float().t()
    GU, H = ops.gemm_glu(A.to(DEV), B.to(DEV), None if A2 is None else A2.to(DEV),
                         None if B2 is None else B2.to(DEV))
    assert max_rel(GU, ref) < 8e-3
    g, u = GU[:, :I].float(), GU[:, I:].float()
    want = (g * torch.sigmoid(g) * u).to(torch.bfloat16)
    assert max_rel(H, want) < 8e-3
    # bf16 rounding of the same fp32 value: at most one ulp apart
    assert ((H.float() - want.float()).abs() <= want.float().abs() * 2 ** -7 + 1e-30).all()
    GU2, H2 = ops.gemm_glu(A.to(DEV), B.to(DEV), None if A2 is None else A2.to(DEV),
                           None if B2 is None else B2.to(DEV), with_h=False)
    assert H2 is None and torch.equal(GU2, GU)


def test_rmsnorm_fwd_bwd():
    from deltaserve_amd import ops
    x = _bf(_rnd(77, 1024, seed=11) * 3)
    w = _bf(1 + _rnd(1024, seed=12).abs() * 0.1)
    g32 = _rnd(77, 1024, seed=13)
    r = _bf(_rnd(77, 1024, seed=14))
    eps = 1e-5
    y = ops.rmsnorm(x.to(DEV), w.to(DEV), eps)
    assert max_rel(y, O.rmsnorm(x.float(), w.float(), eps)) < 8e-3
    dx = ops.rmsnorm_backward(x.to(DEV), g32.to(DEV), w.to(DEV), eps, resid=r.to(DEV))
    ref = O.rmsnorm_backward(x.float(), g32, w.float(), eps) + r.float()
    assert max_rel(dx, ref) < 8e-3
    dxb = ops.rmsnorm_backward(x.to(DEV), _bf(g32).to(DEV), w.to(DEV), eps)
    assert max_rel(dxb, O.rmsnorm_backward(x.float(), _bf(g32).float(), w.float(), eps)) < 8e-3


@pytest.mark.parametrize("scaling", [None, {"rope_type": "llama3", "factor": 8.0,
                                            "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                            "original_max_position_embeddings": 8192.0}])
def test_rope_table(scaling):
    from deltaserve_amd import ops
    pos = torch.tensor(list(range(300)) + list(range(8000, 8192)), dtype=torch.int32)
    inv = ops.rope_inv_freq(128, 5e5, scaling)
    assert max_rel(inv, O.rope_inv_freq(128, 5e5, scaling)) < 1e-6
    c, s = ops.rope_cos_sin(pos.to(DEV), inv.to(DEV))
    rc, rs = O.rope_cos_sin(pos, 128, 5e5, scaling)
    assert (c.cpu() - rc).abs().max().item() < 2e-3
    assert (s.cpu() - rs).abs().max().item() < 2e-3


@pytest.mark.parametrize("hd", [128, 64])
@pytest.mark.parametrize("qk_norm", [False, True])
def test_rope_fwd_bwd(qk_norm, hd):
    """head_dim 64: four lanes per head, 16 heads per wave (6 heads: one
    partly filled wave per token)."""
    from deltaserve_amd import ops
    n, Hq, Hkv = 50, 4, 2
    q, kv = Hq * hd, Hkv * hd
    pre = _bf(_rnd(n, q + 2 * kv, seed=21))
    pos = torch.arange(n, dtype=torch.int32)
    cos, sin = O.rope_cos_sin(pos, hd, 1e6)
    qn = _bf(1 + _rnd(hd, seed=22).abs() * 0.2) if qk_norm else None
    kn = _bf(1 + _rnd(hd, seed=23).abs() * 0.2) if qk_norm else None
    out = ops.apply_rope(pre.to(DEV), Hq, Hkv, cos.to(DEV), sin.to(DEV),
                         None if qn is None else qn.to(DEV), None if kn is None else kn.to(DEV), 1e-6)
    qp = pre.float()[:, :q].view(n, Hq, hd)
    kp = pre.float()[:, q:q + kv].view(n, Hkv, hd)
    if qk_norm:
        qp = O.rmsnorm(qp, qn.float(), 1e-6)
        kp = O.rmsnorm(kp, kn.float(), 1e-6)
    ref = torch.cat([O.apply_rope(qp, cos, sin).reshape(n, q), O.apply_rope(kp, cos, sin).reshape(n, kv)], 1)
    assert max_rel(out, ref) < 1e-2
    g = _bf(_rnd(n, q + 2 * kv, seed=24))
    gd = g.to(DEV).clone()
    ops.rope_backward_(gd, pre.to(DEV), Hq, Hkv, cos.to(DEV), sin.to(DEV),
                       None if qn is None else qn.to(DEV), None if kn is None else kn.to(DEV), 1e-6)
    gq = O.rope_backward(g.float()[:, :q].view(n, Hq, hd), cos, sin)
    gk = O.rope_backward(g.float()[:, q:q + kv].view(n, Hkv, hd), cos, sin)
    if qk_norm:
        gq = O.rmsnorm_backward(pre.float()[:, :q].view(n, Hq, hd), gq, qn.float(), 1e-6)
        gk = O.rmsnorm_backward(pre.float()[:, q:q + kv].view(n, Hkv, hd), gk, kn.float(), 1e-6)
    assert max_rel(gd[:, :q], gq.reshape(n, q)) < 1e-2
    assert max_rel(gd[:, q:q + kv], gk.reshape(n, kv)) < 1e-2
    assert torch.equal(gd[:, q + kv:].cpu(), g[:, q + kv:])  # v columns untouched


# group sizes Hq/Hkv 1..8: forward and dQ blocks take four (32-query subtile,
# q-head) pairs of one kv head, so G = 3 and 5 mix subtiles within a block
# head_dim 64 (last three cases): heads zero-padded to 128 inside the kernels
@pytest.mark.parametrize("seq_lens,Hq,Hkv,hd", [([37, 128, 1, 200, 64], 4, 2, 128),
                                                ([300], 8, 2, 128), ([5, 129, 256], 2, 1, 128),
                                                ([1, 1, 2], 4, 4, 128),
                                                ([33, 95, 160, 1, 250], 10, 2, 128),
                                                ([70, 31, 129], 6, 2, 128), ([200, 64], 8, 1, 128),
                                                ([37, 128, 1, 200, 64], 4, 2, 64),
                                                ([300, 5], 8, 2, 64),
                                                ([33, 95, 160, 1, 250], 10, 2, 64)])
def test_attention(seq_lens, Hq, Hkv, hd):
    from deltaserve_amd import ops
    n = sum(seq_lens)
    b_start, *_ = O.pack(seq_lens)
    qh = _bf(_rnd(n, Hq, hd, seed=31))
    kh = _bf(_rnd(n, Hkv, hd, seed=32))
    vh = _bf(_rnd(n, Hkv, hd, seed=33))
    ctx, o32, lse = ops.attn_forward(qh.reshape(n, -1).to(DEV), kh.reshape(n, -1).to(DEV),
                                     vh.reshape(n, -1).to(DEV), seq_lens, Hq, Hkv)
    ref = O.attn_forward(qh.float(), kh.float(), vh.float(), seq_lens, b_start, Hq, Hkv)
    assert max_rel(o32, ref) < 1e-2
    assert cosine(o32, ref) > 0.9999
    assert max_rel(ctx, ref) < 1.5e-2
    g = _bf(_rnd(n, Hq * hd, seed=34))
    dq, dk, dv = ops.attn_backward(qh.reshape(n, -1).to(DEV), kh.reshape(n, -1).to(DEV),
                                   vh.reshape(n, -1).to(DEV), o32, lse, g.to(DEV), seq_lens, Hq, Hkv)
    rq, rk, rv = O.attn_backward(qh.float(), kh.float(), vh.float(), g.float(), seq_lens, b_start,
                                 Hq, Hkv)
    for got, want in ((dq, rq), (dk, rk), (dv, rv)):
        want = want.reshape(n, -1)
        assert max_rel(got, want) < 2e-2
        assert cosine(got, want) > 0.999


def test_attention_two_8192_token_sequences():
    """C5's packing (2 x 8192 tokens) at op level: every kernel's long-sequence
    path (128 key tiles per query block, 64 q tiles per dK/dV block) against
    the fp32 oracle run on the device (8 q-heads over 2 kv heads keep its
    [heads, 8192, 8192] score tensors at 2 GiB each)."""
    from deltaserve_amd import ops
    seq_lens, Hq, Hkv = [8192, 8192], 8, 2
    n = sum(seq_lens)
    b_start, *_ = O.pack(seq_lens)
    qh = _bf(_rnd(n, Hq, 128, seed=51)).to(DEV)
    kh = _bf(_rnd(n, Hkv, 128, seed=52)).to(DEV)
    vh = _bf(_rnd(n, Hkv, 128, seed=53)).to(DEV)
    ctx, o32, lse = ops.attn_forward(qh.reshape(n, -1), kh.reshape(n, -1), vh.reshape(n, -1),
                                     seq_lens, Hq, Hkv)
    with torch.no_grad():
        ref = O.attn_forward(qh.float(), kh.float(), vh.float(), seq_lens, b_start, Hq, Hkv)
    assert max_rel(o32, ref) < 1e-2
    assert cosine(o32, ref) > 0.9999
    g = _bf(_rnd(n, Hq * 128, seed=54)).to(DEV)
    dq, dk, dv = ops.attn_backward(qh.reshape(n, -1), kh.reshape(n, -1), vh.reshape(n, -1), o32,
                                   lse, g, seq_lens, Hq, Hkv)
    with torch.no_grad():
        rq, rk, rv = O.attn_backward(qh.float(), kh.float(), vh.float(), g.float(), seq_lens,
                                     b_start, Hq, Hkv)
    for name, got, want in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        want = want.reshape(n, -1)
        print(f"[attn 2x8192] {name}: max-rel {max_rel(got, want):.2e} cos "
              f"{cosine(got, want):.6f}", flush=True)
        assert max_rel(got, want) < 2e-2
        assert cosine(got, want) > 0.999


@pytest.mark.parametrize("V,vchunk", [(1000, 0), (211, 0), (1027, 0), (1027, 256), (5000, 768),
                                      (2304, 512)])
def test_head(V, vchunk):
    """The streamed head against fp32 logits/softmax, with the vocabulary in
    one chunk or several (including a last chunk that is not a multiple of
    256 or of 8 columns)."""
    from deltaserve_amd import ops
    seq_lens = [5, 1, 64, 300]
    n, D = sum(seq_lens), 256
    normed = _bf(_rnd(n, D, seed=41))
    W = _bf(_rnd(V, D, seed=42) * 0.05)
    ids = torch.randint(0, V, (n,), generator=torch.Generator().manual_seed(43))
    # targets in the first and last vocab columns too
    ids[1], ids[6] = 0, V - 1
    loss, nv, dH = ops.head_backward(normed.to(DEV), W.to(DEV), ids.to(DEV), seq_lens,
                                     vocab_chunk=vchunk)
    _, _, rows, tgt, n_valid = O.pack(seq_lens)
    logits = normed.float()[rows] @ W.float().t()
    ref_loss = torch.nn.functional.cross_entropy(logits, ids[tgt], reduction="sum").item() / n_valid
    p = torch.softmax(logits, -1)
    p[torch.arange(n_valid), ids[tgt]] -= 1
    p /= n_valid
    ref_dH = torch.zeros(n, D)
    ref_dH[rows] = p @ W.float()
    assert nv == n_valid
    assert abs(loss - ref_loss) / ref_loss < 1e-4
    assert max_rel(dH, ref_dH) < 1e-2
    assert cosine(dH, ref_dH) > 0.9999
    last = [sum(seq_lens[:i + 1]) - 1 for i in range(len(seq_lens))]
    assert dH[last].abs().max().item() == 0.0  # rows that predict nothing


@pytest.mark.parametrize("n,R,C", [(333, 24, 520), (8192, 16, 4096), (1000, 48, 1024), (17, 96, 256)])
def test_lora_tn(n, R, C):
    from deltaserve_amd import ops
    P = _bf(_rnd(n, R, seed=51)).to(DEV)
    X = _bf(_rnd(n, C, seed=52)).to(DEV)
    ref = P.float().cpu().t() @ X.float().cpu()
    rg = R // 3 if R % 3 == 0 else R
    ng = R // rg
    outs = [torch.empty(rg, C, device=DEV) for _ in range(ng)]
    ops.lora_tn(P, X, rg, False, outs)
    assert max_rel(torch.cat([o.cpu() for o in outs], 0), ref) < 1e-5
    outT = torch.empty(C, R, device=DEV)
    ops.lora_tn(P, X, R, True, [outT], scale=2.0)
    assert max_rel(outT, 2.0 * ref.t()) < 1e-5


@pytest.mark.parametrize("n,R,K", [(333, 24, 520), (8192, 48, 4096), (100, 16, 14336), (5, 64, 64),
                                   (256, 48, 5120), (504, 16, 4096), (77, 32, 4200)])
def test_lora_skinny(n, R, K):
    """Z = X·Bᵀ; short token ranges over long rows (100, 256, 504 and 77 rows)
    split K into 8, 5, 4 and 4 slices (the last with a partial 128-column
    chunk) and add the fp32 slices in a second launch, as the cycle does."""
    from deltaserve_amd import ops
    X = _bf(_rnd(n, K, seed=53)).to(DEV)
    B = _bf(_rnd(R, K, seed=54)).to(DEV)
    Z = ops.lora_skinny(X, B)
    ref = X.float().cpu() @ B.float().cpu().t()
    assert max_rel(Z, ref) < 8e-3


@pytest.mark.parametrize("n,r,C", [(700, 16, 1536), (8192, 16, 14336), (333, 32, 520), (33, 16, 1024),
                                   (4100, 32, 4096)])
def test_lora_dual(n, r, C):
    """One pass over G for grad_Z and grad_B: against fp32 products on the
    CPU and against the separate skinny / TN kernels."""
    from deltaserve_amd import ops
    G = _bf(_rnd(n, C, seed=55)).to(DEV)
    Z = _bf(_rnd(n, r, seed=56)).to(DEV)
    BT = _bf(_rnd(r, C, seed=57) * 0.1).to(DEV)
    gZ, gB = ops.lora_dual(G, Z, BT, scale=2.0)
    Gc, Zc, Bc = G.float().cpu(), Z.float().cpu(), BT.float().cpu()
    assert max_rel(gZ, Gc @ Bc.t()) < 8e-3
    assert max_rel(gB, 2.0 * (Gc.t() @ Zc)) < 1e-5
    gZ2 = ops.lora_skinny(G, BT)
    gB2 = torch.empty(C, r, device=DEV)
    ops.lora_tn(Z, G, r, True, [gB2], scale=2.0)
    assert max_rel(gZ, gZ2) < 8e-3
    assert max_rel(gB, gB2) < 1e-5
    # the same pass over xin for Z and grad_A ([r, C])
    _, gA = ops.lora_dual(G, Z, BT, scale=1.0, transpose_out=False)
    assert max_rel(gA, Zc.t() @ Gc) < 1e-5


@pytest.mark.parametrize("r", [16, 32])
def test_lora_dual_batched_passes(r):
    """The cycle's batched q/k/v launch: three passes in one launch, each
    reading a column slice of one strided [n, q + 2kv] gradient, with Z and
    grad_Z interleaved at a row stride of 3r, the live row count read from
    device memory and the partials laid out for n_alloc > n rows."""
    from deltaserve_amd import ops
    n, n_alloc, q, kv = 1000, 1500, 1024, 256
    W3 = q + 2 * kv
    G = _bf(_rnd(n_alloc, W3, seed=58)).to(DEV)
    Zall = _bf(_rnd(n_alloc, 3 * r, seed=59)).to(DEV)
    BTs = [_bf(_rnd(r, c, seed=60 + i) * 0.1).to(DEV) for i, c in enumerate((q, kv, kv))]
    gZall = torch.full((n_alloc, 3 * r), 7.0, dtype=torch.bfloat16, device=DEV)
    cols = [(0, q), (q, kv), (q + kv, kv)]
    gBs = [torch.empty(c, r, device=DEV) for _, c in cols]
    passes = [(G[:, c0:c0 + c], Zall[:, i * r:(i + 1) * r], BTs[i], gZall[:, i * r:(i + 1) * r],
               gBs[i], 2.0, True) for i, (c0, c) in enumerate(cols)]
    ops.lora_dual_batch(passes, n, n_alloc)
    Gc, Zc = G.float().cpu()[:n], Zall.float().cpu()[:n]
    for i, (c0, c) in enumerate(cols):
        Gi, Zi = Gc[:, c0:c0 + c], Zc[:, i * r:(i + 1) * r]
        assert max_rel(gZall[:n, i * r:(i + 1) * r], Gi @ BTs[i].float().cpu().t()) < 8e-3
        assert max_rel(gBs[i], 2.0 * (Gi.t() @ Zi)) < 1e-5
    # rows past the live count are not written
    assert (gZall[n:].float() == 7.0).all()


def test_clip_adamw():
    from deltaserve_amd import ops
    shapes = [(8, 64), (96, 8), (8, 4100), (33,)]
    groups = [0, 0, 1, 2]
    ws = [_rnd(*s, seed=60 + i) for i, s in enumerate(shapes)]
    gs = [_rnd(*s, seed=70 + i) * (3.0 if i < 2 else 0.01) for i, s in enumerate(shapes)]
    ms = [_rnd(*s, seed=80 + i) * 0.1 for i, s in enumerate(shapes)]
    vs = [_rnd(*s, seed=90 + i).abs() * 0.1 for i, s in enumerate(shapes)]
    dw, dg, dm, dv = ([t.clone().to(DEV) for t in x] for x in (ws, gs, ms, vs))
    ops.clip_adamw_(dw, dg, dm, dv, groups, lr=1e-3, step=3, wd=0.01)
    for gi in range(3):
        idx = [i for i, g in enumerate(groups) if g == gi]
        O.clip_([gs[i] for i in idx], 1.0)
    for i in range(len(ws)):
        O.adamw_(ws[i], gs[i], ms[i], vs[i], 3, 1e-3, wd=0.01)
        assert max_rel(dg[i], gs[i]) < 1e-5
        assert max_rel(dm[i], ms[i]) < 1e-5
        assert max_rel(dv[i], vs[i]) < 1e-5
        assert max_rel(dw[i], ws[i]) < 1e-5
