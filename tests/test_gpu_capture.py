"""The forward-side capture on the GPU: the save op and its index refresh.

Mirrors the reference's own capture test (tests/test_ft_save_op.py): a graph
captured once with the persistent index tensors replays with DIFFERENT index
contents and the saved rows follow the contents; a capture with no active
state records no work; interleaved rows, the residual sum and the scratch
row. Every check is bit-exact against the oracle's restatement of the op
(ft_save_op.py:84-89) on the same inputs, and a store filled through the op
trains exactly as the same activations handed over directly.
"""

import numpy as np
import pytest
import torch

from harness import O, bf16_round_acts, build_service, gpu_activations, tiny_meta

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _capture():
    from deltaserve_amd import capture

    return capture


def _oracle_save(x, r, buf, src, dst):
    cpu = buf.cpu()
    O.save_rows_(x.cpu(), None if r is None else r.cpu(), cpu, src.cpu(), dst.cpu())
    return cpu


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("width,ld_pad", [(4096, 0), (256, 8), (100, 0), (136, 3)])
@pytest.mark.parametrize("resid", [False, True])
def test_save_rows_bit_exact_vs_oracle(xdt, width, ld_pad, resid):
    C = _capture()
    g = torch.Generator().manual_seed(width + ld_pad)
    T, M, off = 300, 64, 10
    xf = (torch.randn(T, width + ld_pad, generator=g) * 4).to(xdt)
    rf = (torch.randn(T, width + ld_pad, generator=g) * 4).to(xdt) if resid else None
    x, r = xf[:, :width], None if rf is None else rf[:, :width]
    pos = torch.randperm(T, generator=g)[:70]  # more rows than fit after the offset
    src, dst, n = O.capture_index(pos.tolist(), 70, off, M)
    assert n == M - off
    buf = torch.randn(M + 1, width, generator=g).to(torch.bfloat16)
    want = _oracle_save(x, r, buf.clone(), src, dst)
    gbuf = buf.cuda()
    gx = xf.cuda()[:, :width]  # row stride width + ld_pad on the device too
    gr = None if rf is None else rf.cuda()[:, :width]
    assert gx.stride(0) == width + ld_pad
    C.save_rows(gx, gr, gbuf, src.cuda(), dst.cuda())
    torch.cuda.synchronize()
    got = gbuf.cpu()
    assert torch.equal(got[:M], want[:M])
    assert torch.equal(got[M], buf[M])  # the scratch row is not written


def test_capture_follows_index_contents():
    """tests/test_ft_save_op.py:40-90 on the MI355X op: capture once, replay
    with other positions and offsets; a stateless capture records nothing."""
    C = _capture()
    S, D, T = 16, 8, 32
    store = C.ActivationStore(num_layers=1, hidden_size=D, max_saved=S)
    x = torch.randn(T, D, device="cuda").to(torch.bfloat16)
    r = torch.randn(T, D, device="cuda").to(torch.bfloat16)
    slot = store.slot(0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with C.active_state(None):
            g0 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g0, stream=s):
                C.dserve_save_rows(x, r, store.marker, slot)
        with C.active_state(store.capture_state()):
            for _ in range(2):
                C.dserve_save_rows(x, r, store.marker, slot)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                C.dserve_save_rows(x, r, store.marker, slot)
    torch.cuda.synchronize()
    buf = store.layer_in[0]
    assert buf[:S].abs().sum().item() == 0  # warm-up and capture hit the scratch row only
    g0.replay()
    torch.cuda.synchronize()
    assert buf[:S].abs().sum().item() == 0
    cases = [([3, 7, 20], 5), ([31, 0], 12), ([1, 2, 3, 4, 5, 6, 7, 8], 11), ([], 0),
             (list(range(31, 15, -1)), 0)]
    want = buf.cpu().clone()
    for pos, off in cases:
        store.arm_op_step(np.array(pos, dtype=np.int64), len(pos), off)
        g.replay()
        torch.cuda.synchronize()
        src, dst, n = O.capture_index(pos, len(pos), off, S)
        O.save_rows_(x.cpu(), r.cpu(), want, src, dst)
        assert torch.equal(buf[:S].cpu(), want[:S]), (pos, off)
    assert store.num_saved == S


def test_final_ids_through_the_index_pair():
    """accumulate.py:598-622 on a graph-padded id vector with interleaved FT rows."""
    C = _capture()
    S = 16
    store = C.ActivationStore(num_layers=1, hidden_size=8, max_saved=S)
    ids = torch.arange(100, 124, device="cuda", dtype=torch.int64)  # padded to 24
    st = store.arm_op_step([1, 7, 15], 3, 3)
    store.save_final_ids(ids, st)
    st = store.arm_op_step([0, 23, 2, 9], 4, 14)  # two rows fit
    store.save_final_ids(ids, st)
    torch.cuda.synchronize()
    got = store.concat_input_ids.cpu().tolist()
    assert got[3:6] == [101, 107, 115] and got[14:16] == [100, 123]
    assert all(v == 0 for i, v in enumerate(got) if i not in (3, 4, 5, 14, 15))


def test_out_of_range_source_rows_are_skipped():
    C = _capture()
    x = torch.randn(10, 64, device="cuda").to(torch.bfloat16)
    buf = torch.zeros(9, 64, device="cuda", dtype=torch.bfloat16)
    src = torch.tensor([2, 10, 11, 3, 0, 0, 0, 0], device="cuda")
    dst = torch.tensor([0, 1, 2, 3, 8, 8, 8, 8], device="cuda")
    C.save_rows(x, None, buf, src, dst)
    ids = torch.arange(10, device="cuda")
    out = torch.zeros(8, dtype=torch.int64, device="cuda")
    C.save_ids(ids, src, dst, out)
    torch.cuda.synchronize()
    assert torch.equal(buf[0], x[2]) and torch.equal(buf[3], x[3])
    assert buf[1:3].abs().sum().item() == 0 and buf[4:].abs().sum().item() == 0
    assert out.tolist() == [2, 0, 0, 3, 0, 0, 0, 0]


@pytest.mark.parametrize("contiguous", [True, False])
def test_eager_hooks_match_the_op_path(contiguous):
    """The eager step (begin_step + per-hook save, accumulate.py:421-446 and
    :581-596) and the op path produce the same buffers."""
    C = _capture()
    S, D, T = 32, 128, 48
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, D, generator=g).to(torch.bfloat16).cuda()
    r = torch.randn(T, D, generator=g).to(torch.bfloat16).cuda()
    ids = torch.randint(0, 999, (T,), generator=g).cuda()
    if contiguous:
        start, nft = 5, 20
        pos = list(range(start, start + nft))
    else:
        start, pos = 0, sorted(torch.randperm(T, generator=g)[:20].tolist())
        nft = len(pos)
    mask = torch.zeros(T, dtype=torch.bool)
    mask[pos] = True
    a = C.ActivationStore(2, D, S)
    b = C.ActivationStore(2, D, S)
    a.begin_step(mask.cuda(), nft, offset=7, start=start, contiguous=contiguous)
    a.save(a.slot(0), x)
    a.save(a.slot(1), x, r)
    a.save(a.final_slot, r)
    a.accumulate_final(ids)
    a.end_step()
    a.save(a.slot(0), r)  # disarmed: no effect
    st = b.arm_op_step(pos, nft, 7)
    with C.active_state(st):
        C.dserve_save_rows(x, None, b.marker, b.slot(0))
        C.dserve_save_rows(x, r, b.marker, b.slot(1))
        C.dserve_save_rows(r, None, b.marker, b.final_slot)
        C.dserve_save_rows(x, r, b.marker, b.slot(0, 3))  # a slot with no buffer
    b.save_final_ids(ids, st)
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(a.layer_in[i][:S], b.layer_in[i][:S])
    assert torch.equal(a.final_in[:S], b.final_in[:S])
    assert torch.equal(a.concat_input_ids, b.concat_input_ids)
    assert torch.equal(a.layer_in[0][7:27].cpu(), x[pos].cpu())
    a.zero_offset_range(10, 5)
    assert a.layer_in[1][10:15].abs().sum().item() == 0 and a.concat_input_ids[10:15].sum() == 0


SEQ = [37, 128, 1, 200, 64]


def test_store_filled_by_the_op_trains_like_a_direct_handoff():
    """Two mixed forward steps (FT rows interleaved with inference rows, the
    fused add-norm's (hidden, residual) pair at layers > 0) fill the store
    through the op; the buffers equal the oracle's, and a backward cycle on
    them gives the same loss, gradients and masters as the same activations
    handed over directly."""
    C = _capture()
    meta = tiny_meta(family="llama3", L=2)
    model = O.make_model(meta, seed=9, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    S, D, Lyr = meta["max_saved_finetuning_tokens"], meta["hidden_size"], 2
    n = sum(SEQ)
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=g)
    acts = O.forward_capture(model, ids, SEQ)
    store = C.ActivationStore(Lyr, D, S)
    want = {"layer_in": [torch.zeros(S + 1, D, dtype=torch.bfloat16) for _ in range(Lyr)],
            "final_in": torch.zeros(S + 1, D, dtype=torch.bfloat16),
            "concat_input_ids": torch.zeros(S, dtype=torch.int64)}
    splits = [(0, 230), (230, n)]  # FT rows of step 1, then of step 2
    for (a, b), T in zip(splits, (300, 260)):
        nft = b - a
        pos = sorted(torch.randperm(T, generator=g)[:nft].tolist())
        flat_ids = torch.randint(0, meta["vocab_size"], (T,), generator=g)
        flat_ids[pos] = ids[a:b]
        st = store.arm_op_step(pos, nft, a)
        src, dst, _ = O.capture_index(pos, nft, a, S)
        for i in range(Lyr + 1):
            val = (acts["layer_in"][i] if i < Lyr else acts["final_in"])[a:b]
            flat = torch.randn(T, D, generator=g)
            flat[pos] = val
            if i == 0:
                h, r = flat.to(torch.bfloat16), None
            else:  # hidden + residual, the fused add-norm's pre-hook arguments
                r = (torch.randn(T, D, generator=g) * 0.5).to(torch.bfloat16)
                h = (flat - r.float()).to(torch.bfloat16)
            slot = store.slot(i) if i < Lyr else store.final_slot
            with C.active_state(st):
                C.dserve_save_rows(h.cuda(), None if r is None else r.cuda(), store.marker, slot)
            O.save_rows_(h, r, want["layer_in"][i] if i < Lyr else want["final_in"], src, dst)
        store.save_final_ids(flat_ids.cuda(), st)
        want["concat_input_ids"].index_copy_(0, dst[dst < S], flat_ids[src[dst < S]])
    torch.cuda.synchronize()
    assert store.num_saved == n
    for i in range(Lyr):
        assert torch.equal(store.layer_in[i][:S].cpu(), want["layer_in"][i][:S]), i
    assert torch.equal(store.final_in[:S].cpu(), want["final_in"][:S])
    assert torch.equal(store.concat_input_ids.cpu(), want["concat_input_ids"])
    assert torch.equal(store.concat_input_ids[:n].cpu(), ids)

    direct = gpu_activations({"layer_in": [t[:n].float() for t in want["layer_in"]],
                              "final_in": want["final_in"][:n].float(),
                              "concat_input_ids": ids}, S)
    one, two = build_service(model, "llama3"), build_service(model, "llama3")
    try:
        l1, n1 = one.process_backward(store.activations(), SEQ, n, epoch=0)
        l2, n2 = two.process_backward(direct, SEQ, n, epoch=0)
        assert n1 == n2 and l1 == l2, (l1, l2)
        for i, d in one.lora.items():
            for p, dd in d.items():
                for ab, t in dd.items():
                    u = two.lora[i][p][ab]
                    assert torch.equal(t.detach(), u.detach()) and torch.equal(t.grad, u.grad)
    finally:
        one.close()
        two.close()


def test_gate_up_slot_feeds_the_saved_path():
    """A store built with the intermediate size has the reference's default
    mlp_gate_up save point (accumulate.py:174, :210-212): the gate‖up
    projection output saved through the op lands bit-exact in its buffer,
    ``activations()`` hands it to the backward, and the cycle on the store
    equals the same activations (gate‖up included) handed over directly; the
    saved path's loss agrees with the recompute path's."""
    C = _capture()
    meta = tiny_meta(family="llama3", L=2)
    model = O.make_model(meta, seed=4, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    S, D, Lyr, inter = (meta["max_saved_finetuning_tokens"], meta["hidden_size"], 2,
                        meta["intermediate_size"])
    n = sum(SEQ)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(4))
    acts = O.forward_capture(model, ids, SEQ, save_gate_up=True)
    store = C.ActivationStore(Lyr, D, S, intermediate_size=inter)
    assert len(store.mlp_gate_up) == Lyr and store.mlp_gate_up[0].shape == (S + 1, 2 * inter)
    st = store.arm_op_step(list(range(n)), n, 0)
    with C.active_state(st):
        for i in range(Lyr):
            C.dserve_save_rows(acts["layer_in"][i].to(torch.bfloat16).cuda(), None,
                               store.marker, store.slot(i))
            C.dserve_save_rows(acts["mlp_gate_up"][i].to(torch.bfloat16).cuda(), None,
                               store.marker, store.slot(i, C.SLOT_GATE_UP))
        C.dserve_save_rows(acts["final_in"].to(torch.bfloat16).cuda(), None, store.marker,
                           store.final_slot)
    store.save_final_ids(ids.cuda(), st)
    torch.cuda.synchronize()
    for i in range(Lyr):
        assert torch.equal(store.mlp_gate_up[i][:n].cpu(), acts["mlp_gate_up"][i].to(torch.bfloat16))
        assert not store.mlp_gate_up[i][n:S].any()
    got = store.activations()
    assert "mlp_gate_up" in got

    direct = gpu_activations(acts, S)
    recompute = {k: v for k, v in direct.items() if k != "mlp_gate_up"}
    one, two, three = (build_service(model, "llama3") for _ in range(3))
    try:
        l1, n1 = one.process_backward(got, SEQ, n, epoch=0)
        l2, n2 = two.process_backward(direct, SEQ, n, epoch=0)
        l3, n3 = three.process_backward(recompute, SEQ, n, epoch=0)
        assert n1 == n2 == n3 and l1 == l2, (l1, l2)
        assert abs(l1 - l3) / abs(l3) < 1e-3, (l1, l3)
        for i, d in one.lora.items():
            for p, dd in d.items():
                for ab, t in dd.items():
                    assert torch.equal(t.grad, two.lora[i][p][ab].grad)
    finally:
        one.close()
        two.close()
        three.close()


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_every_save_point_filled_by_the_op_feeds_the_cycle(family):
    """A store with every opt-in save point (accumulate.py:213-235): the
    op writes q/k/v (Llama-3 after RoPE, Qwen3 before the q/k-norm), the
    attention context, the post-attention residual and the final hidden
    state into their slots bit-exact; ``activations()`` hands them over;
    with the worker's save_attn_qkv / save_resid_mid meta keys the cycle on
    the store equals the same buffers handed over directly, and the capture
    check (verify_activations, trainer.py:806-826) passes on it."""
    C = _capture()
    meta = tiny_meta(family=family, L=2)
    model = O.make_model(meta, seed=21, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    S, D, Lyr = meta["max_saved_finetuning_tokens"], meta["hidden_size"], 2
    q_size = meta["num_attention_heads"] * 128
    kv_size = meta["num_key_value_heads"] * 128
    n = sum(SEQ)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(21))
    acts = O.forward_capture(model, ids, SEQ, save_gate_up=True, save_attn_qkv=True,
                             save_attn_ctx=True, save_resid_mid=True)
    final_hidden = O.rmsnorm(acts["final_in"], model.norm_w, meta["rms_norm_eps"])
    store = C.ActivationStore(Lyr, D, S, intermediate_size=meta["intermediate_size"],
                              q_size=q_size, kv_size=kv_size, save_attn_qkv=True,
                              save_attn_ctx=True, save_resid_mid=True, save_final_hidden=True)
    slots = {"layer_in": C.SLOT_LAYER_IN, "mlp_gate_up": C.SLOT_GATE_UP,
             "resid_mid": C.SLOT_RESID_MID, "attn_qh": C.SLOT_QH, "attn_kh": C.SLOT_KH,
             "attn_vh": C.SLOT_VH, "attn_ctx": C.SLOT_CTX}
    st = store.begin_step(None, n, 0, start=0, contiguous=True)
    for i in range(Lyr):
        for name, kind in slots.items():
            store.save(store.slot(i, kind), acts[name][i].to(torch.bfloat16).cuda())
    store.save(store.final_slot, acts["final_in"].to(torch.bfloat16).cuda())
    store.accumulate_final(ids.cuda(), final_hidden.to(torch.bfloat16).cuda())
    store.end_step()
    torch.cuda.synchronize()
    got = store.activations()
    for name in slots:
        for i in range(Lyr):
            assert torch.equal(got[name][i][:n].cpu(), acts[name][i].to(torch.bfloat16)), (name, i)
    assert torch.equal(got["final_hidden"][:n].cpu(), final_hidden.to(torch.bfloat16))
    assert st.src.shape[0] == S

    direct = gpu_activations(bf16_round_acts(acts), S)
    svcs = [build_service(model, family) for _ in range(2)]
    try:
        for svc in svcs:
            svc.shared["meta"].update(save_attn_qkv=True, save_resid_mid=True)
        checks = svcs[0].verify_activations(got, n)
        assert checks and all(ok for _, _, ok in checks), checks
        l1, n1 = svcs[0].process_backward(got, SEQ, n, epoch=0)
        l2, n2 = svcs[1].process_backward(direct, SEQ, n, epoch=0)
        assert svcs[0].saved_points == ["attn_ctx", "attn_kh", "attn_qh", "attn_vh",
                                        "mlp_gate_up", "resid_mid"]
        assert n1 == n2 and l1 == l2, (l1, l2)
        for i, d in svcs[0].lora.items():
            for p, dd in d.items():
                for ab, t in dd.items():
                    assert torch.equal(t.grad, svcs[1].lora[i][p][ab].grad), (i, p, ab)
    finally:
        for svc in svcs:
            svc.close()
