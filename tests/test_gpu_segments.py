"""Pause points and the served-slot publish on the GPU.

* The segmented cycle (dsb_step_begin / dsb_step_segment / dsb_step_end, one
  captured graph per segment, the reference's _maybe_pause once per LM-head
  vocab chunk in both passes and at every layer boundary, head.py:78-80,
  :92-94, base.py:148-208) computes exactly what the single-graph cycle
  computes: same kernels in the same order, so loss, gradients and updated
  masters agree bit for bit, for any run-ahead bound.
* The attention backward's dK/dV pass runs on a second stream beside the
  dQ pass (parallel graph branches, or two streams in an eager cycle); the
  per-kernel timing mode runs them in order. All three give the same loss,
  gradients and masters bit for bit (the passes share only inputs).
* Each layer's recompute runs on a third stream beside the backward of the
  layer before it in the cycle, into the other of two buffer sets; with
  ``backward_serial_layers`` it runs right before its own backward. Both
  orders give the same loss, gradients and masters bit for bit.
* A cleared GPU grant holds the cycle at a boundary until it is set again.
* Every cycle ends by writing clamp(A) and clamp(s·B) (bf16) into the bound
  rows of vLLM's stacked LoRA buffers (trainer.py:760-802) and nothing else.
"""

import threading
import time

import pytest
import torch

from harness import O, bf16_round_acts, build_service, config_meta, gpu_activations, tiny_meta

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


SEQ = [37, 128, 1, 200, 64]


def _setup(family="llama3", seed=5, vocab_chunk=0):
    meta = tiny_meta(family=family, L=2, vocab_chunk=vocab_chunk)
    model = O.make_model(meta, seed=seed, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    n = sum(SEQ)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(seed))
    acts = bf16_round_acts(O.forward_capture(model, ids, SEQ))
    return meta, model, gpu_activations(acts, meta["max_saved_finetuning_tokens"])


def _state(svc):
    return {(i, p, ab): (t.detach().clone(), t.grad.detach().clone())
            for i, d in svc.lora.items() for p, dd in d.items() for ab, t in dd.items()}


@pytest.mark.parametrize("family,run_ahead,vchunk", [("llama3", 0, 0), ("llama3", 2, 256),
                                                     ("qwen3", 1, 512)])
def test_segmented_cycle_equals_single_graph(family, run_ahead, vchunk):
    meta, model, gacts = _setup(family, vocab_chunk=vchunk)
    n = sum(SEQ)
    one = build_service(model, family)
    seg = build_service(model, family)
    seg.shared["meta"]["backward_pause_boundaries"] = True
    seg.shared["meta"]["backward_run_ahead_boundaries"] = run_ahead
    try:
        for _ in range(2):
            l1, n1 = one.process_backward(gacts, SEQ, n, epoch=0)
            l2, n2 = seg.process_backward(gacts, SEQ, n, epoch=0)
            assert "segments" in seg._last_mode and "segments" not in one._last_mode
            assert n1 == n2 and l1 == l2, (l1, l2)
            s1, s2 = _state(one), _state(seg)
            for k in s1:
                assert torch.equal(s1[k][0], s2[k][0]), ("master", k)
                assert torch.equal(s1[k][1], s2[k][1]), ("grad", k)
    finally:
        one.close()
        seg.close()


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_concurrent_attention_backward_equals_in_order(family):
    meta, model, gacts = _setup(family)
    n = sum(SEQ)
    graph = build_service(model, family)
    eager = build_service(model, family, meta_extra={"backward_hip_graph": False})
    timed = build_service(model, family)
    timed.set_kernel_timing(True)
    svcs = [graph, eager, timed]
    try:
        for _ in range(2):
            out = [s.process_backward(gacts, SEQ, n, epoch=0) for s in svcs]
            assert graph.last_cycle_info["graph"]
            assert not eager.last_cycle_info["graph"] and not timed.last_cycle_info["graph"]
            for o in out[1:]:
                assert o == out[0], (o, out[0])
            ref = _state(graph)
            for s in svcs[1:]:
                st = _state(s)
                for k in ref:
                    assert torch.equal(ref[k][0], st[k][0]), ("master", k)
                    assert torch.equal(ref[k][1], st[k][1]), ("grad", k)
    finally:
        for s in svcs:
            s.close()


def test_pause_points_per_vocab_chunk_and_layer():
    """With V = 1000 in chunks of 256 (4 chunks) and 2 layers, the cycle
    checks the grant before each of the 4 + 4 head segments and the 2 layer
    segments (plus once on entry, trainer.py:504), not before the optimizer."""
    from deltaserve_amd import _lib as L

    meta, model, gacts = _setup(vocab_chunk=256)
    n = sum(SEQ)
    svc = build_service(model, "llama3")
    svc.shared["meta"]["backward_pause_boundaries"] = True
    calls = []
    svc._maybe_pause = lambda: calls.append(1)
    try:
        svc.process_backward(gacts, SEQ, n, epoch=0)
        assert L.load().dsb_num_segments(svc._h) == 2 * 4 + 2 + 1
        assert len(calls) == 1 + 2 * 4 + 2
    finally:
        svc.close()


def test_cleared_grant_holds_the_cycle_until_set():
    meta, model, gacts = _setup()
    n = sum(SEQ)
    ref = build_service(model, "llama3")
    svc = build_service(model, "llama3")
    grant = threading.Event()  # cleared: an inference prefill holds the GPU
    svc._gpu_grant = grant
    try:
        rl, _ = ref.process_backward(gacts, SEQ, n, epoch=0)
        timer = threading.Timer(0.3, grant.set)
        t0 = time.perf_counter()
        timer.start()
        loss, _ = svc.process_backward(gacts, SEQ, n, epoch=0)
        dt = time.perf_counter() - t0
        timer.join()
        assert dt >= 0.25, dt
        assert loss == rl
        # grant set: no hold
        t0 = time.perf_counter()
        svc.process_backward(gacts, SEQ, n, epoch=0)
        assert time.perf_counter() - t0 < 0.25
    finally:
        ref.close()
        svc.close()


def _served_buffers(svc, slots=2, extra=8, sentinel=7.0):
    """vLLM-style stacked buffers: lora_a [slots, 1, r + extra, in + extra],
    lora_b [slots, 1, out + extra, r + extra], bf16, filled with a sentinel."""
    layers = {}
    for i, d in svc.lora.items():
        layers[i] = {}
        for p, t in d.items():
            r, fin = t["A"].shape
            fout = t["B"].shape[0]
            a = torch.full((slots, 1, r + extra, fin + extra), sentinel, dtype=torch.bfloat16,
                           device="cuda")
            b = torch.full((slots, 1, fout + extra, r + extra), sentinel, dtype=torch.bfloat16,
                           device="cuda")
            layers[i][p] = {"a": a, "b": b}
    return {"slot": 1, "layers": layers}


def _check_published(svc, bufs, sentinel=7.0):
    slot = bufs["slot"]
    for i, d in bufs["layers"].items():
        for p, buf in d.items():
            A, B = svc.lora[i][p]["A"].detach(), svc.lora[i][p]["B"].detach()
            r, fin = A.shape
            fout = B.shape[0]
            want_a = A.clamp(-6.5e4, 6.5e4).to(torch.bfloat16)
            want_b = (B * svc.scaling).clamp(-6.5e4, 6.5e4).to(torch.bfloat16)
            a, b = buf["a"], buf["b"]
            assert torch.equal(a[slot, 0, :r, :fin], want_a), (i, p, "A")
            assert torch.equal(b[slot, 0, :fout, :r], want_b), (i, p, "B")
            # nothing outside the slot's rows is written
            assert (a[slot, 0, r:] == sentinel).all() and (a[slot, 0, :, fin:] == sentinel).all()
            assert (b[slot, 0, fout:] == sentinel).all() and (b[slot, 0, :, r:] == sentinel).all()
            assert (a[0] == sentinel).all() and (b[0] == sentinel).all()


@pytest.mark.parametrize("segmented", [False, True])
def test_cycle_publishes_into_the_served_slot(segmented):
    meta, model, gacts = _setup()
    n = sum(SEQ)
    svc = build_service(model, "llama3")
    if segmented:
        svc.shared["meta"]["backward_pause_boundaries"] = True
    try:
        bufs = _served_buffers(svc)
        svc.lora_buffers = bufs
        svc._on_lora_buffers()
        # one master beyond the clamp range exercises the ±6.5e4 clamp
        with torch.no_grad():
            svc.lora[0]["q"]["A"][0, 0] = 7.0e4
            svc.lora[1]["down"]["B"][3, 1] = -4.0e4  # s·B = -8e4 → clamped
        svc.process_backward(gacts, SEQ, n, epoch=0)
        torch.cuda.synchronize()
        _check_published(svc, bufs)
        assert svc.lora_buffers["layers"][0]["q"]["a"][1, 0, 0, 0].item() == 65024.0
        # outside a cycle (the switch_adapter path): new masters, explicit publish
        with torch.no_grad():
            for d in svc.lora.values():
                for t in d.values():
                    t["A"].mul_(-0.5)
                    t["B"].add_(0.01)
        svc._publish_to_served()
        torch.cuda.synchronize()
        _check_published(svc, bufs)
    finally:
        svc.close()


@pytest.mark.parametrize("case", ["llama3", "qwen3", "c4s"])
def test_layer_overlap_equals_serial(case):
    """Three layers, two cycles. The c4s case (256 tokens at Qwen3-14B widths)
    takes the split-K products and the skinny kernel's K split in the
    recompute, whose scratch the side stream has its own copy of."""
    if case == "c4s":
        meta, seq = config_meta("c4s", L=3)
        dev = "cuda"
    else:
        meta, seq, dev = tiny_meta(family=case, L=3), SEQ, "cpu"
    model = O.make_model(meta, seed=3, w_std=0.02, b_std=0.01, device=dev)
    n = sum(seq)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(3))
    acts = bf16_round_acts(O.forward_capture(model, ids.to(dev), seq))
    gacts = gpu_activations(acts, meta["max_saved_finetuning_tokens"])
    del acts
    family = meta["family"]
    over = build_service(model, family)
    serial = build_service(model, family, meta_extra={"backward_serial_layers": True})
    try:
        for _ in range(2):
            l1, n1 = over.process_backward(gacts, seq, n, epoch=0)
            l2, n2 = serial.process_backward(gacts, seq, n, epoch=0)
            assert over.last_cycle_info["graph"] and serial.last_cycle_info["graph"]
            assert n1 == n2 and l1 == l2, (l1, l2)
            s1, s2 = _state(over), _state(serial)
            for k in s1:
                assert torch.equal(s1[k][0], s2[k][0]), ("master", k)
                assert torch.equal(s1[k][1], s2[k][1]), ("grad", k)
    finally:
        over.close()
        serial.close()
