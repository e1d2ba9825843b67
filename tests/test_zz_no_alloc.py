"""The allocation-free entry point dsb_op_lora_dual_noalloc against
dsb_op_lora_dual, through the C-ABI: same passes, same kernels, so the
outputs agree bit for bit — on two calls in a row (the second with fewer
rows and columns, over the same scratch array), including the batched
three-pass q/k/v form; and captured into a graph, as the process's first
call of the entry point (its device lookup then runs under the capture),
replayed with new inputs."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _inputs(n_alloc, cols, r, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    W3 = sum(cols)
    G = torch.randn(n_alloc, W3, generator=g, device=DEV).to(torch.bfloat16)
    Z = torch.randn(n_alloc, len(cols) * r, generator=g, device=DEV).to(torch.bfloat16)
    BTs = [(torch.randn(r, c, generator=g, device=DEV) * 0.1).to(torch.bfloat16) for c in cols]
    return G, Z, BTs


def _run(entry, G, Z, BTs, cols, r, n, n_alloc):
    from deltaserve_amd import ops

    gZ = torch.full((n_alloc, len(cols) * r), 3.0, dtype=torch.bfloat16, device=DEV)
    gBs = [torch.full((c, r), 5.0, device=DEV) for c in cols]
    passes, c0 = [], 0
    for i, c in enumerate(cols):
        passes.append((G[:, c0:c0 + c], Z[:, i * r:(i + 1) * r], BTs[i],
                       gZ[:, i * r:(i + 1) * r], gBs[i], 2.0, i != 1))
        c0 += c
    ops.lora_dual_batch(passes, n, n_alloc, entry=entry)
    torch.cuda.synchronize()
    return gZ, gBs


def test_noalloc_captured_in_a_graph_first_then_replayed():
    """Runs first in this file: no other test calls the entry point, so in a
    fresh process the capture below is its first call on the device."""
    from deltaserve_amd import ops

    cols, r, n, n_alloc = (1024, 256, 256), 16, 1500, 2048
    G, Z, BTs = _inputs(n_alloc, cols, r, seed=7)
    gZ = torch.zeros(n_alloc, len(cols) * r, dtype=torch.bfloat16, device=DEV)
    gBs = [torch.zeros(c, r, device=DEV) for c in cols]
    passes, c0 = [], 0
    for i, c in enumerate(cols):
        passes.append((G[:, c0:c0 + c], Z[:, i * r:(i + 1) * r], BTs[i],
                       gZ[:, i * r:(i + 1) * r], gBs[i], 2.0, i != 1))
        c0 += c
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=side):
        ops.lora_dual_batch(passes, n, n_alloc, entry="dsb_op_lora_dual_noalloc")
    for rep in range(3):
        g = torch.Generator(device=DEV).manual_seed(50 + rep)
        G.copy_(torch.randn(G.shape, generator=g, device=DEV).to(torch.bfloat16))
        Z.copy_(torch.randn(Z.shape, generator=g, device=DEV).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        want = _run("dsb_op_lora_dual", G, Z, BTs, cols, r, n, n_alloc)
        assert torch.equal(gZ[:n], want[0][:n]), ("grad_Z", rep)
        for i in range(len(cols)):
            assert torch.equal(gBs[i], want[1][i]), ("grad_B", rep, i)
        # eager work between the replays, as a serving loop has
        _run("dsb_op_lora_dual_noalloc", G, Z, BTs, cols, r, n // 2, n_alloc)
    # a second capture, now after eager calls, replayed alongside the first
    graph2 = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph2, stream=side):
        ops.lora_dual_batch(passes, n // 3, n_alloc, entry="dsb_op_lora_dual_noalloc")
    graph2.replay()
    torch.cuda.synchronize()
    want = _run("dsb_op_lora_dual", G, Z, BTs, cols, r, n // 3, n_alloc)
    assert torch.equal(gZ[:n // 3], want[0][:n // 3])
    assert all(torch.equal(gBs[i], want[1][i]) for i in range(len(cols)))


@pytest.mark.parametrize("r", [16, 32])
def test_noalloc_equals_allocating_entry(r):
    cases = [((1024, 256, 256), 3000, 4096), ((520, 136), 700, 800)]  # second call smaller
    for k, (cols, n, n_alloc) in enumerate(cases):
        G, Z, BTs = _inputs(n_alloc, cols, r, seed=100 + k)
        want = _run("dsb_op_lora_dual", G, Z, BTs, cols, r, n, n_alloc)
        got = _run("dsb_op_lora_dual_noalloc", G, Z, BTs, cols, r, n, n_alloc)
        assert torch.equal(got[0], want[0]), ("grad_Z", k)
        for i in range(len(cols)):
            assert torch.equal(got[1][i], want[1][i]), ("grad_B", k, i)
        # rows past n untouched by both
        assert (got[0][n:].float() == 3.0).all()
        # and the result is the product itself
        Gc, Zc = G.float()[:n], Z.float()[:n]
        ref = 2.0 * (Gc[:, :cols[0]].t() @ Zc[:, :r])
        assert ((got[1][0] - ref).abs().max() / ref.abs().max()).item() < 1e-5
