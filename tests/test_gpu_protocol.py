"""The trainer child on the GPU, driven through its pipe by the reference
parent's own messages (``ParentSide``, restated from
``backward_process.py:266-495``): weights, the activation store and vLLM's
served LoRA buffers are shared the way the worker shares them, a
``process_activations`` trains (loss against the oracle), the served slot is
written with the cycle's updated masters, the store is zeroed, and the
job-switch / export / save commands the parent checks reply as it expects.

The child loop runs in a thread of this process over an in-process pipe, so
the shared tensors stay shared, as CUDA IPC keeps them between the reference's
processes.
"""

import os
import time

import pytest
import torch

from harness import (O, bf16_round_acts, gpu_activations, peft_key, shared_from_model,
                     tiny_meta)
from parent_protocol import InlinePipe

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


SEQ = [37, 128, 1, 200, 64]


def _served_payload(ft, scaling_slots=2, extra=4, sentinel=3.0):
    """vLLM's stacked LoRA buffers for every adapted (layer, projection):
    a [slots, 1, r + extra, in + extra], b [slots, 1, out + extra, r + extra]."""
    layers = {}
    for key, t in ft.items():
        if ".lora_A." not in key:
            continue
        i = int(key.split("layers.")[1].split(".")[0])
        proj = key.split("_proj.lora_A")[0].rsplit(".", 1)[1]
        r, fin = t.shape
        fout = ft[key.replace("lora_A", "lora_B")].shape[0]
        a = torch.full((scaling_slots, 1, r + extra, fin + extra), sentinel,
                       dtype=torch.bfloat16, device="cuda")
        b = torch.full((scaling_slots, 1, fout + extra, r + extra), sentinel,
                       dtype=torch.bfloat16, device="cuda")
        layers.setdefault(i, {})[proj] = {"a": a, "b": b}
    return {"slot": 1, "layers": layers}


def _assert_published(svc, payload):
    slot = payload["slot"]
    for i, projd in payload["layers"].items():
        for proj, buf in projd.items():
            A, B = svc.lora[i][proj]["A"].detach(), svc.lora[i][proj]["B"].detach()
            r, fin = A.shape
            fout = B.shape[0]
            assert torch.equal(buf["a"][slot, 0, :r, :fin],
                               A.clamp(-6.5e4, 6.5e4).to(torch.bfloat16)), (i, proj)
            assert torch.equal(buf["b"][slot, 0, :fout, :r],
                               (B * svc.scaling).clamp(-6.5e4, 6.5e4).to(torch.bfloat16)), (i, proj)


@pytest.mark.parametrize("family", ["llama3", "qwen3"])
def test_child_trains_and_publishes_through_the_parent_protocol(tmp_path, family):
    from deltaserve_amd.bwd_services.registry import get_service

    meta = tiny_meta(family=family, L=2)
    model = O.make_model(meta, seed=11, w_std=0.05, b_std=0.02, norm_jitter=0.2)
    n = sum(SEQ)
    ids = torch.randint(0, meta["vocab_size"], (n,), generator=torch.Generator().manual_seed(12))
    acts = bf16_round_acts(O.forward_capture(model, ids, SEQ))
    base, ft, smeta = shared_from_model(model)
    buffers = gpu_activations(acts, meta["max_saved_finetuning_tokens"])
    payload = _served_payload(ft)

    svc = get_service(family)(0)
    pipe = InlinePipe(svc, by_reference=True)
    parent = pipe.parent
    try:
        assert parent.ready()["event"] == "ready"
        got = parent.share_weights(base, ft, meta=smeta)
        assert got["event"] == "weights_received" and got["error"] is None, got
        assert parent.share_activations(buffers)["num_layers"] == meta["num_hidden_layers"]
        assert parent.share_lora_buffers(payload)["num_layers"] == meta["num_hidden_layers"]
        parent.set_corpus_meta(10 * n)

        parent.notify_buffer_full(n, SEQ, epoch=0)
        ack = parent.poll_response(timeout=300)
        assert ack["event"] == "activations_processed", ack
        rloss, rnv, _ = O.process_backward(model, acts, SEQ, n, lr=meta["learning_rate"],
                                           step=1, update=False)
        assert ack["loss"] is not None and abs(ack["loss"] - rloss) / abs(rloss) < 1e-3, \
            (ack["loss"], rloss)
        assert ack["n"] == n and ack["samples"] == len(SEQ) and ack["gpu_ms"] > 0
        assert svc.last_cycle_info["n_valid"] == rnv
        torch.cuda.synchronize()
        # the served slot holds the cycle's updated masters; the store is zeroed
        _assert_published(svc, payload)
        assert not any(t.any() for t in buffers["layer_in"]) and not buffers["final_in"].any()
        assert not buffers["concat_input_ids"].any()

        # end of the job: snapshot, save a shard, switch to the next adapter
        state = parent.export_lora()
        assert set(state) == set(ft)
        assert all(torch.equal(state[k], p.detach().cpu()) for k, p in svc.masters())
        shard = tmp_path / "shard" / "rank0.safetensors"
        assert parent.save_lora(str(shard))["tensors"] == len(ft)
        for _ in range(1000):
            if shard.exists():
                break
            time.sleep(0.01)
        assert shard.exists() and not os.path.exists(str(shard) + ".error")
        nxt = {k: (0.5 * v).cuda() for k, v in ft.items()}
        sw = parent.switch_adapter(nxt, {"learning_rate": 2e-4, "weight_decay": 0.0,
                                         "gamma": 1.0, "lora_scaling": svc.scaling})
        assert sw["event"] == "adapter_switched" and sw["tensors"] == len(ft)
        torch.cuda.synchronize()
        i0 = min(payload["layers"])
        assert torch.equal(svc.lora[i0]["q"]["A"].detach(),
                           nxt[peft_key(i0, "q", "A")].float())
        _assert_published(svc, payload)
        with pytest.raises(RuntimeError, match="refused the adapter"):
            parent.switch_adapter({k: v[:1] for k, v in nxt.items()},
                                  {"learning_rate": 1e-4, "weight_decay": 0.0, "gamma": 1.0})
        assert parent.shutdown()["event"] == "bye"
        pipe.join()
    finally:
        close = getattr(svc, "close", None)
        if close is not None:
            close()
