"""Host-side surface of the drop-in backward child, on the CPU: service
registry (registry.py:15-49), PEFT adapter checkpoints and their periodic
schedule (adapter_io.py:95-159, trainer.py:336-437), the pipe protocol and
per-cycle wrapper of BackwardService driven by the reference parent's own
messages (backward_process.py:266-495, base.py:297-633), the capture
fingerprints, the pause points, the handover line and the workload configs."""

from __future__ import annotations

import json
import os
import types

import pytest
import torch

from deltaserve_amd import checkpoint as adapter_io
from deltaserve_amd import configs
from deltaserve_amd.bwd_services import registry
from deltaserve_amd.bwd_services.base import BackwardService


# ------------------------------------------------------------------ registry

def test_registry_resolves_architectures():
    for arch in ("LlamaForCausalLM", "llama3", "Qwen3ForCausalLM", "qwen3"):
        cls = registry.get_service(arch)
        assert cls.family is not None and cls.__name__.endswith("BackwardService")
    assert registry.get_service("ipc") is BackwardService
    assert registry.get_family("qwen3").name == "qwen3"
    assert registry.get_family("GPT2LMHeadModel") is None


def test_registry_unknown_lists_supported():
    with pytest.raises(NotImplementedError, match="LlamaForCausalLM"):
        registry.get_service("MistralForCausalLM")


# ------------------------------------------------------------------ adapter files

def _tensors(r=4):
    g = torch.Generator().manual_seed(0)
    p = "base_model.model.model.layers.0."
    return {p + "self_attn.q_proj.lora_A.weight": torch.randn(r, 32, generator=g),
            p + "self_attn.q_proj.lora_B.weight": torch.randn(48, r, generator=g),
            p + "mlp.down_proj.lora_A.weight": torch.randn(r, 64, generator=g),
            p + "mlp.down_proj.lora_B.weight": torch.randn(32, r, generator=g)}


def test_write_peft_adapter_roundtrip(tmp_path):
    from safetensors.torch import load_file

    t = _tensors()
    out = tmp_path / "ckpt-1"
    adapter_io.write_peft_adapter(str(out), t, source_dir=None, scaling=2.0,
                                  state={"save_id": "s1", "reason": "manual", "epoch": 0})
    back = load_file(str(out / adapter_io.WEIGHTS_FILE))
    assert sorted(back) == sorted(t)
    for k in t:
        assert back[k].dtype == torch.float32 and torch.equal(back[k], t[k])
    cfg = json.loads((out / adapter_io.CONFIG_FILE).read_text())
    assert cfg["r"] == 4 and cfg["lora_alpha"] == 8.0
    assert cfg["target_modules"] == ["down_proj", "q_proj"]
    st = json.loads((out / adapter_io.STATE_FILE).read_text())
    assert st["num_tensors"] == 4 and st["save_id"] == "s1"
    res = adapter_io.read_save_result(str(out), "s1")
    assert res["saved"] is True
    assert adapter_io.read_save_result(str(out), "other") is None
    assert sorted(os.listdir(out)) == sorted([adapter_io.WEIGHTS_FILE, adapter_io.CONFIG_FILE,
                                              adapter_io.STATE_FILE])


def test_adapter_config_copied_from_source(tmp_path):
    src = tmp_path / "src"
    src.mkdir()
    (src / adapter_io.CONFIG_FILE).write_text(json.dumps({"r": 4, "lora_alpha": 99}))
    adapter_io.write_peft_adapter(str(tmp_path / "o"), _tensors(), source_dir=str(src),
                                  scaling=2.0, state={"save_id": "x"})
    assert json.loads((tmp_path / "o" / adapter_io.CONFIG_FILE).read_text())["lora_alpha"] == 99


def test_save_error_and_prune(tmp_path):
    adapter_io.write_save_error(str(tmp_path / "e"), "s9", "disk full")
    res = adapter_io.read_save_result(str(tmp_path / "e"), "s9")
    assert res["saved"] is False and res["error"] == "disk full"
    for i in (1, 2, 10, 3):
        (tmp_path / f"step-{i}").mkdir()
    (tmp_path / "step-x").mkdir()
    removed = adapter_io.prune_checkpoints(str(tmp_path), "step-", 2)
    assert sorted(os.path.basename(p) for p in removed) == ["step-1", "step-2"]
    assert sorted(os.listdir(tmp_path)) == ["e", "step-10", "step-3", "step-x"]


class _Owner:
    """The attributes AdapterCheckpointer reads from a trainer."""

    def __init__(self, root):
        self.scaling = 2.0
        self.lr = 1e-4
        self._total_tokens_trained = 0
        self._last_loss = None
        self.shared = {"meta": {"adapter_save_path": str(root),
                                "adapter_save_every_backwards": 2,
                                "adapter_save_every_epoch": True,
                                "adapter_save_keep_last": 2}}
        self.w = torch.zeros(4, 8)

    def masters(self):
        yield "base_model.model.model.layers.0.self_attn.q_proj.lora_A.weight", self.w


def test_checkpoint_schedule(tmp_path):
    """trainer.py:405-437: the epoch checkpoint holds the state left by the
    previous epoch's last cycle (captured when the next epoch's first cycle
    starts, written after it); every 2nd attempted cycle writes
    backward-NNNNNN, keeping the newest 2."""
    from safetensors.torch import load_file

    o = _Owner(tmp_path)
    ck = adapter_io.AdapterCheckpointer(o)
    ck.configure(o.shared["meta"])
    for cycle, epoch in enumerate([0, 0, 0, 1, 1, 1], start=1):
        ck.before_cycle(epoch)
        o.w += 1.0  # the cycle's update
        o._total_tokens_trained += 10
        ck.after_cycle(epoch)
    assert sorted(os.listdir(tmp_path)) == ["backward-000004", "backward-000006", "epoch-0"]
    ep = json.loads((tmp_path / "epoch-0" / adapter_io.STATE_FILE).read_text())
    assert ep["reason"] == "epoch" and ep["epoch"] == 0 and ep["backward_cycles"] == 3
    assert ep["tokens_trained"] == 30 and ep["save_id"] == "epoch-0"
    w = load_file(str(tmp_path / "epoch-0" / adapter_io.WEIGHTS_FILE))
    assert float(next(iter(w.values()))[0, 0]) == 3.0  # after cycle 3, not cycle 4
    last = json.loads((tmp_path / "backward-000006" / adapter_io.STATE_FILE).read_text())
    assert last["reason"] == "every_backwards" and last["backward_cycles"] == 6


def test_checkpoint_schedule_off_without_root(tmp_path):
    o = _Owner(tmp_path)
    ck = adapter_io.AdapterCheckpointer(o)
    ck.configure({})
    for epoch in (0, 1, 2):
        ck.before_cycle(epoch)
        ck.after_cycle(epoch)
    assert os.listdir(tmp_path) == [] and ck.schedule.attempted == 3


# ------------------------------------------------------------------ pipe protocol
#
# The child is driven by ``ParentSide``, which sends the reference parent's
# exact message dicts and checks the replies the way the parent does.

class _CpuTrainer(BackwardService):
    """A protocol-level trainer on the CPU: fp32 masters in a dict, a cycle
    that records its inputs and returns a known loss."""

    def __init__(self):
        super().__init__(0)
        self.calls = []
        self.masters_ = {}

    def _on_weights_shared(self):
        if not self.shared["ft"]:
            return "ValueError: the FT adapter holds no LoRA tensors"
        self.masters_ = {k: v.clone().float() for k, v in self.shared["ft"].items()}
        return None

    def process_backward(self, activations, sample_lens, n, epoch):
        self.calls.append((list(sample_lens), n, epoch,
                           float(activations["layer_in"][0][:n].sum())))
        if epoch == 3:
            raise RuntimeError("planted failure")
        return 1.25, sum(max(s - 1, 0) for s in sample_lens)

    def export_lora_state(self):
        return {k: v.clone() for k, v in self.masters_.items()}

    def switch_adapter(self, ft, hparams):
        if set(ft) != set(self.masters_):
            raise ValueError("different target modules")
        self.masters_ = {k: v.clone().float() for k, v in ft.items()}
        self.ledger.restart(int(hparams.get("total_tokens_per_epoch", 0)))
        return {"tensors": len(ft)}


def _buffers(rows=9, width=4):
    return {"layer_in": [torch.ones(rows, width), 2 * torch.ones(rows, width)],
            "final_in": torch.ones(rows, width),
            "concat_input_ids": torch.arange(rows - 1)}


def _adapter():
    p = "base_model.model.model.layers.{}.self_attn.q_proj.lora_{}.weight"
    g = torch.Generator().manual_seed(3)
    return {p.format(i, ab): torch.randn(4, 8, generator=g) for i in (0, 1) for ab in "AB"}


def test_child_speaks_the_reference_parents_protocol(tmp_path):
    from parent_protocol import InlinePipe
    from safetensors.torch import load_file

    svc = _CpuTrainer()
    pipe = InlinePipe(svc)
    parent = pipe.parent
    ready = parent.ready()
    assert ready["event"] == "ready" and ready["pid"] == os.getpid()
    assert {"mps_percentage", "max_connections"} <= set(ready)
    pong = parent.ping({"x": 1})
    assert pong == {"event": "pong", "pid": os.getpid(), "data": {"x": 1}}

    ft = _adapter()
    base = {"model.layers.0.mlp.fc1.weight": torch.ones(2, 2),
            "model.layers.5.mlp.fc1.weight": torch.zeros(2, 2)}
    got = parent.share_weights(base, ft, print_hash=True, meta={"tp_rank": 0})
    assert got["event"] == "weights_received" and got["error"] is None
    assert got["base_num"] == 2 and got["ft_num"] == 4 and got["ft_numel"] == 128
    assert set(got["hash_report"]) == {"base_ffn_fc1_first", "base_ffn_fc1_last",
                                       "ft_q_loraA_first", "ft_q_loraA_last"}
    assert got["hash_report"]["base_ffn_fc1_last"][0] == 5
    assert abs(parent.checksum("ft") - float(sum(t.double().sum() for t in ft.values()))) < 1e-9

    buffers = _buffers()
    assert parent.share_activations(buffers) == {"event": "activations_received",
                                                 "num_layers": 2}
    payload = {"slot": 1, "layers": {0: {"q": {"a": torch.zeros(2, 1, 4, 8),
                                               "b": torch.zeros(2, 1, 8, 4)}}}}
    assert parent.share_lora_buffers(payload) == {"event": "lora_buffers_received",
                                                  "num_layers": 1}
    assert svc.lora_buffers["slot"] == 1  # the pipe pickles CPU tensors: the child holds a copy
    report = parent.hash_activations(7)
    assert set(report) == {"layer_in_first", "layer_in_last", "final_in", "concat_input_ids"}
    parent.set_corpus_meta(100)

    parent.notify_buffer_full(7, [3, 4], epoch=0)
    ack = parent.poll_response(timeout=60)
    assert ack["event"] == "activations_processed"
    assert ack["n"] == 7 and ack["loss"] == 1.25 and ack["samples"] == 2
    assert ack["gpu_ms"] is not None and ack["wall_ms"] >= 0
    assert svc.calls == [([3, 4], 7, 0, 28.0)]
    assert svc._total_tokens_trained == 7 and svc.ledger.meter() == "7/100"
    # every shared activation buffer (the child's view) is zeroed after the cycle
    mine = svc.activations
    assert not any(t.any() for t in mine["layer_in"]) and not mine["final_in"].any()
    assert not mine["concat_input_ids"].any()

    new = {k: v + 1 for k, v in ft.items()}
    sw = parent.switch_adapter(new, {"learning_rate": 1e-4, "weight_decay": 0.0, "gamma": 1.0,
                                     "total_tokens_per_epoch": 50})
    assert sw == {"event": "adapter_switched", "tensors": 4}
    assert svc.ledger.meter() == "0/50"
    state = parent.export_lora()
    assert set(state) == set(new) and all(torch.equal(state[k], new[k]) for k in new)
    shard = tmp_path / "job" / "rank0.safetensors"
    assert parent.save_lora(str(shard)) == {"event": "lora_save_started", "tensors": 4}
    for _ in range(500):
        if shard.exists():
            break
        import time
        time.sleep(0.01)
    back = load_file(str(shard))
    assert all(torch.equal(back[k], new[k]) for k in new)
    with pytest.raises(RuntimeError, match="refused the adapter: ValueError"):
        parent.switch_adapter({"other": torch.zeros(1)}, {})

    parent.conn.send({"cmd": "bogus"})
    assert parent.poll_response(timeout=30) == {"event": "error", "msg": "unknown cmd 'bogus'"}
    assert parent.shutdown() == {"event": "bye", "pid": os.getpid()}
    pipe.join()


def test_cycle_skipped_and_failed_acks_carry_no_loss():
    from parent_protocol import InlinePipe

    svc = _CpuTrainer()
    pipe = InlinePipe(svc)
    parent = pipe.parent
    parent.ready()
    # no activations shared yet: the cycle is skipped
    parent.notify_buffer_full(5, [5], epoch=0)
    ack = parent.poll_response(timeout=60)
    assert ack["loss"] is None and ack["gpu_ms"] is None and svc.calls == []
    parent.share_activations(_buffers())
    parent.notify_buffer_full(0, [], epoch=0)  # nothing to train
    assert parent.poll_response(timeout=60)["loss"] is None
    parent.notify_buffer_full(5, [5], epoch=3)  # process_backward raises
    ack = parent.poll_response(timeout=60)
    assert ack["event"] == "activations_processed" and ack["loss"] is None
    assert svc._total_tokens_trained == 0 and len(svc.calls) == 1
    parent.shutdown()
    pipe.join()


def test_weights_error_travels_back_and_protocol_only_service(tmp_path):
    from parent_protocol import InlinePipe

    from deltaserve_amd import checkpoint

    svc = _CpuTrainer()
    pipe = InlinePipe(svc)
    parent = pipe.parent
    parent.ready()
    got = parent.share_weights({}, {}, meta={})
    assert got["error"].startswith("ValueError") and got["hash_report"] == {}
    parent.shutdown()
    pipe.join()

    # the registry's protocol-only child trains nothing and says so
    proto = registry.get_service("ipc")(0)
    pipe = InlinePipe(proto)
    parent = pipe.parent
    parent.ready()
    parent.share_weights({}, {}, meta={"tp_rank": 0})
    with pytest.raises(RuntimeError, match="does not train an adapter"):
        parent.switch_adapter({}, {})
    assert parent.export_lora() == {}
    parent.request_save_adapter(str(tmp_path / "s"), "id1")
    assert parent.ping()["event"] == "pong"  # the fire-and-forget command was handled first
    res = checkpoint.read_save_result(str(tmp_path / "s"), "id1")
    assert res["saved"] is False and "trains no adapter" in res["error"]
    parent.shutdown()
    pipe.join()


def test_child_exits_when_the_parent_closes_the_pipe():
    from parent_protocol import InlinePipe

    pipe = InlinePipe(_CpuTrainer())
    pipe.parent.ready()
    pipe.parent_end.close()
    pipe.join()


def test_service_main_runs_the_protocol_child():
    """The spawn entry (base.py:48-68) on the protocol-only service, over a
    real multiprocessing pipe, in a thread of this process."""
    import multiprocessing as mp
    import threading

    from deltaserve_amd.bwd_services import service_main

    parent, child = mp.Pipe()
    t = threading.Thread(target=service_main, args=(child, 100, 0, "ipc", None))
    t.start()
    assert parent.recv()["event"] == "ready"
    parent.send({"cmd": "ping"})
    assert parent.recv()["event"] == "pong"
    parent.send({"cmd": "shutdown"})
    assert parent.recv()["event"] == "bye"
    t.join(10)
    assert not t.is_alive()


# ------------------------------------------------------------------ fingerprints

def test_digest_is_sha1_of_fp32_bytes():
    """backward_process.py:44-47: SHA-1 over the values as fp32, first 16 hex
    digits, whatever the dtype; checked against hashlib over numpy bytes."""
    import hashlib

    import numpy as np

    from deltaserve_amd import integrity

    t = torch.arange(12, dtype=torch.bfloat16).reshape(3, 4) / 7
    want = hashlib.sha1(np.asarray(t.float().tolist(), dtype="<f4").tobytes()).hexdigest()[:16]
    assert integrity.tensor_digest(t) == want
    assert integrity.tensor_digest(t.float()) == want
    assert integrity.tensor_digest(t[:, :2]) != want


def test_hash_reports_pick_the_extreme_layers():
    from deltaserve_amd import integrity

    base = {f"model.layers.{i}.mlp.fc1.{suffix}": torch.full((2,), float(i))
            for i in (3, 0, 11) for suffix in ("weight", "bias")}
    base["model.layers.20.mlp.fc1.lora_A.weight"] = torch.zeros(2)
    ft = {f"base_model.model.model.layers.{i}.self_attn.q_proj.lora_A.weight": torch.ones(2) * i
          for i in (2, 7)}
    rep = integrity.weight_hash_report(base, ft)
    assert rep["base_ffn_fc1_first"][:2] == (0, "model.layers.0.mlp.fc1.weight")
    assert rep["base_ffn_fc1_last"][:2] == (11, "model.layers.11.mlp.fc1.weight")
    assert rep["ft_q_loraA_first"][0] == 2 and rep["ft_q_loraA_last"][0] == 7
    assert rep["base_ffn_fc1_last"][2] == integrity.tensor_digest(torch.full((2,), 11.0))
    acts = {"layer_in": [torch.ones(5, 2), torch.zeros(5, 2)],
            "mlp_gate_up": [torch.ones(5, 4)], "concat_input_ids": torch.arange(5)}
    rep = integrity.activation_hash_report(acts, 3)
    assert rep["layer_in_first"] == integrity.tensor_digest(torch.ones(3, 2))
    assert rep["layer_in_last"] == integrity.tensor_digest(torch.zeros(3, 2))
    assert rep["mlp_gate_up_first"] == rep["mlp_gate_up_last"]
    assert integrity.activation_hash_report(acts, 0) == {}


# ------------------------------------------------------------------ pause points

class _Counter:
    def __init__(self):
        self.value = 0

    def read(self):
        return self.value


class _Clock:
    def __init__(self):
        self.t = 0.0

    def __call__(self):
        return self.t


def test_arrival_watch_holds_until_the_prefill_pause_ends():
    """base.py:224-262: an arrival holds the cycle until the worker's pause for
    its prefill is over, or 0.1 s when no pause follows."""
    from deltaserve_amd.pause import ArrivalWatch

    c, clk = _Counter(), _Clock()
    w = ArrivalWatch(c, clock=clk)
    assert not w.blocks(True)
    c.value = 1                      # a request arrives
    assert w.blocks(True)            # waiting for the worker to pause us
    clk.t = 0.05
    assert w.blocks(False)           # paused for its prefill
    clk.t = 5.0
    assert w.blocks(False)           # still paused: no time limit here
    assert not w.blocks(True)        # the prefill is over
    assert not w.blocks(True)
    c.value = 2                      # another arrival, no pause follows
    clk.t = 6.0
    assert w.blocks(True)
    clk.t = 6.05
    assert w.blocks(True)
    clk.t = 6.2
    assert not w.blocks(True)        # grace elapsed
    c.value = 5
    w.rebase()                       # a new cycle: earlier arrivals are not its business
    assert not w.blocks(True)


def test_pause_gate_waits_for_the_grant_and_for_arrivals(monkeypatch):
    import threading
    import time

    from multiprocessing import shared_memory

    from deltaserve_amd import pause

    grant = threading.Event()
    gate = pause.PauseGate(grant, lambda: {})
    threading.Timer(0.05, grant.set).start()
    t0 = time.monotonic()
    gate.hold()
    assert grant.is_set() and time.monotonic() - t0 >= 0.04

    # pause_on_arrival through a real shared-memory counter
    shm = shared_memory.SharedMemory(create=True, size=8)
    try:
        shm.buf[:8] = (0).to_bytes(8, "little")
        monkeypatch.setenv(pause.ARRIVAL_ENV, shm.name)
        gate = pause.PauseGate(grant, lambda: {"pause_on_arrival": True})
        gate.cycle_started()
        assert gate.watch() is not None
        gate.hold()                                  # nothing arrived
        shm.buf[:8] = (1).to_bytes(8, "little")
        t0 = time.monotonic()
        gate.hold()                                  # arrival, no prefill: the 0.1 s grace
        assert 0.08 <= time.monotonic() - t0 < 2.0
        gate.watch().counter.close()
    finally:
        shm.close()
        shm.unlink()
    # without the meta flag the counter is never attached
    gate = pause.PauseGate(grant, lambda: {})
    assert gate.watch() is None


def test_service_holds_at_pause_points_while_the_grant_is_cleared():
    import threading
    import time

    svc = _CpuTrainer()
    grant = threading.Event()
    svc._gpu_grant = grant
    threading.Timer(0.05, grant.set).start()
    t0 = time.monotonic()
    svc._maybe_pause()
    assert time.monotonic() - t0 >= 0.04


# ------------------------------------------------------------------ handover line

def test_handover_line_save_switch_ping(tmp_path, monkeypatch):
    """handover_channel.py:77-103 over a real unix socket with the engine's
    authkey rule."""
    from multiprocessing.connection import Client

    from safetensors.torch import load_file, save_file

    from deltaserve_amd import handover

    sock_dir = tmp_path / "h"
    sock_dir.mkdir()
    monkeypatch.setenv(handover.ENV, str(sock_dir))
    svc = _CpuTrainer()
    svc.shared = {"base": {}, "ft": _adapter(), "meta": {}}
    svc._on_weights_shared()
    line = handover.open_line(svc)
    assert line is not None
    path = handover.socket_path(str(sock_dir), 0)
    with Client(path, family="AF_UNIX", authkey=handover.authkey(path)) as c:
        c.send(("ping",))
        assert c.recv() == ("ok", {"pid": os.getpid()})
        shard = tmp_path / "out" / "rank0.safetensors"
        c.send(("save", str(shard)))
        assert c.recv() == ("ok", {"tensors": 4})
        assert sorted(load_file(str(shard))) == sorted(_adapter())
        adir = tmp_path / "next"
        adir.mkdir()
        nxt = {k: v * 2 for k, v in _adapter().items()}
        save_file(nxt, str(adir / "adapter_model.safetensors"))
        (adir / "adapter_config.json").write_text(json.dumps({"r": 4, "lora_alpha": 8}))
        c.send(("switch", str(adir), {"total_tokens_per_epoch": 9}))
        assert c.recv() == ("ok", {"tensors": 4})
        assert all(torch.equal(svc.masters_[k], nxt[k]) for k in nxt)
        c.send(("nonsense",))
        assert c.recv() == ("error", "unknown request 'nonsense'")
    line.close()
    assert handover.adapter_scaling(str(adir)) == 2.0
    assert handover.adapter_scaling(None) == 1.0
    monkeypatch.delenv(handover.ENV)
    assert handover.open_line(svc) is None


# ------------------------------------------------------------------ configs

@pytest.mark.parametrize("name", sorted(configs.CONFIGS))
def test_config_lengths(name):
    c = configs.CONFIGS[name]
    a = configs.draw_lengths(c["nseq"], c["lo"], c["hi"], c["total"], seed=0)
    b = configs.draw_lengths(c["nseq"], c["lo"], c["hi"], c["total"], seed=0)
    assert a == b and len(a) == c["nseq"]
    assert all(c["lo"] <= x <= c["hi"] for x in a)
    if c["total"] is not None:
        assert sum(a) == c["total"]


def test_c3_algorithmic_flops():
    c = configs.CONFIGS["c3"]
    lens = configs.draw_lengths(c["nseq"], c["lo"], c["hi"], c["total"], seed=0)
    f = configs.algorithmic_flops(c, lens)
    # Frozen dense products: 32 layers × 8192 rows × (4·4096·6144 + 4·4096·4096 + 10·4096·14336)
    assert f["dense"] == 32 * 8192 * (4 * 4096 * 6144 + 4 * 4096 * 4096 + 10 * 4096 * 14336)
    assert f["head"] == 4 * (8192 - 32) * 4096 * 128256
    assert 218e12 < f["total"] < 221e12
