"""Host-side surface of the drop-in backward child, on the CPU: service
registry (registry.py:15-49), PEFT adapter checkpoints and their periodic
schedule (adapter_io.py:95-159, trainer.py:336-437), the pipe protocol and
per-cycle wrapper of BackwardService (base.py:297-408, :468-633) and the
workload configs."""

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

class _Conn:
    def __init__(self, msgs):
        self.inbox, self.sent = list(msgs), []

    def recv(self):
        return self.inbox.pop(0)

    def send(self, m):
        self.sent.append(m)


class _Recorder(BackwardService):
    def __init__(self):
        super().__init__(0)
        self.calls = []

    def process_backward(self, activations, sample_lens, n, epoch):
        self.calls.append((list(sample_lens), n, epoch,
                           float(activations["layer_in"][0][:n].sum())))
        if epoch == 3:
            raise RuntimeError("planted failure")
        return 1.25, sum(max(s - 1, 0) for s in sample_lens)


def _acts():
    return {"layer_in": [torch.ones(9, 4)], "final_in": torch.ones(9, 4),
            "concat_input_ids": torch.arange(8)}


def test_cycle_wrapper_protocol():
    acts = _acts()
    conn = _Conn([
        {"cmd": "ping"},
        {"cmd": "share_activations", "activations": acts},
        {"cmd": "set_corpus_meta", "total_tokens_per_epoch": 100},
        {"cmd": "process_activations", "n": 7, "sample_lens": [3, 4], "epoch": 0},
        {"cmd": "process_activations", "n": 0, "sample_lens": [], "epoch": 0},
        {"cmd": "bogus"},
        {"cmd": "shutdown"},
    ])
    svc = _Recorder()
    svc.run(conn)
    ev = [m["event"] for m in conn.sent]
    assert ev == ["ready", "pong", "activations_received", "activations_processed",
                  "activations_processed", "error", "shutdown_ack"]
    ack = conn.sent[3]
    assert ack["n"] == 7 and ack["loss"] == 1.25 and ack["samples"] == 2
    assert ack["gpu_ms"] is not None and ack["wall_ms"] >= 0
    assert svc.calls == [([3, 4], 7, 0, 28.0)]
    # token accounting counts raw rows (base.py:540-548); buffers zeroed after the cycle
    assert svc._total_tokens_trained == 7
    assert not acts["layer_in"][0].any() and not acts["final_in"].any()
    skipped = conn.sent[4]
    assert skipped["loss"] is None and skipped["gpu_ms"] is None


def test_cycle_failure_acks_with_no_loss():
    svc = _Recorder()
    conn = _Conn([{"cmd": "share_activations", "activations": _acts()},
                  {"cmd": "process_activations", "n": 5, "sample_lens": [5], "epoch": 3},
                  {"cmd": "shutdown"}])
    svc.run(conn)
    ack = conn.sent[2]
    assert ack["event"] == "activations_processed" and ack["loss"] is None
    assert svc._total_tokens_trained == 0


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


def test_service_main_runs_the_protocol_child():
    """The spawn entry (base.py:48-70) on the protocol-only service, over a
    real multiprocessing pipe in this process."""
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
    assert parent.recv()["event"] == "shutdown_ack"
    t.join(10)
    assert not t.is_alive()
