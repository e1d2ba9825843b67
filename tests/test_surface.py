"""Host-side surface of the drop-in backward child, on the CPU: service
registry (registry.py:15-49), backward meta (ft_meta.py:24-213), PEFT adapter
checkpoints (adapter_io.py:95-159), the parent's bwd_log row
(coordinator.py:1079-1109), the pipe protocol and per-cycle wrapper of
BackwardService (base.py:297-408, :468-633) and the workload configs."""

from __future__ import annotations

import csv
import json
import os
import types

import pytest
import torch

from deltaserve_amd import adapter_io, bwd_log, configs, ft_meta
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


# ------------------------------------------------------------------ meta

def _cfg(**kw):
    base = dict(num_attention_heads=32, num_key_value_heads=8, hidden_size=4096,
                intermediate_size=14336, num_hidden_layers=32, vocab_size=128256,
                rms_norm_eps=1e-5)
    base.update(kw)
    return types.SimpleNamespace(**base)


def test_rope_scaling_normalisation():
    assert ft_meta.rope_scaling_of(_cfg(rope_parameters={"rope_type": "default",
                                                         "rope_theta": 5e5})) is None
    rs = ft_meta.rope_scaling_of(_cfg(rope_scaling={"type": "llama3", "factor": 8,
                                                    "low_freq_factor": 1, "high_freq_factor": 4,
                                                    "original_max_position_embeddings": 8192}))
    assert rs == {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                  "high_freq_factor": 4.0, "original_max_position_embeddings": 8192.0}
    assert ft_meta.rope_scaling_of(_cfg(rope_scaling={"rope_type": "linear",
                                                      "factor": 2})) == {"rope_type": "linear",
                                                                          "factor": 2.0}


@pytest.mark.parametrize("rp", [{"rope_type": "yarn", "factor": 4.0},
                                {"rope_type": "default", "partial_rotary_factor": 0.5},
                                {"rope_type": "default", "mrope_section": [16, 24, 24]},
                                {"rope_type": "llama3", "factor": 8.0}])
def test_rope_scaling_rejects_what_the_backward_cannot_reproduce(rp):
    with pytest.raises(ValueError):
        ft_meta.rope_scaling_of(_cfg(rope_parameters=rp))


def test_rope_theta_sources():
    assert ft_meta.rope_theta_of(_cfg(rope_parameters={"rope_theta": 1e6})) == 1e6
    assert ft_meta.rope_theta_of(_cfg(rope_theta=5e5)) == 5e5
    assert ft_meta.rope_theta_of(_cfg()) == 10000.0


def test_lora_scaling_from_adapter_config(tmp_path):
    assert ft_meta.read_lora_scaling(None) == 1.0
    assert ft_meta.read_lora_scaling(str(tmp_path)) == 1.0
    (tmp_path / "adapter_config.json").write_text(json.dumps({"r": 16, "lora_alpha": 32}))
    assert ft_meta.read_lora_scaling(str(tmp_path)) == 2.0


def test_backward_meta_keys():
    ft = types.SimpleNamespace(learning_rate=2e-4, max_saved_finetuning_tokens=8192,
                               backward_max_seqs=32)
    m = ft_meta.build_backward_meta(_cfg(rope_parameters={"rope_theta": 5e5}), ft,
                                    lm_head_key="lm_head.weight",
                                    embed_weight_key="model.embed_tokens.weight",
                                    has_final_norm=True, lora_scaling=2.0)
    assert m["head_dim"] == 128 and m["rope_theta"] == 5e5 and m["rope_scaling"] is None
    assert m["learning_rate"] == 2e-4 and m["max_saved_finetuning_tokens"] == 8192
    assert m["norm_weight_key"] == "model.norm.weight" and m["tp_size"] == 1


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
    assert not [f for f in os.listdir(out) if ".tmp-" in f]


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


# ------------------------------------------------------------------ bwd_log

def test_bwd_log_rows(tmp_path):
    path = tmp_path / "m" / "bwd_log.csv"
    log = bwd_log.BwdLog(str(path))
    log.write_row(0, 100, 2.5)
    log.write_row(1, 50, None)
    rows = list(csv.reader(open(path)))
    assert rows[0] == bwd_log.HEADER
    assert rows[1][1:] == ["0", "1", "100", "2.5", "100"]
    assert rows[2][1:] == ["1", "2", "50", "", "150"]


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
