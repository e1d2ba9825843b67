"""Trained-adapter checkpoints in PEFT format (adapter_io.py:95-159 of the
reference): ``adapter_model.safetensors`` (fp32 masters under the source
adapter's keys, B unscaled), ``adapter_config.json`` (the source's, or a
minimal LoRA config), and ``trainer_state.json`` written last as the
completion marker. Each file is written to a temporary name and renamed."""

from __future__ import annotations

import json
import os
import re
import shutil
import time

import torch

STATE_FILE = "trainer_state.json"
ERROR_FILE = "save_error.json"
WEIGHTS_FILE = "adapter_model.safetensors"
CONFIG_FILE = "adapter_config.json"


def _replace_atomically(path: str, writer) -> None:
    tmp = f"{path}.tmp-{os.getpid()}"
    try:
        writer(tmp)
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise


def _write_json(path: str, obj) -> None:
    def w(tmp):
        with open(tmp, "w") as f:
            json.dump(obj, f, indent=2, sort_keys=True)
    _replace_atomically(path, w)


def adapter_config(source_dir: str | None, tensors: dict, scaling: float) -> dict:
    if source_dir:
        src = os.path.join(source_dir, CONFIG_FILE)
        if os.path.isfile(src):
            with open(src) as f:
                return json.load(f)
    r = next((t.shape[0] for k, t in tensors.items() if "lora_A" in k), 1)
    targets = sorted({m.group(1) for k in tensors
                      if (m := re.search(r"\.(\w+_proj)\.lora_", k))})
    return {"peft_type": "LORA", "task_type": "CAUSAL_LM", "r": int(r),
            "lora_alpha": float(scaling) * int(r), "target_modules": targets,
            "lora_dropout": 0.0, "bias": "none"}


def write_peft_adapter(out_dir: str, tensors: dict, *, source_dir: str | None,
                       scaling: float, state: dict) -> str:
    from safetensors.torch import save_file

    os.makedirs(out_dir, exist_ok=True)
    cpu = {k: v.detach().to("cpu", torch.float32).contiguous() for k, v in tensors.items()}
    _replace_atomically(os.path.join(out_dir, WEIGHTS_FILE),
                        lambda tmp: save_file(cpu, tmp, metadata={"format": "pt"}))
    _write_json(os.path.join(out_dir, CONFIG_FILE), adapter_config(source_dir, cpu, scaling))
    err = os.path.join(out_dir, ERROR_FILE)
    if os.path.exists(err):
        os.remove(err)
    _write_json(os.path.join(out_dir, STATE_FILE),
                {**state, "saved_unix_time": time.time(), "num_tensors": len(cpu)})
    return out_dir


def write_save_error(out_dir: str, save_id: str, message: str) -> None:
    try:
        os.makedirs(out_dir, exist_ok=True)
        _write_json(os.path.join(out_dir, ERROR_FILE),
                    {"save_id": save_id, "error": message, "unix_time": time.time()})
    except OSError:
        pass


def read_save_result(out_dir: str, save_id: str) -> dict | None:
    for name, ok in ((STATE_FILE, True), (ERROR_FILE, False)):
        try:
            with open(os.path.join(out_dir, name)) as f:
                d = json.load(f)
        except (OSError, ValueError):
            continue
        if d.get("save_id") == save_id:
            return {"saved": ok, **d}
    return None


def prune_checkpoints(root: str, prefix: str, keep_last: int) -> list[str]:
    if keep_last <= 0 or not os.path.isdir(root):
        return []
    found = []
    for name in os.listdir(root):
        m = re.fullmatch(re.escape(prefix) + r"(\d+)", name)
        if m and os.path.isdir(os.path.join(root, name)):
            found.append((int(m.group(1)), os.path.join(root, name)))
    found.sort()
    removed = [p for _, p in found[:-keep_last]]
    for p in removed:
        shutil.rmtree(p, ignore_errors=True)
    return removed
