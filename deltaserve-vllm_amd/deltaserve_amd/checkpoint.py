"""Trained-adapter checkpoints of the backward child.

On-disk contract (what the reference's readers and PEFT loaders expect,
``deltaserve-plugin/deltaserve/adapter_io.py:95-159``):

* ``adapter_model.safetensors`` — the fp32 LoRA masters under the source
  adapter's PEFT keys, B unscaled (PEFT applies ``lora_alpha / r`` itself);
* ``adapter_config.json`` — the source adapter's config, or a minimal LoRA
  config built from the tensors;
* ``trainer_state.json`` — training progress plus the request's ``save_id``,
  written last: its appearance is the completion marker;
* ``save_error.json`` — ``{save_id, error, unix_time}`` when a save failed.

Every file appears whole (written beside its final name, then renamed).

The periodic policy (meta ``adapter_save_path``, ``adapter_save_every_backwards``,
``adapter_save_every_epoch``, ``adapter_save_keep_last``; reference
``trainer.py:405-437``) is a small state machine, :class:`CheckpointSchedule`:
when the first cycle of a new epoch starts, the state left by the previous
epoch's last cycle is captured and written once that cycle has replied, and
every N-th attempted cycle writes ``backward-NNNNNN`` and prunes the oldest.
"""

from __future__ import annotations

import contextlib
import json
import os
import re
import shutil
import time
from dataclasses import dataclass, field

import torch

WEIGHTS_FILE = "adapter_model.safetensors"
CONFIG_FILE = "adapter_config.json"
STATE_FILE = "trainer_state.json"
ERROR_FILE = "save_error.json"

_TARGET_RE = re.compile(r"\.(\w+_proj)\.lora_")


@contextlib.contextmanager
def _staged(final_path: str):
    """Yields a sibling path to write; on success it replaces ``final_path``
    in one rename, on failure it is removed."""
    staging = f"{final_path}.part{os.getpid()}"
    try:
        yield staging
        os.replace(staging, final_path)
    finally:
        with contextlib.suppress(FileNotFoundError):
            os.remove(staging)


def _put_json(path: str, payload: dict) -> None:
    with _staged(path) as tmp, open(tmp, "w") as fh:
        fh.write(json.dumps(payload, indent=2, sort_keys=True))


def lora_config_for(tensors: dict, scaling: float, source_dir: str | None = None) -> dict:
    """The source adapter's ``adapter_config.json`` when there is one (the
    trained factors keep its shapes), else a minimal PEFT LoRA config whose
    rank, alpha = scaling · r and target modules come from ``tensors``."""
    if source_dir:
        path = os.path.join(source_dir, CONFIG_FILE)
        if os.path.isfile(path):
            with open(path) as fh:
                return json.load(fh)
    rank = 1
    for key, t in tensors.items():
        if "lora_A" in key:
            rank = int(t.shape[0])
            break
    modules = sorted({m.group(1) for m in map(_TARGET_RE.search, tensors) if m})
    return {"peft_type": "LORA", "task_type": "CAUSAL_LM", "r": rank,
            "lora_alpha": float(scaling) * rank, "target_modules": modules,
            "lora_dropout": 0.0, "bias": "none"}


def write_peft_adapter(out_dir: str, tensors: dict, *, source_dir: str | None,
                       scaling: float, state: dict) -> str:
    """Writes one checkpoint directory (weights, config, then the state file
    that marks it complete); clears a stale error file. Returns ``out_dir``."""
    from safetensors.torch import save_file

    os.makedirs(out_dir, exist_ok=True)
    host = {key: t.detach().float().cpu().contiguous() for key, t in tensors.items()}
    with _staged(os.path.join(out_dir, WEIGHTS_FILE)) as tmp:
        save_file(host, tmp, metadata={"format": "pt"})
    _put_json(os.path.join(out_dir, CONFIG_FILE), lora_config_for(host, scaling, source_dir))
    with contextlib.suppress(FileNotFoundError):
        os.remove(os.path.join(out_dir, ERROR_FILE))
    done = dict(state)
    done["num_tensors"] = len(host)
    done["saved_unix_time"] = time.time()
    _put_json(os.path.join(out_dir, STATE_FILE), done)
    return out_dir


def write_save_error(out_dir: str, save_id: str, message: str) -> None:
    """Leaves the failure where a waiting save request looks for it; an
    unwritable directory is ignored (there is nowhere else to report it)."""
    with contextlib.suppress(OSError):
        os.makedirs(out_dir, exist_ok=True)
        _put_json(os.path.join(out_dir, ERROR_FILE),
                  {"save_id": save_id, "error": message, "unix_time": time.time()})


def read_save_result(out_dir: str, save_id: str) -> dict | None:
    """``{"saved": True, **state}`` or ``{"saved": False, "error": ...}`` once
    save ``save_id`` has finished, ``None`` before."""
    for fname, saved in ((STATE_FILE, True), (ERROR_FILE, False)):
        try:
            with open(os.path.join(out_dir, fname)) as fh:
                record = json.load(fh)
        except (OSError, ValueError):
            continue
        if record.get("save_id") == save_id:
            return {"saved": saved, **record}
    return None


def prune_checkpoints(root: str, prefix: str, keep_last: int) -> list[str]:
    """Removes every ``root/<prefix><number>`` directory but the ``keep_last``
    highest-numbered (``keep_last <= 0`` keeps all). Returns what was removed."""
    if keep_last <= 0 or not os.path.isdir(root):
        return []
    pattern = re.compile(re.escape(prefix) + r"(\d+)")
    numbered = []
    for entry in os.scandir(root):
        m = pattern.fullmatch(entry.name)
        if m and entry.is_dir():
            numbered.append((int(m.group(1)), entry.path))
    numbered.sort()
    doomed = [path for _, path in numbered[:max(0, len(numbered) - keep_last)]]
    for path in doomed:
        shutil.rmtree(path, ignore_errors=True)
    return doomed


@dataclass
class Snapshot:
    """An adapter and its training progress, frozen at one moment."""
    tensors: dict | None
    error: str | None
    state: dict


@dataclass
class CheckpointSchedule:
    """The periodic-save state machine of one backward child."""
    root: str | None = None
    every_cycles: int = 0
    every_epoch: bool = False
    keep_last: int = 0
    attempted: int = 0
    last_epoch: int | None = None
    pending: tuple | None = field(default=None, repr=False)  # (epoch, Snapshot)

    @classmethod
    def from_meta(cls, meta: dict) -> "CheckpointSchedule":
        return cls(root=meta.get("adapter_save_path") or None,
                   every_cycles=int(meta.get("adapter_save_every_backwards") or 0),
                   every_epoch=bool(meta.get("adapter_save_every_epoch") or False),
                   keep_last=int(meta.get("adapter_save_keep_last") or 0))

    def epoch_rolled(self, epoch: int) -> int | None:
        """The finished epoch to checkpoint when a cycle of ``epoch`` starts."""
        if not (self.root and self.every_epoch) or self.last_epoch is None:
            return None
        return self.last_epoch if epoch > self.last_epoch else None

    def cycle_done(self, epoch: int) -> str | None:
        """Counts an attempted cycle; the periodic checkpoint name it is due."""
        self.attempted += 1
        self.last_epoch = epoch
        if self.root and self.every_cycles > 0 and self.attempted % self.every_cycles == 0:
            return f"backward-{self.attempted:06d}"
        return None


class AdapterCheckpointer:
    """Snapshots a trainer's masters and writes them under the contract above.

    ``owner`` provides ``masters()`` (PEFT key → fp32 tensor), ``scaling``,
    the progress counters and ``shared["meta"]``."""

    def __init__(self, owner) -> None:
        self.owner = owner
        self.schedule = CheckpointSchedule()

    def configure(self, meta: dict) -> None:
        attempted, last = self.schedule.attempted, self.schedule.last_epoch
        self.schedule = CheckpointSchedule.from_meta(meta or {})
        self.schedule.attempted, self.schedule.last_epoch = attempted, last

    @torch.no_grad()
    def snapshot(self, reason: str, epoch: int) -> Snapshot:
        o = self.owner
        try:
            tensors = {key: t.detach().to("cpu", copy=True) for key, t in o.masters()}
            error = None
        except Exception as e:  # noqa: BLE001 — reported through the error file
            tensors, error = None, f"rank 0: {type(e).__name__}: {e}"
        state = {"reason": reason, "epoch": int(epoch),
                 "backward_cycles": int(self.schedule.attempted),
                 "tokens_trained": int(o._total_tokens_trained),
                 "last_loss": o._last_loss, "learning_rate": float(o.lr), "tp_size": 1,
                 "source_adapter": (o.shared.get("meta") or {}).get("finetuning_lora_path")}
        return Snapshot(tensors, error, state)

    def write(self, out_dir: str, save_id: str, snap: Snapshot) -> bool:
        from deltaserve_amd import dprint

        reason = snap.state["reason"]
        problem = snap.error
        if problem is None:
            try:
                write_peft_adapter(out_dir, snap.tensors,
                                   source_dir=snap.state.get("source_adapter"),
                                   scaling=self.owner.scaling,
                                   state={**snap.state, "save_id": save_id})
                dprint(f"[backward] adapter saved ({reason}) → {out_dir}")
                return True
            except Exception as e:  # noqa: BLE001
                problem = f"{type(e).__name__}: {e}"
        dprint(f"[backward] adapter save ({reason}) to {out_dir} FAILED: {problem}")
        write_save_error(out_dir, save_id, problem)
        return False

    # ---- the cycle hooks
    def before_cycle(self, epoch: int) -> None:
        done = self.schedule.epoch_rolled(epoch)
        if done is not None:
            self.schedule.pending = (done, self.snapshot("epoch", done))

    def after_cycle(self, epoch: int) -> None:
        import os as _os

        due = self.schedule.cycle_done(epoch)
        root = self.schedule.root
        if self.schedule.pending is not None:
            done, snap = self.schedule.pending
            self.schedule.pending = None
            self.write(_os.path.join(root, f"epoch-{done}"), f"epoch-{done}", snap)
        if due is not None:
            self.write(_os.path.join(root, due), due, self.snapshot("every_backwards", epoch))
            prune_checkpoints(root, "backward-", self.schedule.keep_last)
