"""The engine's direct line to the backward child for the adapter handover.

At the end of a finetuning job the engine saves the trained adapter and hands
the child the next job's, from a background thread of its own and not through
the worker's command pipe (``deltaserve-plugin/deltaserve/handover_channel.py``).
The child side is a unix-socket listener served by daemon threads beside the
command loop. The engine's client fixes the contract this module keeps:

* socket ``<$DSERVE_HANDOVER_DIR>/rank<N>.sock`` (N = the child's rank; one GPU
  per model here, so the device index), authkey = SHA-256 of
  ``b"deltaserve-handover" + path`` (handover_channel.py:49-56);
* requests ``("ping",)``, ``("save", shard_path)``,
  ``("switch", adapter_dir, hparams)``; replies ``("ok", payload)`` or
  ``("error", message)`` (handover_channel.py:77-103).

Callers only use the line while no backward is in flight (the job's training
stage is over), the same rule as for the pipe's ``save_lora`` / ``switch_adapter``.
"""

from __future__ import annotations

import hashlib
import json
import os
import threading
from multiprocessing.connection import Listener

from deltaserve_amd import dprint

ENV = "DSERVE_HANDOVER_DIR"


def socket_path(directory: str, rank: int) -> str:
    return os.path.join(directory, f"rank{int(rank)}.sock")


def authkey(path: str) -> bytes:
    return hashlib.sha256(b"deltaserve-handover" + path.encode()).digest()


def write_shard(state: dict, path: str) -> int:
    """The adapter ``state`` as fp32 safetensors at ``path``; the file gets its
    name only once complete. Returns the tensor count."""
    from safetensors.torch import save_file

    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    partial = path + ".tmp"
    save_file({k: v.detach().float().cpu().contiguous() for k, v in state.items()}, partial)
    os.replace(partial, path)
    return len(state)


def write_shard_in_background(state: dict, path: str) -> threading.Thread:
    """``write_shard`` on a daemon thread; a failure leaves ``path + ".error"``
    with the reason instead of the file (base.py:72-91 of the reference)."""
    def job():
        try:
            write_shard(state, path)
        except Exception as e:  # noqa: BLE001 — the engine reads the reason file
            try:
                with open(path + ".error", "w") as f:
                    f.write(f"{type(e).__name__}: {e}")
            except OSError:
                pass

    t = threading.Thread(target=job, daemon=True, name="deltaserve-shard-writer")
    t.start()
    return t


def adapter_scaling(adapter_dir: str | None) -> float:
    """alpha / r from ``adapter_config.json`` (1.0 without one; ft_meta.py:89-101)."""
    cfg = os.path.join(adapter_dir or "", "adapter_config.json")
    if not adapter_dir or not os.path.exists(cfg):
        return 1.0
    with open(cfg) as f:
        conf = json.load(f)
    r = float(conf.get("r", 1) or 1)
    return float(conf.get("lora_alpha", r)) / r


def _load_adapter(svc, adapter_dir: str) -> dict:
    import torch
    from safetensors.torch import load_file

    where = f"cuda:{svc.device_index}" if torch.cuda.is_available() else "cpu"
    raw = load_file(os.path.join(adapter_dir, "adapter_model.safetensors"), device=where)
    return {k: v.float() for k, v in raw.items()}


def answer(svc, request) -> tuple:
    """One request against the service; never raises."""
    try:
        op = request[0]
        if op == "ping":
            return ("ok", {"pid": os.getpid()})
        if op == "save":
            return ("ok", {"tensors": write_shard(svc.export_lora_state(), request[1])})
        if op == "switch":
            adapter_dir, hparams = request[1], dict(request[2] or {})
            hparams["lora_scaling"] = adapter_scaling(adapter_dir)
            return ("ok", svc.switch_adapter(_load_adapter(svc, adapter_dir), hparams))
        return ("error", f"unknown request {op!r}")
    except Exception as e:  # noqa: BLE001 — reported to the engine
        return ("error", f"{type(e).__name__}: {e}")


class HandoverLine:
    """The child's listener: one thread accepts, one thread per connection
    answers its requests in order."""

    def __init__(self, svc, path: str) -> None:
        self.svc, self.path = svc, path
        try:
            os.unlink(path)
        except OSError:
            pass
        self._listener = Listener(path, family="AF_UNIX", authkey=authkey(path))
        os.chmod(path, 0o600)
        threading.Thread(target=self._accept, daemon=True,
                         name="deltaserve-handover-accept").start()

    def _accept(self) -> None:
        while True:
            try:
                conn = self._listener.accept()
            except Exception:  # noqa: BLE001 — listener closed: the child is leaving
                return
            threading.Thread(target=self._serve, args=(conn,), daemon=True,
                             name="deltaserve-handover").start()

    def _serve(self, conn) -> None:
        with conn:
            while True:
                try:
                    request = conn.recv()
                except (EOFError, OSError):
                    return
                try:
                    conn.send(answer(self.svc, request))
                except OSError:
                    return

    def close(self) -> None:
        try:
            self._listener.close()
        except OSError:
            pass


def open_line(svc, rank: int | None = None) -> HandoverLine | None:
    """Listen for the engine when it offers a directory (``$DSERVE_HANDOVER_DIR``);
    None otherwise, or when the socket cannot be created (the handover then
    goes through the command pipe)."""
    directory = os.environ.get(ENV)
    if not directory or not os.path.isdir(directory):
        return None
    path = socket_path(directory, svc.device_index if rank is None else rank)
    try:
        return HandoverLine(svc, path)
    except Exception as e:  # noqa: BLE001 — never keeps the child from starting
        dprint(f"[backward] no handover line ({type(e).__name__}: {e})")
        return None
