"""The backward child: its command loop and the wrapper around each cycle.

The parent is the reference's ``BackwardProcess``
(``deltaserve-plugin/deltaserve/backward_process.py:184-480``); this module
speaks its pipe protocol unchanged, so pointing the reference's service
registry at this package is the whole integration. The protocol, as the
parent sends and checks it:

=====================  ===========================  ======================================
command ``cmd``        keys read                    reply ``event`` (keys)
=====================  ===========================  ======================================
(on start)                                          ``ready`` (pid, mps_percentage,
                                                    max_connections)
``ping``               data                         ``pong`` (pid, data)
``share_weights``      base, ft, meta, print_hash   ``weights_received`` (base_num, ft_num,
                                                    hash_report, error [+ summary])
``checksum``           which                        ``checksum`` (which, value)
``share_activations``  buffers, print_hash          ``activations_received`` (num_layers)
``share_lora_buffers`` payload                      ``lora_buffers_received`` (num_layers)
``hash_activations``   n                            ``activation_hashes`` (hash_report)
``set_corpus_meta``    total_tokens_per_epoch       none
``process_activations`` n, sample_lens, epoch       ``activations_processed`` (n, loss,
                                                    samples, gpu_ms, wall_ms, mem)
``switch_adapter``     ft, hparams                  ``adapter_switched`` (+ result) or
                                                    ``error`` (msg)
``save_lora``          path                         ``lora_save_started`` (tensors) or
                                                    ``lora_save_failed`` (msg)
``export_lora``                                     ``lora_state`` (state)
``save_adapter``       path, save_id                none (the result goes to a file)
``shutdown``                                        ``bye`` (pid), then the loop ends
anything else                                       ``error`` (msg)
=====================  ===========================  ======================================

(backward_process.py:272-480 for the sends and the checks on the replies;
bwd_services/base.py:297-408 for the reference child.) A closed pipe ends the
loop. The ``[backward] start:`` and per-cycle ``[backward] <ms>ms (<mode>)
loss=…`` log lines keep the reference's format, which log readers parse.

A cycle (``process_activations``) runs the subclass's ``process_backward``
over the first ``n`` rows of the shared activation store, then zeroes every
shared activation buffer, then acks; the ack reopens FT admission, so
checkpoint writing (``_after_cycle``) happens after it. A failing cycle is
logged and acked with ``loss=None``. Throughput counts raw rows ``n``, not
the loss rows ``n_valid``.
"""

from __future__ import annotations

import math
import os
import time
import traceback
from dataclasses import dataclass, field

import torch

from deltaserve_amd import dprint, handover, integrity, mark_backward_process
from deltaserve_amd.pause import PauseGate

# Environment the child inherits from the parent's MPS wrapping; echoed in
# ``ready`` so the parent can log what the child got.
_ECHOED_ENV = ("CUDA_MPS_ACTIVE_THREAD_PERCENTAGE", "CUDA_DEVICE_MAX_CONNECTIONS")


def _die_with_parent() -> None:
    """Ask Linux to SIGKILL this child when its parent dies, so a killed
    engine leaves no child holding GPU memory."""
    import ctypes
    import signal
    import sys

    if not sys.platform.startswith("linux"):
        return
    try:
        pr_set_pdeathsig = 1
        ctypes.CDLL("libc.so.6", use_errno=True).prctl(pr_set_pdeathsig, signal.SIGKILL)
    except Exception as e:  # noqa: BLE001
        dprint(f"[backward child] parent-death signal not armed: {e}")
        return
    if os.getppid() == 1:
        dprint("[backward child] parent already gone at startup; exiting")
        os._exit(1)


def service_main(conn, mps_percentage: int, device_index: int, service_name: str,
                 gpu_grant=None) -> None:
    """Spawn target of the parent (bwd_services/base.py:48-68): choose the
    service by architecture string, bind the device and the GPU grant, run
    the loop. ``mps_percentage`` is the parent's argument; the MI355X child
    does not partition CUs."""
    from deltaserve_amd.bwd_services.registry import get_service

    import multiprocessing

    mark_backward_process()
    if multiprocessing.parent_process() is not None:  # a spawned child, not a thread
        _die_with_parent()
    if torch.cuda.is_available():
        torch.cuda.set_device(device_index)
    svc = get_service(service_name)(device_index)
    svc._gpu_grant = gpu_grant
    try:
        svc.run(conn)
    except KeyboardInterrupt:
        dprint("[backward] child interrupted by shutdown; exiting")
    finally:
        close = getattr(svc, "close", None)
        if close is not None:
            close()


# ---------------------------------------------------------------- bookkeeping

@dataclass
class TokenLedger:
    """Rows trained: since the child started, and in the current epoch out of
    the corpus size the parent announced (``set_corpus_meta``)."""

    total: int = 0
    epoch: int = 0
    in_epoch: int = 0
    per_epoch: int = 0

    def see_epoch(self, epoch: int) -> None:
        # a new epoch restarts the meter before the cycle's rows are added
        if epoch > self.epoch:
            self.epoch, self.in_epoch = epoch, 0

    def add(self, rows: int) -> None:
        self.total += rows
        self.in_epoch += rows

    def restart(self, per_epoch: int) -> None:
        """A new adapter (job): epoch and meter start over."""
        self.epoch, self.in_epoch, self.per_epoch = 0, 0, int(per_epoch)

    def meter(self) -> str:
        return f"{self.in_epoch}/{self.per_epoch if self.per_epoch > 0 else '?'}"


class CycleClock:
    """Device time of the wrapped region (HIP events on the current stream),
    or host time without a GPU. ``ms()`` waits for the end event only."""

    def __init__(self) -> None:
        self._events = None
        self._host = None

    def __enter__(self) -> "CycleClock":
        if torch.cuda.is_available():
            self._events = (torch.cuda.Event(enable_timing=True),
                            torch.cuda.Event(enable_timing=True))
            self._events[0].record()
        else:
            self._host = [time.perf_counter(), None]
        return self

    def __exit__(self, exc_type, exc, tb) -> bool:
        if exc_type is not None:
            self._events = self._host = None
        elif self._events is not None:
            self._events[1].record()
        else:
            self._host[1] = time.perf_counter()
        return False

    def ms(self) -> float | None:
        if self._events is not None:
            self._events[1].synchronize()
            return float(self._events[0].elapsed_time(self._events[1]))
        if self._host is not None and self._host[1] is not None:
            return (self._host[1] - self._host[0]) * 1000.0
        return None


@dataclass
class Cycle:
    """One ``process_activations`` request and what became of it."""

    n: int
    sample_lens: list
    epoch: int
    t_wall: float = field(default_factory=time.perf_counter)
    loss: object = None
    n_valid: int = 0
    clock: CycleClock | None = None

    @classmethod
    def of(cls, msg: dict) -> "Cycle":
        return cls(n=int(msg.get("n", 0)), sample_lens=list(msg.get("sample_lens") or []),
                   epoch=int(msg.get("epoch", 0)))

    def gpu_ms(self) -> float | None:
        ms = self.clock.ms() if self.clock is not None else None
        return None if ms is None or ms != ms else ms

    def ack(self, gpu_ms: float | None, mem: dict | None) -> dict:
        reply = {"event": "activations_processed", "n": self.n, "loss": self.loss,
                 "samples": len(self.sample_lens), "gpu_ms": gpu_ms,
                 "wall_ms": (time.perf_counter() - self.t_wall) * 1000.0}
        if mem is not None:
            reply["mem"] = mem
        return reply


# Command name -> handler method name. Handlers take the message and return
# the reply (or None for fire-and-forget commands); subclasses override the
# methods, not the table.
_COMMANDS: dict[str, str] = {}


def _command(name: str):
    def register(fn):
        _COMMANDS[name] = fn.__name__
        return fn
    return register


def _as_float(loss) -> float:
    try:
        return float(loss.item() if hasattr(loss, "item") else loss)
    except Exception:  # noqa: BLE001
        return float("nan")


class BackwardService:
    """The protocol-only child (registry name ``ipc``); trainers subclass it
    and implement ``process_backward`` and the adapter hooks."""

    def __init__(self, device_index: int) -> None:
        self.device_index = int(device_index)
        # The IPC-mapped dicts are held here for the child's lifetime, which
        # keeps the mappings alive.
        self.shared: dict = {"base": None, "ft": None, "meta": {}}
        self.activations: dict | None = None
        self.lora_buffers: dict | None = None
        self.current_epoch = 0
        self.ledger = TokenLedger()
        self._verify = False
        self._last_loss: float | None = None
        self._last_mode = "eager"
        self._pause = PauseGate(None, lambda: (self.shared or {}).get("meta") or {})
        self._after_reply: list = []
        self._handover = None

    # -- attributes other parts of the child read
    @property
    def _gpu_grant(self):
        return self._pause.grant

    @_gpu_grant.setter
    def _gpu_grant(self, grant) -> None:
        self._pause.grant = grant

    @property
    def _total_tokens_trained(self) -> int:
        return self.ledger.total

    # -- pause points (called by process_backward between its segments)
    def _maybe_pause(self) -> None:
        self._pause.hold()

    def _run_ahead(self) -> int:
        """Segments the host may queue ahead of the GPU while pause points are
        on (meta ``backward_run_ahead_boundaries``; 0 = unbounded)."""
        meta = (self.shared or {}).get("meta") or {}
        return max(0, int(meta.get("backward_run_ahead_boundaries", 0) or 0))

    # -- hooks for trainers
    def _on_weights_shared(self) -> str | None:
        """Build the training state; a returned string is sent back as the
        ``weights_received`` error (the worker then refuses to serve FT)."""
        return None

    def _on_lora_buffers(self) -> None:
        pass

    def _before_cycle(self, epoch: int, attempted: bool) -> None:
        pass

    def _after_cycle(self, epoch: int, attempted: bool) -> None:
        pass

    def verify_activations(self, activations: dict, n: int) -> None:
        pass

    def process_backward(self, activations, sample_lens, n, epoch):
        raise NotImplementedError(f"{type(self).__name__} trains nothing")

    def export_lora_state(self) -> dict:
        return {}

    def switch_adapter(self, ft: dict, hparams: dict) -> dict:
        raise NotImplementedError("this backward service does not train an adapter")

    def _handle_save_adapter(self, msg) -> None:
        from deltaserve_amd.checkpoint import write_save_error

        if int(((self.shared or {}).get("meta") or {}).get("tp_rank", 0)) == 0:
            write_save_error(msg.get("path"), msg.get("save_id"),
                             f"{type(self).__name__} trains no adapter")

    # -- the loop
    def run(self, conn) -> None:
        pid = os.getpid()
        echoed = {k: os.environ.get(k) for k in _ECHOED_ENV}
        dprint(f"[backward] {type(self).__name__} started pid={pid} device={self.device_index} "
               + " ".join(f"{k}={v}" for k, v in echoed.items()))
        conn.send({"event": "ready", "pid": pid,
                   "mps_percentage": echoed[_ECHOED_ENV[0]],
                   "max_connections": echoed[_ECHOED_ENV[1]]})
        self._handover = handover.open_line(self)
        if self._handover is not None:
            dprint(f"[backward] pid={pid} handover line {self._handover.path}")
        try:
            while True:
                try:
                    msg = conn.recv()
                except EOFError:
                    break  # the parent is gone
                cmd = msg.get("cmd") if isinstance(msg, dict) else None
                if cmd == "shutdown":
                    dprint(f"[backward] pid={pid} shutting down")
                    conn.send({"event": "bye", "pid": pid})
                    break
                handler = _COMMANDS.get(cmd)
                reply = (getattr(self, handler)(msg) if handler is not None
                         else {"event": "error", "msg": f"unknown cmd {cmd!r}"})
                if reply is not None:
                    conn.send(reply)
                while self._after_reply:
                    self._after_reply.pop(0)()
        finally:
            if self._handover is not None:
                self._handover.close()
            close = getattr(conn, "close", None)
            if close is not None:
                close()

    # -- commands
    @_command("ping")
    def _cmd_ping(self, msg):
        return {"event": "pong", "pid": os.getpid(), "data": msg.get("data")}

    @_command("share_weights")
    def _cmd_share_weights(self, msg):
        base, ft = msg.get("base") or {}, msg.get("ft") or {}
        self.shared = {"base": base, "ft": ft, "meta": msg.get("meta") or {}}
        error = self._on_weights_shared()
        reply = {"event": "weights_received", "base_num": len(base), "ft_num": len(ft),
                 "hash_report": {}, "error": error}
        if msg.get("print_hash"):
            reply["hash_report"] = integrity.weight_hash_report(base, ft)
            integrity.print_hash_report(reply["hash_report"], "child")
            reply.update(integrity.weights_summary(base, ft))
        return reply

    @_command("checksum")
    def _cmd_checksum(self, msg):
        which = msg.get("which", "ft")
        return {"event": "checksum", "which": which,
                "value": integrity.checksum((self.shared or {}).get(which) or {})}

    @_command("share_activations")
    def _cmd_share_activations(self, msg):
        self.activations = msg.get("buffers")
        self._verify = bool(msg.get("print_hash"))
        layers = len((self.activations or {}).get("layer_in") or [])
        if self._verify:
            dprint(f"[backward] received activation buffers: layer_in x {layers} "
                   f"+ {', '.join(k for k in (self.activations or {}) if k != 'layer_in')}")
        return {"event": "activations_received", "num_layers": layers}

    @_command("share_lora_buffers")
    def _cmd_share_lora_buffers(self, msg):
        self.lora_buffers = msg.get("payload")
        layers = len((self.lora_buffers or {}).get("layers") or {})
        dprint(f"[backward] received served LoRA buffers: {layers} layers "
               f"(slot {(self.lora_buffers or {}).get('slot')})")
        self._on_lora_buffers()
        return {"event": "lora_buffers_received", "num_layers": layers}

    @_command("hash_activations")
    def _cmd_hash_activations(self, msg):
        report = integrity.activation_hash_report(self.activations or {}, int(msg.get("n", 0)))
        integrity.print_hash_report(report, "child")
        return {"event": "activation_hashes", "hash_report": report}

    @_command("set_corpus_meta")
    def _cmd_set_corpus_meta(self, msg):
        self.ledger.per_epoch = int(msg.get("total_tokens_per_epoch", 0))
        dprint(f"[backward] corpus meta: total_tokens_per_epoch={self.ledger.per_epoch}")
        return None

    @_command("switch_adapter")
    def _cmd_switch_adapter(self, msg):
        try:
            result = self.switch_adapter(msg.get("ft") or {}, msg.get("hparams") or {})
        except Exception as e:  # noqa: BLE001 — the job fails, the child lives on
            return {"event": "error", "msg": f"{type(e).__name__}: {e}"}
        return {"event": "adapter_switched", **result}

    @_command("save_lora")
    def _cmd_save_lora(self, msg):
        # The snapshot to host memory happens now, while no backward runs;
        # the file is written on a thread so the caller does not wait for it.
        try:
            state = self.export_lora_state()
        except Exception as e:  # noqa: BLE001
            return {"event": "lora_save_failed", "msg": f"{type(e).__name__}: {e}"}
        handover.write_shard_in_background(state, msg["path"])
        return {"event": "lora_save_started", "tensors": len(state)}

    @_command("export_lora")
    def _cmd_export_lora(self, msg):
        return {"event": "lora_state", "state": self.export_lora_state()}

    @_command("save_adapter")
    def _cmd_save_adapter(self, msg):
        self._handle_save_adapter(msg)
        return None

    @_command("process_activations")
    def _cmd_process_activations(self, msg):
        cyc = Cycle.of(msg)
        self._pause.cycle_started()
        grant = self._gpu_grant
        gate = "n/a" if grant is None else ("SET" if grant.is_set() else "CLEAR")
        dprint(f"[backward] start: n={cyc.n} samples={len(cyc.sample_lens)} epoch={cyc.epoch} "
               f"gpu_grant={gate}" + ("  (will block until released)" if gate == "CLEAR" else ""))
        self.ledger.see_epoch(cyc.epoch)
        runnable = self._has_rows(cyc)
        self._before_cycle(cyc.epoch, runnable)
        if runnable:
            self._train(cyc)
        else:
            dprint(f"[backward] skipped (n={cyc.n}, no data / save_activations off)")
        # the zero fill is queued behind the cycle; the clock's end event
        # was recorded before it, so it is not timed
        self._wipe_activations()
        gpu_ms = None
        if cyc.loss is not None:
            gpu_ms = cyc.gpu_ms()
            self._report(cyc, gpu_ms)
        self._after_reply.append(lambda: self._after_cycle(cyc.epoch, runnable))
        return cyc.ack(gpu_ms, self._memory())

    # -- cycle steps
    def _has_rows(self, cyc: Cycle) -> bool:
        acts = self.activations
        return (cyc.n > 0 and bool(cyc.sample_lens) and acts is not None
                and acts.get("concat_input_ids") is not None)

    def _train(self, cyc: Cycle) -> None:
        clock = CycleClock()
        try:
            if self._verify:
                self.verify_activations(self.activations, cyc.n)
            with clock:
                cyc.loss, cyc.n_valid = self.process_backward(
                    self.activations, cyc.sample_lens, cyc.n, cyc.epoch)
        except Exception as e:  # noqa: BLE001 — the cycle is acked with loss=None
            dprint(f"[backward] backward failed: {e}")
            traceback.print_exc()
            cyc.loss = None
            return
        cyc.clock = clock
        self.ledger.add(cyc.n)

    def _wipe_activations(self) -> None:
        for value in (self.activations or {}).values():
            for t in (value if isinstance(value, (list, tuple)) else [value]):
                if torch.is_tensor(t):
                    t.zero_()

    def _report(self, cyc: Cycle, gpu_ms: float | None) -> None:
        loss = _as_float(cyc.loss)
        self._last_loss = loss
        ms = float("nan") if gpu_ms is None else gpu_ms
        dprint(f"[backward] {ms:.1f}ms ({self._last_mode}) loss={loss:.6f} "
               f"total_trained={self.ledger.total} n={cyc.n} epoch={cyc.epoch} "
               f"{self.ledger.meter()} tokens")
        if not math.isfinite(loss):
            dprint(f"[backward] !!! NON-FINITE LOSS ({loss}) at epoch={cyc.epoch} n={cyc.n} — "
                   "training diverged; the FT adapter published to the served slot is now "
                   "NaN-tainted. Lower the learning rate or disable FT to recover.")

    def _memory(self) -> dict | None:
        if not torch.cuda.is_available():
            return None
        return {"alloc": torch.cuda.memory_allocated(),
                "peak": torch.cuda.max_memory_allocated(),
                "reserved": torch.cuda.memory_reserved(),
                "lora_train_state": getattr(self, "_train_state_bytes", 0)}
