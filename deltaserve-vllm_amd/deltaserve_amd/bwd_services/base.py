"""The model-agnostic backward-child loop: pipe protocol and the per-cycle wrapper.

Restates ``deltaserve-plugin/deltaserve/bwd_services/base.py`` for the MI355X
backward: the child receives the shared weights / activation store / served
LoRA buffers over its pipe, and on ``process_activations`` runs the
subclass's ``process_backward`` (libdsb's hipGraph cycle), zeroes the shared
activation buffers, prints the one-line cycle log and replies with the
``activations_processed`` ack (base.py:468-633).
"""

from __future__ import annotations

import math
import time

import torch

from deltaserve_amd import dprint, mark_backward_process


def service_main(conn, mps_percentage: int, device_index: int, service_name: str,
                 gpu_grant=None) -> None:
    """Child-process entry point (base.py:48-70): select the service by
    architecture string, bind the GPU-yield event and run the pipe loop.
    ``mps_percentage`` is accepted for signature compatibility; the MI355X
    child does not partition CUs."""
    from deltaserve_amd.bwd_services.registry import get_service

    mark_backward_process()
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


class BackwardService:
    """Base class: recv/dispatch loop + cycle wrapper (base.py:93-633)."""

    def __init__(self, device_index: int) -> None:
        self.device_index = int(device_index)
        self.shared: dict = {"base": None, "ft": None, "meta": {}}
        self.activations: dict | None = None
        self._verify = False
        self.current_epoch = 0
        self._total_tokens_trained = 0
        self.lora_buffers: dict | None = None
        self._gpu_grant = None
        self._cur_epoch_seen = 0
        self._epoch_processed_tokens = 0
        self._total_tokens_per_epoch = 0
        self._last_loss = None
        self._last_mode = "graph"

    # -- GPU-yield contract (base.py:148-208): at a segment boundary, block
    # (bounded, 5 s) while the grant is cleared. The run-ahead bound of the
    # reference's event ring is applied by libdsb between segment launches
    # (dsb_step_segment's run_ahead, from meta backward_run_ahead_boundaries).
    def _maybe_pause(self) -> None:
        grant = self._gpu_grant
        if grant is None or grant.is_set():
            return
        deadline = time.monotonic() + 5.0
        while not grant.is_set() and time.monotonic() < deadline:
            grant.wait(timeout=0.002)

    def _run_ahead(self) -> int:
        meta = (self.shared or {}).get("meta") or {}
        return max(0, int(meta.get("backward_run_ahead_boundaries", 0) or 0))

    def _on_lora_buffers(self) -> None:  # trainer overrides
        pass

    # -- pipe loop (base.py:297-408)
    def run(self, conn) -> None:
        conn.send({"event": "ready", "device": self.device_index})
        while True:
            msg = conn.recv()
            cmd = msg.get("cmd") if isinstance(msg, dict) else msg
            if cmd == "shutdown":
                conn.send({"event": "shutdown_ack"})
                break
            if cmd == "ping":
                conn.send({"event": "pong"})
            elif cmd == "share_weights":
                self.shared = {"base": msg.get("base"), "ft": msg.get("ft"),
                               "meta": msg.get("meta") or {}}
                err = self._on_weights_shared()
                conn.send({"event": "weights_received", "error": err})
            elif cmd == "share_activations":
                self._handle_share_activations(conn, msg)
            elif cmd == "share_lora_buffers":
                self.lora_buffers = msg.get("buffers")
                self._on_lora_buffers()
                conn.send({"event": "lora_buffers_received"})
            elif cmd == "set_corpus_meta":
                self._total_tokens_per_epoch = int(msg.get("total_tokens_per_epoch", 0))
            elif cmd == "process_activations":
                self._handle_process_activations(conn, msg)
            elif cmd == "save_adapter":
                self._handle_save_adapter(msg)
            else:
                conn.send({"event": "error", "error": f"unknown command {cmd!r}"})

    def _on_weights_shared(self) -> str | None:
        return None

    def _handle_share_activations(self, conn, msg) -> None:
        self.activations = msg.get("activations")
        self._verify = bool(msg.get("print_hash"))
        nlayers = len((self.activations or {}).get("layer_in", []))
        conn.send({"event": "activations_received", "num_layers": nlayers})

    def _handle_save_adapter(self, msg) -> None:  # trainer overrides
        pass

    def _before_cycle(self, epoch: int, attempted: bool) -> None:
        pass

    def _after_cycle(self, epoch: int, attempted: bool) -> None:
        pass

    def verify_activations(self, activations: dict, n: int) -> None:
        pass

    def process_backward(self, activations, sample_lens, n, epoch):
        """Protocol-only service: nothing to train."""
        return 0.0, 0

    # -- the cycle wrapper (base.py:468-633)
    def _handle_process_activations(self, conn, msg) -> None:
        t_wall0 = time.perf_counter()
        n = int(msg.get("n", 0))
        sample_lens = msg.get("sample_lens") or []
        epoch = int(msg.get("epoch", 0))
        _grant_set = self._gpu_grant.is_set() if self._gpu_grant is not None else None
        gate = "SET" if _grant_set else ("CLEAR" if _grant_set is False else "n/a")
        dprint(f"[backward] start: n={n} samples={len(sample_lens)} epoch={epoch} "
               f"gpu_grant={gate}" + ("  (will block until released)"
                                      if _grant_set is False else ""))
        if epoch > self._cur_epoch_seen:
            self._epoch_processed_tokens = 0
            self._cur_epoch_seen = epoch
        loss = None
        total_ms = None
        start_evt = end_evt = None
        cpu_elapsed_ms = None
        can_compute = (n > 0 and self.activations is not None
                       and self.activations.get("concat_input_ids") is not None
                       and bool(sample_lens))
        self._before_cycle(epoch, can_compute)
        if can_compute:
            try:
                if self._verify:
                    self.verify_activations(self.activations, n)
                if torch.cuda.is_available():
                    start_evt = torch.cuda.Event(enable_timing=True)
                    end_evt = torch.cuda.Event(enable_timing=True)
                    start_evt.record()
                    loss, _n_valid = self.process_backward(self.activations, sample_lens, n, epoch)
                    end_evt.record()
                else:
                    t0 = time.perf_counter()
                    loss, _n_valid = self.process_backward(self.activations, sample_lens, n, epoch)
                    cpu_elapsed_ms = (time.perf_counter() - t0) * 1000.0
                # Throughput counts raw token rows n, not n_valid (base.py:540-548).
                self._total_tokens_trained += n
                self._epoch_processed_tokens += n
            except Exception as e:  # noqa: BLE001 — keep the cycle alive, ack loss=None
                import traceback
                dprint(f"[backward] backward failed: {e}")
                traceback.print_exc()
                loss = None
                start_evt = end_evt = None
        else:
            dprint(f"[backward] skipped (n={n}, no data / save_activations off)")

        if self.activations:
            for value in self.activations.values():
                for t in (value if isinstance(value, list) else [value]):
                    if torch.is_tensor(t):
                        t.zero_()

        if can_compute and loss is not None:
            if start_evt is not None and end_evt is not None:
                end_evt.synchronize()
                total_ms = start_evt.elapsed_time(end_evt)
            elif cpu_elapsed_ms is not None:
                total_ms = cpu_elapsed_ms
            else:
                total_ms = float("nan")
            try:
                loss_f = loss.item() if hasattr(loss, "item") else float(loss)
            except Exception:  # noqa: BLE001
                loss_f = float("nan")
            self._last_loss = loss_f
            total = self._total_tokens_per_epoch
            progress = (f"{self._epoch_processed_tokens}/{total}" if total > 0
                        else f"{self._epoch_processed_tokens}/?")
            dprint(f"[backward] {total_ms:.1f}ms ({self._last_mode}) loss={loss_f:.6f} "
                   f"total_trained={self._total_tokens_trained} n={n} epoch={epoch} "
                   f"{progress} tokens")
            if not math.isfinite(loss_f):
                dprint(f"[backward] !!! NON-FINITE LOSS ({loss_f}) at epoch={epoch} n={n} — "
                       "training diverged; the FT adapter published to vLLM is now "
                       "NaN-tainted. Lower the learning rate or disable FT to recover.")

        resp = {"event": "activations_processed", "n": n, "loss": loss,
                "samples": len(sample_lens),
                "gpu_ms": (None if total_ms is None or total_ms != total_ms
                           else float(total_ms)),
                "wall_ms": (time.perf_counter() - t_wall0) * 1000.0}
        if torch.cuda.is_available():
            resp["mem"] = {"alloc": torch.cuda.memory_allocated(),
                           "peak": torch.cuda.max_memory_allocated(),
                           "reserved": torch.cuda.memory_reserved(),
                           "lora_train_state": getattr(self, "_train_state_bytes", 0)}
        conn.send(resp)
        self._after_cycle(epoch, can_compute)
