"""When the backward child must leave the GPU to inference.

Two signals hold a cycle at its next pause point (between vocabulary chunks
of the LM head and between layers):

* the **GPU grant**, a shared ``multiprocessing.Event`` the worker clears
  around an inference prefill (set = the child may run;
  ``deltaserve-plugin/deltaserve/backward_process.py:197-205``, ``:448-458``);
* with meta ``pause_on_arrival``, the engine's **arrival counter**: an
  inference request that arrived during the cycle holds it from the arrival
  until the worker's pause for that request's prefill has ended, or for at
  most 0.1 s if no pause follows (the reference's ``_arrival_blocked``,
  ``bwd_services/base.py:224-262``). The counter is an 8-byte little-endian
  count in POSIX shared memory named by ``$DSERVE_FT_ARRIVAL_SHM``, written
  by the engine's input thread (``coordinator.py:64-115``).

A hold polls every 2 ms and gives up after 5 s, so a grant that is never set
again cannot hang the backward. How far the host may queue work ahead of the
GPU is bounded inside libdsb (``dsb_step_segment``'s ``run_ahead``), not here.
"""

from __future__ import annotations

import enum
import os
import struct
import time

from deltaserve_amd import dprint

ARRIVAL_ENV = "DSERVE_FT_ARRIVAL_SHM"
_U64 = struct.Struct("<Q")


class ArrivalCounter:
    """Reader of the engine's arrival count in shared memory."""

    def __init__(self, name: str) -> None:
        from multiprocessing import resource_tracker, shared_memory

        self._shm = shared_memory.SharedMemory(name=name, create=False)
        # Attaching registers the segment with this process's resource
        # tracker, which would unlink the engine's segment when the child
        # exits; the engine owns it.
        try:
            resource_tracker.unregister(self._shm._name, "shared_memory")
        except Exception:  # noqa: BLE001
            pass

    def read(self) -> int:
        return _U64.unpack_from(self._shm.buf, 0)[0]

    def close(self) -> None:
        try:
            self._shm.close()
        except Exception:  # noqa: BLE001
            pass


class _Arrival(enum.Enum):
    NONE = 0           # nothing pending
    AWAITING_PAUSE = 1  # a request arrived; the worker has not paused us for it yet
    PAUSED = 2         # the worker paused us for its prefill


class ArrivalWatch:
    """The pause_on_arrival state of one child. ``blocks(grant_set)`` is
    asked at every pause point and on every poll while held."""

    GRACE_S = 0.1

    def __init__(self, counter, clock=time.monotonic) -> None:
        self.counter = counter
        self.clock = clock
        self.state = _Arrival.NONE
        self.seen = counter.read()
        self.since = 0.0

    def rebase(self) -> None:
        """A cycle starts: arrivals before it are covered by the prefill pause."""
        self.seen = self.counter.read()
        self.state = _Arrival.NONE

    def _settle(self) -> bool:
        self.state = _Arrival.NONE
        self.seen = self.counter.read()
        return False

    def blocks(self, grant_set: bool) -> bool:
        now = self.clock()
        if self.state is _Arrival.NONE:
            if self.counter.read() == self.seen:
                return False
            self.state, self.since = _Arrival.AWAITING_PAUSE, now
        if self.state is _Arrival.AWAITING_PAUSE:
            if not grant_set:
                self.state = _Arrival.PAUSED
            elif now - self.since > self.GRACE_S:
                return self._settle()     # no prefill followed the arrival
        if self.state is _Arrival.PAUSED and grant_set:
            return self._settle()         # its prefill is over
        return True


class PauseGate:
    """The child's pause points: ``hold()`` returns at once while the grant is
    set and no arrival is pending, else polls until both clear (at most
    ``LIMIT_S``)."""

    LIMIT_S = 5.0
    POLL_S = 0.002

    def __init__(self, grant=None, meta_of=None) -> None:
        self.grant = grant
        self._meta_of = meta_of or (lambda: {})
        self._watch: ArrivalWatch | None = None
        self._watch_resolved = False

    def watch(self) -> ArrivalWatch | None:
        """The arrival watch, attached on first use when meta asks for it."""
        if not self._watch_resolved:
            self._watch_resolved = True
            name = os.environ.get(ARRIVAL_ENV)
            if (self._meta_of() or {}).get("pause_on_arrival") and name:
                try:
                    self._watch = ArrivalWatch(ArrivalCounter(name))
                except Exception as e:  # noqa: BLE001
                    dprint(f"[backward] pause_on_arrival off: {e}")
        return self._watch

    def cycle_started(self) -> None:
        w = self.watch()
        if w is not None:
            w.rebase()

    def _arrival_blocks(self) -> bool:
        w = self.watch()
        return w is not None and w.blocks(self.grant.is_set())

    def _clear_to_run(self) -> bool:
        """One poll while held."""
        arrival = self._arrival_blocks()
        if not self.grant.is_set():
            self.grant.wait(timeout=self.POLL_S)
            return False
        if arrival:
            time.sleep(self.POLL_S)
            return False
        return True

    def hold(self) -> None:
        g = self.grant
        if g is None:
            return
        if g.is_set() and not self._arrival_blocks():
            return
        give_up = time.monotonic() + self.LIMIT_S
        while time.monotonic() < give_up and not self._clear_to_run():
            pass
