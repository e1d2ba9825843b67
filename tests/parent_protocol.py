"""The reference parent's side of the backward pipe, restated for tests.

``ParentSide`` sends exactly the message dicts the reference's
``BackwardProcess`` sends (``deltaserve-plugin/deltaserve/backward_process.py``,
cited per method) and checks the replies the way it does, raising where it
raises. Driving the child through it shows that the child is a drop-in for
the real parent, not only for this build's own idea of the protocol.

It talks over any object with ``send``/``recv``/``poll``: a
``multiprocessing`` pipe end, or ``InlinePipe``, which runs the child's loop
in a thread of the test process.
"""

from __future__ import annotations

import multiprocessing as mp
import queue
import threading


class ParentSide:
    def __init__(self, conn, timeout: float = 120.0) -> None:
        self.conn, self.timeout = conn, timeout

    def _reply(self, what: str):
        if not self.conn.poll(self.timeout):
            raise TimeoutError(f"[deltaserve] {what} timed out")
        return self.conn.recv()

    def ready(self) -> dict:  # start(): the handshake (backward_process.py:266)
        return self._reply("ready")

    def ping(self, data=None) -> dict:  # :270-275
        self.conn.send({"cmd": "ping", "data": data})
        return self._reply("ping")

    def share_weights(self, base, ft, print_hash=False, meta=None) -> dict:  # :277-296
        self.conn.send({"cmd": "share_weights", "base": base, "ft": ft,
                        "print_hash": bool(print_hash), "meta": meta or {}})
        return self._reply("share_weights")

    def switch_adapter(self, ft, hparams) -> dict:  # :298-312
        self.conn.send({"cmd": "switch_adapter", "ft": ft, "hparams": hparams})
        reply = self._reply("switch_adapter")
        if reply.get("event") != "adapter_switched":
            raise RuntimeError(f"backward child refused the adapter: "
                               f"{reply.get('msg', reply.get('event'))}")
        return reply

    def export_lora(self) -> dict:  # :314-325
        self.conn.send({"cmd": "export_lora"})
        reply = self._reply("export_lora")
        if reply.get("event") != "lora_state":
            raise RuntimeError(f"unexpected reply to export_lora: {reply.get('event')!r}")
        return reply["state"]

    def save_lora(self, path) -> dict:  # :327-340
        self.conn.send({"cmd": "save_lora", "path": path})
        reply = self._reply("save_lora")
        if reply.get("event") != "lora_save_started":
            raise RuntimeError(f"backward child could not snapshot the adapter: "
                               f"{reply.get('msg', reply.get('event'))}")
        return reply

    def checksum(self, which="ft") -> float:  # :342-347
        self.conn.send({"cmd": "checksum", "which": which})
        return self._reply("checksum")["value"]

    def share_activations(self, buffers, print_hash=False) -> dict:  # :349-367
        self.conn.send({"cmd": "share_activations", "buffers": buffers,
                        "print_hash": bool(print_hash)})
        return self._reply("share_activations")

    def share_lora_buffers(self, payload) -> dict:  # :369-383
        self.conn.send({"cmd": "share_lora_buffers", "payload": payload})
        return self._reply("share_lora_buffers")

    def hash_activations(self, n) -> dict:  # :385-390
        self.conn.send({"cmd": "hash_activations", "n": int(n)})
        return self._reply("hash_activations")["hash_report"]

    def set_corpus_meta(self, total_tokens_per_epoch) -> None:  # :392-407, no reply
        self.conn.send({"cmd": "set_corpus_meta",
                        "total_tokens_per_epoch": int(total_tokens_per_epoch)})

    def request_save_adapter(self, path, save_id) -> None:  # :409-422, no reply
        self.conn.send({"cmd": "save_adapter", "path": str(path), "save_id": str(save_id)})

    def notify_buffer_full(self, n, sample_lens=None, epoch=0) -> None:  # :424-446
        self.conn.send({"cmd": "process_activations", "n": int(n),
                        "sample_lens": list(sample_lens or []), "epoch": int(epoch)})

    def poll_response(self, timeout: float = 0.0):  # :460-473
        return self.conn.recv() if self.conn.poll(timeout) else None

    def shutdown(self) -> dict:  # :475-495
        self.conn.send({"cmd": "shutdown"})
        return self._reply("shutdown")


class _QueueEnd:
    """One end of an in-process pipe: messages pass by reference, as CUDA
    tensors do between the reference's processes (CUDA IPC maps the same
    memory), so a buffer the child writes is the parent's buffer."""

    _CLOSED = object()

    def __init__(self, inbox: queue.Queue, outbox: queue.Queue) -> None:
        self._in, self._out, self._pending = inbox, outbox, []

    def send(self, msg) -> None:
        self._out.put(msg)

    def poll(self, timeout: float = 0.0) -> bool:
        if not self._pending:
            try:
                self._pending.append(self._in.get(timeout=timeout) if timeout
                                     else self._in.get_nowait())
            except queue.Empty:
                return False
        return True

    def recv(self):
        msg = self._pending.pop(0) if self._pending else self._in.get()
        if msg is self._CLOSED:
            raise EOFError
        return msg

    def close(self) -> None:
        self._out.put(self._CLOSED)


def queue_pipe():
    a, b = queue.Queue(), queue.Queue()
    return _QueueEnd(a, b), _QueueEnd(b, a)


class InlinePipe:
    """A pipe whose child end runs ``svc.run`` in a thread of this process:
    a real ``multiprocessing`` pipe (messages pickled), or with
    ``by_reference`` the in-process queue pipe (shared tensors stay shared)."""

    def __init__(self, svc, by_reference: bool = False) -> None:
        self.parent_end, child_end = queue_pipe() if by_reference else mp.Pipe()
        self.thread = threading.Thread(target=svc.run, args=(child_end,), daemon=True)
        self.thread.start()
        self.parent = ParentSide(self.parent_end, timeout=300.0)

    def join(self, timeout: float = 30.0) -> None:
        self.thread.join(timeout)
        assert not self.thread.is_alive(), "the child loop did not end"
