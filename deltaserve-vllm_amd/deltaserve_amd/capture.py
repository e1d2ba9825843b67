"""The serving side of the activation handoff: the save op and its index refresh.

Mirrors the graph-capturable path of the reference's forward-side capture
(paths under ``deltaserve-plugin/deltaserve/``):

* ``FtSaveState`` / ``active_state`` / ``dserve_save_rows`` follow
  ``ft_save_op.py:47-93``: the op gathers a FIXED number of rows (max_saved)
  of ``x`` (+ ``r``, the fused add-norm's residual) through a persistent
  source-index tensor and writes them, as bf16, into the activation buffer of
  ``slot`` through a persistent destination-index tensor. Both index tensors
  and the slot table come from the active state, never from a captured
  graph, so a graph replays the gathers with the indices of each step.
* ``ActivationStore`` holds the buffers the backward reads (``layer_in`` per
  layer, ``final_in``, ``concat_input_ids``; ``accumulate.py:196-262``) and
  the op-path pieces of the reference's accumulator: the slot table
  (``install_save_points``, accumulate.py:276-315, 7 slots per layer + the
  final norm), ``capture_state`` (:317-323), ``arm_op_step`` (:325-343) and
  the final ids save (``accumulate_final``, :598-622).

The gathers run as the HIP kernels of ``libdsb`` (``dsb_save_rows``,
``dsb_save_ids``; the host-side index build is ``dsb_capture_index``), on
the current torch stream, with no host synchronisation. Nothing here falls
back to PyTorch indexing.
"""

from __future__ import annotations

from contextlib import contextmanager
from ctypes import c_void_p
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib as L

_DT = {torch.bfloat16: L.DT_BF16, torch.float16: L.DT_F16, torch.float32: L.DT_F32}

# Per-layer slot numbers of the reference's table (accumulate.py:289-300).
SLOT_LAYER_IN, SLOT_RESID_MID, SLOT_GATE_UP, SLOT_QH, SLOT_KH, SLOT_VH, SLOT_CTX = range(7)
SLOTS_PER_LAYER = 7


@dataclass
class FtSaveState:
    """What the op reads on a step that saves activations (ft_save_op.py:47-53)."""

    src: torch.Tensor  # int64 [max_saved]: rows of x to gather
    dst: torch.Tensor  # int64 [max_saved]: rows of the buffer to write
    bufs: list  # slot -> bf16 buffer [max_saved + 1, width] or None


_ACTIVE: FtSaveState | None = None


@contextmanager
def active_state(state: FtSaveState | None):
    """Make ``state`` what the op reads for the duration of the block."""
    global _ACTIVE
    prev, _ACTIVE = _ACTIVE, state
    try:
        yield
    finally:
        _ACTIVE = prev


def _stream():
    return c_void_p(torch.cuda.current_stream().cuda_stream)


def save_rows(x: torch.Tensor, r: Optional[torch.Tensor], buf: torch.Tensor,
              src: torch.Tensor, dst: torch.Tensor) -> None:
    """``buf[dst[i]] = bf16(x[src[i]] (+ r[src[i]]))`` for every index slot, as
    ``buf.index_copy_(0, dst, (x.index_select(0, src) + ...).to(buf.dtype))``
    (ft_save_op.py:84-89), except that slots aimed at the scratch row
    ``buf[-1]`` are not written (nothing reads that row) and slots whose source
    row lies outside ``x`` are skipped instead of faulting."""
    if x.dtype not in _DT:
        raise TypeError(f"save_rows: x must be bf16, fp16 or fp32, got {x.dtype}")
    if buf.dtype != torch.bfloat16:
        raise TypeError("save_rows: activation buffers are bf16")
    if x.dim() != 2 or buf.dim() != 2 or x.stride(1) != 1 or buf.stride(1) != 1:
        raise ValueError("save_rows: x and buf must be 2-D with contiguous rows")
    if x.shape[1] != buf.shape[1]:
        raise ValueError(f"save_rows: width {x.shape[1]} != buffer width {buf.shape[1]}")
    if r is not None and (r.shape != x.shape or r.dtype != x.dtype or r.stride(1) != 1):
        raise ValueError("save_rows: r must match x in shape and dtype")
    for t in (src, dst):
        if t.dtype != torch.int64 or not t.is_contiguous() or t.dim() != 1:
            raise ValueError("save_rows: src/dst are contiguous int64 vectors")
    if src.shape != dst.shape:
        raise ValueError("save_rows: src and dst differ in length")
    if not (x.is_cuda and buf.is_cuda and src.is_cuda and dst.is_cuda):
        raise ValueError("save_rows takes CUDA (HIP) tensors")
    lib = L.load()
    L.check(lib.dsb_save_rows(
        c_void_p(x.data_ptr()), x.stride(0),
        None if r is None else c_void_p(r.data_ptr()), 0 if r is None else r.stride(0),
        x.shape[0], _DT[x.dtype], c_void_p(src.data_ptr()), c_void_p(dst.data_ptr()),
        src.shape[0], x.shape[1], c_void_p(buf.data_ptr()), buf.stride(0), buf.shape[0],
        _stream()), what="dsb_save_rows")


def save_ids(ids: torch.Tensor, src: torch.Tensor, dst: torch.Tensor,
             out: torch.Tensor) -> None:
    """``out[dst[i]] = ids[src[i]]`` for the slots with ``dst[i] < len(out)``
    (the final save point's ids, accumulate.py:609-622, through the step's
    index pair)."""
    for t in (ids, src, dst, out):
        if t.dtype != torch.int64 or not t.is_contiguous() or t.dim() != 1 or not t.is_cuda:
            raise ValueError("save_ids takes contiguous int64 CUDA vectors")
    if src.shape != dst.shape:
        raise ValueError("save_ids: src and dst differ in length")
    lib = L.load()
    L.check(lib.dsb_save_ids(c_void_p(ids.data_ptr()), ids.shape[0], c_void_p(src.data_ptr()),
                             c_void_p(dst.data_ptr()), src.shape[0], c_void_p(out.data_ptr()),
                             out.shape[0], _stream()), what="dsb_save_ids")


def dserve_save_rows(x: torch.Tensor, r: Optional[torch.Tensor], marker: torch.Tensor,
                     slot: int) -> None:
    """The save op (ft_save_op.py:72-89): a no-op without an active state or
    for a slot with no buffer; otherwise the gather of the active indices into
    the slot's buffer. ``marker`` exists for graph compilers (the reference
    declares it mutated so the call is kept) and is not touched."""
    fs = _ACTIVE
    if fs is None:
        return
    buf = fs.bufs[slot] if slot < len(fs.bufs) else None
    if buf is None:
        return
    save_rows(x, r, buf, fs.src, fs.dst)


def capture_index(positions, num_ft: int, offset: int, max_saved: int):
    """The host-side index build of ``arm_op_step`` (accumulate.py:332-340), via
    ``dsb_capture_index``: returns (src, dst, n) as CPU int64 tensors of
    length max_saved and the number of rows the step saves."""
    lib = L.load()
    pos = torch.as_tensor(positions, dtype=torch.int64).reshape(-1).contiguous()
    if pos.shape[0] < max(int(num_ft), 0):
        raise ValueError("capture_index: fewer positions than num_ft")
    src = torch.empty(max_saved, dtype=torch.int64)
    dst = torch.empty(max_saved, dtype=torch.int64)
    n = lib.dsb_capture_index(c_void_p(pos.data_ptr()) if pos.numel() else None, int(num_ft),
                              int(offset), int(max_saved), c_void_p(src.data_ptr()),
                              c_void_p(dst.data_ptr()))
    if n < 0:
        raise ValueError(f"capture_index: {L.last_error()}")
    return src, dst, n


class ActivationStore:
    """The buffers a backward cycle reads and the op-path state that fills
    them (accumulate.py:196-343).

    ``layer_in[i]`` and ``final_in`` are bf16 ``[max_saved + 1, hidden]``
    (row ``max_saved`` is the scratch row), ``concat_input_ids`` is int64
    ``[max_saved]``. With ``intermediate_size`` > 0 (the reference saves it
    whenever the MLP's gate_up modules exist, accumulate.py:174, :210-212)
    ``mlp_gate_up[i]`` is bf16 ``[max_saved + 1, 2·intermediate]``, the gate‖up
    projection output the backward then reads instead of recomputing it.

    The opt-in save points (accumulate.py:213-235), each per layer:
    ``save_attn_qkv`` → ``attn_qh`` / ``attn_kh`` / ``attn_vh`` bf16
    ``[max_saved + 1, q_size | kv_size]`` (the attention call's q, k, v; for a
    family whose backward needs the pre-transform q/k, the q/k-norm inputs),
    ``save_attn_ctx`` → ``attn_ctx`` ``[max_saved + 1, q_size]`` (the attention
    output), ``save_resid_mid`` → ``resid_mid`` ``[max_saved + 1, hidden]``
    (the post-attention residual), and ``save_final_hidden`` →
    ``final_hidden`` (the final norm's output, for the debug capture check).
    The slot table has the reference's 7 slots per layer plus the final
    norm's; the slots of save points that are off hold no buffer, so their
    save calls are no-ops, as in the reference.
    """

    STAGES = 4  # pinned staging slots for the index refresh (accumulate.py:262)

    def __init__(self, num_layers: int, hidden_size: int, max_saved: int, device="cuda",
                 intermediate_size: int = 0, q_size: int = 0, kv_size: int = 0,
                 save_attn_qkv: bool = False, save_attn_ctx: bool = False,
                 save_resid_mid: bool = False, save_final_hidden: bool = False):
        if max_saved <= 0 or num_layers <= 0 or hidden_size <= 0 or intermediate_size < 0:
            raise ValueError("ActivationStore: sizes must be positive")
        if (save_attn_qkv and (q_size <= 0 or kv_size <= 0)) or (save_attn_ctx and q_size <= 0):
            raise ValueError("ActivationStore: the q/k/v and context save points need "
                             "q_size (and kv_size)")
        self.num_layers, self.hidden_size, self.max_saved = num_layers, hidden_size, max_saved
        self.intermediate_size = intermediate_size
        self.device = torch.device(device)

        def buf(width=hidden_size):
            return torch.zeros(max_saved + 1, width, dtype=torch.bfloat16, device=self.device)

        self.layer_in = [buf() for _ in range(num_layers)]
        self.mlp_gate_up = ([buf(2 * intermediate_size) for _ in range(num_layers)]
                            if intermediate_size > 0 else [])
        per_layer = lambda on, width: [buf(width) for _ in range(num_layers)] if on else []  # noqa: E731
        self.attn_qh = per_layer(save_attn_qkv, q_size)
        self.attn_kh = per_layer(save_attn_qkv, kv_size)
        self.attn_vh = per_layer(save_attn_qkv, kv_size)
        self.attn_ctx = per_layer(save_attn_ctx, q_size)
        self.resid_mid = per_layer(save_resid_mid, hidden_size)
        self.final_hidden = buf() if save_final_hidden else None
        self.final_in = buf()
        self.concat_input_ids = torch.zeros(max_saved, dtype=torch.int64, device=self.device)
        self.ft_src = torch.zeros(max_saved, dtype=torch.int64, device=self.device)
        self.ft_dst = torch.full((max_saved,), max_saved, dtype=torch.int64, device=self.device)
        self._idx_pin = torch.empty((self.STAGES, 2, max_saved), dtype=torch.int64,
                                    pin_memory=self.device.type == "cuda")
        self._idx_evt = [None] * self.STAGES
        self._idx_pin_pos = 0
        bufs: list = [None] * (SLOTS_PER_LAYER * num_layers + 1)
        for i in range(num_layers):
            for kind, per in ((SLOT_LAYER_IN, self.layer_in), (SLOT_GATE_UP, self.mlp_gate_up),
                              (SLOT_RESID_MID, self.resid_mid), (SLOT_QH, self.attn_qh),
                              (SLOT_KH, self.attn_kh), (SLOT_VH, self.attn_vh),
                              (SLOT_CTX, self.attn_ctx)):
                if per:
                    bufs[SLOTS_PER_LAYER * i + kind] = per[i]
        bufs[SLOTS_PER_LAYER * num_layers] = self.final_in
        self.op_bufs = bufs
        self.marker = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.num_saved = 0  # rows filled so far (max over offset + n of the armed steps)
        self._eager: FtSaveState | None = None

    def slot(self, layer: int, kind: int = SLOT_LAYER_IN) -> int:
        return SLOTS_PER_LAYER * layer + kind

    @property
    def final_slot(self) -> int:
        return SLOTS_PER_LAYER * self.num_layers

    def capture_state(self) -> FtSaveState:
        """The persistent index tensors as they are, and the slot table
        (accumulate.py:317-323): what a graph capture runs under."""
        return FtSaveState(src=self.ft_src, dst=self.ft_dst, bufs=self.op_bufs)

    def arm_op_step(self, positions, num_ft: int, offset: int) -> FtSaveState:
        """Refresh the index tensors for a step (accumulate.py:325-343):
        ``positions`` are the step's FT rows in the flat batch (any order),
        written to buffer rows ``offset .. offset+n``; unused slots aim at
        the scratch row. One pinned staging slot and one non-blocking copy on
        the current stream; a staging slot is reused only after its previous
        copy has completed."""
        slot = self._idx_pin_pos
        self._idx_pin_pos = (slot + 1) % self.STAGES
        if self._idx_evt[slot] is not None:
            self._idx_evt[slot].synchronize()
        stage = self._idx_pin[slot]
        lib = L.load()
        pos = torch.as_tensor(positions, dtype=torch.int64).reshape(-1).contiguous()
        if pos.shape[0] < max(int(num_ft), 0):
            raise ValueError("arm_op_step: fewer positions than num_ft")
        n = lib.dsb_capture_index(c_void_p(pos.data_ptr()) if pos.numel() else None,
                                  int(num_ft), int(offset), self.max_saved,
                                  c_void_p(stage[0].data_ptr()), c_void_p(stage[1].data_ptr()))
        if n < 0:
            raise ValueError(f"arm_op_step: {L.last_error()}")
        self.ft_src.copy_(stage[0], non_blocking=True)
        self.ft_dst.copy_(stage[1], non_blocking=True)
        evt = torch.cuda.Event()
        evt.record()
        self._idx_evt[slot] = evt
        self.num_saved = max(self.num_saved, int(offset) + n)
        return self.capture_state()

    # ---- the eager path (hooks on an un-captured forward, accumulate.py:421-457)

    def begin_step(self, mask_gpu, num_ft: int, offset: int = 0, start: int = 0,
                   contiguous: bool = False) -> FtSaveState:
        """Arm an eager step (accumulate.py:581-596): the FT rows are the span
        ``[start, start + num_ft)`` when ``contiguous``, else the set rows of
        ``mask_gpu`` in ascending order (which costs one device-to-host read of
        the mask, as the reference's boolean-mask gather does). The hooks then
        call ``save`` per save point; the rows go through the same index pair
        and kernel as the graph path."""
        if contiguous:
            positions = torch.arange(int(start), int(start) + int(num_ft), dtype=torch.int64)
        else:
            positions = torch.nonzero(mask_gpu.reshape(-1).to("cpu")).reshape(-1)
            if positions.shape[0] != int(num_ft):
                raise ValueError(f"begin_step: mask has {positions.shape[0]} rows, num_ft={num_ft}")
        self._eager = self.arm_op_step(positions, int(num_ft), int(offset))
        return self._eager

    def save(self, slot: int, x: torch.Tensor, r: Optional[torch.Tensor] = None) -> None:
        """One save point on an armed eager step (the hook body,
        accumulate.py:421-446): the residual stream entering the module,
        ``x (+ r)``, for the step's FT rows."""
        fs = self._eager
        if fs is None:
            return
        buf = fs.bufs[slot] if slot < len(fs.bufs) else None
        if buf is not None:
            save_rows(x, r, buf, fs.src, fs.dst)

    def end_step(self) -> None:
        self._eager = None

    def accumulate_final(self, input_ids_flat: torch.Tensor,
                         hidden_states: Optional[torch.Tensor] = None) -> None:
        """The ids of the armed eager step's FT rows, and with a
        ``final_hidden`` buffer the model output's rows (accumulate.py:598-622)."""
        fs = self._eager
        if fs is not None:
            save_ids(input_ids_flat, fs.src, fs.dst, self.concat_input_ids)
            if self.final_hidden is not None and hidden_states is not None:
                save_rows(hidden_states, None, self.final_hidden, fs.src, fs.dst)

    def zero_offset_range(self, off: int, n: int) -> None:
        """Zero rows ``[off, off + n)`` of every buffer after an aborted forward
        (accumulate.py:632-656)."""
        if n <= 0 or off < 0:
            return
        n = min(n, self.max_saved - off)
        if n <= 0:
            return
        for b in self._all_buffers():
            b[off:off + n].zero_()
        self.concat_input_ids[off:off + n].zero_()

    def save_final_ids(self, input_ids_flat: torch.Tensor, state: FtSaveState | None = None):
        """The final save point's ids through the step's index pair
        (accumulate.py:598-622 on the op path): concat_input_ids[offset + i]
        = input_ids_flat[positions[i]]."""
        fs = state or self.capture_state()
        save_ids(input_ids_flat, fs.src, fs.dst, self.concat_input_ids)

    def _all_buffers(self) -> list:
        out = (self.layer_in + self.mlp_gate_up + self.attn_qh + self.attn_kh + self.attn_vh
               + self.attn_ctx + self.resid_mid + [self.final_in])
        return out + ([self.final_hidden] if self.final_hidden is not None else [])

    def activations(self) -> dict:
        """The activation dict a backward cycle takes (the ``buffers`` of the
        share_activations message, accumulate.py:236-252)."""
        out = {"layer_in": self.layer_in, "final_in": self.final_in,
               "concat_input_ids": self.concat_input_ids}
        for name in ("mlp_gate_up", "attn_qh", "attn_kh", "attn_vh", "attn_ctx", "resid_mid"):
            if getattr(self, name):
                out[name] = getattr(self, name)
        if self.final_hidden is not None:
            out["final_hidden"] = self.final_hidden
        return out


def _register_torch_op():
    """Register ``deltaserve::dserve_save_rows`` with ``marker`` declared mutated
    (the reference registers the same signature as ``vllm::dserve_save_rows``,
    ft_save_op.py:97-102), so a compiled forward keeps the call opaque."""
    try:
        lib = torch.library.Library("deltaserve", "FRAGMENT")
        lib.define("dserve_save_rows(Tensor x, Tensor? r, Tensor(a!) marker, int slot) -> ()")
        lib.impl("dserve_save_rows", dserve_save_rows, "CompositeExplicitAutograd")
        lib.impl("dserve_save_rows", lambda x, r, marker, slot: None, "Meta")
        return lib
    except RuntimeError:  # already registered in this process
        return None


_TORCH_LIB = _register_torch_op()
