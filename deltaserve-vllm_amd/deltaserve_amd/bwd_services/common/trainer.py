"""``LoraSftTrainerService`` — the drop-in LoRA-SFT backward child on MI355X.

Same surface as the reference's ``bwd_services/common/trainer.py``:
``_build_state`` turns the shared ``base``/``ft``/``meta`` dicts into bound
state, ``process_backward(activations, sample_lens, n, epoch) -> (loss,
n_valid)`` runs one cycle, and ``save_adapter`` / ``export_lora_state`` /
``switch_adapter`` / ``_publish_to_served`` keep their behaviour. The fp32
LoRA masters stay torch ``nn.Parameter``s (their ``.grad`` holds the clipped
gradient after a cycle) so every reader of them is unchanged.

What differs is where the cycle runs: ``libdsb.so`` executes the whole
head → reversed-layer → clip → AdamW sequence as one captured hipGraph of
hand-written gfx950 kernels (``include/dsb.h``). There is no eager PyTorch
path and no CPU path: if the library is missing the service fails to build.
"""

from __future__ import annotations

import ctypes
import os
import re
from ctypes import byref, c_float, c_int, c_void_p

import torch
import torch.nn as nn

from deltaserve_amd import _lib as L
from deltaserve_amd import dprint
from deltaserve_amd.bwd_services.base import BackwardService
from deltaserve_amd.bwd_services.common.family import LORA_PROJS, Family
from deltaserve_amd.checkpoint import AdapterCheckpointer, write_save_error
from deltaserve_amd.ops import rope_inv_freq  # noqa: F401  (re-exported for callers)

# PEFT adapter keys turned into fp32 masters (trainer.py:46-47, extended to the
# MLP projections).
_LORA_KEY_RE = re.compile(
    r"layers\.(\d+)\.(?:self_attn|mlp)\.(q|k|v|o|gate|up|down)_proj\.lora_([AB])\.weight")


def _graph_enabled(meta: dict) -> bool:
    """One captured hipGraph per cycle unless the worker asked for eager
    launches: this build's ``backward_hip_graph`` key when given, else the
    reference config's ``backward_cuda_graph`` (config.py:94), else on."""
    for key in ("backward_hip_graph", "backward_cuda_graph"):
        if key in meta and meta[key] is not None:
            return bool(meta[key])
    return True


class LoraSftTrainerService(BackwardService):
    """Backward child that trains the FT LoRA adapter for one model family."""

    family: Family = None

    def __init__(self, device_index: int) -> None:
        super().__init__(device_index)
        assert self.family is not None, f"{type(self).__name__} must set ``family``"
        self._built = False
        self.lora: dict = {}
        self._grads: dict = {}
        self._ft_keys: dict = {}
        self._ckpt = AdapterCheckpointer(self)
        self._h = None
        self._act_key = None
        self._served_key = None
        self._opt_step = 0
        self._keep: list = []
        self.lr = 0.0
        self.weight_decay = 0.0
        self.gamma = 1.0
        self.last_cycle_info = None

    # ------------------------------------------------------------ build
    def _on_weights_shared(self) -> str | None:
        """trainer.py:98-110: a build failure is returned to the worker."""
        try:
            self._build_state()
            self._built = True
            return None
        except Exception as e:  # noqa: BLE001 — reported to the worker
            import traceback
            dprint(f"[backward] {self.family.name} state build failed: {e}")
            traceback.print_exc()
            return f"{type(e).__name__}: {e}"

    def _build_state(self) -> None:
        meta = self.shared["meta"]
        base = self.shared["base"] or {}
        ft = self.shared["ft"] or {}
        fam = self.family
        if int(meta.get("tp_size", 1)) != 1:
            raise NotImplementedError("the MI355X backward runs one GPU per model (tp_size 1)")
        self.tp_size, self.tp_rank = 1, 0
        self.D = int(meta["hidden_size"])
        self.L = int(meta["num_hidden_layers"])
        self.Hq = int(meta["num_attention_heads"])
        self.Hkv = int(meta["num_key_value_heads"])
        # head_dim as ft_meta.py:144-145 states it (hidden / heads when absent)
        self.Hd = int(meta.get("head_dim") or self.D // self.Hq)
        self.q_size, self.kv_size = self.Hq * self.Hd, self.Hkv * self.Hd
        self.inter = int(meta["intermediate_size"])
        self.theta = float(meta["rope_theta"])
        self.rope_scaling = meta.get("rope_scaling")
        self.eps = float(meta["rms_norm_eps"])
        self.scaling = float(meta.get("lora_scaling", 1.0))
        self.vocab = int(meta["vocab_size"])
        self.lr = float(meta["learning_rate"])
        self.weight_decay = float(meta.get("weight_decay", 0.0))
        self.gamma = float(meta.get("gamma", 1.0))
        if meta.get("backward_fp32"):
            dprint("[backward] backward_fp32 requested: the MI355X path computes every "
                   "product with bf16 operands and fp32 accumulation")

        bn = {k.replace(".base_layer.", "."): v for k, v in base.items()}

        def bw(name):
            if name not in bn:
                raise KeyError(f"base weight {name!r} not found (have e.g. "
                               f"{list(bn)[:4]} … {len(bn)} keys)")
            t = bn[name]
            if t.dtype != torch.bfloat16 or not t.is_cuda:
                raise TypeError(f"base weight {name!r} must be a bf16 CUDA tensor")
            return t

        self.lm_w = bw(meta.get("lm_head_key") or "lm_head.weight")[:self.vocab].contiguous()
        self.norm_w = bw(meta.get("norm_weight_key") or "model.norm.weight")

        layers = []
        for i in range(self.L):
            p = f"model.layers.{i}."
            lw = {}
            for key, rel in fam.layer_weights.items():
                if key == "qkv" and p + rel not in bn:
                    parts = [bw(p + f"self_attn.{x}_proj.weight") for x in ("q", "k", "v")]
                    lw[key] = torch.cat(parts, 0).contiguous()
                elif key == "gate_up" and p + rel not in bn:
                    parts = [bw(p + f"mlp.{x}_proj.weight") for x in ("gate", "up")]
                    lw[key] = torch.cat(parts, 0).contiguous()
                else:
                    lw[key] = bw(p + rel).contiguous()
            layers.append(lw)
        self._base_layers = layers

        params = []
        rank = None
        for key, t in ft.items():
            m = _LORA_KEY_RE.search(key)
            if m is None:
                continue
            layer, proj, ab = int(m.group(1)), m.group(2), m.group(3)
            param = nn.Parameter(t.detach().to(self.lm_w.device, torch.float32).clone().contiguous())
            grad = torch.zeros_like(param)
            param.grad = grad
            self.lora.setdefault(layer, {}).setdefault(proj, {})[ab] = param
            self._grads[(layer, proj, ab)] = grad
            self._ft_keys[(layer, proj, ab)] = key
            params.append(param)
            r = param.shape[0] if ab == "A" else param.shape[1]
            if rank is not None and r != rank:
                raise ValueError(f"LoRA tensors disagree on the rank ({rank} vs {r})")
            rank = r
        if rank is None:
            raise ValueError("the FT adapter holds no LoRA tensors")
        self.rank = rank
        self._train_state_bytes = 4 * 4 * sum(p.numel() for p in params)

        s_max = int(meta.get("max_saved_finetuning_tokens", 0) or 0)
        self._s_max = s_max
        self._ckpt.configure(meta)
        if s_max > 0:
            self._create_handle(s_max)
        dprint(f"[backward] {fam.name} built: {self.L} layers, {len(params)} LoRA tensors, "
               f"r={self.rank}, scaling={self.scaling}, rope="
               f"{(self.rope_scaling or {}).get('rope_type', 'default')}(theta={self.theta:g}), "
               f"lr={self.lr}, wd={self.weight_decay}, gamma={self.gamma}")

    def _create_handle(self, s_max: int) -> None:
        lib = L.load()
        rs = self.rope_scaling or {}
        rtype = rs.get("rope_type", "default") or "default"
        codes = {"default": L.ROPE_DEFAULT, "linear": L.ROPE_LINEAR, "llama3": L.ROPE_LLAMA3}
        if rtype not in codes:
            raise NotImplementedError(f"RoPE type {rtype!r} is not supported")
        d = L.DsbDesc()
        d.abi_version = L.ABI_VERSION
        d.family = self.family.dsb_family
        d.n_layers, d.hidden, d.n_heads, d.n_kv_heads = self.L, self.D, self.Hq, self.Hkv
        d.head_dim, d.intermediate, d.vocab, d.lora_rank = self.Hd, self.inter, self.vocab, self.rank
        d.lora_scaling, d.rms_eps, d.rope_theta = self.scaling, self.eps, self.theta
        d.rope_type = codes[rtype]
        d.rope_factor = float(rs.get("factor", 1.0))
        d.rope_low_freq_factor = float(rs.get("low_freq_factor", 1.0))
        d.rope_high_freq_factor = float(rs.get("high_freq_factor", 1.0))
        d.rope_orig_max_pos = float(rs.get("original_max_position_embeddings", 1.0))
        meta = self.shared["meta"]
        # every sequence of a cycle holds at least one of its s_max tokens, so
        # s_max sequences admit any packing (backward_max_seqs may lower it:
        # it only sizes the attention tile table)
        d.s_max = int(s_max)
        d.max_seqs = int(meta.get("backward_max_seqs") or s_max)
        d.beta1, d.beta2, d.adam_eps = 0.9, 0.999, 1e-8
        d.weight_decay, d.max_grad_norm = self.weight_decay, 1.0
        d.flags = L.FLAG_GRAPH if _graph_enabled(meta) else 0
        if meta.get("backward_serial_layers"):
            d.flags |= L.FLAG_SERIAL_LAYERS
        d.vocab_chunk = int(meta.get("backward_vocab_chunk") or 0)
        d.gemm_tile = int(meta.get("backward_gemm_tile") or 0)
        h = c_void_p()
        L.check(lib.dsb_create(byref(d), byref(h)), None, "dsb_create")
        self._h = h
        self._s_max = int(s_max)
        for i, lw in enumerate(self._base_layers):
            w = L.DsbLayerWeights()
            for key in ("qkv", "o", "gate_up", "down", "in_ln", "post_ln", "q_norm", "k_norm"):
                t = lw.get(key)
                setattr(w, key, None if t is None else t.data_ptr())
            L.check(lib.dsb_bind_weights(h, i, byref(w)), h, "dsb_bind_weights")
        L.check(lib.dsb_bind_head(h, self.lm_w.data_ptr(), self.norm_w.data_ptr()), h,
                "dsb_bind_head")
        for (layer, proj, ab), _ in self._ft_keys.items():
            if ab != "A":
                continue
            pa, pb = self.lora[layer][proj]["A"], self.lora[layer][proj]["B"]
            t = L.DsbLoraTensors(pa.data_ptr(), pb.data_ptr(), self._grads[(layer, proj, "A")].data_ptr(),
                                 self._grads[(layer, proj, "B")].data_ptr())
            L.check(lib.dsb_bind_lora(h, layer, L.PROJ_INDEX[proj], byref(t)), h, "dsb_bind_lora")

    def _saved_points(self, activations) -> dict:
        """The optional save points the cycle consumes, gated as the reference
        trainer gates them (trainer.py:160-177, :532-552): ``mlp_gate_up``
        and ``attn_ctx`` whenever the store carries them, q/k/v only with the
        worker's ``save_attn_qkv`` (all three buffers), ``resid_mid`` only
        with ``save_resid_mid``. Returns name -> (per-layer list, width)."""
        meta = self.shared.get("meta") or {}
        want = {"mlp_gate_up": 2 * self.inter, "attn_ctx": self.q_size}
        if meta.get("save_attn_qkv") and self.family.supports_saved_qkv and all(
                activations.get(k) is not None for k in ("attn_qh", "attn_kh", "attn_vh")):
            want.update(attn_qh=self.q_size, attn_kh=self.kv_size, attn_vh=self.kv_size)
        if meta.get("save_resid_mid"):
            want["resid_mid"] = self.D
        out = {}
        for name, width in want.items():
            bufs = activations.get(name)
            if bufs is None or (isinstance(bufs, (list, tuple)) and not bufs):
                continue
            if len(bufs) != self.L:
                raise ValueError(f"{name} carries {len(bufs)} layers, the model has {self.L}")
            ld = bufs[0].stride(0)
            for t in bufs:
                if (t.dtype != torch.bfloat16 or not t.is_cuda or t.stride(0) != ld
                        or t.stride(1) != 1 or t.shape[1] != width):
                    raise TypeError(f"{name} buffers must be bf16 CUDA [rows, {width}] with one "
                                    "row stride")
            out[name] = (bufs, ld)
        return out

    def _bind_activations(self, activations) -> None:
        li = activations["layer_in"]
        fi = activations["final_in"]
        ids = activations["concat_input_ids"]
        if len(li) != self.L:
            raise ValueError(f"activations carry {len(li)} layer inputs, the model has {self.L}")
        ld = fi.stride(0)
        for t in list(li) + [fi]:
            if t.dtype != torch.bfloat16 or not t.is_cuda or t.stride(0) != ld or t.stride(1) != 1:
                raise TypeError("activation buffers must be bf16 CUDA [rows, D] with one row stride")
        if ids.dtype != torch.int64 or not ids.is_cuda:
            raise TypeError("concat_input_ids must be an int64 CUDA tensor")
        saved = self._saved_points(activations)
        key = (tuple(t.data_ptr() for t in li), fi.data_ptr(), ids.data_ptr(), ld,
               tuple((name, tuple(t.data_ptr() for t in bufs), sld)
                     for name, (bufs, sld) in sorted(saved.items())))
        if key == self._act_key:
            return
        keep = []  # the pointer arrays must outlive the bind call

        def ptrs(bufs):
            arr = (c_void_p * self.L)(*[t.data_ptr() for t in bufs])
            keep.append(arr)
            return ctypes.cast(arr, ctypes.POINTER(c_void_p))

        a = L.DsbActivations()
        a.layer_in, a.final_in, a.input_ids, a.ld = ptrs(li), fi.data_ptr(), ids.data_ptr(), ld
        fields = {"mlp_gate_up": ("mlp_gate_up", "ld_gate_up"), "attn_qh": ("attn_q", "ld_q"),
                  "attn_kh": ("attn_k", "ld_k"), "attn_vh": ("attn_v", "ld_v"),
                  "attn_ctx": ("attn_ctx", "ld_ctx"), "resid_mid": ("resid_mid", "ld_resid_mid")}
        for name, (bufs, sld) in saved.items():
            f_ptr, f_ld = fields[name]
            setattr(a, f_ptr, ptrs(bufs))
            setattr(a, f_ld, sld)
        L.check(L.load().dsb_bind_activations(self._h, byref(a)), self._h, "dsb_bind_activations")
        self._act_ptrs = keep
        self._act_key = key
        self.saved_points = sorted(saved)

    # ------------------------------------------------------------ the cycle
    def process_backward(self, activations, sample_lens, n, epoch):
        """trainer.py:503-678 — one backward + AdamW step; returns (loss, n_valid)."""
        self._maybe_pause()
        if not self._built:
            raise RuntimeError(
                f"{self.family.name} backward state not built (weights not shared)")
        self._last_mode = "graph"
        # zero-length samples hold no rows and predict nothing
        seq_lens = [int(s) for s in sample_lens if int(s) > 0]
        n = int(n)
        if self._h is None:
            self._create_handle(int(activations["final_in"].shape[0]) - 1)
        if n > self._s_max:
            raise ValueError(f"n={n} exceeds the backward capacity s_max={self._s_max}")
        self._bind_activations(activations)
        self._bind_served_buffers()
        self._opt_step += 1
        loss = c_float(0.0)
        nv = c_int(0)
        info = L.DsbCycleInfo()
        stream = c_void_p(torch.cuda.current_stream().cuda_stream)
        lib = L.load()
        if self._use_segments():
            rc = self._run_segmented(lib, seq_lens, n, stream, loss, nv, info)
            what = "segmented cycle"
        else:
            rc = lib.dsb_step(self._h, L.i32_array(seq_lens), len(seq_lens), n, float(self.lr),
                              int(self._opt_step), stream, byref(loss), byref(nv), byref(info))
            what = "dsb_step"
        if rc != 0:
            self._opt_step -= 1
            L.check(rc, self._h, what)
        self.last_cycle_info = {"gpu_ms": info.gpu_ms, "graph": bool(info.graph),
                                "n_valid": info.n_valid}
        self._last_mode = ("graph" if info.graph else "eager") + (
            "/segments" if what != "dsb_step" else "")
        if epoch > self.current_epoch:
            self.lr *= self.gamma  # StepLR(step_size=1, gamma) stepped per epoch advance
            self.current_epoch = epoch
        # the served LoRA slots were written inside the cycle, after AdamW
        return float(loss.value), int(nv.value)

    def _use_segments(self) -> bool:
        """Pause points (one graph per segment) when a GPU grant is wired in
        (co-located with serving) or meta asks for them; otherwise the whole
        cycle is one graph."""
        meta = self.shared.get("meta") or {}
        if meta.get("backward_single_graph"):
            return False
        return self._gpu_grant is not None or bool(meta.get("backward_pause_boundaries"))

    def _run_segmented(self, lib, seq_lens, n, stream, loss, nv, info) -> int:
        """trainer.py:503-678 with _maybe_pause before the cycle (:504), once
        per vocab chunk in both LM-head passes (head.py:78-80, :92-94) and at
        every layer boundary (:577-581); the last segment is the optimizer
        and publish."""
        rc = lib.dsb_step_begin(self._h, L.i32_array(seq_lens), len(seq_lens), n,
                                float(self.lr), int(self._opt_step), stream)
        if rc != 0:
            return rc
        run_ahead = self._run_ahead()
        nseg = lib.dsb_num_segments(self._h)
        for seg in range(nseg):
            # a pause point before every head vocab chunk (both passes) and
            # every layer; the optimizer segment runs straight after the last
            if seg < nseg - 1:
                self._maybe_pause()
            rc = lib.dsb_step_segment(self._h, seg, run_ahead)
            if rc != 0:
                break
        rc_end = lib.dsb_step_end(self._h, stream, byref(loss), byref(nv), byref(info))
        return rc if rc != 0 else rc_end

    # ------------------------------------------------------------ capture checks
    VERIFY_TOL = 5e-2  # relative; bf16 round trips of the capture path stay well inside

    def verify_activations(self, activations: dict, n: int) -> list[tuple[str, float, bool]]:
        """Debug-gated capture checks (trainer.py:806-826; on with the
        ``print_hash`` of ``share_activations``): the first layer's saved
        input must be the embedding rows of the saved ids, and the final
        norm of ``final_in`` must be the saved ``final_hidden``. Logs each
        check and returns ``(name, relative error, ok)``."""
        meta = self.shared.get("meta") or {}
        base = {k.replace(".base_layer.", "."): v for k, v in (self.shared.get("base") or {}).items()}
        out = []

        def judge(name, got, want):
            err = float((got.float() - want.float()).abs().max())
            rel = err / (float(want.float().abs().max()) + 1e-6)
            ok = rel < self.VERIFY_TOL
            dprint(f"[verify] {name}: max|d|={err:.3e} rel={rel:.3e} {'OK' if ok else 'FAIL'}")
            out.append((name, rel, ok))

        ids = activations["concat_input_ids"][:n].long()
        layer_in = activations.get("layer_in") or []
        embed = base.get(meta.get("embed_weight_key") or "model.embed_tokens.weight")
        if layer_in and embed is not None:
            judge("layer_in[0] vs embed[ids]", layer_in[0][:n], embed[ids])
        final_in, final_hidden = activations.get("final_in"), activations.get("final_hidden")
        norm_w = base.get(meta.get("norm_weight_key") or "model.norm.weight")
        if final_in is not None and final_hidden is not None and norm_w is not None and n > 0:
            from deltaserve_amd import ops

            normed = ops.rmsnorm(final_in[:n], norm_w, float(meta.get("rms_norm_eps", 1e-5)))
            judge("RMSNorm(final_in) vs final_hidden", normed, final_hidden[:n])
        return out

    # ------------------------------------------------------------ checkpoints
    def masters(self):
        """(PEFT key, fp32 master) pairs of the adapter being trained."""
        for (layer, proj, ab), key in self._ft_keys.items():
            yield key, self.lora[layer][proj][ab]

    def save_adapter(self, out_dir: str, save_id: str, reason: str = "manual") -> None:
        """A PEFT checkpoint of the current masters (trainer.py:386-391)."""
        if not self._built:
            write_save_error(out_dir, save_id, "trainer state not built")
            return
        self._ckpt.write(out_dir, save_id, self._ckpt.snapshot(reason, self.current_epoch))

    def _handle_save_adapter(self, msg) -> None:
        self.save_adapter(str(msg.get("path")), str(msg.get("save_id")))

    def _before_cycle(self, epoch: int, attempted: bool) -> None:
        if attempted and self._built:
            self._ckpt.before_cycle(epoch)

    def _after_cycle(self, epoch: int, attempted: bool) -> None:
        if attempted:
            if self._built:
                self._ckpt.after_cycle(epoch)
            else:
                self._ckpt.schedule.cycle_done(epoch)

    @property
    def _cycles_attempted(self) -> int:
        return self._ckpt.schedule.attempted

    # ------------------------------------------------------------ adapters
    def export_lora_state(self) -> dict:
        """trainer.py:749-754: the plain PEFT factors as fp32 CPU tensors."""
        return {key: p.detach().float().cpu().clone() for key, p in self.masters()}

    def _matched_adapter(self, ft: dict) -> dict:
        """Pairs each master with the incoming adapter's tensor; ValueError
        unless the adapter has exactly the launch adapter's LoRA tensors and
        shapes (the rank and target modules are baked into the handle)."""
        incoming = {}
        for key, t in ft.items():
            m = _LORA_KEY_RE.search(key)
            if m is not None:
                incoming[(int(m.group(1)), m.group(2), m.group(3))] = (key, t)
        ours = {(layer, proj, ab): p for layer, projs in self.lora.items()
                for proj, pair in projs.items() for ab, p in pair.items()}
        if incoming.keys() != ours.keys():
            raise ValueError(f"the adapter has {len(incoming)} LoRA tensors, the launch adapter "
                             f"{len(ours)} (different target modules or layers)")
        bad = [(k, tuple(incoming[k][1].shape), tuple(p.shape)) for k, p in ours.items()
               if tuple(incoming[k][1].shape) != tuple(p.shape)]
        if bad:
            k, got, want = bad[0]
            raise ValueError(f"LoRA tensor {k} has shape {got}, the launch adapter's is {want} "
                             f"(different rank?)")
        return {k: (ours[k], incoming[k][0], incoming[k][1]) for k in ours}

    def switch_adapter(self, ft: dict, hparams: dict) -> dict:
        """trainer.py:680-742: train another adapter of the launch adapter's
        shape. Its weights are copied into the existing masters (so the
        handle, its graphs and the served slots stay valid), the optimizer
        and schedule restart, and the new weights are published."""
        if not self._built:
            raise RuntimeError("the trainer was never built (no adapter at launch)")
        alpha_r = float(hparams.get("lora_scaling", self.scaling))
        if abs(alpha_r - self.scaling) > 1e-9:
            raise ValueError(f"the adapter's alpha/r is {alpha_r}, the launch adapter's is "
                             f"{self.scaling}; they must match")
        matched = self._matched_adapter(ft)
        if hparams.get("dry_run"):
            return {"tensors": len(matched), "dry_run": True}
        with torch.no_grad():
            for k, (param, _, t) in matched.items():
                param.copy_(t.to(param.device, torch.float32))
                self._grads[k].zero_()
        self._ft_keys = {k: key for k, (_, key, _) in matched.items()}
        self.lr = float(hparams["learning_rate"])
        self.weight_decay = float(hparams["weight_decay"])
        self.gamma = float(hparams["gamma"])
        self._opt_step = 0
        if self._h is not None:
            L.check(L.load().dsb_reset_optimizer(self._h, self.weight_decay), self._h,
                    "dsb_reset_optimizer")
        self.current_epoch = 0
        self.ledger.restart(int(hparams.get("total_tokens_per_epoch", 0)))
        self._publish_to_served()
        dprint(f"[backward] switched to a new adapter: {len(matched)} LoRA tensors, "
               f"lr={self.lr}, wd={self.weight_decay}, gamma={self.gamma}")
        return {"tensors": len(matched)}

    def _on_lora_buffers(self) -> None:
        self._served_key = None
        if self._h is not None:
            self._bind_served_buffers()

    def _bind_served_buffers(self) -> None:
        """Registers vLLM's stacked LoRA slot rows with libdsb (trainer.py:760-802:
        a_buf[slot, 0, :r, :in] = clamp(A), b_buf[slot, 0, :out, :r] = clamp(s·B),
        bf16) so every cycle publishes inside its graph, after AdamW."""
        bufs = self.lora_buffers
        if not bufs or self._h is None:
            return
        slot = int(bufs["slot"])
        key = (slot, tuple((int(i), p, buf["a"].data_ptr(), buf["b"].data_ptr())
                           for i, projd in sorted(bufs["layers"].items(), key=lambda kv: int(kv[0]))
                           for p, buf in sorted(projd.items())))
        if key == self._served_key:
            return
        lib = L.load()
        for i, projd in bufs["layers"].items():
            i = int(i)
            for proj, buf in projd.items():
                if proj not in self.lora.get(i, {}):
                    continue
                a, b = buf["a"][slot, 0], buf["b"][slot, 0]
                for t in (a, b):
                    if t.dtype != torch.bfloat16 or not t.is_cuda or t.stride(1) != 1:
                        raise TypeError("served LoRA buffers must be bf16 CUDA tensors with "
                                        "contiguous rows")
                pa, pb = self.lora[i][proj]["A"], self.lora[i][proj]["B"]
                if a.shape[0] < pa.shape[0] or a.shape[1] < pa.shape[1] or \
                        b.shape[0] < pb.shape[0] or b.shape[1] < pb.shape[1]:
                    raise ValueError(f"served slot of layer {i} {proj} is smaller than the adapter")
                L.check(lib.dsb_bind_served(self._h, i, L.PROJ_INDEX[proj], a.data_ptr(),
                                            a.stride(0), b.data_ptr(), b.stride(0)),
                        self._h, "dsb_bind_served")
        self._served_key = key

    def _publish_to_served(self) -> None:
        """Publishes the current masters into the served slots now, outside a
        cycle (the switch_adapter path; cycles publish inside their graph)."""
        if not self.lora_buffers or self._h is None:
            return
        self._bind_served_buffers()
        stream = c_void_p(torch.cuda.current_stream().cuda_stream)
        L.check(L.load().dsb_publish(self._h, stream), self._h, "dsb_publish")

    def kernel_stats(self) -> list[dict]:
        """Per-kernel-class timing (meta ``backward_kernel_timing``): calls,
        total ms, algorithmic flops and HBM bytes over the cycles run so far."""
        return L.kernel_stats(self._h) if self._h is not None else []

    def set_kernel_timing(self, on: bool) -> None:
        """Per-kernel timing on eager replays of the cycle (off: graph replays)."""
        if self._h is not None:
            L.check(L.load().dsb_set_kernel_timing(self._h, int(bool(on))), self._h,
                    "dsb_set_kernel_timing")

    def reset_kernel_stats(self) -> None:
        if self._h is not None:
            L.check(L.load().dsb_kernel_stats_reset(self._h), self._h, "dsb_kernel_stats_reset")

    def close(self) -> None:
        if self._h is not None:
            L.load().dsb_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass
