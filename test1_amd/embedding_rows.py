"""Row-sparse embedding unit: only the rows a batch uses cross the host link.

Mixed into ``LayerRuntimeState``.  The reference stages the whole embedding
table for every lookup (layer_state.py:296-314) and offloads its whole
gradient (layer_state.py:367-393); here the lookup gathers the batch's rows
from the pinned host table with one kernel and the backward sends back only
the batch's gradient rows, and the host AdamW updates the table with zero
gradient elsewhere (the dense update's bits).
"""

from __future__ import annotations

import threading
from concurrent import futures
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import _native, kernels
from .pinned import pinned_empty
from .staging import _new_event
from .update_executor import EARLY_UPDATE_PRIORITY, _LinkQuiet


class RowSparseEmbedding:
    """Methods of a ``LayerRuntimeState`` whose unit is an ``nn.Embedding``
    moved row by row (``enable_row_sparse``)."""

    def enable_row_sparse(self) -> None:
        """Move only the rows a batch uses, for an ``nn.Embedding`` unit.

        Forward: ``gather_rows`` reads the batch's rows straight from the
        pinned host table (fp32 master, or its bf16 copy) with one kernel and
        rounds them to bf16: the lookup's output, bit for bit, without staging
        the table (reference layer_state.py:296-314 stages all of it, 2 or 4
        bytes per parameter).  Backward: ``offload_rows`` computes the dense
        table gradient on the device as the lookup's own backward does and
        sends only the batch's rows to host; the host AdamW then updates the
        whole table with zero gradient elsewhere (``sf_adam_update_rows``),
        which is the dense update's result."""
        emb = self.layer
        if not isinstance(emb, nn.Embedding) or emb.max_norm is not None or emb.scale_grad_by_freq or emb.sparse:
            raise ValueError("enable_row_sparse: a plain nn.Embedding unit is required")
        V, H = emb.weight.shape
        if H % 16 != 0 or len(self._params) != 1:
            raise ValueError("enable_row_sparse: the row length must be a multiple of 16")
        self.row_sparse = True
        self._rows_shape = (V, H)
        self._bad_ids = pinned_empty(1, torch.int32)
        self._bad_ids.zero_()
        self._rows_host: Optional[torch.Tensor] = None
        self._ids_host: Optional[torch.Tensor] = None
        # The batch's ids on the host, copied at the lookup (pinned, event),
        # for the early part of the update; the early part itself, once queued.
        self._ids_early_host: Optional[torch.Tensor] = None
        self._lookup_ids: Optional[Tuple[torch.Tensor, torch.cuda.Event]] = None
        self._early: Optional[Dict[str, Any]] = None
        self._early_lock = threading.Lock()

    def host_buffers_fit(self, ntok: int) -> bool:
        """The pinned buffers of a batch of ``ntok`` tokens (gradient rows and
        ids, lookup ids) exist and are large enough."""
        return all(b is not None and b.shape[0] >= ntok
                   for b in (self._rows_host, self._ids_host, self._ids_early_host))

    def has_host_buffers(self) -> bool:
        return any(b is not None for b in (self._rows_host, self._ids_host, self._ids_early_host))

    def alloc_host_buffers(self, ntok: int) -> None:
        """Pin the buffers of a batch of ``ntok`` tokens.  Called before a
        step's first copy (``SlideFSDP.forward``), with nothing in flight that
        reads or writes the buffers it replaces, so that no pinned memory is
        allocated while copies run (the lookup and the backward allocate them
        only if this was not called)."""
        n = max(int(ntok), 1)
        self._rows_host = pinned_empty((n, self._rows_shape[1]), torch.bfloat16)
        self._ids_host = pinned_empty(n, torch.int64)
        self._ids_early_host = pinned_empty(n, torch.int64)

    def _host_table(self) -> torch.Tensor:
        V, H = self._rows_shape
        src = self._cpu_params_bf16 if self._cpu_params_bf16 is not None else self._cpu_params_flat
        return src.view(V, H)

    def gather_rows(self, ids: torch.Tensor) -> torch.Tensor:
        """Forward lookup: [*ids.shape, H] bf16 rows of the current master."""
        self.wait_for_update()
        self.settle_orphaned_early()
        V, H = self._rows_shape
        flat = ids.reshape(-1)
        if flat.dtype != torch.int64:
            flat = flat.long()
        if not flat.is_contiguous():
            flat = flat.contiguous()
        out = torch.empty(tuple(ids.shape) + (H,), dtype=torch.bfloat16, device=self.runtime.device)
        # The flag's previous writer (last step's lookup) finished before that
        # step's update, which wait_for_update has just waited for.
        self._bad_ids.zero_()
        lt = self.runtime.link_timing
        cur = torch.cuda.current_stream()
        if lt is not None:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(cur)
        kernels.gather_rows(self._host_table(), flat, out.view(-1, H), bad=self._bad_ids, stream=cur)
        if lt is not None:
            t1 = torch.cuda.Event(enable_timing=True)
            t1.record(cur)
            lt["rows_h2d"].append((t0, t1, flat.numel() * H * self._host_table().element_size()))
        self._copy_lookup_ids(flat)
        self._bwd_compute_done = False
        self._grads_offloaded = False
        self.runtime.log("h2d", self.layer_idx, False)
        self.runtime.mark("h2d_issued", self.layer_idx)
        return out

    def _copy_lookup_ids(self, flat: torch.Tensor) -> None:
        """Copy the batch's ids to pinned host memory on the D2H stream, for
        the early part of this step's update.  The buffer's previous reader
        (last step's update) finished before this lookup, which waited for
        it."""
        rt = self.runtime
        ntok = flat.numel()
        if self._ids_early_host is None or self._ids_early_host.numel() < ntok:
            self._ids_early_host = pinned_empty(max(ntok, 1), torch.int64)
        ready = _new_event()
        ready.record(torch.cuda.current_stream())
        rt.d2h_stream.wait_event(ready)
        kernels.memcpy_async(self._ids_early_host[:ntok], flat, rt.d2h_stream)
        flat.record_stream(rt.d2h_stream)
        copied = _new_event()
        copied.record(rt.d2h_stream)
        self._lookup_ids = (self._ids_early_host[:ntok], copied)

    def start_early_update(self) -> None:
        """Queue the part of this step's update that needs no gradient: the
        table rows the batch did not touch (zero gradient) get their AdamW
        update now, at the lowest priority, so the host AdamW does it while
        it would otherwise wait for the backward's first gradients; the
        batch's rows follow once their gradient has landed (``step_rows_early``
        then ``step_rows``: the bits of the whole update).  It waits for the
        host link to have no unit copy queued, so that its host-memory traffic
        does not slow the copies the forward is waiting for.  Called by the
        model right before its backward, which is then certain to reach the
        lookup (not in the reference, whose update of the whole table waits
        for the gradient)."""
        if not self.row_sparse:
            return   # a unit staged whole updates in one part, after its gradient
        rt = self.runtime
        opt = self.layer_optimizer
        lookup, self._lookup_ids = self._lookup_ids, None
        if (lookup is None or opt is None or not getattr(opt, "reference_order", False)
                or not self.layer.weight.requires_grad):
            return
        if getattr(opt, "offloader", None) is not None:
            # moments on storage: the two parts would read the table's moments
            # back twice, and that step is bound by storage, not by this wait
            return
        ids, copied = lookup
        early = {"ids": ids, "ready": copied, "state": "queued"}
        self._early = early
        early["future"] = rt.update_executor.submit(EARLY_UPDATE_PRIORITY, self._do_update_rows_early, early,
                                                    ready=_LinkQuiet(copied, rt.stager))

    def _do_update_rows_early(self, early: Dict[str, Any]) -> bool:
        """Update thread: the early part queued by ``start_early_update``
        (nothing if the late part has already run it or it was cancelled).
        States: queued -> running -> applied, skipped (ids out of range: the
        late part raises for them) or failed; queued -> cancelled."""
        with self._early_lock:
            if early["state"] != "queued":
                return False
            early["state"] = "running"
        rt = self.runtime
        V, H = self._rows_shape
        try:
            kernels.wait_event(early["ready"], rt.wait_timeout, f"unit {self.layer_idx}: lookup ids")
            ids = early["ids"]
            if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= V):
                early["state"] = "skipped"
                return False
            rt.mark("early_update_start", self.layer_idx)
            slot = torch.full((V,), _native.SF_ROW_ZERO, dtype=torch.int64)
            slot[ids] = _native.SF_ROW_SKIP
            if rt.capturing(self.layer_idx):
                early["master_before"] = self._cpu_params_flat.clone()
            rt.set_adam_threads()
            with self.update_lock:
                self.layer_optimizer.step_rows_early(self.layer_idx, slot,
                                                     param_view=self._cpu_params_flat.view(V, H),
                                                     bf16_view=None if self._cpu_params_bf16 is None
                                                     else self._cpu_params_bf16.view(V, H))
            early["state"] = "applied"
        except BaseException:
            early["state"] = "failed"
            raise
        rt.mark("early_update_done", self.layer_idx)
        return True

    def settle_orphaned_early(self) -> None:
        """Close an early part whose late part will never run: the step's
        backward failed before it reached the lookup.  A part still queued is
        cancelled; one that ran began the table's step (its untouched rows
        were updated with zero gradient), which is completed here with zero
        gradient for the batch's rows as well, so that every row of the table
        has taken the same step and the next step starts from a consistent
        table and step counter.  Waits for a part that is running, so that no
        update writes the table while the next lookup reads it."""
        early, self._early = getattr(self, "_early", None), None
        if early is None:
            return
        rt = self.runtime
        with self._early_lock:
            cancelled = early["state"] == "queued"
            if cancelled:
                early["state"] = "cancelled"
        f = early.get("future")
        if cancelled:
            if f is not None:
                f.cancel()   # the worker skips it (or finds it cancelled)
        elif f is not None:
            try:
                f.result(timeout=rt.wait_timeout)
            except futures.TimeoutError:
                raise TimeoutError(f"Layer {self.layer_idx}: early update not finished after "
                                   f"{rt.wait_timeout:g} s") from None
            except Exception:
                pass   # its state says what happened
        opt = self.layer_optimizer
        if early["state"] == "applied":
            V, H = self._rows_shape
            row_slot = torch.full((V,), _native.SF_ROW_SKIP, dtype=torch.int64)
            row_slot[early["ids"]] = _native.SF_ROW_ZERO
            no_rows = torch.empty((0, H), dtype=torch.bfloat16)
            with self.update_lock:
                opt.step_rows(self.layer_idx, row_slot, no_rows, param_view=self._cpu_params_flat.view(V, H),
                              bf16_view=None if self._cpu_params_bf16 is None else self._cpu_params_bf16.view(V, H))
        elif early["state"] == "failed":
            opt.abandon_early_step(self.layer_idx)

    def offload_rows(self, grad_out: torch.Tensor, ids: torch.Tensor) -> None:
        """Backward of the lookup: dense table gradient on the device (as the
        lookup's backward computes it), its batch rows to pinned host slots,
        then the update is queued."""
        rt = self.runtime
        V, H = self._rows_shape
        flat = ids.reshape(-1)
        ntok = flat.numel()
        pad = self.layer.padding_idx if self.layer.padding_idx is not None else -1
        # ids outside the table were flagged by the lookup (the update raises
        # for them); clamped here so that the dense backward never indexes
        # outside the table.  Valid ids are unchanged.
        dense = torch.ops.aten.embedding_dense_backward(grad_out.reshape(ntok, H), flat.clamp(0, V - 1), V, pad,
                                                        False)
        if rt.capturing(self.layer_idx):
            rt.capture[("device_grads", self.layer_idx)] = [dense.detach().clone().view(V, H)]
        if self._rows_host is None or self._rows_host.shape[0] < ntok:
            self._rows_host = pinned_empty((ntok, H), torch.bfloat16)
            self._ids_host = pinned_empty(ntok, torch.int64)
        grad_ready = _new_event()
        grad_ready.record(torch.cuda.current_stream())
        with self._grad_lock:
            self._post_called = True
            self._bwd_armed = False
        self.update_finished.clear()
        rt.log("d2h", self.layer_idx)
        rt.mark("post_backward", self.layer_idx)
        rt.d2h_stream.wait_event(grad_ready)
        lt = rt.link_timing
        if lt is not None:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(rt.d2h_stream)
        kernels.gather_rows(dense, flat, self._rows_host[:ntok], stream=rt.d2h_stream,
                            max_workgroups=rt.d2h_workgroups)
        if lt is not None:
            t1 = torch.cuda.Event(enable_timing=True)
            t1.record(rt.d2h_stream)
            lt["rows_d2h"].append((t0, t1, ntok * H * 2))
        kernels.memcpy_async(self._ids_host[:ntok], flat, rt.d2h_stream)
        dense.record_stream(rt.d2h_stream)
        flat.record_stream(rt.d2h_stream)
        done = _new_event()
        done.record(rt.d2h_stream)
        self._grads_offloaded = True
        self._bwd_compute_done = True
        # this step's early part (if any) now belongs to the late part
        early, self._early = self._early, None
        self._update_future = rt.update_executor.submit(rt.update_priority(self.layer_idx), self._do_update_rows,
                                                        done, ntok, early, ready=self._update_ready(done))

    def _do_update_rows(self, d2h_done: torch.cuda.Event, ntok: int, early: Optional[Dict[str, Any]]) -> bool:
        rt = self.runtime
        V, H = self._rows_shape
        try:
            rt.mark("update_start", self.layer_idx)
            kernels.wait_event(d2h_done, rt.wait_timeout, f"unit {self.layer_idx}: gradient rows")
            if int(self._bad_ids[0]) != 0:
                raise ValueError(f"embedding unit {self.layer_idx}: input ids outside [0, {V})")
            ids = self._ids_host[:ntok]
            rows = self._rows_host[:ntok]
            if early is not None and early["state"] == "queued":
                self._do_update_rows_early(early)   # not run yet: now, on this thread
            applied = early is not None and early["state"] == "applied"
            if early is not None and early["state"] == "failed":
                raise RuntimeError(f"embedding unit {self.layer_idx}: the early part of the update failed")
            row_slot = torch.full((V,), _native.SF_ROW_SKIP if applied else _native.SF_ROW_ZERO, dtype=torch.int64)
            row_slot[ids] = torch.arange(ntok, dtype=torch.int64)
            if rt.capturing(self.layer_idx):
                dense = torch.zeros(V, H, dtype=rows.dtype)
                dense[ids] = rows
                before = early["master_before"] if applied else self._cpu_params_flat.clone()
                rt.capture[self.layer_idx] = (dense.view(-1), before)
            rt.set_adam_threads()
            with self.update_lock:
                if self.layer_optimizer is not None:
                    self.layer_optimizer.step_rows(self.layer_idx, row_slot, rows,
                                                   param_view=self._cpu_params_flat.view(V, H),
                                                   bf16_view=None if self._cpu_params_bf16 is None
                                                   else self._cpu_params_bf16.view(V, H))
            rt.mark("adam_done", self.layer_idx)
        finally:
            self.update_finished.set()
        return True
