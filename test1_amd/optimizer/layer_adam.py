"""LayerAdam: one host AdamW for all units, stepped one unit at a time.

Drop-in for reference optimizer/layer_adam/layer_adam.py:9-442: same
constructor, ``param_groups`` / ``state`` / ``exp_avg_flat`` layout and the
methods ``add_layer_params``, ``step``, ``step_with_grad_views``,
``update_learning_rate`` and ``torch_adam_update``.  The arithmetic runs in
``libsf_cpu.so`` (AVX-512 + OpenMP) through the ``cpu_adam`` shim.

Differences, all deliberate:
  * ``step_with_grad_views`` hands bf16 grad views to the native update
    as they are; the reference first materialises ``grad.float()``
    (layer_adam.py:404).  Widening is exact, so the bits are the same and a
    full fp32 copy of every layer's grads per step is saved.
  * param groups are also looked up by the ``layer_idx`` they were added
    with, so a unit without parameters (``add_layer_params`` returning -1)
    does not shift later indices.
  * each instance owns its own native optimizer id (the reference always
    uses 0, layer_adam.py:59), so two instances in one process do not share
    or destroy each other's bias-correction state.
  * ``reference_order = True`` computes each update's bias corrections as
    the reference's call order would (last unit first, once per step)
    instead of from the native call-order-dependent beta^t state, so a
    caller may update units in any order and keep the reference's bits.
  * NVMe offload (``nvme_offload_fraction > 0``) keeps the reference's
    choice of moments (exp_avg, plus exp_avg_sq above 0.5) but stores them
    through the native storage engine (``StateOffloader``) instead of
    tensornvme, with ``nvme_buffers`` host buffers as a write-back cache;
    callers that update out of order name the next units with
    ``prefetch_states``.
"""

from __future__ import annotations

import itertools
import math
from collections import OrderedDict, defaultdict
from typing import Any, DefaultDict, Dict, Iterable, Optional

import torch

from . import cpu_adam as _cpu_adam
from .state_offload import StateOffloader


class LayerAdam:
    """Layer-wise AdamW over fp32 host parameters (reference layer_adam.py:9-27)."""

    _ids = itertools.count()

    def __init__(
        self,
        lr=1e-3,
        bias_correction=True,
        betas=(0.9, 0.999),
        eps=1e-8,
        weight_decay=0,
        adamw_mode=True,
        fp32_optimizer_state=True,
        num_layer: int = 0,
        nvme_offload_fraction: float = 0.0,
        offload_dir: str = "/NVME1",
        prefetch: bool = True,
        nvme_buffers: int = 4,
    ):
        self.defaults = dict(lr=lr, bias_correction=bias_correction, betas=betas, eps=eps,
                             weight_decay=weight_decay, adamw_mode=adamw_mode)
        self.param_groups = []
        self._groups_by_layer: Dict[int, dict] = {}
        self.cpu_adam = _cpu_adam
        # One native optimizer for every layer, as the reference (which always
        # uses id 0); ids are unique per instance here so that the destructor
        # of one LayerAdam cannot remove another's state.
        self.optimizer_id = next(LayerAdam._ids)
        self.cpu_adam.create_adam(self.optimizer_id, lr, betas[0], betas[1], eps, weight_decay, adamw_mode, True)
        self.fp32_optimizer_state = fp32_optimizer_state
        self.num_layer = num_layer
        # False: the native stateful update, whose bias corrections depend on
        # the order of calls, as in the reference.  True (set by callers that
        # update units out of order, not in the reference): each call gets
        # the scalars the reference's order -- last unit first, once per
        # step -- would give it.
        self.reference_order = False
        # units whose current step was begun by step_rows_early on their
        # gradient-free rows and awaits step_rows: {unit: (step, lr)}
        self._early_rows: Dict[int, tuple] = {}
        self.state: DefaultDict[torch.Tensor, Any] = defaultdict(dict)
        if not 0.0 <= nvme_offload_fraction <= 1.0:
            raise ValueError("nvme_offload_fraction must be in [0, 1]")
        self.nvme_offload_fraction = nvme_offload_fraction
        self.prefetch = prefetch
        self.pin_memory = nvme_offload_fraction > 0.0
        self.exp_avg_flat: "OrderedDict[int, torch.Tensor]" = OrderedDict()
        self.exp_avg_sq_flat: "OrderedDict[int, torch.Tensor]" = OrderedDict()
        # Moments offloaded to storage: exp_avg when the fraction is > 0, and
        # exp_avg_sq too when it is > 0.5 (reference layer_adam.py:209-218).
        self._offloaded = ()
        self._hinted = False
        if nvme_offload_fraction > 0.0:
            if offload_dir is None:
                raise ValueError("offload_dir cannot be None")
            self._offloaded = ("exp_avg", "exp_avg_sq") if nvme_offload_fraction > 0.5 else ("exp_avg",)
            self.offload_dir = offload_dir
            self.offloader = StateOffloader(offload_dir, len(self._offloaded), n_buffers=nvme_buffers)
        else:
            self.offload_dir = None
            self.offloader = None

    def __del__(self):
        try:
            self.cpu_adam.destroy_adam(self.optimizer_id)
        except Exception:
            pass
        try:
            if self.offloader is not None:
                self.offloader.close()
        except Exception:
            pass

    # ------------------------------------------------------------------
    def _group(self, layer_idx: int) -> dict:
        g = self._groups_by_layer.get(layer_idx)
        if g is None:
            raise IndexError(f"LayerAdam: no parameters registered for layer {layer_idx}")
        return g

    def _get_layer_numel(self, layer_idx: int) -> int:
        return sum(p.numel() for p in self._group(layer_idx)["params"])

    def add_layer_params(self, layer_idx: int, params: Iterable[torch.nn.Parameter]) -> int:
        """Register one unit: a param group with its own step counter and zeroed
        flat fp32 moments laid out in parameter order (reference
        layer_adam.py:131-195).  Returns ``layer_idx``, or -1 without params."""
        params = list(params)
        if not params:
            return -1
        group = {"params": params, "layer_idx": layer_idx, "step": 0, **self.defaults}
        self.param_groups.append(group)
        self._groups_by_layer[layer_idx] = group
        numel = sum(p.numel() for p in params)
        state_type = torch.float32 if self.fp32_optimizer_state else params[0].dtype
        if self._offloaded and state_type != torch.float32:
            raise ValueError("LayerAdam: NVMe offload keeps fp32 moments")
        # Offloaded moments have no host tensor between steps (the
        # reference frees their storage after the write, layer_adam.py:205-207).
        for name, flat in (("exp_avg", self.exp_avg_flat), ("exp_avg_sq", self.exp_avg_sq_flat)):
            flat[layer_idx] = (torch.empty(0, dtype=state_type) if name in self._offloaded
                               else torch.zeros(numel, dtype=state_type))
        if self._offloaded:
            self.offloader.register(layer_idx, numel)
        self._bind_states(layer_idx)
        return layer_idx

    def _bind_states(self, layer_idx: int) -> None:
        """Point ``state[p]`` at the unit's flat moments (empty views for
        moments that are on storage)."""
        off = 0
        m_flat, v_flat = self.exp_avg_flat[layer_idx], self.exp_avg_sq_flat[layer_idx]
        for p in self._group(layer_idx)["params"]:
            n = p.numel()
            st = self.state[p]
            for name, flat in (("exp_avg", m_flat), ("exp_avg_sq", v_flat)):
                st[name] = flat[off:off + n].view(p.shape) if flat.numel() else flat
            off += n

    # ------------------------------------------------------------------
    # Storage offload (reference layer_adam.py:197-244)
    def prefetch_states(self, layer_idx: int, priority: float = 0.0) -> None:
        """Start reading ``layer_idx``'s moments from storage (not in the
        reference, whose ``_pre_step`` always prefetches ``layer_idx - 1``):
        a caller that knows its update order names the units itself, after
        which steps no longer guess."""
        if self.offloader is not None:
            self._hinted = True
            self.offloader.prefetch(layer_idx, priority)

    def states_ready(self, layer_idx: int) -> bool:
        """True if a step of ``layer_idx`` would not wait for storage."""
        return self.offloader is None or self.offloader.ready(layer_idx)

    def _pre_step(self, layer_idx: int) -> None:
        if self.offloader is None:
            return
        if self.prefetch and not self._hinted:
            # the reference's order: updates run in descending unit order
            units = self.offloader.units()
            prev = layer_idx - 1 if layer_idx - 1 in self._groups_by_layer else max(units)
            if prev != layer_idx:
                self.offloader.prefetch(prev, 0.0)
        moments = self.offloader.acquire(layer_idx)
        for name, t in zip(self._offloaded, moments):
            (self.exp_avg_flat if name == "exp_avg" else self.exp_avg_sq_flat)[layer_idx] = t
        self._bind_states(layer_idx)

    def _post_step(self, layer_idx: int) -> None:
        if self.offloader is None:
            return
        for name in self._offloaded:
            (self.exp_avg_flat if name == "exp_avg" else self.exp_avg_sq_flat)[layer_idx] = torch.empty(0)
        self._bind_states(layer_idx)
        self.offloader.release(layer_idx)

    def layer_states(self, layer_idx: int):
        """Copies of ``layer_idx``'s (exp_avg, exp_avg_sq), from storage when
        they are offloaded (not in the reference)."""
        if self.offloader is None:
            return self.exp_avg_flat[layer_idx].clone(), self.exp_avg_sq_flat[layer_idx].clone()
        moments = dict(zip(self._offloaded, self.offloader.read_back(layer_idx)))
        return (moments.get("exp_avg", self.exp_avg_flat[layer_idx].clone()),
                moments.get("exp_avg_sq", self.exp_avg_sq_flat[layer_idx].clone()))

    def torch_adam_update(self, data, grad, exp_avg, exp_avg_sq, lr, beta1, beta2, eps,
                          weight_decay, bias_correction1, bias_correction2):
        """Pure-torch Adam(W) on any device (reference layer_adam.py:247-265)."""
        grad = grad.to(data.dtype)
        if weight_decay != 0:
            if self.defaults["adamw_mode"]:
                data.mul_(1 - lr * weight_decay)
            else:
                grad = grad.add(data, alpha=weight_decay)
        exp_avg.mul_(beta1).add_(grad, alpha=1 - beta1)
        exp_avg_sq.mul_(beta2).addcmul_(grad, grad, value=1 - beta2)
        denom = (exp_avg_sq.sqrt() / math.sqrt(bias_correction2)).add_(eps)
        data.addcdiv_(exp_avg, denom, value=-(lr / bias_correction1))

    def _groups_to_update(self, layer_idx: Optional[int]):
        if layer_idx is not None:
            return [self._group(layer_idx)]
        if self.offloader is not None:
            # reference layer_adam.py:289-290
            raise RuntimeError("LayerAdam: with NVMe offload, step one layer at a time")
        return list(self.param_groups)

    def _update_param(self, group: dict, p: torch.Tensor, grad: torch.Tensor,
                      data: Optional[torch.Tensor] = None, data_bf16: Optional[torch.Tensor] = None) -> None:
        data = p.data if data is None else data
        if data.device.type != "cpu":
            raise RuntimeError(f"LayerAdam: unsupported device type {data.device.type}")
        if data.numel() != grad.numel():
            raise ValueError("LayerAdam: parameter and gradient sizes differ")
        beta1, beta2 = group["betas"]
        st = self.state[p]
        if self.reference_order:
            hp = _cpu_adam.hparams_in_reference_order(
                group["step"], group["lr"], beta1, beta2, group["eps"], group["weight_decay"],
                group["bias_correction"], self.defaults["adamw_mode"], self._first_of_step(group, p))
            if not grad.is_contiguous():
                grad = grad.contiguous()
            _cpu_adam.adam_step(data, grad, st["exp_avg"], st["exp_avg_sq"], hp, params_bf16=data_bf16)
            return
        self.cpu_adam.adam_update(self.optimizer_id, group["step"], group["lr"], beta1, beta2, group["eps"],
                                  group["weight_decay"], group["bias_correction"], data, grad,
                                  st["exp_avg"], st["exp_avg_sq"], params_bf16=data_bf16)

    def _first_of_step(self, group: dict, p) -> bool:
        """Whether the reference's update order (last unit first, parameters
        in order) makes this the first native call of the step."""
        return group["layer_idx"] == max(self._groups_by_layer) and p is group["params"][0]

    @torch.no_grad()
    def step(self, layer_idx: Optional[int] = None, closure=None):
        """Update one unit (or all) from ``p.grad`` (reference layer_adam.py:267-356)."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        groups = self._groups_to_update(layer_idx)
        self._pre_step(layer_idx)
        try:
            for group in groups:
                group["step"] += 1
                for p in group["params"]:
                    if p.grad is None:
                        continue
                    self._update_param(group, p, p.grad.data)
        finally:
            self._post_step(layer_idx)
        return loss

    @torch.no_grad()
    def step_with_grad_views(self, layer_idx: Optional[int] = None,
                             grad_views: Optional[Dict[torch.nn.Parameter, torch.Tensor]] = None, closure=None,
                             param_views: Optional[Dict[torch.nn.Parameter, torch.Tensor]] = None,
                             bf16_views: Optional[Dict[torch.nn.Parameter, torch.Tensor]] = None,
                             pieces=None, before_piece=None, after_piece=None):
        """Update one unit from per-parameter grad views into a host staging
        buffer (reference layer_adam.py:358-425).  bf16 views are read in place.

        ``param_views`` (not in the reference) names the fp32 host tensors to
        update per parameter; without it ``p.data`` is updated, which must then
        be the host master, as in the reference.  ``bf16_views`` (not in the
        reference) names bf16 host tensors that receive the rounded params in
        the same pass.

        ``pieces`` (not in the reference): a list of pieces, each a list of
        ``(param, lo, hi)`` flat element ranges, together covering the unit
        in order.  With ``reference_order`` the update runs piece by piece,
        calling ``before_piece(j)`` before piece ``j`` (e.g. to wait for its
        gradients) and ``after_piece(j)`` after it (e.g. to send its new
        weights on).  Every ``lo`` that is not a parameter's start must be a
        multiple of 16: each element then gets the same vector or tail
        arithmetic as in the whole-tensor call, so the bits are the same.
        Without ``reference_order`` the unit is updated at once, between all
        ``before_piece`` and all ``after_piece`` calls."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        groups = self._groups_to_update(layer_idx)
        self._pre_step(layer_idx)
        try:
            if pieces is not None and self.reference_order and len(groups) == 1:
                groups[0]["step"] += 1
                self._step_pieces(groups[0], grad_views, param_views, bf16_views, pieces,
                                  before_piece, after_piece)
                return loss
            n_pieces = 0 if pieces is None else len(pieces)
            if before_piece is not None:
                for j in range(n_pieces):
                    before_piece(j)
            for group in groups:
                group["step"] += 1
                for p in group["params"]:
                    grad = grad_views.get(p) if grad_views else None
                    if grad is None:
                        print(f"Warning: no gradient view for a parameter of shape {tuple(p.shape)}; skipped")
                        continue
                    self._update_param(group, p, grad, None if param_views is None else param_views[p],
                                       None if bf16_views is None else bf16_views[p])
            if after_piece is not None:
                for j in range(n_pieces):
                    after_piece(j)
        finally:
            self._post_step(layer_idx)
        return loss

    def _step_pieces(self, group, grad_views, param_views, bf16_views, pieces, before_piece, after_piece) -> None:
        beta1, beta2 = group["betas"]
        covered: Dict[Any, int] = {}
        hps: Dict[Any, Any] = {}
        for j, piece in enumerate(pieces):
            if before_piece is not None:
                before_piece(j)
            for p, lo, hi in piece:
                grad = grad_views.get(p) if grad_views else None
                if grad is None:
                    if lo == 0:
                        print(f"Warning: no gradient view for a parameter of shape {tuple(p.shape)}; skipped")
                    continue
                if covered.get(p, 0) != lo or hi <= lo or hi > p.numel() or (hi < p.numel() and hi % 16):
                    raise ValueError(f"LayerAdam: piece range [{lo}, {hi}) of a parameter of {p.numel()} "
                                     "elements does not continue the previous one on a 16-element boundary")
                covered[p] = hi
                data = p.data if param_views is None else param_views[p]
                if data.device.type != "cpu":
                    raise RuntimeError(f"LayerAdam: unsupported device type {data.device.type}")
                if data.numel() != grad.numel():
                    raise ValueError("LayerAdam: parameter and gradient sizes differ")
                hp = hps.get(p)
                if hp is None:
                    hp = hps[p] = _cpu_adam.hparams_in_reference_order(
                        group["step"], group["lr"], beta1, beta2, group["eps"], group["weight_decay"],
                        group["bias_correction"], self.defaults["adamw_mode"], self._first_of_step(group, p))
                st = self.state[p]
                pb = None if bf16_views is None else bf16_views[p].view(-1)[lo:hi]
                _cpu_adam.adam_step(data.view(-1)[lo:hi], grad.reshape(-1)[lo:hi],
                                    st["exp_avg"].view(-1)[lo:hi], st["exp_avg_sq"].view(-1)[lo:hi], hp,
                                    params_bf16=pb)
            if after_piece is not None:
                after_piece(j)
        for p in group["params"]:
            if grad_views and grad_views.get(p) is not None and covered.get(p, 0) != p.numel():
                raise ValueError(f"LayerAdam: the pieces leave part of a parameter of {p.numel()} elements out")

    @torch.no_grad()
    def step_rows_early(self, layer_idx: int, row_slot: torch.Tensor, param_view: torch.Tensor,
                        bf16_view: Optional[torch.Tensor] = None):
        """Begin a step of a one-parameter [V, H] unit with the part that needs
        no gradient (not in the reference): the step counter advances, and
        every row whose ``row_slot`` is ``SF_ROW_ZERO`` gets this step's
        zero-gradient update now.  Rows marked ``SF_ROW_SKIP`` are left for
        the ``step_rows`` call that completes the step, with the same step
        and learning rate; it must mark these early rows ``SF_ROW_SKIP`` in
        turn.  Together the two give the bits of one ``step_rows`` over all
        rows.  Needs ``reference_order`` (the scalars then depend only on the
        step and the learning rate)."""
        if not self.reference_order:
            raise RuntimeError("step_rows_early: needs reference_order")
        if bool((row_slot >= 0).any()):
            raise ValueError("step_rows_early: rows with a gradient belong to step_rows")
        group = self._group(layer_idx)
        if len(group["params"]) != 1:
            raise ValueError("step_rows_early: the unit must hold exactly one parameter")
        self._pre_step(layer_idx)
        try:
            group["step"] += 1
            # a step begun here and never completed (its backward failed) is dropped
            self._early_rows[layer_idx] = (group["step"], group["lr"])
            p = group["params"][0]
            st = self.state[p]
            beta1, beta2 = group["betas"]
            shape = param_view.shape
            hp = _cpu_adam.hparams_in_reference_order(
                group["step"], group["lr"], beta1, beta2, group["eps"], group["weight_decay"],
                group["bias_correction"], self.defaults["adamw_mode"], self._first_of_step(group, p))
            no_rows = torch.empty((0, shape[1]), dtype=torch.bfloat16)
            _cpu_adam.adam_step_rows(param_view, st["exp_avg"].view(shape), st["exp_avg_sq"].view(shape),
                                     row_slot, no_rows, hp, params_bf16=bf16_view)
        finally:
            self._post_step(layer_idx)

    def abandon_early_step(self, layer_idx: int) -> None:
        """Forget a step begun by ``step_rows_early`` that will not be
        completed (its early part failed); the next ``step_rows`` then starts
        a step of its own."""
        self._early_rows.pop(layer_idx, None)

    @torch.no_grad()
    def step_rows(self, layer_idx: int, row_slot: torch.Tensor, rows: torch.Tensor,
                  param_view: torch.Tensor, bf16_view: Optional[torch.Tensor] = None):
        """Update a one-parameter unit (a [V, H] table) whose gradient is zero
        outside the rows that ``row_slot`` maps into ``rows`` (not in the
        reference: the dense ``step_with_grad_views`` on the scattered
        gradient gives the same bits).  After ``step_rows_early`` it completes
        that step, with its step and learning rate: the rows updated early
        must be marked ``SF_ROW_SKIP``."""
        group = self._group(layer_idx)
        if len(group["params"]) != 1:
            raise ValueError("step_rows: the unit must hold exactly one parameter")
        early = self._early_rows.pop(layer_idx, None)
        if early is not None and not self.reference_order:
            raise RuntimeError("step_rows: an early part needs reference_order")
        self._pre_step(layer_idx)
        try:
            if early is None:
                group["step"] += 1
                step, lr = group["step"], group["lr"]
            else:
                step, lr = early
            p = group["params"][0]
            st = self.state[p]
            beta1, beta2 = group["betas"]
            shape = param_view.shape
            if self.reference_order:
                hp = _cpu_adam.hparams_in_reference_order(
                    step, lr, beta1, beta2, group["eps"], group["weight_decay"],
                    group["bias_correction"], self.defaults["adamw_mode"], self._first_of_step(group, p))
                _cpu_adam.adam_step_rows(param_view, st["exp_avg"].view(shape), st["exp_avg_sq"].view(shape),
                                         row_slot, rows, hp, params_bf16=bf16_view)
            else:
                self.cpu_adam.adam_update_rows(self.optimizer_id, group["step"], group["lr"], beta1, beta2,
                                               group["eps"], group["weight_decay"], group["bias_correction"],
                                               param_view, st["exp_avg"].view(shape), st["exp_avg_sq"].view(shape),
                                               row_slot, rows, params_bf16=bf16_view)
        finally:
            self._post_step(layer_idx)

    def update_learning_rate(self, new_lr):
        """Set the learning rate of every group (reference layer_adam.py:427-442)."""
        self.defaults["lr"] = new_lr
        for group in self.param_groups:
            group["lr"] = new_lr
