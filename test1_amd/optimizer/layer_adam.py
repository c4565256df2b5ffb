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
"""

from __future__ import annotations

import itertools
import math
from collections import OrderedDict, defaultdict
from typing import Any, DefaultDict, Dict, Iterable, Optional

import torch

from . import cpu_adam as _cpu_adam


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
        self.state: DefaultDict[torch.Tensor, Any] = defaultdict(dict)
        if not 0.0 <= nvme_offload_fraction <= 1.0:
            raise ValueError("nvme_offload_fraction must be in [0, 1]")
        self.nvme_offload_fraction = nvme_offload_fraction
        self.prefetch = prefetch
        self.pin_memory = nvme_offload_fraction > 0.0
        self.exp_avg_flat: "OrderedDict[int, torch.Tensor]" = OrderedDict()
        self.exp_avg_sq_flat: "OrderedDict[int, torch.Tensor]" = OrderedDict()
        if nvme_offload_fraction > 0.0:
            # NVMe state offload is not part of this build; the reference needs
            # tensornvme for it (layer_adam.py:89-98) and raises the same way.
            raise ModuleNotFoundError("Please install tensornvme to use NVMeOptimizer")
        self.offload_dir = None
        self.offloader = None

    def __del__(self):
        try:
            self.cpu_adam.destroy_adam(self.optimizer_id)
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
        self.exp_avg_flat[layer_idx] = torch.zeros(numel, dtype=state_type)
        self.exp_avg_sq_flat[layer_idx] = torch.zeros(numel, dtype=state_type)
        off = 0
        for p in params:
            n = p.numel()
            st = self.state[p]
            st["exp_avg"] = self.exp_avg_flat[layer_idx][off:off + n].view(p.shape)
            st["exp_avg_sq"] = self.exp_avg_sq_flat[layer_idx][off:off + n].view(p.shape)
            off += n
        return layer_idx

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
        self.cpu_adam.adam_update(self.optimizer_id, group["step"], group["lr"], beta1, beta2, group["eps"],
                                  group["weight_decay"], group["bias_correction"], data, grad,
                                  st["exp_avg"], st["exp_avg_sq"], params_bf16=data_bf16)

    @torch.no_grad()
    def step(self, layer_idx: Optional[int] = None, closure=None):
        """Update one unit (or all) from ``p.grad`` (reference layer_adam.py:267-356)."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self._groups_to_update(layer_idx):
            group["step"] += 1
            for p in group["params"]:
                if p.grad is None:
                    continue
                self._update_param(group, p, p.grad.data)
        return loss

    @torch.no_grad()
    def step_with_grad_views(self, layer_idx: Optional[int] = None,
                             grad_views: Optional[Dict[torch.nn.Parameter, torch.Tensor]] = None, closure=None,
                             param_views: Optional[Dict[torch.nn.Parameter, torch.Tensor]] = None,
                             bf16_views: Optional[Dict[torch.nn.Parameter, torch.Tensor]] = None):
        """Update one unit from per-parameter grad views into a host staging
        buffer (reference layer_adam.py:358-425).  bf16 views are read in place.

        ``param_views`` (not in the reference) names the fp32 host tensors to
        update per parameter; without it ``p.data`` is updated, which must then
        be the host master, as in the reference.  ``bf16_views`` (not in the
        reference) names bf16 host tensors that receive the rounded params in
        the same pass."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self._groups_to_update(layer_idx):
            group["step"] += 1
            for p in group["params"]:
                grad = grad_views.get(p) if grad_views else None
                if grad is None:
                    print(f"Warning: no gradient view for a parameter of shape {tuple(p.shape)}; skipped")
                    continue
                self._update_param(group, p, grad, None if param_views is None else param_views[p],
                                   None if bf16_views is None else bf16_views[p])
        return loss

    @torch.no_grad()
    def step_rows(self, layer_idx: int, row_slot: torch.Tensor, rows: torch.Tensor,
                  param_view: torch.Tensor, bf16_view: Optional[torch.Tensor] = None):
        """Update a one-parameter unit (a [V, H] table) whose gradient is zero
        outside the rows that ``row_slot`` maps into ``rows`` (not in the
        reference: the dense ``step_with_grad_views`` on the scattered
        gradient gives the same bits)."""
        group = self._group(layer_idx)
        if len(group["params"]) != 1:
            raise ValueError("step_rows: the unit must hold exactly one parameter")
        group["step"] += 1
        p = group["params"][0]
        st = self.state[p]
        beta1, beta2 = group["betas"]
        shape = param_view.shape
        self.cpu_adam.adam_update_rows(self.optimizer_id, group["step"], group["lr"], beta1, beta2, group["eps"],
                                       group["weight_decay"], group["bias_correction"], param_view,
                                       st["exp_avg"].view(shape), st["exp_avg_sq"].view(shape), row_slot, rows,
                                       params_bf16=bf16_view)

    def update_learning_rate(self, new_lr):
        """Set the learning rate of every group (reference layer_adam.py:427-442)."""
        self.defaults["lr"] = new_lr
        for group in self.param_groups:
            group["lr"] = new_lr
