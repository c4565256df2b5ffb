"""Tensor-level shim with the reference's native ``cpu_adam`` module interface.

Reference optimizer/layer_adam/csrc/cpu_adam.cpp:8-13 binds three functions
through pybind11; the same three are offered here over the C ABI of
``libsf_cpu.so`` (include/slidefsdp.h):

  create_adam(id, alpha, beta1, beta2, eps, weight_decay, adamw_mode, should_log) -> 0
  adam_update(id, step, lr, beta1, beta2, eps, weight_decay, bias_correction,
              params, grads, exp_avg, exp_avg_sq) -> 0
  destroy_adam(id) -> 0

Supported dtypes: fp32 params and fp32 moments (the combination LayerAdam
uses, layer_adam.py:158 with fp32_optimizer_state=True), with fp32, bf16 or
fp16 grads; 16-bit grads are widened exactly, so they give the bits of the
reference's ``grad.float()`` call.  Other combinations raise the reference's
RuntimeError.  Deliberate differences from the reference: a non-contiguous
params/exp_avg/exp_avg_sq raises ValueError instead of silently updating a
``.contiguous()`` copy (cpu_adam_impl.cpp:224-227), and an unknown id raises
RuntimeError instead of dereferencing a null pointer (cpu_adam_impl.cpp:229-231).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from .. import _native


def _lib():
    return _native.cpu()


def _check(status: int, what: str) -> None:
    _native.check(status, what, _lib())


def create_adam(optimizer_id: int, alpha: float = 1e-3, beta1: float = 0.9, beta2: float = 0.999,
                eps: float = 1e-8, weight_decay: float = 0.0, adamw_mode: bool = True,
                should_log: bool = False) -> int:
    _check(_lib().sf_adam_create(int(optimizer_id), alpha, beta1, beta2, eps, weight_decay,
                                 1 if adamw_mode else 0, 1 if should_log else 0), "create_adam")
    return 0


def destroy_adam(optimizer_id: int) -> int:
    _check(_lib().sf_adam_destroy(int(optimizer_id)), "destroy_adam")
    return 0


def _grad_dtype_code(g: torch.Tensor) -> int:
    if g.dtype == torch.float32:
        return _native.SF_DTYPE_F32
    if g.dtype == torch.bfloat16:
        return _native.SF_DTYPE_BF16
    if g.dtype == torch.float16:
        return _native.SF_DTYPE_F16
    return -1


def adam_update(optimizer_id: int, step: int, lr: float, beta1: float, beta2: float, eps: float,
                weight_decay: float, bias_correction: bool, params: torch.Tensor, grads: torch.Tensor,
                exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
                params_bf16: Optional[torch.Tensor] = None) -> int:
    """The reference's ``adam_update``.  ``params_bf16`` (not in the
    reference): a contiguous bf16 CPU tensor of the params' size that receives
    the round-to-nearest-even bf16 of every updated param in the same pass."""
    if params.dtype != torch.float32 or exp_avg.dtype != torch.float32 or exp_avg_sq.dtype != torch.float32:
        raise RuntimeError(
            f"Adam optimizer with param type {params.dtype} and state type {exp_avg.dtype} "
            "is not supported on current hardware"
        )
    gcode = _grad_dtype_code(grads)
    if gcode < 0:
        raise RuntimeError(f"Adam optimizer with grad type {grads.dtype} is not supported on current hardware")
    for t, name in ((params, "params"), (grads, "grads"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if t.device.type != "cpu":
            raise RuntimeError(f"adam_update: {name} must be a CPU tensor, got {t.device}")
    for t, name in ((params, "params"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if not t.is_contiguous():
            raise ValueError(f"adam_update: {name} is updated in place and must be contiguous")
    n = params.numel()
    if grads.numel() != n or exp_avg.numel() != n or exp_avg_sq.numel() != n:
        raise ValueError("adam_update: params, grads and moments must have the same numel")
    if not grads.is_contiguous():
        grads = grads.contiguous()
    pb = None
    if params_bf16 is not None:
        if (params_bf16.dtype != torch.bfloat16 or params_bf16.device.type != "cpu"
                or not params_bf16.is_contiguous() or params_bf16.numel() != n):
            raise ValueError("adam_update: params_bf16 must be a contiguous bf16 CPU tensor of the params' size")
        pb = params_bf16.data_ptr()
    _check(_lib().sf_adam_update_cast(int(optimizer_id), int(step), lr, beta1, beta2, eps, weight_decay,
                                      1 if bias_correction else 0, params.data_ptr(), grads.data_ptr(), gcode,
                                      exp_avg.data_ptr(), exp_avg_sq.data_ptr(), pb, n), "adam_update")
    return 0


def adam_update_rows(optimizer_id: int, step: int, lr: float, beta1: float, beta2: float, eps: float,
                     weight_decay: float, bias_correction: bool, params: torch.Tensor, exp_avg: torch.Tensor,
                     exp_avg_sq: torch.Tensor, row_slot: torch.Tensor, grads: torch.Tensor,
                     params_bf16: Optional[torch.Tensor] = None) -> int:
    """``adam_update`` of a 2-D ``params`` [n_rows, row_len] whose gradient is
    zero except in the rows named by ``row_slot`` (int64 [n_rows]: the row of
    ``grads`` [k, row_len] holding row r's gradient, or -1).  Gives the bits
    of the dense update with the scattered gradient."""
    if params.dim() != 2:
        raise ValueError("adam_update_rows: params must be 2-D")
    n_rows, row_len = params.shape
    for t, name in ((params, "params"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if t.dtype != torch.float32 or t.device.type != "cpu" or not t.is_contiguous() or t.numel() != params.numel():
            raise ValueError(f"adam_update_rows: {name} must be a contiguous fp32 CPU tensor of params' size")
    if row_slot.dtype != torch.int64 or row_slot.numel() != n_rows or not row_slot.is_contiguous():
        raise ValueError("adam_update_rows: row_slot must be a contiguous int64 tensor of n_rows")
    gcode = _grad_dtype_code(grads)
    if gcode < 0:
        raise RuntimeError(f"Adam optimizer with grad type {grads.dtype} is not supported on current hardware")
    if grads.device.type != "cpu" or not grads.is_contiguous() or grads.numel() % max(1, row_len):
        raise ValueError("adam_update_rows: grads must be a contiguous CPU tensor of whole rows")
    pb = None
    if params_bf16 is not None:
        if (params_bf16.dtype != torch.bfloat16 or params_bf16.device.type != "cpu"
                or not params_bf16.is_contiguous() or params_bf16.numel() != params.numel()):
            raise ValueError("adam_update_rows: params_bf16 must be a contiguous bf16 CPU tensor of the params' size")
        pb = params_bf16.data_ptr()
    _check(_lib().sf_adam_update_rows(int(optimizer_id), int(step), lr, beta1, beta2, eps, weight_decay,
                                      1 if bias_correction else 0, params.data_ptr(), exp_avg.data_ptr(),
                                      exp_avg_sq.data_ptr(), pb, n_rows, row_len, row_slot.data_ptr(),
                                      grads.data_ptr(), grads.numel() // max(1, row_len), gcode),
           "adam_update_rows")
    return 0


def hparams_in_reference_order(step: int, lr: float, beta1: float, beta2: float, eps: float,
                               weight_decay: float, bias_correction: bool, adamw_mode: bool,
                               first_of_step: bool) -> "_native.SfAdamHparams":
    """Scalars of one update of ``step`` as the reference's stateful call
    sequence gives them when units are stepped last unit first
    (``first_of_step``: the last unit's first parameter); no optimizer state
    is involved, so any update order gets the reference's bits."""
    hp = _native.SfAdamHparams()
    _check(_lib().sf_adam_hparams_in_order(int(step), lr, beta1, beta2, eps, weight_decay,
                                           1 if bias_correction else 0, 1 if adamw_mode else 0,
                                           1 if first_of_step else 0, ctypes.byref(hp)),
           "sf_adam_hparams_in_order")
    return hp


def _check_step_tensors(params, grads, exp_avg, exp_avg_sq, params_bf16, what):
    for t, name in ((params, "params"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if t.dtype != torch.float32 or t.device.type != "cpu" or not t.is_contiguous() or t.numel() != params.numel():
            raise ValueError(f"{what}: {name} must be a contiguous fp32 CPU tensor of the params' size")
    gcode = _grad_dtype_code(grads)
    if gcode < 0:
        raise RuntimeError(f"Adam optimizer with grad type {grads.dtype} is not supported on current hardware")
    if grads.device.type != "cpu" or not grads.is_contiguous():
        raise ValueError(f"{what}: grads must be a contiguous CPU tensor")
    pb = None
    if params_bf16 is not None:
        if (params_bf16.dtype != torch.bfloat16 or params_bf16.device.type != "cpu"
                or not params_bf16.is_contiguous() or params_bf16.numel() != params.numel()):
            raise ValueError(f"{what}: params_bf16 must be a contiguous bf16 CPU tensor of the params' size")
        pb = params_bf16.data_ptr()
    return gcode, pb


def adam_step(params: torch.Tensor, grads: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
              hp: "_native.SfAdamHparams", params_bf16: Optional[torch.Tensor] = None) -> None:
    """One update with caller-given scalars (``hparams_in_reference_order``)."""
    gcode, pb = _check_step_tensors(params, grads, exp_avg, exp_avg_sq, params_bf16, "adam_step")
    if grads.numel() != params.numel():
        raise ValueError("adam_step: params and grads must have the same numel")
    _check(_lib().sf_cpu_adam_step_cast(params.data_ptr(), grads.data_ptr(), gcode, exp_avg.data_ptr(),
                                        exp_avg_sq.data_ptr(), pb, params.numel(), ctypes.byref(hp)),
           "sf_cpu_adam_step_cast")


def adam_step_rows(params: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor, row_slot: torch.Tensor,
                   grads: torch.Tensor, hp: "_native.SfAdamHparams",
                   params_bf16: Optional[torch.Tensor] = None) -> None:
    """``adam_update_rows`` with caller-given scalars."""
    if params.dim() != 2:
        raise ValueError("adam_step_rows: params must be 2-D")
    n_rows, row_len = params.shape
    gcode, pb = _check_step_tensors(params, grads, exp_avg, exp_avg_sq, params_bf16, "adam_step_rows")
    if row_slot.dtype != torch.int64 or row_slot.numel() != n_rows or not row_slot.is_contiguous():
        raise ValueError("adam_step_rows: row_slot must be a contiguous int64 tensor of n_rows")
    if grads.numel() % max(1, row_len):
        raise ValueError("adam_step_rows: grads must hold whole rows")
    _check(_lib().sf_cpu_adam_step_rows(params.data_ptr(), exp_avg.data_ptr(), exp_avg_sq.data_ptr(), pb,
                                        n_rows, row_len, row_slot.data_ptr(), grads.data_ptr(),
                                        grads.numel() // max(1, row_len), gcode, ctypes.byref(hp)),
           "sf_cpu_adam_step_rows")


def cast_f32_bf16(src: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    """``dst`` = round-to-nearest-even bf16 of ``src`` (NaN -> 0xFFFF), on the
    host AdamW's threads.  Both contiguous CPU tensors of the same size."""
    if src.dtype != torch.float32 or dst.dtype != torch.bfloat16:
        raise TypeError("cast_f32_bf16: expects fp32 src and bf16 dst")
    if src.device.type != "cpu" or dst.device.type != "cpu":
        raise RuntimeError("cast_f32_bf16: CPU tensors only")
    if not (src.is_contiguous() and dst.is_contiguous()) or src.numel() != dst.numel():
        raise ValueError("cast_f32_bf16: contiguous tensors of the same size")
    _check(_lib().sf_cpu_cast_f32_bf16(src.data_ptr(), dst.data_ptr(), src.numel()), "sf_cpu_cast_f32_bf16")
    return dst


def set_num_threads(n: int) -> None:
    """OpenMP team size of the host AdamW (<= 0 restores the default)."""
    _check(_lib().sf_cpu_set_threads(int(n)), "sf_cpu_set_threads")


def has_avx512() -> bool:
    return bool(_lib().sf_cpu_has_avx512())
