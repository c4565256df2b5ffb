"""ctypes bindings to the C ABI in include/slidefsdp.h.

``libsf_hip.so`` (device kernels, copies, pinned memory) and ``libsf_cpu.so``
(host AdamW) live in ``test1_amd/lib`` and are built by ``test1_amd.build``.
There is no fallback: a missing library raises at first use.

``libsf_hip.so`` must share torch's HIP runtime, so torch is imported before
it is loaded: the dynamic loader then resolves its ``libamdhip64.so.7`` to the
copy torch already mapped, and streams, events and device pointers are
interchangeable between the two.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads torch's HIP runtime first; see above)

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
HIP_LIB = os.path.join(LIB_DIR, "libsf_hip.so")
CPU_LIB = os.path.join(LIB_DIR, "libsf_cpu.so")

SF_COPY_H2D = 1
SF_COPY_D2H = 2
SF_COPY_D2D = 3
SF_DTYPE_F32 = 0
SF_DTYPE_BF16 = 1
SF_DTYPE_F16 = 2
SF_MAX_SEGS = 64
SF_IO_READ = 0
SF_IO_WRITE = 1
SF_IO_ALIGN = 4096
SF_EINVAL = 9001
SF_ETOOMANY = 9002
SF_EALIGN = 9007
SF_ETOOBIG = 9008
SF_ETIMEDOUT = 9009
SF_STAGE_SCRATCH_ELEMS = 16 << 20
# row_slot markers of the row-wise AdamW: a zero-gradient row, a row left as it is
SF_ROW_ZERO = -1
SF_ROW_SKIP = -2


class SfSeg(ctypes.Structure):
    _fields_ = [("src", ctypes.c_uint64), ("dst", ctypes.c_uint64), ("n", ctypes.c_uint64)]


class SfAdamHparams(ctypes.Structure):
    _fields_ = [
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("step_size", ctypes.c_float),
        ("bias_correction2", ctypes.c_float),
        ("lr", ctypes.c_float),
        ("adamw_mode", ctypes.c_int),
    ]


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i = ctypes.c_int
_f = ctypes.c_float

# name -> (argtypes) for every entry point; restype is int unless listed in
# _RESTYPES.
HIP_SIGNATURES = {
    "sf_error_string": [_i],
    "sf_abi_version": [],
    "sf_cast_f32_bf16": [_vp, _vp, _sz, _vp],
    "sf_cast_f32_bf16_timed": [_vp, _vp, _sz, _vp, _vp, _vp],
    "sf_cast_f32_f16": [_vp, _vp, _sz, _vp],
    "sf_cast_f32_f16_timed": [_vp, _vp, _sz, _vp, _vp, _vp],
    "sf_event_create": [ctypes.POINTER(ctypes.c_void_p)],
    "sf_event_destroy": [_vp],
    "sf_event_elapsed_ms": [_vp, _vp, ctypes.POINTER(ctypes.c_float)],
    "sf_cast_scatter_f32_bf16": [ctypes.POINTER(SfSeg), _i, _vp],
    "sf_pack_b16": [ctypes.POINTER(SfSeg), _i, _vp, _i, _vp],
    "sf_unpack_b16": [_vp, ctypes.POINTER(SfSeg), _i, _i, _vp],
    "sf_copy_segs_b16": [ctypes.POINTER(SfSeg), _i, _i, _vp],
    "sf_fill_b16": [_vp, _sz, ctypes.c_uint16, _vp],
    "sf_gather_rows_f32_bf16": [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _i, _vp],
    "sf_gather_rows_b16": [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _i, _vp],
    "sf_stage_f32_bf16": [_vp, _vp, _sz, _vp, _sz, _vp],
    "sf_stage_f32_bf16_noalloc": [_vp, _vp, _sz, _sz, _vp],
    "sf_memcpy_async": [_vp, _vp, _sz, _i, _vp],
    "sf_host_alloc": [ctypes.POINTER(_vp), _sz],
    "sf_host_free": [_vp],
    "sf_host_device_pointer": [_vp, ctypes.POINTER(_vp)],
    "sf_dma_init": [_i],
    "sf_dma_set_engines": [ctypes.c_uint32],
    "sf_dma_get_engines": [ctypes.POINTER(ctypes.c_uint32)],
    "sf_dma_set_avoid_held": [_i],
    "sf_dma_choose_engines": [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _i],
    "sf_dma_copy_d2h": [ctypes.POINTER(SfSeg), _i, ctypes.POINTER(ctypes.c_uint64), _i, ctypes.POINTER(_i)],
    "sf_dma_wait": [ctypes.POINTER(ctypes.c_uint64), _i, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64),
                    ctypes.POINTER(ctypes.c_uint64)],
    "sf_dma_query": [ctypes.POINTER(ctypes.c_uint64), _i, ctypes.POINTER(ctypes.c_int)],
    "sf_dma_enable_timing": [_i],
    "sf_dma_clock_ns": [ctypes.POINTER(ctypes.c_uint64)],
}

CPU_SIGNATURES = {
    "sf_error_string": [_i],
    "sf_abi_version": [],
    "sf_cpu_adam_step": [_vp, _vp, _i, _vp, _vp, _sz, ctypes.POINTER(SfAdamHparams)],
    "sf_adam_create": [_i, _f, _f, _f, _f, _f, _i, _i],
    "sf_adam_update": [_i, _sz, _f, _f, _f, _f, _f, _i, _vp, _vp, _i, _vp, _vp, _sz],
    "sf_adam_destroy": [_i],
    "sf_adam_update_cast": [_i, _sz, _f, _f, _f, _f, _f, _i, _vp, _vp, _i, _vp, _vp, _vp, _sz],
    "sf_cpu_adam_step_cast": [_vp, _vp, _i, _vp, _vp, _vp, _sz, ctypes.POINTER(SfAdamHparams)],
    "sf_cpu_cast_f32_bf16": [_vp, _vp, _sz],
    "sf_adam_update_rows": [_i, _sz, _f, _f, _f, _f, _f, _i, _vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _sz, _i],
    "sf_adam_hparams_in_order": [_sz, _f, _f, _f, _f, _f, _i, _i, _i, ctypes.POINTER(SfAdamHparams)],
    "sf_cpu_adam_step_rows": [_vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _sz, _i, ctypes.POINTER(SfAdamHparams)],
    "sf_cpu_set_threads": [_i],
    "sf_cpu_has_avx512": [],
    "sf_io_create": [_i, _sz, ctypes.POINTER(_vp)],
    "sf_io_destroy": [_vp],
    "sf_io_open": [ctypes.c_char_p, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "sf_io_reserve": [_i, ctypes.c_uint64],
    "sf_io_close": [_i],
    "sf_io_submit": [_vp, _i, _i, _vp, _sz, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
    "sf_io_query": [_vp, ctypes.c_uint64, ctypes.POINTER(_i)],
    "sf_io_wait": [_vp, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
    "sf_io_stats": [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                    ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
}

_lock = threading.Lock()
_hip = None
_cpu = None

_RESTYPES = {"sf_error_string": ctypes.c_char_p, "sf_dma_choose_engines": ctypes.c_uint32}


def _bind(path: str, sigs: dict) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise RuntimeError(
            f"native library not built: {path}. Build it with `python -c \"import "
            f"__graft_entry__ as g; g.build()\"` (or `python -m test1_amd.build`)."
        )
    lib = ctypes.CDLL(path)
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    return lib


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        with _lock:
            if _hip is None:
                _hip = _bind(HIP_LIB, HIP_SIGNATURES)
    return _hip


def cpu() -> ctypes.CDLL:
    global _cpu
    if _cpu is None:
        with _lock:
            if _cpu is None:
                _cpu = _bind(CPU_LIB, CPU_SIGNATURES)
    return _cpu


class NativeError(RuntimeError):
    """A nonzero status from the C ABI (``status`` holds it)."""

    def __init__(self, msg: str, status: int = 0):
        super().__init__(msg)
        self.status = status


# hipErrorOutOfMemory, as the HIP entry points return it
HIP_ERROR_OUT_OF_MEMORY = 2


def check(status: int, what: str, lib: ctypes.CDLL | None = None) -> None:
    if status != 0:
        lib = lib or hip()
        msg = lib.sf_error_string(status).decode(errors="replace")
        raise NativeError(f"{what} failed: {msg} (status {status})", status)
