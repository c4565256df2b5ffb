"""Exact-size pinned host memory as torch CPU tensors.

torch's pinned-memory allocator rounds every request up to a power of two
(ATen CachingHostAllocator), which for the fp32 masters of an 8B model would
pin ~43 GB instead of 32 GB.  ``pinned_empty`` allocates exactly the bytes
asked for through ``sf_host_alloc`` (hipHostMalloc) and wraps them as a CPU
tensor without a copy.  The allocation is released when the last tensor
viewing it is garbage-collected, so views (for example ``param.data``
pointing into a flat master) keep it alive.

Replaces ``torch.empty(..., pin_memory=True)`` at reference
layer_state.py:203-208, slide_fsdp.py:174-186 and slide_fsdp.py:480-503.
"""

from __future__ import annotations

import ctypes
import math
import sys
import threading

import torch

from . import _native

_stats_lock = threading.Lock()
_live_bytes = 0


def pinned_bytes_live() -> int:
    """Bytes of pinned memory currently held by pinned_empty allocations."""
    return _live_bytes


def _owned_array(addr: int, nbytes: int):
    base = ctypes.c_ubyte * nbytes

    class _PinnedBlock(base):  # one class per block: ctypes array types are sized
        def __del__(self):
            global _live_bytes
            if sys.is_finalizing():
                return  # the HIP runtime may already be gone; the OS reclaims it
            try:
                _native.hip().sf_host_free(ctypes.c_void_p(addr))
            finally:
                with _stats_lock:
                    _live_bytes -= nbytes

    return _PinnedBlock.from_address(addr)


def pinned_empty(shape, dtype: torch.dtype) -> torch.Tensor:
    """An uninitialised pinned CPU tensor of exactly ``numel * itemsize`` bytes."""
    global _live_bytes
    if isinstance(shape, int):
        shape = (shape,)
    shape = tuple(int(s) for s in shape)
    numel = math.prod(shape)
    itemsize = torch.empty((), dtype=dtype).element_size()
    nbytes = numel * itemsize
    if nbytes == 0:
        return torch.empty(shape, dtype=dtype)
    ptr = ctypes.c_void_p()
    _native.check(_native.hip().sf_host_alloc(ctypes.byref(ptr), nbytes), f"sf_host_alloc({nbytes} B)")
    with _stats_lock:
        _live_bytes += nbytes
    block = _owned_array(ptr.value, nbytes)
    flat = torch.frombuffer(block, dtype=torch.uint8)
    return flat.view(dtype).view(shape)
