"""Tensor-level wrappers over the device entry points of the C ABI.

Every wrapper checks dtype, device, contiguity and sizes on the host before
anything is launched, passes raw pointers and the stream handle, and turns a
nonzero status into ``NativeError`` (a ``RuntimeError``).  The work is
asynchronous on ``stream`` (default: the current stream).
"""

from __future__ import annotations

import ctypes
import threading
import time
import os
from typing import Callable, List, Optional, Sequence, Tuple

import torch

from . import _native

_B16 = (torch.bfloat16, torch.float16, torch.int16, torch.uint16)


def _stream_ptr(stream: Optional[torch.cuda.Stream]) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _require_cuda(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what} must be a GPU tensor, got {t.device}")


def _require_contig(t: torch.Tensor, what: str) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


class KernelTimer:
    """A pair of HIP timing events that a launch stamps around its kernels'
    own dispatch (``cast_f32_bf16_(..., timer=t)``): ``elapsed_ms`` is then
    the kernels' duration alone, not what the stream waited for first."""

    def __init__(self):
        lib = _native.hip()
        self._lib = lib
        self.start, self.stop = ctypes.c_void_p(), ctypes.c_void_p()
        _native.check(lib.sf_event_create(ctypes.byref(self.start)), "sf_event_create")
        try:
            _native.check(lib.sf_event_create(ctypes.byref(self.stop)), "sf_event_create")
        except BaseException:
            lib.sf_event_destroy(self.start)
            raise

    def elapsed_ms(self) -> float:
        """Milliseconds from the first kernel's start to the last one's end
        (the launch must have completed)."""
        ms = ctypes.c_float(0.0)
        _native.check(self._lib.sf_event_elapsed_ms(self.start, self.stop, ctypes.byref(ms)), "sf_event_elapsed_ms")
        return float(ms.value)

    def __del__(self):
        lib = getattr(self, "_lib", None)
        if lib is not None:
            for ev in (getattr(self, "start", None), getattr(self, "stop", None)):
                if ev is not None and ev.value:
                    lib.sf_event_destroy(ev)


_CASTS = {torch.bfloat16: ("sf_cast_f32_bf16", "sf_cast_f32_bf16_timed"),
          torch.float16: ("sf_cast_f32_f16", "sf_cast_f32_f16_timed")}


def cast_f32_16_(dst: torch.Tensor, src: torch.Tensor, stream: Optional[torch.cuda.Stream] = None,
                 timer: Optional[KernelTimer] = None) -> torch.Tensor:
    """dst[:] = src rounded to nearest even into dst's 16-bit float type
    (bfloat16 or float16); both flat-contiguous GPU tensors of equal numel.
    With ``timer``, its events are stamped around the cast kernels."""
    if src.dtype != torch.float32 or dst.dtype not in _CASTS:
        raise TypeError(f"cast_f32_16_: need float32 -> bfloat16 or float16, got {src.dtype} -> {dst.dtype}")
    _require_cuda(src, "src")
    _require_cuda(dst, "dst")
    _require_contig(src, "src")
    _require_contig(dst, "dst")
    if src.numel() != dst.numel():
        raise ValueError(f"cast_f32_16_: numel mismatch {src.numel()} vs {dst.numel()}")
    plain, timed = _CASTS[dst.dtype]
    if timer is None:
        _native.check(getattr(_native.hip(), plain)(src.data_ptr(), dst.data_ptr(), src.numel(),
                                                    _stream_ptr(stream)), plain)
    else:
        _native.check(getattr(_native.hip(), timed)(src.data_ptr(), dst.data_ptr(), src.numel(), _stream_ptr(stream),
                                                    timer.start, timer.stop), timed)
    return dst


def cast_f32_bf16_(dst: torch.Tensor, src: torch.Tensor, stream: Optional[torch.cuda.Stream] = None,
                   timer: Optional[KernelTimer] = None) -> torch.Tensor:
    """dst[:] = RNE-bf16(src), both flat-contiguous GPU tensors of equal numel.
    With ``timer``, its events are stamped around the cast kernels."""
    if src.dtype != torch.float32 or dst.dtype != torch.bfloat16:
        raise TypeError(f"cast_f32_bf16_: need float32 -> bfloat16, got {src.dtype} -> {dst.dtype}")
    return cast_f32_16_(dst, src, stream, timer)


def _check_stage_args(dst: torch.Tensor, host_src: torch.Tensor) -> None:
    if host_src.dtype != torch.float32 or dst.dtype != torch.bfloat16:
        raise TypeError(f"stage_f32_bf16_: need float32 -> bfloat16, got {host_src.dtype} -> {dst.dtype}")
    if host_src.device.type != "cpu" or (host_src.numel() and not host_src.is_pinned()):
        raise ValueError("stage_f32_bf16_: the source must be a pinned host tensor")
    _require_cuda(dst, "dst")
    _require_contig(host_src, "host_src")
    _require_contig(dst, "dst")
    if host_src.numel() != dst.numel():
        raise ValueError(f"stage_f32_bf16_: numel mismatch {host_src.numel()} vs {dst.numel()}")


def stage_f32_bf16_(dst: torch.Tensor, host_src: torch.Tensor, workspace: torch.Tensor,
                    stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """dst[:] = RNE-bf16(host_src) for a pinned fp32 host tensor and a bf16 GPU
    tensor: copied piece by piece through the fp32 GPU tensor ``workspace``
    (pieces of its size rounded down to 8 elements) and cast from there, all
    in order on ``stream``; ``workspace`` is free again once the stream has
    passed the call."""
    _check_stage_args(dst, host_src)
    if workspace.dtype != torch.float32 or workspace.numel() < 8:
        raise ValueError("stage_f32_bf16_: the workspace must be a float32 GPU tensor of at least 8 elements")
    _require_cuda(workspace, "workspace")
    _require_contig(workspace, "workspace")
    _native.check(_native.hip().sf_stage_f32_bf16(host_src.data_ptr(), dst.data_ptr(), host_src.numel(),
                                                  workspace.data_ptr(), workspace.numel(), _stream_ptr(stream)),
                  "sf_stage_f32_bf16")
    return dst


def stage_f32_bf16_noalloc_(dst: torch.Tensor, host_src: torch.Tensor, chunk_elems: int = 0,
                            stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """``stage_f32_bf16_`` through the library's own device scratch buffer
    (pieces of ``chunk_elems``, at most ``_native.SF_STAGE_SCRATCH_ELEMS``;
    0: that size), allocating nothing.  Calls on one device share the
    buffer: keep them on one stream or otherwise ordered."""
    _check_stage_args(dst, host_src)
    _native.check(_native.hip().sf_stage_f32_bf16_noalloc(host_src.data_ptr(), dst.data_ptr(), host_src.numel(),
                                                          int(chunk_elems), _stream_ptr(stream)),
                  "sf_stage_f32_bf16_noalloc")
    return dst


def _seg_array(segs: Sequence[Tuple[int, int, int]]):
    arr = (_native.SfSeg * max(1, len(segs)))()
    for i, (s, d, n) in enumerate(segs):
        arr[i].src, arr[i].dst, arr[i].n = s, d, n
    return arr


def cast_scatter_f32_bf16(pairs: Sequence[Tuple[torch.Tensor, torch.Tensor]],
                          stream: Optional[torch.cuda.Stream] = None) -> None:
    """For each (src fp32, dst bf16) pair of contiguous GPU tensors: dst = RNE(src)."""
    segs = []
    for k, (src, dst) in enumerate(pairs):
        if src.dtype != torch.float32 or dst.dtype != torch.bfloat16:
            raise TypeError(f"pair {k}: need float32 -> bfloat16")
        _require_cuda(src, f"pair {k} src")
        _require_cuda(dst, f"pair {k} dst")
        _require_contig(src, f"pair {k} src")
        _require_contig(dst, f"pair {k} dst")
        if src.numel() != dst.numel():
            raise ValueError(f"pair {k}: numel mismatch")
        segs.append((src.data_ptr(), dst.data_ptr(), src.numel()))
    arr = _seg_array(segs)
    _native.check(_native.hip().sf_cast_scatter_f32_bf16(arr, len(segs), _stream_ptr(stream)),
                  "sf_cast_scatter_f32_bf16")


def _check_b16(t: torch.Tensor, what: str, host_ok: bool = False) -> None:
    if t.dtype not in _B16:
        raise TypeError(f"{what}: need a 16-bit dtype, got {t.dtype}")
    if host_ok and t.device.type == "cpu":
        if not t.is_pinned():
            raise ValueError(f"{what}: a host tensor must be pinned to be written by a kernel")
    else:
        _require_cuda(t, what)
    _require_contig(t, what)


def device_address(t: torch.Tensor) -> int:
    """Address at which a kernel reaches ``t``: its data pointer for a GPU
    tensor, the mapped device address of pinned host memory otherwise."""
    if t.device.type == "cuda":
        return t.data_ptr()
    base = t.untyped_storage().data_ptr()
    dev = ctypes.c_void_p()
    _native.check(_native.hip().sf_host_device_pointer(ctypes.c_void_p(base), ctypes.byref(dev)),
                  "sf_host_device_pointer")
    return dev.value + (t.data_ptr() - base)


def pack_b16(srcs: Sequence[torch.Tensor], dst: torch.Tensor,
             stream: Optional[torch.cuda.Stream] = None, max_workgroups: int = 0) -> torch.Tensor:
    """dst[off_k : off_k + n_k] = srcs[k].flatten(), offsets in order from 0.

    ``dst`` may be pinned host memory (then pass a small ``max_workgroups``)."""
    _check_b16(dst, "dst", host_ok=True)
    total = 0
    segs = []
    for k, s in enumerate(srcs):
        _check_b16(s, f"srcs[{k}]")
        segs.append((s.data_ptr(), 0, s.numel()))
        total += s.numel()
    if total > dst.numel():
        raise ValueError(f"pack_b16: {total} elements do not fit in dst of {dst.numel()}")
    arr = _seg_array(segs)
    _native.check(_native.hip().sf_pack_b16(arr, len(segs), device_address(dst), int(max_workgroups),
                                            _stream_ptr(stream)), "sf_pack_b16")
    return dst


def copy_segs_b16(pairs: Sequence[Tuple[torch.Tensor, torch.Tensor]],
                  stream: Optional[torch.cuda.Stream] = None, max_workgroups: int = 0) -> None:
    """For each (src, dst) pair of contiguous 16-bit tensors of equal numel,
    dst = src, all in one launch.  Sources are GPU tensors; destinations are
    GPU tensors or pinned host tensors."""
    segs = []
    for k, (src, dst) in enumerate(pairs):
        _check_b16(src, f"pair {k} src")
        _check_b16(dst, f"pair {k} dst", host_ok=True)
        if src.numel() != dst.numel():
            raise ValueError(f"pair {k}: numel mismatch {src.numel()} vs {dst.numel()}")
        segs.append((src.data_ptr(), device_address(dst), src.numel()))
    if not segs:
        return
    arr = _seg_array(segs)
    _native.check(_native.hip().sf_copy_segs_b16(arr, len(segs), int(max_workgroups), _stream_ptr(stream)),
                  "sf_copy_segs_b16")


def unpack_b16(src: torch.Tensor, dsts: Sequence[torch.Tensor],
               stream: Optional[torch.cuda.Stream] = None, max_workgroups: int = 0) -> None:
    """dsts[k].flatten() = src[off_k : off_k + n_k], the inverse of pack_b16.
    ``src`` may be pinned host memory."""
    _check_b16(src, "src", host_ok=True)
    total = 0
    segs = []
    for k, d in enumerate(dsts):
        _check_b16(d, f"dsts[{k}]")
        segs.append((0, d.data_ptr(), d.numel()))
        total += d.numel()
    if total > src.numel():
        raise ValueError(f"unpack_b16: src of {src.numel()} holds fewer than {total} elements")
    arr = _seg_array(segs)
    _native.check(_native.hip().sf_unpack_b16(device_address(src), arr, len(segs), int(max_workgroups),
                                              _stream_ptr(stream)), "sf_unpack_b16")


def fill_b16_(dst: torch.Tensor, value: int = 0, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """dst[:] = value (a 16-bit pattern), as a kernel (graph-capture safe)."""
    _check_b16(dst, "dst")
    _native.check(_native.hip().sf_fill_b16(dst.data_ptr(), dst.numel(), int(value) & 0xFFFF, _stream_ptr(stream)),
                  "sf_fill_b16")
    return dst


def gather_rows(table: torch.Tensor, ids: torch.Tensor, dst: torch.Tensor, bad: Optional[torch.Tensor] = None,
                stream: Optional[torch.cuda.Stream] = None, max_workgroups: int = 0) -> torch.Tensor:
    """``dst[t] = table[ids[t]]`` for a 2-D ``table`` (fp32: rounded to bf16;
    16-bit: copied) into a 16-bit ``dst`` of shape [len(ids), row_len].

    ``table`` and ``dst`` may be pinned host tensors (read or written over the
    host link by the kernel); ``ids`` is an int64 GPU tensor.  An id out of
    range yields a row of 0xFFFF and sets ``bad[0] = 1`` (``bad``: a uint32/
    int32 tensor of one element, GPU or pinned host)."""
    if table.dim() != 2:
        raise ValueError("gather_rows: table must be 2-D")
    nrows, row_len = table.shape
    _require_contig(table, "table")
    _require_contig(dst, "dst")
    _require_cuda(ids, "ids")
    _require_contig(ids, "ids")
    if ids.dtype != torch.int64:
        raise TypeError("gather_rows: ids must be int64")
    if dst.element_size() != 2 or dst.numel() < ids.numel() * row_len:
        raise ValueError("gather_rows: dst must be 16-bit with room for len(ids) rows")
    for t, what in ((table, "table"), (dst, "dst")):
        if t.device.type == "cpu" and not t.is_pinned():
            raise ValueError(f"gather_rows: a host {what} must be pinned")
    bad_ptr = None
    if bad is not None:
        if bad.element_size() != 4 or bad.numel() < 1:
            raise ValueError("gather_rows: bad must hold one 32-bit word")
        if bad.device.type == "cpu" and not bad.is_pinned():
            raise ValueError("gather_rows: a host bad flag must be pinned")
        bad_ptr = device_address(bad)
    if table.dtype == torch.float32:
        fn = _native.hip().sf_gather_rows_f32_bf16
    elif table.element_size() == 2:
        fn = _native.hip().sf_gather_rows_b16
    else:
        raise TypeError(f"gather_rows: unsupported table dtype {table.dtype}")
    _native.check(fn(device_address(table), ids.data_ptr(), ids.numel(), row_len, nrows, device_address(dst),
                     bad_ptr, int(max_workgroups), _stream_ptr(stream)), "sf_gather_rows")
    return dst


def memcpy_async(dst: torch.Tensor, src: torch.Tensor, stream: Optional[torch.cuda.Stream] = None,
                 nbytes: Optional[int] = None) -> None:
    """Asynchronous byte copy between contiguous tensors on ``stream``.

    Host tensors must be pinned for the copy to overlap; direction is taken
    from the devices.
    """
    _require_contig(src, "src")
    _require_contig(dst, "dst")
    n = nbytes if nbytes is not None else src.numel() * src.element_size()
    if n > src.numel() * src.element_size() or n > dst.numel() * dst.element_size():
        raise ValueError(f"memcpy_async: {n} bytes exceed a buffer")
    sd, dd = src.device.type, dst.device.type
    if sd == "cpu" and dd == "cuda":
        kind = _native.SF_COPY_H2D
    elif sd == "cuda" and dd == "cpu":
        kind = _native.SF_COPY_D2H
    elif sd == "cuda" and dd == "cuda":
        kind = _native.SF_COPY_D2D
    else:
        raise ValueError(f"memcpy_async: unsupported direction {sd} -> {dd}")
    _native.check(_native.hip().sf_memcpy_async(dst.data_ptr(), src.data_ptr(), n, kind, _stream_ptr(stream)),
                  "sf_memcpy_async")


# ---------------------------------------------------------------------------
# SDMA device -> pinned host copies (not stream-ordered; see include/slidefsdp.h)
# ---------------------------------------------------------------------------
_dma_ready = set()
# Routing mode last set through ``dma_set_avoid_held`` (0: off).
_avoid_held_mode = 0


def avoid_held_from_env(value: Optional[str]) -> int:
    """The routing mode an ``SF_DMA_AVOID_HELD`` value asks for: unset or
    empty is 0; otherwise an integer in 0..2 (``ValueError`` for anything
    else)."""
    if value is None or value.strip() == "":
        return 0
    try:
        mode = int(value.strip())
    except ValueError:
        raise ValueError(f"SF_DMA_AVOID_HELD={value!r}: expected 0, 1 or 2") from None
    if mode not in (0, 1, 2):
        raise ValueError(f"SF_DMA_AVOID_HELD={value!r}: expected 0, 1 or 2")
    return mode


ROUTING_DISABLED = (
    "SDMA engine routing (SF_DMA_AVOID_HELD 1 or 2, sf_dma_set_avoid_held) is disabled for training: with it "
    "on, the step-1 gradients of the full-size Qwen2.5-14B step differed from a non-offloaded run's in about a "
    "third of the test runs, for a cause not found; unset SF_DMA_AVOID_HELD or set it to 0")


def dma_init(device: Optional[torch.device] = None) -> None:
    """Bind the SDMA copies to ``device`` (once per process).  The library
    picks engine 3 (HIP's own copies take engines 0, 1, 2 in turn, and a copy
    queued behind one of them that waits on an event waits as long);
    ``SF_DMA_ENGINES`` (e.g. "3" or "2,3") overrides it.  ``SF_DMA_AVOID_HELD`` other than
    0 raises ``RuntimeError``: engine routing is disabled (see
    ``ROUTING_DISABLED``)."""
    mode = avoid_held_from_env(os.environ.get("SF_DMA_AVOID_HELD"))
    if mode != 0:
        raise RuntimeError(ROUTING_DISABLED)
    idx = (device.index if device is not None and device.index is not None else torch.cuda.current_device())
    if idx in _dma_ready:
        return
    engines = engines_from_env(os.environ.get("SF_DMA_ENGINES"))
    _native.check(_native.hip().sf_dma_init(int(idx)), "sf_dma_init")
    if engines is not None:
        _native.check(_native.hip().sf_dma_set_engines(_engine_mask(engines)), "sf_dma_set_engines")
    _dma_ready.add(idx)


def engines_from_env(value: Optional[str]) -> Optional[List[int]]:
    """The engines ``SF_DMA_ENGINES`` names ("3", "2,3"), or None when it is
    unset or empty; anything but comma-separated engine numbers 0-15 raises
    ``ValueError``."""
    if value is None or value.strip() == "":
        return None
    try:
        engines = [int(e) for e in value.split(",")]
    except ValueError:
        raise ValueError(f"SF_DMA_ENGINES={value!r}: expected engine numbers 0-15 separated by commas") from None
    _engine_mask(engines, f"SF_DMA_ENGINES={value!r}: ")
    return engines


def _engine_mask(engines: Sequence[int], what: str = "") -> int:
    mask = 0
    for e in engines:
        if not 0 <= int(e) < 16:
            raise ValueError(f"{what}SDMA engine {e} out of range 0..15")
        mask |= 1 << int(e)
    return mask


def require_routing_off() -> None:
    """Raise ``RuntimeError`` if engine routing is on (set through
    ``dma_set_avoid_held`` or the environment): the training runtime does
    not run with it."""
    if _avoid_held_mode != 0 or avoid_held_from_env(os.environ.get("SF_DMA_AVOID_HELD")) != 0:
        raise RuntimeError(ROUTING_DISABLED)


def dma_engines() -> list:
    """SDMA engines used for device -> host copies ([] : runtime's choice)."""
    m = ctypes.c_uint32(0)
    _native.check(_native.hip().sf_dma_get_engines(ctypes.byref(m)), "sf_dma_get_engines")
    return [e for e in range(16) if m.value >> e & 1]


def dma_set_engines(engines: Sequence[int]) -> None:
    """Select the SDMA engines for device -> host copies ([] : runtime's choice)."""
    _native.check(_native.hip().sf_dma_set_engines(_engine_mask(engines)), "sf_dma_set_engines")


def dma_set_avoid_held(mode: int) -> None:
    """Route device -> host copies around engines another client holds: 0 no
    (default), 1 onto free engines 0-3, 2 also onto slower free engines from
    4 up when none of 0-3 is free.  For single-copy tests of the engine
    choice only: ``SlideFSDP`` refuses to run while it is not 0."""
    global _avoid_held_mode
    _native.check(_native.hip().sf_dma_set_avoid_held(int(mode)), "sf_dma_set_avoid_held")
    _avoid_held_mode = int(mode)


def dma_enable_timing(on: bool) -> None:
    _native.check(_native.hip().sf_dma_enable_timing(1 if on else 0), "sf_dma_enable_timing")


class DmaCopiesOutstanding(TimeoutError):
    """SDMA copies that had not completed when a bounded wait for them ended.
    Their destinations must not be reused nor their sources freed: an engine
    may still be moving the bytes."""


def _poll(done: Callable[[], bool], timeout: Optional[float]) -> bool:
    """Poll ``done`` with short sleeps (10 us doubling to 100 us) until it is
    true (returns True) or ``timeout`` seconds have passed (False); None
    waits without limit."""
    deadline = None if timeout is None else time.monotonic() + timeout
    pause = 10e-6
    while not done():
        if deadline is not None and time.monotonic() >= deadline:
            return False
        time.sleep(pause)
        pause = min(pause * 2, 100e-6)
    return True


def wait_event(ev, timeout: Optional[float], what: str) -> None:
    """Block until the device event ``ev`` has completed: ``synchronize()``
    without a limit, else polling ``query()`` until ``timeout`` seconds,
    then ``TimeoutError`` naming ``what``."""
    if timeout is None:
        ev.synchronize()
        return
    if not _poll(ev.query, timeout):
        raise TimeoutError(f"{what}: not complete after {timeout:g} s")


def dma_clock_ns() -> int:
    """The HSA system clock in ns, the clock of the SDMA copy times."""
    t = ctypes.c_uint64(0)
    _native.check(_native.hip().sf_dma_clock_ns(ctypes.byref(t)), "sf_dma_clock_ns")
    return t.value


def dma_copy_d2h(pairs: Sequence[Tuple[torch.Tensor, torch.Tensor]], timeout: Optional[float] = None):
    """Start SDMA copies of each contiguous GPU ``src`` into the pinned host
    ``dst`` of equal byte size.  The sources must already be complete on the
    device.  Returns a handle for ``dma_wait``; keep the tensors alive until
    then.  If the library fails after issuing some of the copies, they are
    waited for (up to ``timeout`` seconds, else ``DmaCopiesOutstanding``) and
    released before the error is raised, so no copy outlives the call."""
    segs = []
    for k, (src, dst) in enumerate(pairs):
        _require_cuda(src, f"pair {k} src")
        _require_contig(src, f"pair {k} src")
        _require_contig(dst, f"pair {k} dst")
        if dst.device.type != "cpu" or not dst.is_pinned():
            raise ValueError(f"pair {k}: dst must be a pinned host tensor")
        nb = src.numel() * src.element_size()
        if nb != dst.numel() * dst.element_size():
            raise ValueError(f"pair {k}: byte size mismatch")
        segs.append((src.data_ptr(), dst.data_ptr(), nb))
    arr = _seg_array(segs)
    cap = 16 * max(1, len(segs))
    handles = (ctypes.c_uint64 * cap)()
    count = ctypes.c_int(0)
    rc = _native.hip().sf_dma_copy_d2h(arr, len(segs), handles, cap, ctypes.byref(count))
    return _issued_or_raise(rc, handles, count.value, timeout)


def _issued_or_raise(rc: int, handles, n: int, timeout: Optional[float]):
    """The handle of the ``n`` copies an ``sf_dma_copy_d2h`` call started; if
    the call failed, those copies are waited for and released first, and the
    call's error is raised (``DmaCopiesOutstanding`` if they do not complete
    within ``timeout`` seconds)."""
    if rc != 0:
        if n > 0:
            issued = (handles, n)
            if not _poll(lambda: dma_query(issued), timeout):
                raise DmaCopiesOutstanding(f"sf_dma_copy_d2h failed (status {rc}) with {n} copies issued that "
                                           f"did not complete within {timeout:g} s")
            dma_wait(issued)
        _native.check(rc, "sf_dma_copy_d2h")
    return (handles, n)


def dma_query(handle) -> bool:
    """True once every copy of ``handle`` has completed (does not release it)."""
    handles, n = handle
    done = ctypes.c_int(0)
    _native.check(_native.hip().sf_dma_query(handles, n, ctypes.byref(done)), "sf_dma_query")
    return bool(done.value)


class DmaReady:
    """``query()`` / ``synchronize()`` view of an SDMA copy handle, the
    interface of a device event.  Completion is remembered once seen, so
    several threads may ask; ``release`` (``dma_wait``, which frees the copy's
    signals) is allowed only after completion was seen, and later queries
    then never touch the freed signals."""

    def __init__(self, handle, timeout: Optional[float] = None):
        self.handle = handle
        self.timeout = timeout
        self._done = False
        self._released = False
        self._lock = threading.Lock()

    def query(self) -> bool:
        with self._lock:
            if not self._done:
                self._done = dma_query(self.handle)
            return self._done

    def synchronize(self) -> None:
        """Wait until the copies have completed, at most ``timeout`` seconds
        (then ``DmaCopiesOutstanding``)."""
        if not _poll(self.query, self.timeout):
            raise DmaCopiesOutstanding(f"{self.handle[1]} SDMA copies not complete after {self.timeout:g} s")

    def release(self) -> Tuple[int, int]:
        """Wait for the copies, free their signals and return their (start,
        end) ns as ``dma_wait``."""
        self.synchronize()
        with self._lock:
            if self._released:
                raise RuntimeError("DmaReady: released twice")
            self._released = True
            return dma_wait(self.handle)


def dma_wait(handle, timeout: Optional[float] = None) -> Tuple[int, int]:
    """Wait for the copies of ``handle`` (at most ``timeout`` seconds, then
    ``DmaCopiesOutstanding`` with every copy still held; None: no limit)
    and release them; returns (start_ns, end_ns) when timing is enabled,
    else (0, 0)."""
    handles, n = handle
    t0, t1 = ctypes.c_uint64(0), ctypes.c_uint64(0)
    ns = 0 if timeout is None else max(1, int(timeout * 1e9))
    rc = _native.hip().sf_dma_wait(handles, n, ns, ctypes.byref(t0), ctypes.byref(t1))
    if rc == _native.SF_ETIMEDOUT:
        raise DmaCopiesOutstanding(f"{n} SDMA copies not complete after {timeout:g} s")
    _native.check(rc, "sf_dma_wait")
    return t0.value, t1.value
