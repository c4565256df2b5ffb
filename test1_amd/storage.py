"""Files on local storage for offloaded data: the Python side of the native
storage engine (``sf_io_*`` in ``libsf_cpu.so``).

The reference offloads checkpointed activations with kvikio (GPUDirect
Storage, sliding_checkpoint.py:133-202) and LayerAdam's moments with
tensornvme's ``DiskOffloader`` (optimizer/layer_adam/layer_adam.py:89-103,
197-244).  Neither exists for ROCm and there is no GPU-to-storage DMA here, so
both go through host memory and this engine: worker threads moving chunks of
a request with pread/pwrite on files opened with O_DIRECT (where the file
system allows it), so the page cache does not take back the host memory the
offload frees.

O_DIRECT needs 4 KiB-aligned buffers, sizes and offsets: ``aligned_empty``
makes such host tensors, and file layouts put every region at an aligned
offset with an aligned length.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

from . import _native

ALIGN = _native.SF_IO_ALIGN


def align_up(n: int, a: int = ALIGN) -> int:
    return (int(n) + a - 1) // a * a


def aligned_empty(numel: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Host tensor of at least ``numel`` elements whose first byte is
    ALIGN-aligned and whose byte length is a multiple of ALIGN (the tail
    beyond ``numel`` is padding that transfers carry along)."""
    esize = torch.empty((), dtype=dtype).element_size()
    nbytes = align_up(max(1, numel) * esize)
    raw = torch.empty(nbytes + ALIGN, dtype=torch.uint8)
    skip = (-raw.data_ptr()) % ALIGN
    return raw[skip:skip + nbytes].view(dtype)


def _cpu():
    return _native.cpu()


def _check(status: int, what: str) -> None:
    _native.check(status, what, _cpu())


class IoRequest:
    """One queued transfer.  Holds the buffer alive until it completes."""

    __slots__ = ("_engine", "ticket", "_keep", "nbytes", "op", "_status", "submit_ns", "done_ns", "_lock")

    def __init__(self, engine: "IoEngine", ticket: int, keep, nbytes: int, op: int):
        self._engine = engine
        self.ticket = ticket
        self._keep = keep
        self.nbytes = nbytes
        self.op = op
        self._status: Optional[int] = None
        self.submit_ns = 0
        self.done_ns = 0
        self._lock = threading.Lock()

    def done(self) -> bool:
        """True once the transfer finished (raises if it failed)."""
        with self._lock:
            if self._status is not None:
                return True
            flag = ctypes.c_int(0)
            st = _cpu().sf_io_query(self._engine.handle, self.ticket, ctypes.byref(flag))
            if not flag.value:
                _check(st, "sf_io_query")
                return False
        self.wait()
        return True

    def wait(self) -> None:
        """Block until the transfer finished; raise if it failed."""
        with self._lock:
            if self._status is None:
                t0, t1 = ctypes.c_uint64(0), ctypes.c_uint64(0)
                self._status = _cpu().sf_io_wait(self._engine.handle, self.ticket, ctypes.byref(t0), ctypes.byref(t1))
                self.submit_ns, self.done_ns = t0.value, t1.value
                self._keep = None
            status = self._status
        _check(status, "file " + ("write" if self.op == _native.SF_IO_WRITE else "read"))

    # the interface of a device event, for schedulers that poll readiness
    query = done
    synchronize = wait


class OffloadFile:
    """A file opened for offload (``kvikio.CuFile`` / a ``DiskOffloader``
    file).  With ``unlink=True`` its name is removed at once: the space is
    returned when it is closed or the process ends."""

    def __init__(self, engine: "IoEngine", path: str, direct: bool = True, unlink: bool = True):
        self.engine = engine
        self.path = path
        fd, d = ctypes.c_int(-1), ctypes.c_int(0)
        _check(_cpu().sf_io_open(path.encode(), int(direct), int(unlink), ctypes.byref(fd), ctypes.byref(d)),
               f"sf_io_open({path})")
        self.fd = fd.value
        self.direct = bool(d.value)
        self.size = 0

    def reserve(self, nbytes: int) -> None:
        """Grow the file to ``nbytes`` (unwritten ranges read as zeros)."""
        if nbytes > self.size:
            _check(_cpu().sf_io_reserve(self.fd, int(nbytes)), "sf_io_reserve")
            self.size = int(nbytes)

    def _submit(self, op: int, t: torch.Tensor, offset: int, nbytes: Optional[int]) -> IoRequest:
        if t.device.type != "cpu" or not t.is_contiguous():
            raise ValueError("offload file: host tensors that are contiguous expected")
        if nbytes is None:
            nbytes = t.numel() * t.element_size()
        return self.engine.submit(self.fd, op, t.data_ptr(), int(nbytes), int(offset), keep=t)

    def write(self, t: torch.Tensor, offset: int, nbytes: Optional[int] = None) -> IoRequest:
        """Queue ``nbytes`` (default: all of ``t``) from ``t`` to ``offset``."""
        return self._submit(_native.SF_IO_WRITE, t, offset, nbytes)

    def read(self, t: torch.Tensor, offset: int, nbytes: Optional[int] = None) -> IoRequest:
        """Queue ``nbytes`` (default: all of ``t``) from ``offset`` into ``t``."""
        return self._submit(_native.SF_IO_READ, t, offset, nbytes)

    def close(self) -> None:
        if self.fd >= 0:
            _check(_cpu().sf_io_close(self.fd), "sf_io_close")
            self.fd = -1

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class IoEngine:
    """Worker threads moving requests between host buffers and files."""

    def __init__(self, n_threads: int = 8, chunk_bytes: int = 8 << 20):
        h = ctypes.c_void_p(0)
        _check(_cpu().sf_io_create(int(n_threads), int(chunk_bytes), ctypes.byref(h)), "sf_io_create")
        self.handle = h
        self.n_threads = n_threads

    def open(self, path: str, direct: bool = True, unlink: bool = True) -> OffloadFile:
        return OffloadFile(self, path, direct=direct, unlink=unlink)

    def submit(self, fd: int, op: int, ptr: int, nbytes: int, offset: int, keep=None) -> IoRequest:
        if not self.handle:
            raise RuntimeError("IoEngine: closed")
        t = ctypes.c_uint64(0)
        _check(_cpu().sf_io_submit(self.handle, fd, op, ctypes.c_void_p(ptr), nbytes, offset, ctypes.byref(t)),
               "sf_io_submit")
        return IoRequest(self, t.value, keep, nbytes, op)

    def stats(self) -> dict:
        """Bytes read / written by completed requests, the seconds during
        which at least one request was in flight, and the bytes copied through
        a worker's staging buffer (caller memory the kernel cannot pin for
        direct I/O, such as hipHostMalloc'd slots)."""
        r, w, b, st = ctypes.c_uint64(0), ctypes.c_uint64(0), ctypes.c_uint64(0), ctypes.c_uint64(0)
        _check(_cpu().sf_io_stats(self.handle, ctypes.byref(r), ctypes.byref(w), ctypes.byref(b), ctypes.byref(st)),
               "sf_io_stats")
        return {"bytes_read": r.value, "bytes_written": w.value, "busy_s": b.value * 1e-9,
                "bytes_staged": st.value}

    def close(self) -> None:
        if self.handle:
            _check(_cpu().sf_io_destroy(self.handle), "sf_io_destroy")
            self.handle = ctypes.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_default: Optional[IoEngine] = None
_default_lock = threading.Lock()


def default_engine() -> IoEngine:
    """The process's shared engine (``SF_IO_THREADS`` workers, default 8),
    created on first use."""
    global _default
    with _default_lock:
        if _default is None:
            raw = os.environ.get("SF_IO_THREADS", "").strip() or "8"
            if not raw.isdigit() or int(raw) < 1:
                raise ValueError(f"SF_IO_THREADS={raw!r}: expected a positive thread count")
            _default = IoEngine(n_threads=int(raw))
        return _default
