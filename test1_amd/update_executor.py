"""The worker threads that run gradient offloads and host updates.

The reference runs host updates first in, first out on one executor thread
(slide_fsdp.py:163).  ``PriorityUpdateExecutor`` keeps one worker thread but
runs, among the queued tasks whose input is ready, the one with the lowest
priority value (the unit the next forward needs first).  ``_UpdateReady``
and ``_LinkQuiet`` are readiness objects polled by that worker.
"""

from __future__ import annotations

import threading
import time
from concurrent.futures import Future
from typing import Any, Callable, Optional


# Queue priority of work that may wait until the host AdamW has nothing else
# ready (the gradient-free rows of the embedding's update).
EARLY_UPDATE_PRIORITY = 1 << 30


class PriorityUpdateExecutor:
    """One worker thread that runs queued host updates lowest priority value
    first, among those whose input is ready.

    The reference runs updates first-in first-out, i.e. in backward order
    (slide_fsdp.py:163), so the units the next forward needs first are
    updated last.  Taking the ready unit the next forward needs soonest lets
    the next forward start while later units are still being updated.  Each
    unit's update is independent of the others' within a step, so the order
    does not change any result.

    A task may carry a ``ready`` object with ``query()`` and ``synchronize()``
    (a device event marking the end of its input's production).  Inputs
    complete in submission order (one stream or engine queue), so when no
    queued task is ready the worker waits for the oldest one, never for a
    later one.

    ``gate`` (optional) is called by the worker before each pick, outside the
    lock, and may block until a resource is free (a host gradient slot); its
    result is passed to the picked task as its first argument.  The choice is
    made once the resource is there, so it goes to the most urgent task.
    """

    def __init__(self, name: str, gate: Optional[Callable[[], Any]] = None):
        self._tasks: list = []   # [priority, seq, future, fn, args, ready]
        self._cv = threading.Condition()
        self._seq = 0
        self._stop = False
        self._gate = gate
        self._thread = threading.Thread(target=self._run, name=name, daemon=True)
        self._thread.start()

    def submit(self, priority: int, fn: Callable, *args, ready=None) -> Future:
        f: Future = Future()
        with self._cv:
            if self._stop:
                raise RuntimeError("PriorityUpdateExecutor: shut down")
            self._tasks.append((priority, self._seq, f, fn, args, ready))
            self._seq += 1
            self._cv.notify()
        return f

    @staticmethod
    def _ready(t) -> bool:
        if t[5] is None:
            return True
        try:
            return bool(t[5].query())
        except BaseException:
            return True   # a failed input: the task runs and reports it

    def _pick(self):
        """Under the lock: (task, must_wait).  The lowest-priority ready task,
        else the oldest task, to be waited for outside the lock."""
        for t in sorted(self._tasks, key=lambda t: (t[0], t[1])):
            if self._ready(t):
                return t, False
        return min(self._tasks, key=lambda t: t[1]), True

    def _run(self) -> None:
        while True:
            with self._cv:
                self._cv.wait_for(lambda: self._tasks or self._stop)
                if not self._tasks:
                    return
            token, gate_error = None, None
            if self._gate is not None:
                try:
                    token = self._gate()
                except BaseException as e:  # e.g. no slot freed in time: fail the oldest task
                    gate_error = e
            with self._cv:
                if gate_error is not None:
                    task = min(self._tasks, key=lambda t: t[1])
                    self._tasks.remove(task)
                    if task[2].set_running_or_notify_cancel():
                        task[2].set_exception(gate_error)
                    continue
                task, must_wait = self._pick()
                if not must_wait:
                    self._tasks.remove(task)
            if must_wait and getattr(task[5], "poll_interval", None):
                # Readiness that other queued tasks' progress can bring about
                # (moments read back into buffers they free): pick again until
                # some task is ready instead of committing to the oldest.  If
                # none is for poll_fallback_s, run the oldest anyway (it then
                # waits for its own inputs), so progress never depends on the
                # readiness reports alone.
                deadline = time.monotonic() + task[5].poll_fallback_s
                while must_wait and time.monotonic() < deadline:
                    time.sleep(task[5].poll_interval)
                    with self._cv:
                        task, must_wait = self._pick()
                        if not must_wait:
                            self._tasks.remove(task)
                if must_wait:
                    with self._cv:
                        task = min(self._tasks, key=lambda t: t[1])
                        self._tasks.remove(task)
                    try:
                        task[5].synchronize()
                    except BaseException:
                        pass
            elif must_wait:
                try:
                    task[5].synchronize()
                except BaseException:
                    pass  # the task itself reports the failure when it runs
                with self._cv:
                    task, _ = self._pick()
                    self._tasks.remove(task)
            _, _, f, fn, args, _ = task
            if self._gate is not None:
                args = (token,) + tuple(args)
            if not f.set_running_or_notify_cancel():
                continue
            try:
                f.set_result(fn(*args))
            except BaseException as e:  # delivered to whoever waits on f
                f.set_exception(e)

    def shutdown(self, wait: bool = True, timeout: Optional[float] = None) -> None:
        """Stop taking tasks; the worker finishes the queued ones and exits.
        With ``wait``, join it, for at most ``timeout`` seconds (then
        ``TimeoutError``: a task is still running)."""
        with self._cv:
            self._stop = True
            self._cv.notify_all()
        if wait and self._thread is not threading.current_thread():
            self._thread.join(timeout)
            if self._thread.is_alive():
                raise TimeoutError(f"{self._thread.name}: worker still running after {timeout:g} s")


class _UpdateReady:
    """``query`` is true once the gradients have landed and the moments are
    in memory.  A unit's moments may wait for a buffer that another queued
    unit's update frees, so the executor must not commit to one waiting
    task: ``poll_interval`` makes it pick again until some task is ready.
    ``synchronize`` waits for the gradients only (the update reads moments
    that are still on storage itself)."""

    poll_interval = 200e-6
    poll_fallback_s = 10.0

    def __init__(self, grads_ready, optimizer, unit: int):
        self.grads_ready, self.optimizer, self.unit = grads_ready, optimizer, unit

    def query(self) -> bool:
        try:
            return ((self.grads_ready is None or self.grads_ready.query())
                    and self.optimizer.states_ready(self.unit))
        except BaseException:
            return True  # a failed copy or read: the update runs and reports it

    def synchronize(self) -> None:
        if self.grads_ready is not None:
            self.grads_ready.synchronize()


class _LinkQuiet:
    """Ready once ``first`` has completed and no host-to-device copy of a
    unit is queued.  For update work that may wait (the embedding's
    gradient-free rows): its host-memory traffic would slow the copies the
    forward is waiting for, so it runs once they have landed.  Polled by the
    executor like ``_UpdateReady``; after ``poll_fallback_s`` it runs anyway."""

    poll_interval = 200e-6
    poll_fallback_s = 10.0

    def __init__(self, first, stager):
        self.first, self.stager = first, stager

    def query(self) -> bool:
        return self.first.query() and self.stager.backlog() == 0

    def synchronize(self) -> None:
        self.first.synchronize()
