"""Pinned host slots that a unit's bf16 gradients are offloaded into.

The reference has one shared pinned gradient buffer (slide_fsdp.py:174-179),
so each offload waits for the previous unit's host update
(layer_state.py:362-363).  Here a unit's gradients go into a slot of their
own (``GradSlotsPerUnit``), or, where the host cannot pin that much, into a
ring of decoder-sized slots with slots of their own for the largest units
(``GradSlotRing``); ``GradStagingRing`` is a ring of max-size slots.
"""

from __future__ import annotations

import queue
from typing import Any, Dict, List, Optional

import torch

from . import _native
from .pinned import pinned_empty


class GradStagingRing:
    """``depth`` pinned bf16 host slots of ``max_elems`` for gradient D2H.

    Replaces the single shared ``_cpu_grad_buffer`` of reference
    slide_fsdp.py:174-179; a slot is handed back by the update thread once
    LayerAdam has consumed it.
    """

    def __init__(self, depth: int, max_elems: int, dtype: torch.dtype = torch.bfloat16):
        self.slots = [pinned_empty(max_elems, dtype) for _ in range(depth)]
        self._free: "queue.Queue[int]" = queue.Queue()
        for i in range(depth):
            self._free.put(i)

    def acquire(self, timeout: Optional[float] = None, unit: Optional[int] = None) -> int:
        try:
            return self._free.get(timeout=timeout)
        except queue.Empty:
            raise TimeoutError("GradStagingRing.acquire: no slot released in time") from None

    def release(self, idx: int) -> None:
        self._free.put(idx)


class GradSlotRing:
    """Pinned gradient slots when one per unit does not fit the host's
    pinned memory.  Units more than twice the median unit's size (the output
    unit; a dense embedding) keep a slot of their own; the others share a
    ring of slots of the largest remaining unit, so a ring slot holds one
    decoder's gradients instead of the output unit's.  ``grow`` adds ring
    slots once the step's other pinned buffers exist.  Ring slots have ids
    0, 1, ...; a unit's own slot has the id ``("unit", u)``."""

    def __init__(self, unit_sizes: Dict[int, int], depth: int, dtype: torch.dtype = torch.bfloat16):
        sizes = sorted(unit_sizes.values())
        median = sizes[len(sizes) // 2] if sizes else 1
        self.big = {u: n for u, n in unit_sizes.items() if n > 2 * median}
        small = [n for u, n in unit_sizes.items() if u not in self.big]
        self.slot_elems = max(1, max(small) if small else max(sizes, default=1))
        self.n_small = len(small)
        self._dtype = dtype
        self.slots: Dict[Any, torch.Tensor] = {}
        for u, n in self.big.items():
            self.slots[("unit", u)] = pinned_empty(max(1, n), dtype)
        self._free: "queue.Queue[int]" = queue.Queue()
        self.depth = 0
        for _ in range(depth):
            self._publish(pinned_empty(self.slot_elems, dtype))

    def _publish(self, t: torch.Tensor) -> None:
        i = self.depth
        self.slots[i] = t
        self.depth += 1
        self._free.put(i)

    def grow(self, max_depth: int, headroom_bytes: int) -> int:
        """Pin more ring slots, up to ``max_depth``, until the host refuses;
        then give back enough of the new ones to leave ``headroom_bytes``
        pinnable for buffers allocated later.  Returns the slots added."""
        new: List[torch.Tensor] = []
        refused = False
        while self.depth + len(new) < max_depth:
            try:
                new.append(pinned_empty(self.slot_elems, self._dtype))
            except _native.NativeError as e:
                if e.status != _native.HIP_ERROR_OUT_OF_MEMORY:
                    raise
                refused = True
                break
        if refused:
            per = self.slot_elems * torch.empty((), dtype=self._dtype).element_size()
            for _ in range(min(len(new), -(-headroom_bytes // per))):
                new.pop()
        for t in new:
            self._publish(t)
        return len(new)

    def acquire(self, timeout: Optional[float] = None, unit: Optional[int] = None):
        """A ring slot (blocking), or with ``unit`` a big unit's own slot."""
        if unit is not None and unit in self.big:
            return ("unit", unit)
        try:
            return self._free.get(timeout=timeout)
        except queue.Empty:
            raise TimeoutError("GradSlotRing.acquire: no slot released in time") from None

    def own_slot(self, unit: int):
        """The unit's own slot id, or None for a unit that uses the ring."""
        return ("unit", unit) if unit in self.big else None

    def release(self, idx) -> None:
        if isinstance(idx, tuple):
            return None
        self._free.put(idx)


class GradSlotsPerUnit:
    """One pinned bf16 host slot per unit, sized to the unit.

    A unit has at most one gradient offload outstanding (its next backward
    follows its next forward, which waits for its update), so its slot is
    always free: gradient D2H never waits for the host optimizer, and
    updates may run in any order.  Costs 2 bytes of pinned host memory per
    parameter.
    """

    def __init__(self, unit_sizes: Dict[int, int], dtype: torch.dtype = torch.bfloat16):
        self.slots = {}
        for u, n in unit_sizes.items():
            self.slots[u] = pinned_empty(max(1, n), dtype)

    def acquire(self, timeout: Optional[float] = None, unit: Optional[int] = None) -> int:
        if unit not in self.slots:
            raise KeyError(f"GradSlotsPerUnit: no slot for unit {unit}")
        return unit

    def release(self, idx: int) -> None:
        return None
