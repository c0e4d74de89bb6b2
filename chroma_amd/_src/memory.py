"""Arena planning: pack temporaries with known lifetimes into one buffer.

Lifetimes are inclusive ranges of kernel indices. Allocations are visited in order of their first kernel;
every allocation whose last kernel precedes the current start is released, adjacent free ranges merge, and
the smallest free range that fits is taken (best fit), otherwise the arena grows. This is the reference's
planner (chroma/_src/memory.py:12-50); the known answer in its test (tests/test_runtime.py:287-302) pins it.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Tuple


@dataclass
class Allocation:
    size: int
    start: int
    end: int
    offset: int = 0


def _coalesce(free: List[Tuple[int, int]]) -> List[Tuple[int, int]]:
    merged: List[Tuple[int, int]] = []
    for offset, size in sorted(free):
        if merged and merged[-1][0] + merged[-1][1] == offset:
            start, length = merged.pop()
            merged.append((start, length + size))
        else:
            merged.append((offset, size))
    return merged


def plan_memory(allocations: Dict[str, Allocation]) -> int:
    """Assign ``offset`` to every allocation and return the arena size in bytes."""
    live: List[Allocation] = []
    free: List[Tuple[int, int]] = []
    total = 0
    for allocation in sorted(allocations.values(), key=lambda a: a.start):
        still_live = []
        for other in live:
            if other.end < allocation.start:
                free.append((other.offset, other.size))
            else:
                still_live.append(other)
        live = still_live
        free = _coalesce(free)
        best = None
        for index, (_, size) in enumerate(free):
            if size >= allocation.size and (best is None or size < free[best][1]):
                best = index
        if best is None:
            allocation.offset = total
            total += allocation.size
        else:
            offset, size = free.pop(best)
            allocation.offset = offset
            if size > allocation.size:
                free.append((offset + allocation.size, size - allocation.size))
        live.append(allocation)
    return total
