"""Page-locked host arrays for program results.

Copies between the device and page-locked (pinned) host memory run at the link's DMA rate; copies into
ordinary pageable arrays go through the runtime's pinned staging slots, an extra CPU copy. ``Program``
therefore returns fresh outputs in page-locked blocks from the runtime library
(``chroma_hip_host_alloc``). Blocks are pooled by size: a block goes back to the pool when its array and
every view of it have been garbage collected, and the next call of the same shape reuses it. Blocks are
never handed back to the driver; the pool is bounded, and past the bound (or for arrays above
``BLOCK_LIMIT`` bytes) results are ordinary NumPy arrays.
"""

from __future__ import annotations

import ctypes
import math
import threading
from typing import Dict, List, Sequence, Tuple

import numpy as np

from chroma_amd._src import native

POOL_BYTES = 1 << 30  # page-locked bytes the pool may hold in total, in use or free
BLOCK_LIMIT = 64 << 20  # larger results are ordinary arrays (their copies stream through the staging slots)
PAGE = 4096

_lock = threading.Lock()
_free: Dict[int, List[int]] = {}
_held = 0


class _Lease:
    """Owner of one pooled block; collected together with the last array that views the block (the
    arrays are made from its ``__array_interface__``, so every view keeps it as its base)."""

    __slots__ = ("pointer", "size", "__array_interface__")

    def __init__(self, pointer: int, size: int, shape: Tuple[int, ...], typestr: str) -> None:
        self.pointer, self.size = pointer, size
        self.__array_interface__ = {"shape": shape, "typestr": typestr, "data": (pointer, False), "version": 3}

    def __del__(self) -> None:
        try:
            with _lock:
                _free.setdefault(self.size, []).append(self.pointer)
        except Exception:  # interpreter shutdown: the process is ending and the block with it
            pass


def empty(shape: Sequence[int], dtype: np.dtype) -> np.ndarray:
    """An uninitialised C-contiguous array in page-locked memory (ordinary memory past the pool's bound)."""
    global _held
    dtype = np.dtype(dtype)
    count = math.prod(shape)
    size = -(-max(1, count * dtype.itemsize) // PAGE) * PAGE
    if size > BLOCK_LIMIT:
        return np.empty(shape, dtype)
    with _lock:
        blocks = _free.get(size)
        pointer = blocks.pop() if blocks else None
        if pointer is None:
            if _held + size > POOL_BYTES:
                return np.empty(shape, dtype)
            _held += size
    if pointer is None:
        lib = native.library()
        handle, error = ctypes.c_void_p(), ctypes.create_string_buffer(512)
        if lib.chroma_hip_host_alloc(size, ctypes.byref(handle), error, len(error)) != native.OK or not handle.value:
            with _lock:
                _held -= size
            return np.empty(shape, dtype)
        pointer = handle.value
    array = np.asarray(_Lease(pointer, size, tuple(int(n) for n in shape), dtype.str))
    # A typestr names only the item size of a dtype NumPy does not know by string (bfloat16 reads '<V2').
    return array if array.dtype == dtype else array.view(dtype)


def pooled_bytes() -> int:
    """Page-locked bytes the pool holds (blocks in use and free)."""
    with _lock:
        return _held
