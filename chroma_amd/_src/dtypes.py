"""NumPy-side storage types for compiled programs.

The reference runtime represents bfloat16 arrays with ``ml_dtypes.bfloat16`` (chroma/_src/program.py:15).
That package is optional here: when it is missing, bfloat16 arrays use a one-field structured dtype whose
only field holds the raw 16-bit pattern. It is distinct from ``uint16`` and ``V2``, so a raw bit array is
still rejected as a dtype mismatch, and ``array.view(np.uint16)`` recovers the bits.
"""

from __future__ import annotations

import struct
from typing import Dict

import numpy as np

try:  # pragma: no cover - depends on the environment
    from ml_dtypes import bfloat16 as _ml_bfloat16

    BFLOAT16 = np.dtype(_ml_bfloat16)
except ImportError:  # pragma: no cover - depends on the environment
    BFLOAT16 = np.dtype([("bfloat16", "<u2")])

NUMPY_DTYPES: Dict[str, np.dtype] = {
    "float32": np.dtype(np.float32),
    "bfloat16": BFLOAT16,
    "int64": np.dtype(np.int64),
}


def numpy_dtype(name: str) -> np.dtype:
    return NUMPY_DTYPES[name]


def bf16_bits(value: float) -> int:
    """Round-to-nearest-even float32 -> bfloat16 bit pattern; every NaN becomes 0x7fc0.

    Same rounding as the reference's ``bfloat16_t`` (chroma/_src/core/bfloat16.h:7-17). The value is
    first rounded to float32, as a C++ ``float`` parameter would be.
    """
    word = struct.unpack("<I", struct.pack("<f", value))[0]
    if word & 0x7FFFFFFF > 0x7F800000:
        return 0x7FC0
    return ((word + 0x7FFF + ((word >> 16) & 1)) >> 16) & 0xFFFF


def round_bf16(value: float) -> float:
    """The float value of ``value`` after rounding to bfloat16."""
    return struct.unpack("<f", struct.pack("<I", bf16_bits(value) << 16))[0]


def bf16_to_float32(array: np.ndarray) -> np.ndarray:
    """Widen a bfloat16 array (either representation) to float32 exactly."""
    bits = np.ascontiguousarray(array).view(np.uint16).astype(np.uint32) << 16
    return bits.view(np.float32).reshape(array.shape)


def float32_to_bf16(array: np.ndarray) -> np.ndarray:
    """Round a float32 array to a bfloat16 array with the same RNE/NaN rule as ``bf16_bits``."""
    word = np.ascontiguousarray(array, dtype=np.float32).view(np.uint32)
    rounded = ((word + 0x7FFF + ((word >> 16) & 1)) >> 16).astype(np.uint16)
    rounded = np.where((word & 0x7FFFFFFF) > 0x7F800000, np.uint16(0x7FC0), rounded)
    return rounded.view(BFLOAT16).reshape(np.shape(array))
