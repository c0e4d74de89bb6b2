"""Torch-free artifact metadata shared by the compiler and the runtime loader.

``signature`` hashes the input/output specs exactly as the reference does (chroma/_src/program.py:62-63):
sha256 of the sorted-key JSON of ``{"inputs": ..., "outputs": ...}``.
"""

from __future__ import annotations

import hashlib
import json
import math
from typing import Any, Dict, List

TensorSpec = Dict[str, Any]  # {"name": str, "shape": list[int], "dtype": "float32" | "bfloat16" | "int64"}
Stats = Dict[str, Any]

ITEMSIZE_BY_NAME = {"float32": 4, "bfloat16": 2, "int64": 8}
MANIFEST_VERSION = 2


def signature(inputs: List[TensorSpec], outputs: List[TensorSpec]) -> str:
    return hashlib.sha256(json.dumps({"inputs": inputs, "outputs": outputs}, sort_keys=True).encode()).hexdigest()


def nbytes(spec: TensorSpec) -> int:
    return math.prod(spec["shape"]) * ITEMSIZE_BY_NAME[spec["dtype"]]
