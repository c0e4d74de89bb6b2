"""The codegen plugin protocol the front end drives, and the bookkeeping every backend shares.

A backend receives one call per lowered operation (``extern``, ``weight``, ``elementwise``, ``linear`` ...)
and returns ``Value`` objects. The base class owns what is backend-independent, following the reference
(chroma/_src/codegen/base.py:39-113):

* the weight blob: constants deduplicated by (dtype, shape, sha256 of bytes), each padded to 64 bytes;
* arena allocations: sizes rounded up to 64 bytes, lifetimes as inclusive kernel-index ranges that
  ``record_usage`` extends to the kernel that last reads them;
* output promotion: a temporary that is also a graph output is written straight into the output buffer;
* the compile statistics reported in the manifest.
"""

from __future__ import annotations

import hashlib
import itertools
import math
import shutil
import tempfile
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from chroma_amd._src.memory import Allocation, plan_memory
from chroma_amd._src.spec import Stats, TensorSpec, nbytes
from chroma_amd._src.value import ITEMSIZE, Shape, Value, View, contiguous_strides


class WeightBlob:
    """The constant blob: appended in 64-byte aligned pieces, hashed as it grows, spilled to a temporary
    file once it exceeds ``spill_bytes`` so that multi-gigabyte models never need a host copy of their
    size in memory."""

    def __init__(self, spill_bytes: int = 1 << 30) -> None:
        self._memory = bytearray()
        self._file = None
        self._size = 0
        self._digest = hashlib.sha256()
        self._spill_bytes = spill_bytes

    def __len__(self) -> int:
        return self._size

    def append(self, data) -> None:
        view = memoryview(data).cast("B")
        if self._file is None and self._size + len(view) > self._spill_bytes:
            self._file = tempfile.NamedTemporaryFile(prefix="chroma-weights-", suffix=".bin")
            self._file.write(self._memory)
            self._memory = bytearray()
        if self._file is None:
            self._memory += view
        else:
            self._file.write(view)
        self._digest.update(view)
        self._size += len(view)

    def pad(self, alignment: int) -> None:
        self.append(bytes(-self._size % alignment))

    def hexdigest(self) -> str:
        return self._digest.copy().hexdigest()

    def write_to(self, path: Path) -> None:
        if self._file is None:
            Path(path).write_bytes(self._memory)
            return
        self._file.flush()
        shutil.copyfile(self._file.name, path)

    def __bytes__(self) -> bytes:
        if self._file is None:
            return bytes(self._memory)
        self._file.flush()
        return Path(self._file.name).read_bytes()


@dataclass
class GeneratedCode:
    files: Dict[str, str]
    source_name: str
    flags: List[str]
    stats: Stats
    inputs: List[TensorSpec]
    outputs: List[TensorSpec]
    weights: WeightBlob


def tensor_bytes(tensor: torch.Tensor) -> memoryview:
    """The tensor's bytes without a copy when it is already contiguous (bfloat16 as its bit patterns)."""
    tensor = tensor.detach().contiguous()
    if tensor.dtype == torch.bfloat16:
        tensor = tensor.view(torch.uint16)
    return memoryview(tensor.numpy().reshape(-1)).cast("B")


class Codegen:
    backend = "abstract"

    def __init__(self) -> None:
        self.materialized: Dict[str, Value] = {}
        self.allocations: Dict[str, Allocation] = {}
        self.weights = WeightBlob()
        self.weight_cache: Dict[Tuple[torch.dtype, Shape, bytes], Value] = {}
        self.output_buffers: Dict[str, int] = {}
        self.counter = itertools.count()
        self.kernels = 0
        self.expressions = 0
        self.matrix_contractions = 0

    # -- storage ---------------------------------------------------------------------------------
    def extern(self, tensor: torch.Tensor, kind: str, offset: int) -> Value:
        """Bind an input (``offset`` = input position) or a weight (``offset`` = byte offset in the blob)."""
        raise NotImplementedError

    def weight(self, tensor: torch.Tensor) -> Value:
        data = tensor_bytes(tensor)
        key = (tensor.dtype, tuple(tensor.shape), hashlib.sha256(data).digest())
        cached = self.weight_cache.get(key)
        if cached is not None:
            return cached
        offset = len(self.weights)
        self.weights.append(data)
        self.weights.pad(64)
        value = self.extern(tensor, "weight", offset)
        self.weight_cache[key] = value
        return value

    def allocate(self, shape: Shape, dtype: torch.dtype) -> Value:
        name = f"t{next(self.counter)}"
        size = math.prod(shape) * ITEMSIZE[dtype]
        self.allocations[name] = Allocation(-(-size // 64) * 64, self.kernels, self.kernels)
        return Value(name, tuple(shape), dtype, frozenset({name}), stored=True, view=View(None, contiguous_strides(shape)))

    def expression_value(self, name: str, meta: torch.Tensor, inputs: Sequence[Value]) -> Value:
        self.expressions += 1
        deps: frozenset = frozenset().union(*(value.deps for value in inputs)) if inputs else frozenset()
        depth = 1 + max((value.depth for value in inputs), default=0)
        return Value(name, tuple(meta.shape), meta.dtype, deps, depth=depth)

    def record_usage(self, inputs: Sequence[Value]) -> None:
        for value in inputs:
            for name in value.deps:
                self.allocations[name].end = self.kernels

    def promote_output(self, index: int, value: Value) -> bool:
        if value.name not in self.allocations or value.name in self.output_buffers:
            return False
        self.output_buffers[value.name] = index
        return True

    # -- results -----------------------------------------------------------------------------------
    def finish(self, inputs: List[TensorSpec], outputs: List[TensorSpec], folded_constants: int) -> GeneratedCode:
        for name in self.output_buffers:
            del self.allocations[name]
        workspace = plan_memory(self.allocations)
        stats: Stats = {
            "kernels": self.kernels,
            "expressions": self.expressions,
            "folded_constants": folded_constants,
            "matrix_contractions": self.matrix_contractions,
            "workspace_bytes": workspace,
            "unreused_workspace_bytes": sum(a.size for a in self.allocations.values()),
            "weight_bytes": len(self.weights),
            "output_bytes": sum(map(nbytes, outputs)),
        }
        return self.generate(inputs, outputs, stats)

    def generate(self, inputs: List[TensorSpec], outputs: List[TensorSpec], stats: Stats) -> GeneratedCode:
        raise NotImplementedError

    # -- operations (implemented by backends) -------------------------------------------------------
    def materialize(self, value: Value) -> Value:
        raise NotImplementedError

    def output(self, index: int, value: Value) -> None:
        raise NotImplementedError


def literal(value: float) -> str:
    """A C++ float literal that round-trips ``value`` through float32."""
    value = float(value)
    if math.isnan(value):
        return "NAN"
    if math.isinf(value):
        return "-INFINITY" if value < 0 else "INFINITY"
    return repr(value) + "f"


def optional(value: Optional[Value]) -> List[Value]:
    return [value] if value is not None else []
