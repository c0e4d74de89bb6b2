"""The codegen plugin protocol the front end drives, and the bookkeeping every backend shares.

A backend receives one call per lowered operation (``extern``, ``weight``, ``elementwise``, ``linear`` ...)
and returns ``Value`` objects. The base class owns what is backend-independent, following the reference
(chroma/_src/codegen/base.py:39-113):

* the weight blob: constants deduplicated by (dtype, shape, bytes), each padded to 64 bytes;
* arena allocations: sizes rounded up to 64 bytes, lifetimes as inclusive kernel-index ranges that
  ``record_usage`` extends to the kernel that last reads them;
* output promotion: a temporary that is also a graph output is written straight into the output buffer;
* the compile statistics reported in the manifest.
"""

from __future__ import annotations

import itertools
import math
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
import xxhash

from chroma_amd._src.memory import Allocation, plan_memory
from chroma_amd._src.spec import Stats, TensorSpec, nbytes
from chroma_amd._src.value import ITEMSIZE, Shape, Value, View, contiguous_strides


class WeightBlob:
    """The constant blob as a list of borrowed pieces: each appended buffer is kept by reference (a
    model's parameters are not copied), hashed once with XXH3-128 as it arrives, and only streamed out
    when the artifact is written. A multi-gigabyte model therefore never needs a second host copy of its
    weights, a temporary file, or a cryptographic hash over every byte.

    ``piece_digest`` (XXH3-128 of one buffer) is the deduplication key of a constant; ``hexdigest`` names
    the blob's content as the XXH3-128 of the sequence of (piece digest, piece length), so every byte is
    hashed exactly once."""

    def __init__(self) -> None:
        self._pieces: List[memoryview] = []
        self._size = 0
        self._digest = xxhash.xxh3_128()

    def __len__(self) -> int:
        return self._size

    def append(self, data, digest: Optional[bytes] = None) -> None:
        view = memoryview(data).cast("B")
        if not len(view):
            return
        self._pieces.append(view)
        self._digest.update((digest or self.piece_digest(view)) + len(view).to_bytes(8, "little"))
        self._size += len(view)

    def pad(self, alignment: int) -> None:
        self.append(bytes(-self._size % alignment))

    def hexdigest(self) -> str:
        return self._digest.hexdigest()

    @staticmethod
    def piece_digest(data: memoryview) -> bytes:
        return xxhash.xxh3_128(data).digest()

    def write_to(self, path: Path) -> None:
        with open(path, "wb") as stream:
            for piece in self._pieces:
                stream.write(piece)

    def __bytes__(self) -> bytes:
        return b"".join(self._pieces)


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
    # Graph rewrites (functions of the imported ExportedProgram) this backend wants before lowering.
    graph_passes: Tuple = ()

    def __init__(self) -> None:
        self.materialized: Dict[str, Value] = {}
        self.allocations: Dict[str, Allocation] = {}
        self.weights = WeightBlob()
        self.weight_cache: Dict[Tuple[torch.dtype, Shape, bytes], Value] = {}
        self.weight_data: Dict[Tuple[torch.dtype, Shape, bytes], memoryview] = {}
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
        """Store a constant once per distinct (dtype, shape, bytes): the key carries a 128-bit content
        digest and a hit is confirmed byte for byte before the stored copy is reused."""
        data = tensor_bytes(tensor)
        digest = WeightBlob.piece_digest(data)
        key = (tensor.dtype, tuple(tensor.shape), digest)
        cached = self.weight_cache.get(key)
        if cached is not None and np.array_equal(np.frombuffer(self.weight_data[key], np.uint8), np.frombuffer(data, np.uint8)):
            return cached
        self.weight_data[key] = data
        offset = len(self.weights)
        self.weights.append(data, digest)
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
