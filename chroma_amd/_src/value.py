"""Front-end values: stored buffers, strided views of them, and deferred expressions.

A ``Value`` is what every lowering step hands to the codegen plugin and gets back.
Field meaning follows the reference IR (chroma/_src/value.py:19-37): ``deps`` names the arena
allocations the value reads, ``stored`` says whether it lives in memory, ``depth`` counts fused
expression levels and ``view`` places a stored value inside its root buffer.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, FrozenSet, List, Optional, Sequence, Tuple, Union

import torch

Shape = Tuple[int, ...]
FLOAT_DTYPES = (torch.float32, torch.bfloat16)
# dtype -> manifest name; the three storage types the compiler accepts (reference value.py:12-16).
DTYPE_NAMES: Dict[torch.dtype, str] = {
    torch.float32: "float32",
    torch.bfloat16: "bfloat16",
    torch.int64: "int64",
}
ITEMSIZE: Dict[torch.dtype, int] = {torch.float32: 4, torch.bfloat16: 2, torch.int64: 8}


@dataclass(frozen=True)
class View:
    """Element strides and offset of a stored value relative to ``base`` (None: the value is its own root)."""

    base: Optional["Value"]
    strides: Shape
    offset: int = 0


@dataclass(eq=False)
class Value:
    name: str
    shape: Shape
    dtype: torch.dtype
    deps: FrozenSet[str] = frozenset()
    stored: bool = False
    depth: int = 0
    view: Optional[View] = None

    def spec(self, name: str) -> dict:
        return {"name": name, "shape": list(self.shape), "dtype": DTYPE_NAMES[self.dtype]}

    @property
    def root(self) -> "Value":
        return self.view.base if self.view is not None and self.view.base is not None else self


Operand = Union[Value, float]


def contiguous_strides(shape: Sequence[int]) -> Shape:
    out: List[int] = []
    step = 1
    for size in reversed(shape):
        out.append(step)
        step *= size
    return tuple(reversed(out))


def axis(value: int, rank: int) -> int:
    """Normalise a possibly negative dim; a rank-0 tensor only has axis 0."""
    return value % rank if rank else 0


def contraction(eqn: str, values: Sequence[Value]) -> Tuple[List[str], str, Dict[str, int], List[str]]:
    """Split a two-operand einsum into (operand labels, output labels, label sizes, reduced labels).

    Broadcast labels take their largest size (reference value.py:52-66).
    """
    eqn = eqn.replace(" ", "")
    if len(values) != 2 or "->" not in eqn or "..." in eqn:
        raise NotImplementedError(f"einsum {eqn!r}: two operands, explicit output, no ellipses")
    if any(v.dtype not in FLOAT_DTYPES for v in values):
        raise NotImplementedError("Einsum requires float tensors")
    lhs, output = eqn.split("->")
    labels = lhs.split(",")
    sizes: Dict[str, int] = {}
    for label, value in zip(labels, values):
        if len(label) != len(value.shape):
            raise ValueError(f"einsum {eqn!r}: label {label!r} does not match shape {value.shape}")
        for letter, size in zip(label, value.shape):
            sizes[letter] = max(size, sizes.get(letter, 1))
    return labels, output, sizes, sorted(set(sizes) - set(output))


def matrix_axes(labels: Sequence[str], output: str, reduction: Sequence[str]):
    """Recognise a batched matrix product: one row label, one column label, one contracted label.

    Returns (batch labels in output order, row, column, contracted) or None (reference value.py:69-81).
    """
    left, right = set(labels[0]), set(labels[1])
    rows, columns = left - right, right - left
    batch = [letter for letter in output if letter in left and letter in right]
    if len(reduction) != 1 or len(rows) != 1 or len(columns) != 1:
        return None
    m, n, k = next(iter(rows)), next(iter(columns)), reduction[0]
    if set(output) != set(batch) | {m, n} or k not in (left & right):
        return None
    return batch, m, n, k


def numel(shape: Sequence[int]) -> int:
    return math.prod(shape)
