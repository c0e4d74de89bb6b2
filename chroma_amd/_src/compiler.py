"""Drive a codegen plugin over an imported graph.

Follows the reference compiler (chroma/_src/compiler.py:28-164):

* placeholders: user inputs become ``extern(..., "input", i)``; parameters, buffers and constant tensors
  become compile-time constants;
* constant folding: a node whose inputs are all constants is evaluated with torch at compile time; nodes
  derived from state are folded only up to 1 MiB each and 16 MiB in total;
* liveness: only nodes reachable backwards from the outputs are emitted (layout nodes are always walked
  through, so views of folded constants still resolve);
* an elementwise result with more than one consumer (looking through layout ops) is materialised.
"""

from __future__ import annotations

import operator
import os
from typing import Any, Dict, List, Mapping, Set, Tuple, Union

import torch
from torch.export import ExportedProgram
from torch.fx import Node, map_arg
from torch.utils._pytree import tree_leaves

from chroma_amd._src.codegen.base import Codegen, GeneratedCode
from chroma_amd._src.graph import prepare, validate_tensor
from chroma_amd._src.lowering import OPERATIONS, lower
from chroma_amd._src.value import Value

_NOT_CONSTANT = object()
_STATE_NODE_LIMIT = 1024**2
_STATE_TOTAL_LIMIT = 16 * 1024**2


def consumers(node: Node) -> Set[Node]:
    pending = list(node.users)
    found: Set[Node] = set()
    seen: Set[Node] = set()
    while pending:
        user = pending.pop()
        if user in seen:
            continue
        seen.add(user)
        family = OPERATIONS.get(str(user.target))
        if family == "layout" or user.target == operator.getitem:
            pending.extend(user.users)
        elif family != "metadata":
            found.add(user)
    return found


def _arguments(node: Node, values: Mapping[Node, Any]) -> Tuple[Tuple[Any, ...], Dict[str, Any]]:
    args = map_arg(node.args, values.__getitem__)
    kwargs = map_arg(node.kwargs, values.__getitem__)
    return tuple(args), dict(kwargs)


class Compiler:
    def __init__(self, program: ExportedProgram, codegen: Codegen) -> None:
        self.program = program
        self.codegen = codegen
        self.values: Dict[Node, Any] = {}
        self.constants: Dict[Node, Any] = {}
        self.state_constants: Set[Node] = set()
        self.fold_bytes = 0
        self.folded: Set[str] = set()
        self.inputs: List[dict] = []
        self.outputs: List[dict] = []

    @classmethod
    def from_export(cls, program: Union[ExportedProgram, str, "os.PathLike[str]"], codegen: Codegen) -> "Compiler":
        compiler = cls(prepare(program), codegen)
        for rewrite in codegen.graph_passes:
            rewrite(compiler.program)
        placeholders = [node for node in compiler.program.graph.nodes if node.op == "placeholder"]
        for node, spec in zip(placeholders, compiler.program.graph_signature.input_specs):
            if spec.kind.name == "USER_INPUT":
                value = codegen.extern(node.meta["val"], "input", len(compiler.inputs))
                compiler.inputs.append(value.spec(node.name))
                compiler.values[node] = value
            else:
                source = compiler.program.constants if spec.kind.name == "CONSTANT_TENSOR" else compiler.program.state_dict
                tensor = source[spec.target].detach()
                validate_tensor(tensor)
                compiler.constants[node] = tensor
                compiler.state_constants.add(node)
        return compiler

    def fold_constant(self, node: Node) -> Any:
        if node in self.constants:
            return self.constants[node]
        target = str(node.target)
        if node.op != "call_function" or OPERATIONS.get(target) == "metadata":
            return _NOT_CONSTANT
        size = 0
        if any(n in self.state_constants for n in node.all_input_nodes):
            self.state_constants.add(node)
            size = sum(t.numel() * t.element_size() for t in tree_leaves(node.meta.get("val")) if isinstance(t, torch.Tensor))
            if size > _STATE_NODE_LIMIT or self.fold_bytes + size > _STATE_TOTAL_LIMIT:
                return _NOT_CONSTANT
        if target == "aten.new_full.default":
            meta = node.meta["val"]
            return torch.full(tuple(meta.shape), node.args[2], dtype=meta.dtype)
        args, kwargs = _arguments(node, self.constants)
        if any(value is _NOT_CONSTANT for value in tree_leaves((args, kwargs))):
            return _NOT_CONSTANT
        with torch.no_grad():
            value = node.target(*args, **kwargs)
        self.fold_bytes += size
        return value

    def emit(self, node: Node) -> Any:
        constant = self.constants[node]
        target = str(node.target)
        is_layout = OPERATIONS.get(target) == "layout"
        if constant is not _NOT_CONSTANT and target in ("aten.to.dtype", "aten._to_copy.default"):
            is_layout = False
        if not is_layout and isinstance(constant, torch.Tensor):
            if node.op == "call_function":
                self.folded.add(node.name)
            result: Any = self.codegen.weight(constant)
        elif not is_layout and isinstance(constant, (tuple, list)):
            result = tuple(self.codegen.weight(t) for t in constant)
        else:
            args, kwargs = _arguments(node, self.values)
            result = lower(self.codegen, node.target, node.meta["val"], args, kwargs)
        if isinstance(result, Value) and OPERATIONS.get(target) == "elementwise" and len(consumers(node)) > 1:
            result = self.codegen.materialize(result)
        self.values[node] = result
        return result

    def lower(self) -> GeneratedCode:
        nodes = list(self.program.graph.nodes)
        for node in nodes:
            self.constants[node] = self.fold_constant(node)
        output = next(node for node in nodes if node.op == "output")
        needed = set(output.all_input_nodes)
        for node in reversed(nodes):
            if node in needed and (self.constants[node] is _NOT_CONSTANT or OPERATIONS.get(str(node.target)) == "layout"):
                needed.update(node.all_input_nodes)
        for node in nodes:
            if node in needed and node not in self.values:
                self.emit(node)
        for index, node in enumerate(output.args[0]):
            value = self.values[node]
            self.outputs.append(value.spec(node.name))
            self.codegen.output(index, value)
        return self.codegen.finish(self.inputs, self.outputs, len(self.folded))


def lower_program(program: Union[ExportedProgram, str, "os.PathLike[str]"], codegen: Codegen) -> GeneratedCode:
    """Import ``program`` and lower it through ``codegen``; returns the generated sources and weights."""
    return Compiler.from_export(program, codegen).lower()


def compile_for_backend(program, output, *, blas: bool = True, backend: str = "hip"):
    """``chroma.compile``'s dispatch (reference compiler.py:153-164) with the ``hip`` backend.

    ``blas`` selects the MFMA/tiled matrix kernels (True) or the scalar fallback kernels (False), the
    counterpart of the reference's cuBLAS switch.
    """
    if backend != "hip":
        raise ValueError(f"Unknown runtime backend: {backend}")
    from chroma_amd._src.build import build
    from chroma_amd._src.codegen.hip import HIPCodegen

    return build(lower_program(program, HIPCodegen(blas=blas)), output)
