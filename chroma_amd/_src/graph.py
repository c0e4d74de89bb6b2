"""Import and validate a ``torch.export`` program, and recognise the fp32 RMSNorm chain.

Validation mirrors the reference importer (chroma/_src/graph.py:15-55): decompositions are run with an
empty table; only tensor user inputs and outputs are accepted; mutated inputs or buffers are rejected;
every call must be in ``OPERATIONS``; every tensor must be static, non-empty, on the CPU and of a
supported dtype. ``fuse_norms`` (graph.py:58-95) replaces ``x * rsqrt(mean(x**2, -1, True) + eps) * w``
in float32 with one ``_rmsnorm`` node.
"""

from __future__ import annotations

import operator
import os
from typing import Union

import torch
from torch.export import ExportedProgram
from torch.export.graph_signature import InputKind, OutputKind, TensorArgument
from torch.fx import Node
from torch.utils._pytree import tree_leaves

from chroma_amd._src.lowering import OPERATIONS, _rmsnorm
from chroma_amd._src.value import DTYPE_NAMES


def validate_tensor(tensor: torch.Tensor) -> None:
    if any(type(d) is not int for d in tensor.shape):
        raise ValueError(f"Dynamic shape {tuple(tensor.shape)}")
    if any(d <= 0 for d in tensor.shape):
        raise ValueError(f"empty dim in {tuple(tensor.shape)}")
    if tensor.numel() * tensor.element_size() >= 2**63:
        raise ValueError(f"{tensor.numel()} elements do not fit")
    if tensor.device.type != "cpu":
        raise ValueError(f"export is on {tensor.device.type}")
    if tensor.dtype not in DTYPE_NAMES:
        raise ValueError(f"Unsupported dtype {tensor.dtype}")


def prepare(program: Union[ExportedProgram, str, "os.PathLike[str]"]) -> ExportedProgram:
    if isinstance(program, (str, os.PathLike)):
        program = torch.export.load(program)
    program = program.run_decompositions({})
    signature = program.graph_signature
    for spec in signature.input_specs:
        if spec.kind == InputKind.USER_INPUT and not isinstance(spec.arg, TensorArgument):
            raise TypeError(f"Only tensor inputs are supported, got {spec.arg}")
    for spec in signature.output_specs:
        if spec.kind != OutputKind.USER_OUTPUT:
            raise ValueError(f"Export mutates {spec.target}; mutation of inputs and buffers is unsupported")
        if not isinstance(spec.arg, TensorArgument):
            raise TypeError(f"Only tensor outputs are supported, got {spec.arg}")
    for node in program.graph.nodes:
        if node.op == "call_function" and node.target != operator.getitem and str(node.target) not in OPERATIONS:
            raise NotImplementedError(f"{node.name}: unsupported operator {node.target}")
        for tensor in tree_leaves(node.meta.get("val")):
            if isinstance(tensor, torch.Tensor):
                validate_tensor(tensor)
        if node.op not in ("placeholder", "call_function", "output"):
            raise NotImplementedError(f"{node.name}: unsupported node kind {node.op}")
    fuse_norms(program)
    return program


def _is(node: object, name: str) -> bool:
    return isinstance(node, Node) and str(node.target) == name


def fuse_norms(program: ExportedProgram) -> None:
    for node in program.graph.nodes:
        if not _is(node, "aten.mul.Tensor"):
            continue
        product, weight = node.args
        if not _is(product, "aten.mul.Tensor") or not isinstance(weight, Node):
            continue
        x, inverse = product.args
        if not _is(inverse, "aten.rsqrt.default"):
            continue
        shifted = inverse.args[0]
        if not _is(shifted, "aten.add.Tensor") or len(shifted.args) != 2 or shifted.kwargs:
            continue
        mean, epsilon = shifted.args
        if not _is(mean, "aten.mean.dim") or list(mean.args[1:]) != [[-1], True] or not isinstance(epsilon, (int, float)):
            continue
        squared = mean.args[0]
        if not _is(squared, "aten.pow.Tensor_Scalar") or squared.args != (x, 2):
            continue
        chain = (x, squared, mean, shifted, inverse, product, node)
        if any(part.meta["val"].dtype != torch.float32 for part in chain):
            continue
        if tuple(weight.meta["val"].shape) != (x.meta["val"].shape[-1],):
            continue
        node.target, node.args = _rmsnorm, (x, weight, epsilon)
    program.graph.eliminate_dead_code()
