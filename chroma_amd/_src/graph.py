"""Import and validate a ``torch.export`` program, and recognise the fp32 RMSNorm chain.

Validation mirrors the reference importer (chroma/_src/graph.py:15-55): decompositions are run with an
empty table; only tensor user inputs and outputs are accepted; mutated inputs or buffers are rejected;
every call must be in ``OPERATIONS``; every tensor must be static, non-empty, on the CPU and of a
supported dtype. ``fuse_norms`` (graph.py:58-95) replaces ``x * rsqrt(mean(x**2, -1, True) + eps) * w``
in float32 with one ``_rmsnorm`` node. ``fuse_attention`` (applied by backends that ask for it) replaces
the workload's grouped-query attention chain with one ``_attention`` node.
"""

from __future__ import annotations

import operator
import os
from typing import Optional, Tuple, Union

import torch
from torch.export import ExportedProgram
from torch.export.graph_signature import InputKind, OutputKind, TensorArgument
from torch.fx import Node
from torch.utils._pytree import tree_leaves

from chroma_amd._src.lowering import OPERATIONS, _attention, _rmsnorm
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


def _only_user(node: Node) -> bool:
    return len(node.users) == 1


def _unexpanded(node: object, group: int) -> Optional[Node]:
    """``X`` when ``node`` is ``expand(unsqueeze(X, 2), [-1, -1, group, -1])`` (a grouped-query key or
    value [S, KV, D] repeated over the group axis), else None."""
    if not _is(node, "aten.expand.default") or not _is(node.args[0], "aten.unsqueeze.default"):
        return None
    unsqueezed = node.args[0]
    source = unsqueezed.args[0]
    if unsqueezed.args[1] not in (2, -2) or not isinstance(source, Node) or source.meta["val"].dim() != 3:
        return None
    if tuple(node.meta["val"].shape) != tuple(source.meta["val"].shape[:2]) + (group,) + tuple(source.meta["val"].shape[2:]):
        return None
    return source


def _parts(node: Node) -> Tuple[Optional[Node], Node]:
    """(past, new) when ``node`` concatenates two tensors along axis 0, else (None, node)."""
    if _is(node, "aten.cat.default") and len(node.args[0]) == 2 and (node.args[1] if len(node.args) > 1 else 0) in (0, -3):
        past, new = node.args[0]
        if isinstance(past, Node) and isinstance(new, Node):
            return past, new
    return None, node


def fuse_attention(program: ExportedProgram) -> None:
    """Replace grouped-query attention with sinks - the reference workload's chain (gpt_oss.py:sdpa and
    cached.py:16-51)

        s = einsum("qhmd,khmd->hmqk", q, expand(unsqueeze(k, 2))) * scale + mask
        out = einsum("hmqk,khmd->qhmd", softmax(cat([s, sinks], -1), -1)[..., :-1], expand(unsqueeze(v, 2)))

    - by one ``_attention`` node, so a backend can compute it without storing the [heads, queries, keys]
    scores. Keys and values that are a concatenation of two tensors along the sequence axis (cached keys
    and new keys) are passed as their two parts. Only chains whose intermediate results have no other
    consumer and share one floating dtype are replaced; the node keeps the chain's rounding points."""
    graph = program.graph
    for e2 in list(graph.nodes):
        if not _is(e2, "aten.einsum.default") or e2.args[0].replace(" ", "") != "hmqk,khmd->qhmd":
            continue
        sliced, v_expanded = e2.args[1]
        if not _is(sliced, "aten.slice.Tensor") or not _only_user(sliced):
            continue
        weights = sliced.args[0]
        if not _is(weights, "aten.softmax.int") or not _only_user(weights) or weights.args[1] not in (3, -1):
            continue
        width = weights.meta["val"].shape[-1]
        bounds = list(sliced.args[2:5])
        start, end, step = bounds + [None, None, 1][len(bounds):]
        if sliced.args[1] not in (3, -1) or start not in (0, None) or end not in (-1, width - 1) or step != 1:
            continue
        joined = weights.args[0]
        if not _is(joined, "aten.cat.default") or not _only_user(joined) or len(joined.args) < 2 or joined.args[1] not in (3, -1):
            continue
        if len(joined.args[0]) != 2:
            continue
        masked, sinks = joined.args[0]
        if not _is(masked, "aten.add.Tensor") or not _only_user(masked) or masked.kwargs or len(masked.args) != 2:
            continue
        scaled, mask = masked.args
        if not _is(scaled, "aten.mul.Tensor") or not _only_user(scaled) or not isinstance(mask, Node):
            continue
        e1, scale = scaled.args
        if not _is(e1, "aten.einsum.default") or not _only_user(e1) or not isinstance(scale, (int, float)):
            continue
        if e1.args[0].replace(" ", "") != "qhmd,khmd->hmqk" or not isinstance(sinks, Node):
            continue
        q, k_expanded = e1.args[1]
        group = q.meta["val"].shape[2]
        k, v = _unexpanded(k_expanded, group), _unexpanded(v_expanded, group)
        if k is None or v is None:
            continue
        chain = (q, k, v, e1, scaled, masked, sinks, joined, weights, sliced, e2, mask)
        dtypes = {part.meta["val"].dtype for part in chain}
        if len(dtypes) != 1 or dtypes.pop() not in (torch.float32, torch.bfloat16):
            continue
        scores = tuple(e1.meta["val"].shape)
        if tuple(sinks.meta["val"].shape) != scores[:3] + (1,) or len(mask.meta["val"].shape) > 4:
            continue
        if torch.broadcast_shapes(tuple(mask.meta["val"].shape), scores) != scores:
            continue
        k_past, k_new = _parts(k)
        v_past, v_new = _parts(v)
        with graph.inserting_before(e2):
            fused = graph.call_function(_attention, (q, k_past, k_new, v_past, v_new, mask, sinks, float(scale)))
        fused.meta["val"] = e2.meta["val"]
        e2.replace_all_uses_with(fused)
        for node in (e2, sliced, weights, joined, masked, scaled, e1):
            graph.erase_node(node)
    graph.eliminate_dead_code()
