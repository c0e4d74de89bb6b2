"""ATen operator table and the lowering of each operator family onto codegen calls.

The accepted operators and their families follow the reference table (chroma/_src/lowering.py:34-86).
Two elementwise operators are added as extensions because torch 2.10's export emits them where the
reference's torch emitted in-table decompositions: ``aten.silu.default`` and ``aten.tanh.default``.
Both backends evaluate them as ``x * (1 / (1 + exp(-x)))`` and ``tanh(x)``. Two more extensions serve
vocabulary-wide log-probabilities: ``aten.log.default`` (``log(x)``) and ``aten.logsumexp.default``
over one axis, with torch's definition ``m + log(sum(exp(x - m)))``, m the maximum along the axis
(0 when it is infinite), float statistics, the result rounded once.

Per-family behaviour (reference lowering.py:112-284):

* layout ops become views (stride/offset mappings) or aliases; ``clone``/``contiguous`` materialise;
  ``to``/``_to_copy`` between float types is a cast;
* elementwise ops take their scalar operands as floats; for bfloat16 results the scalar operands of
  add/sub/rsub/pow and the alpha factor are rounded to bfloat16 first, as torch does; a NaN clamp bound
  turns the clamp into a multiplication by NaN;
* ``embedding`` gathers rows without negative indices, ``index.Tensor`` (one int64 index on axis 0)
  allows them;
* reductions, softmax and top-k normalise their axes; rank-0 softmax/top-k go through a [1] reshape.
"""

from __future__ import annotations

import math
import operator
from typing import Any, Dict, List, Sequence, Tuple, Union

import torch

from chroma_amd._src.dtypes import round_bf16
from chroma_amd._src.value import FLOAT_DTYPES, Value, View, axis, contiguous_strides

ELEMENTWISE = (
    "aten.abs.default",
    "aten.add.Tensor",
    "aten.clamp.default",
    "aten.cos.default",
    "aten.div.Tensor",
    "aten.exp.default",
    "aten.mul.Tensor",
    "aten.neg.default",
    "aten.pow.Scalar",
    "aten.pow.Tensor_Scalar",
    "aten.reciprocal.default",
    "aten.rsub.Scalar",
    "aten.rsqrt.default",
    "aten.sigmoid.default",
    "aten.sin.default",
    "aten.square.default",
    "aten.sub.Tensor",
    # extensions (see module docstring)
    "aten.silu.default",
    "aten.tanh.default",
    "aten.log.default",
)
LAYOUT = (
    "aten.view.default",
    "aten.reshape.default",
    "aten._unsafe_view.default",
    "aten.unsqueeze.default",
    "aten.expand.default",
    "aten.slice.Tensor",
    "aten.permute.default",
    "aten.transpose.int",
    "aten.t.default",
    "aten.to.dtype",
    "aten._to_copy.default",
    "aten.clone.default",
    "aten.contiguous.default",
    "aten.split.Tensor",
    "aten.split_with_sizes.default",
)
OPERATIONS: Dict[str, str] = {name: "elementwise" for name in ELEMENTWISE}
OPERATIONS.update({name: "layout" for name in LAYOUT})
OPERATIONS.update(
    {
        "aten.linear.default": "linear",
        "aten.embedding.default": "gather",
        "aten.index.Tensor": "gather",
        "aten.einsum.default": "einsum",
        "aten.mean.dim": "reduction",
        "aten.mean.default": "reduction",
        "aten.sum.default": "reduction",
        "aten.sum.dim_IntList": "reduction",
        "aten.softmax.int": "softmax",
        "aten.logsumexp.default": "logsumexp",  # extension (see module docstring)
        "aten.topk.default": "topk",
        "aten.cat.default": "cat",
        "aten.arange.default": "constant",
        "aten.arange.start": "constant",
        "aten.arange.start_step": "constant",
        "aten.new_full.default": "constant",
        "aten.full.default": "constant",
        "aten.triu.default": "triangular",
        "aten.tril.default": "triangular",
        "aten._assert_tensor_metadata.default": "metadata",
    }
)

_BF16_ROUNDED_SCALARS = {
    "aten.add.Tensor",
    "aten.sub.Tensor",
    "aten.rsub.Scalar",
    "aten.pow.Tensor_Scalar",
    "aten.pow.Scalar",
}


def _rmsnorm(x: torch.Tensor, weight: torch.Tensor, epsilon: float) -> torch.Tensor:
    """Graph target that ``fuse_norms`` substitutes for the fp32 RMSNorm chain."""
    return x * torch.rsqrt(x.square().mean(-1, keepdim=True) + epsilon) * weight


def _attention(q, k_past, k_new, v_past, v_new, mask, sinks, scale: float) -> torch.Tensor:
    """Graph target that ``fuse_attention`` substitutes for grouped-query attention with sinks: the same
    operations in the same order as the chain it replaces (reference chroma/models/gpt_oss.py sdpa and
    cached.py:38-48), so folding or tracing it gives the chain's result. q [T, KV, G, D]; keys and
    values [S, KV, D], each given whole (past None) or as past and new rows; mask broadcasts to
    [KV, G, T, S]; sinks [KV, G, T, 1]."""
    k = k_new if k_past is None else torch.cat((k_past, k_new))
    v = v_new if v_past is None else torch.cat((v_past, v_new))
    group = q.shape[2]
    k = k[:, :, None, :].expand(-1, -1, group, -1)
    v = v[:, :, None, :].expand(-1, -1, group, -1)
    scores = torch.einsum("qhmd,khmd->hmqk", q, k) * scale + mask
    weights = torch.cat((scores, sinks), dim=-1).softmax(-1)[..., :-1]
    return torch.einsum("hmqk,khmd->qhmd", weights, v)


def _arg(args: Sequence[Any], kwargs: Dict[str, Any], index: int, name: str, default: Any = None) -> Any:
    return args[index] if len(args) > index else kwargs.get(name, default)


def layout_view(codegen, meta: torch.Tensor, x: Value, mapping: Sequence[int], offset: int) -> Value:
    """A strided view of ``x``. Views of stored values are rebased onto their root buffer; a view whose
    strides are contiguous for its shape becomes a plain alias."""
    if x.view is None:
        return codegen.reindex(meta, x, mapping, offset)
    root = x.root
    offset += x.view.offset
    shape = tuple(meta.shape)
    if all(size == 1 or given == natural for size, given, natural in zip(shape, mapping, contiguous_strides(shape))):
        return codegen.alias(meta, root, offset)
    result = codegen.reindex(meta, root, mapping, offset)
    result.view = View(root, tuple(mapping), offset)
    return result


def _lower_layout(codegen, name: str, meta, args, kwargs) -> Union[Value, Tuple[Value, ...]]:
    x: Value = args[0]
    if name in ("aten.to.dtype", "aten._to_copy.default"):
        if x.dtype == meta.dtype:
            return x
        if x.dtype not in FLOAT_DTYPES or meta.dtype not in FLOAT_DTYPES:
            raise NotImplementedError(f"{x.dtype} -> {meta.dtype}")
        return codegen.cast(meta, x)
    if name in ("aten.clone.default", "aten.contiguous.default"):
        return codegen.materialize(x)
    if name in ("aten.view.default", "aten.reshape.default", "aten._unsafe_view.default"):
        return codegen.reshape(meta, x)

    mapping = list(x.view.strides if x.view is not None else contiguous_strides(x.shape))
    if name in ("aten.split.Tensor", "aten.split_with_sizes.default"):
        dim = axis(_arg(args, kwargs, 2, "dim", 0), len(x.shape))
        parts = []
        offset = 0
        for part in meta:
            parts.append(layout_view(codegen, part, x, mapping, offset))
            offset += part.shape[dim] * mapping[dim]
        return tuple(parts)

    shape = tuple(meta.shape)
    offset = 0
    if name == "aten.unsqueeze.default":
        mapping.insert(axis(args[1], len(shape)), 0)
    elif name == "aten.expand.default":
        pad = len(shape) - len(x.shape)
        padded_shape = (1,) * pad + tuple(x.shape)
        padded = [0] * pad + mapping
        mapping = [stride if before == after else 0 for stride, before, after in zip(padded, padded_shape, shape)]
    elif name == "aten.slice.Tensor":
        dim = axis(_arg(args, kwargs, 1, "dim", 0), len(x.shape))
        start, _, step = slice(_arg(args, kwargs, 2, "start"), _arg(args, kwargs, 3, "end"), _arg(args, kwargs, 4, "step", 1)).indices(
            x.shape[dim]
        )
        if step <= 0:
            raise NotImplementedError(f"slice step {step}")
        offset = start * mapping[dim]
        mapping[dim] *= step
    else:
        order = list(range(len(x.shape)))
        if name == "aten.permute.default":
            order = [axis(d, len(x.shape)) for d in args[1]]
        elif len(order) > 1:
            if name == "aten.t.default":
                a, b = 0, 1
            else:
                a, b = axis(args[1], len(order)), axis(args[2], len(order))
            order[a], order[b] = order[b], order[a]
        mapping = [mapping[d] for d in order]
    return layout_view(codegen, meta, x, mapping, offset)


def _lower_elementwise(codegen, name: str, meta, args, kwargs) -> Value:
    if meta.dtype not in FLOAT_DTYPES:
        raise NotImplementedError(name)
    alpha = kwargs.get("alpha", 1)
    if name == "aten.rsub.Scalar":
        alpha = _arg(args, kwargs, 2, "alpha", 1)
    low = high = None
    if name == "aten.clamp.default":
        low, high = _arg(args, kwargs, 1, "min"), _arg(args, kwargs, 2, "max")
        if any(bound is not None and math.isnan(bound) for bound in (low, high)):
            name, args, low, high = "aten.mul.Tensor", (args[0], math.nan), None, None
        else:
            args = args[:1]
    operands = tuple(value for value in args if value is not None)
    if name == "aten.rsub.Scalar":
        operands = operands[:2]
    if meta.dtype == torch.bfloat16 and name in _BF16_ROUNDED_SCALARS:
        operands = tuple(v if isinstance(v, Value) else round_bf16(float(v)) for v in operands)
        alpha = round_bf16(float(alpha))
    return codegen.elementwise(meta, name, operands, alpha=alpha, low=low, high=high)


def lower(codegen, target: Any, meta: Any, args: Tuple[Any, ...], kwargs: Dict[str, Any]) -> Union[Value, Tuple[Value, ...]]:
    if target == operator.getitem:
        return args[0][args[1]]
    if target is _rmsnorm:
        return codegen.norm(meta, args[0], args[1], args[2])
    if target is _attention:
        return codegen.attention(meta, *args)
    name = str(target)
    family = OPERATIONS.get(name)

    if family == "layout":
        return _lower_layout(codegen, name, meta, args, kwargs)
    if family == "elementwise":
        return _lower_elementwise(codegen, name, meta, args, kwargs)
    if family == "gather":
        negative = name == "aten.index.Tensor"
        indices = args[1]
        if negative:
            if len(indices) != 1 or not isinstance(indices[0], Value):
                raise NotImplementedError("index: one tensor, axis 0")
            indices = indices[0]
        if indices.dtype != torch.int64:
            raise NotImplementedError("index wants int64")
        return codegen.gather(meta, args[0], indices, negative)
    if family == "linear":
        if any(v.dtype not in FLOAT_DTYPES for v in args[:2]) or meta.dtype not in FLOAT_DTYPES:
            raise NotImplementedError(name)
        return codegen.linear(meta, args[0], args[1], _arg(args, kwargs, 2, "bias"))
    if family == "reduction":
        x: Value = args[0]
        if x.dtype not in FLOAT_DTYPES or meta.dtype not in FLOAT_DTYPES:
            raise NotImplementedError(name)
        dims = _arg(args, kwargs, 1, "dim", []) or range(len(x.shape))
        axes: List[int] = sorted({axis(d, len(x.shape)) for d in dims}) if x.shape else []
        keepdim = _arg(args, kwargs, 2, "keepdim", False)
        mean = name.startswith("aten.mean.")
        if not mean and x.dtype != meta.dtype:
            x = codegen.cast(meta.new_empty(x.shape), x)
        return codegen.reduction(meta, x, axes, keepdim, mean)
    if family == "einsum":
        return codegen.einsum(meta, args[0], args[1])
    if family == "softmax":
        x = args[0]
        if x.dtype not in FLOAT_DTYPES or meta.dtype not in FLOAT_DTYPES:
            raise NotImplementedError(name)
        dim = axis(args[1], len(x.shape))
        if x.dtype != meta.dtype:
            x = codegen.cast(meta.new_empty(x.shape), x)
        if x.shape:
            return codegen.softmax(meta, x, dim)
        vector = meta.new_empty((1,))
        return codegen.reshape(meta, codegen.softmax(vector, codegen.reshape(vector, x), 0))
    if family == "logsumexp":
        x = args[0]
        if x.dtype not in FLOAT_DTYPES or meta.dtype not in FLOAT_DTYPES or not x.shape:
            raise NotImplementedError(name)
        dims = list(_arg(args, kwargs, 1, "dim", []))
        if len(dims) != 1:
            raise NotImplementedError("logsumexp over one axis")
        if x.dtype != meta.dtype:
            x = codegen.cast(meta.new_empty(x.shape), x)
        return codegen.logsumexp(meta, x, axis(dims[0], len(x.shape)))
    if family == "topk":
        x = args[0]
        dim = axis(_arg(args, kwargs, 2, "dim", -1), len(x.shape))
        width = x.shape[dim] if x.shape else 1
        # the reference's limit (lowering.py:262-264) unless the backend selects over wider rows
        if x.dtype not in FLOAT_DTYPES or width > getattr(codegen, "topk_width_limit", 4096):
            raise NotImplementedError(f"topk axis {width}")
        largest = _arg(args, kwargs, 3, "largest", True)
        sort = _arg(args, kwargs, 4, "sorted", True)
        if x.shape:
            return codegen.topk(meta, x, dim, largest, sort)
        vector = meta[0].new_empty((1,), dtype=x.dtype)
        values, indices = codegen.topk([part.new_empty((1,)) for part in meta], codegen.reshape(vector, x), 0, largest, sort)
        return codegen.reshape(meta[0], values), codegen.reshape(meta[1], indices)
    if family == "cat":
        return codegen.concatenate(meta, args[0], axis(_arg(args, kwargs, 1, "dim", 0), len(meta.shape)))
    if family == "triangular":
        return codegen.triangular(meta, args[0], _arg(args, kwargs, 1, "diagonal", 0), name == "aten.triu.default")
    raise NotImplementedError(f"Unsupported runtime operation {target}")
