"""ORACLE - test infrastructure only. Never imported by the ``chroma_amd`` product path.

CPU restatement of Chroma's CPU backend codegen (chroma/_src/codegen/cpu/codegen.py:77-415): the parity
oracle for the ``hip`` backend and the CPU baseline timed next to it. It plugs into the product's front
end like any backend and emits one C++20 translation unit per graph:

* fused elementwise chains become expression templates (``unary``/``binary``/``reindex``/``gather``);
  an expression is materialised once it is 32 levels deep (codegen.py:93-97);
* ``linear`` materialises its operands and calls ``linear`` (BLAS sgemm or the portable loop);
* ``beck,bk->bec`` / ``beck,bek->bec`` over gathered expert weights call ``expert_linear`` and read the
  selected experts in place (codegen.py:263-294);
* an einsum that is one matrix product per batch index calls ``gemm`` with the view's strides
  (codegen.py:320-392); every other einsum and every reduction is a loop nest;
* softmax, top-k, RMSNorm, triangular masks and concatenation call the header kernels.

The emitted program uses the API of the reference's ``kernels.h``/``expressions.h``; the oracle's own
headers (oracle/include) implement that API, and ``oracle/ref`` compiles the same emitted program against
the reference's headers to pin them.
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Union

import torch

from chroma_amd._src.codegen.base import Codegen, GeneratedCode, literal
from chroma_amd._src.value import Operand, Value, View, contraction, contiguous_strides, matrix_axes

CTYPES = {torch.float32: "float", torch.bfloat16: "chroma::bfloat16_t", torch.int64: "int64_t"}

UNARY = {
    "aten.reciprocal.default": "1.0f / x",
    "aten.rsqrt.default": "1.0f / std::sqrt(x)",
    "aten.sigmoid.default": "1.0f / (1.0f + std::exp(-x))",
    "aten.neg.default": "-x",
    "aten.sin.default": "std::sin(x)",
    "aten.cos.default": "std::cos(x)",
    "aten.exp.default": "std::exp(x)",
    "aten.abs.default": "std::abs(x)",
    "aten.square.default": "x * x",
    # extensions (chroma_amd/_src/lowering.py)
    "aten.tanh.default": "std::tanh(x)",
    "aten.silu.default": "x * (1.0f / (1.0f + std::exp(-x)))",
    "aten.log.default": "std::log(x)",
}
BINARY = {"aten.add.Tensor": "+", "aten.sub.Tensor": "-", "aten.mul.Tensor": "*", "aten.div.Tensor": "/"}


def dims(shape: Sequence[int]) -> str:
    return "dims<" + ", ".join(str(int(d)) for d in shape) + ">"


def scalar(value: float) -> str:
    return f"Scalar<float>{{{literal(value)}}}"


def operand(value: Operand) -> str:
    return value.name if isinstance(value, Value) else scalar(value)


def encode(dtype: torch.dtype, code: str) -> str:
    return f"astype<chroma::bfloat16_t>({code})" if dtype == torch.bfloat16 else code


def loop_nest(out: Value, reduction_shape: Sequence[int], product: str, divisor: int = 1) -> str:
    """One output element per outer iteration; ``product`` is summed in float over the reduction loops."""
    lines = ["{"]
    lines += [f"for (size_t o{i} = 0; o{i} < {size}; ++o{i}) {{" for i, size in enumerate(out.shape)]
    lines.append("float sum = 0.0f;")
    lines += [f"for (size_t r{i} = 0; r{i} < {size}; ++r{i}) {{" for i, size in enumerate(reduction_shape)]
    lines.append(f"sum += {product};")
    lines += ["}"] * len(reduction_shape)
    index = " + ".join(f"o{i} * {stride}" for i, stride in enumerate(contiguous_strides(out.shape))) or "0"
    lines.append(f"{out.name}.data[{index}] = sum / {literal(divisor)};")
    lines += ["}"] * len(out.shape)
    lines.append("}")
    return "\n".join(lines)


class CPUCodegen(Codegen):
    backend = "cpu"

    def __init__(self, *, blas: bool = True) -> None:
        super().__init__()
        self.blas = blas
        self.expert_contractions = 0
        self.lines: List[Union[str, Value]] = []
        self.gathers = {}
        self.extensions = False  # the program uses a kernel of extensions.h

    # -- storage -------------------------------------------------------------------------------------
    def extern(self, tensor: torch.Tensor, kind: str, offset: int) -> Value:
        name = f"v{next(self.counter)}"
        shape = tuple(tensor.shape)
        ctype = CTYPES[tensor.dtype]
        pointer = f"inputs[{offset}]" if kind == "input" else f"weights.data() + {offset}"
        self.lines.append(f"auto {name} = view<const {ctype}, {dims(shape)}>(reinterpret_cast<const {ctype}*>({pointer}));")
        return Value(name, shape, tensor.dtype, stored=True, view=View(None, contiguous_strides(shape)))

    def allocate(self, shape, dtype) -> Value:
        value = super().allocate(shape, dtype)
        self.lines.append(value)
        return value

    def expr(self, meta: torch.Tensor, code: str, inputs: Sequence[Value]) -> Value:
        name = f"e{next(self.counter)}"
        self.lines.append(f"auto {name} = {code};")
        value = self.expression_value(name, meta, inputs)
        return self.materialize(value) if value.depth >= 32 else value

    def record(self, code: str, inputs: Sequence[Value]) -> None:
        self.record_usage(inputs)
        self.lines.append(code)
        self.kernels += 1

    def materialize(self, value: Value) -> Value:
        if value.stored:
            return value
        if value.name not in self.materialized:
            out = self.allocate(value.shape, value.dtype)
            self.record(f"evaluate({out.name}, {value.name});", [value])
            self.materialized[value.name] = out
        return self.materialized[value.name]

    def alias(self, meta: torch.Tensor, root: Value, offset: int) -> Value:
        shape = tuple(meta.shape)
        name = f"v{next(self.counter)}"
        self.lines.append(f"auto {name} = view<const {CTYPES[meta.dtype]}, {dims(shape)}>({root.name}.data + {offset});")
        return Value(name, shape, meta.dtype, root.deps, stored=True, view=View(root, contiguous_strides(shape), offset))

    def reshape(self, meta: torch.Tensor, x: Value) -> Value:
        if x.stored:
            return self.alias(meta, x.root, x.view.offset)
        return self.expr(meta, f"reshape<{dims(meta.shape)}>({x.name})", [x])

    def reindex(self, meta: torch.Tensor, x: Value, mapping: Sequence[int], offset: int) -> Value:
        return self.expr(meta, f"reindex<{dims(meta.shape)}, {dims(mapping)}, {offset}>({x.name})", [x])

    def cast(self, meta: torch.Tensor, x: Value) -> Value:
        return self.expr(meta, f"astype<{CTYPES[meta.dtype]}>({x.name})", [x])

    def output(self, index: int, value: Value) -> None:
        if self.promote_output(index, value):
            return
        ctype = CTYPES[value.dtype]
        target = f"view<{ctype}, {dims(value.shape)}>(reinterpret_cast<{ctype}*>(outputs[{index}]))"
        self.record(f"evaluate({target}, {value.name});", [value])

    # -- elementwise -----------------------------------------------------------------------------------
    def elementwise(self, meta, target: str, args, *, alpha: float = 1, low: Optional[float] = None, high: Optional[float] = None) -> Value:
        values = [value for value in args if isinstance(value, Value)]
        code = [operand(value) for value in args]
        if target in BINARY:
            if alpha != 1:
                code[1] = encode(meta.dtype, f"({code[1]} * {scalar(alpha)})")
            expression = f"{code[0]} {BINARY[target]} {code[1]}"
        elif target == "aten.rsub.Scalar":
            expression = f"{code[1]} - {encode(meta.dtype, f'({code[0]} * {scalar(alpha)})')}"
        elif target in ("aten.pow.Tensor_Scalar", "aten.pow.Scalar"):
            expression = f"binary({code[0]}, {code[1]}, [](float a, float b) {{ return std::pow(a, b); }})"
        elif target == "aten.clamp.default":
            body = "x"
            if low is not None:
                body = f"std::max({body}, {literal(low)})"
            if high is not None:
                body = f"std::min({body}, {literal(high)})"
            expression = f"unary({code[0]}, [](float x) {{ return {body}; }})"
        else:
            expression = f"unary({code[0]}, [](float x) {{ return {UNARY[target]}; }})"
        return self.expr(meta, encode(meta.dtype, expression), values)

    def gather(self, meta, x: Value, indices: Value, negative: bool) -> Value:
        value = self.expr(meta, f"gather<{dims(meta.shape)}, {str(negative).lower()}>({x.name}, {indices.name})", [x, indices])
        if negative and not value.stored:
            self.gathers[value.name] = (x, indices)
        return value

    def triangular(self, meta, x: Value, diagonal: int, upper: bool) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        self.record(f"triangular<{str(upper).lower()}, {diagonal}>({out.name}, {x.name});", [x])
        return out

    # -- whole-tensor kernels ---------------------------------------------------------------------------
    def linear(self, meta, x: Value, weight: Value, bias: Optional[Value]) -> Value:
        x, weight = self.materialize(x), self.materialize(weight)
        bias = self.materialize(bias) if bias is not None else None
        out = self.allocate(tuple(meta.shape), meta.dtype)
        rows, columns, inner = math.prod(x.shape[:-1]), weight.shape[0], weight.shape[1]
        if max(rows, columns, inner) > 2**31 - 1:
            raise ValueError("Matrix dimensions exceed the BLAS integer range")
        bias_pointer = f"{bias.name}.data" if bias is not None else "nullptr"
        code = f"linear({out.name}.data, {x.name}.data, {weight.name}.data, {bias_pointer}, {rows}, {columns}, {inner});"
        self.record(code, [x, weight] + ([bias] if bias is not None else []))
        return out

    def softmax(self, meta, x: Value, dim: int) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        self.record(f"softmax<{dim}>({out.name}, {x.name});", [x])
        return out

    def logsumexp(self, meta, x: Value, dim: int) -> Value:
        """Extension (no reference counterpart): ``extensions.h`` ``logsumexp``."""
        out = self.allocate(tuple(meta.shape), meta.dtype)
        self.extensions = True
        self.record(f"logsumexp<{dim}>({out.name}, {x.name});", [x])
        return out

    def topk(self, meta, x: Value, dim: int, largest: bool, sort: bool):
        values, indices = [self.allocate(tuple(t.shape), t.dtype) for t in meta]
        self.record(f"topk<{dim}, {str(largest).lower()}, {str(sort).lower()}>({values.name}, {indices.name}, {x.name});", [x])
        return values, indices

    def concatenate(self, meta, values: Sequence[Value], dim: int) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        parts, start = [], 0
        for value in values:
            parts.append(f"concat_part<{dim}, {start}>({out.name}, {value.name});")
            start += value.shape[dim]
        self.record("\n".join(parts), values)
        return out

    def norm(self, meta, x: Value, weight: Value, epsilon: float) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        self.record(f"rmsnorm({out.name}, {x.name}, {weight.name}, {literal(epsilon)});", [x, weight])
        return out

    def reduction(self, meta, x: Value, axes: Sequence[int], keepdim: bool, mean: bool) -> Value:
        out = self.allocate(tuple(meta.shape), meta.dtype)
        reduction_shape = tuple(x.shape[d] for d in axes)
        terms, out_dim, reduce_dim = [], 0, 0
        for dim, stride in enumerate(contiguous_strides(x.shape)):
            if dim in axes:
                terms.append(f"r{reduce_dim} * {stride}")
                reduce_dim += 1
            else:
                terms.append(f"o{out_dim} * {stride}")
            if keepdim or dim not in axes:
                out_dim += 1
        product = f"{x.name}[{' + '.join(terms) or '0'}]"
        self.record(loop_nest(out, reduction_shape, product, math.prod(reduction_shape) if mean else 1), [x])
        return out

    # -- contractions ---------------------------------------------------------------------------------
    def einsum(self, meta, eqn: str, values: Sequence[Value]) -> Value:
        labels, output, sizes, reduction = contraction(eqn, values)
        eqn = eqn.replace(" ", "")
        result = self.expert_einsum(meta, eqn, labels, sizes, values)
        if result is None:
            result = self.matrix(meta, labels, output, sizes, reduction, values)
        if result is None:
            result = self.loop_einsum(meta, labels, output, sizes, reduction, values)
        return result

    def expert_einsum(self, meta, eqn, labels, sizes, values) -> Optional[Value]:
        if eqn not in ("beck,bk->bec", "beck,bek->bec"):
            return None
        source = self.gathers.get(values[0].name)
        if source is None:
            return None
        for label, value in zip(labels, values):
            if any(size != sizes[letter] for letter, size in zip(label, value.shape)):
                return None
        weight, indices = source
        weight, indices, x = self.materialize(weight), self.materialize(indices), self.materialize(values[1])
        out = self.allocate(tuple(meta.shape), meta.dtype)
        tokens, selected, channels = out.shape
        inner = weight.shape[-1]
        if max(tokens, selected, channels, inner, weight.shape[0]) > 2**31 - 1:
            raise ValueError("Expert dimensions exceed the BLAS integer range")
        per_expert = str(eqn == "beck,bek->bec").lower()
        self.record(
            f"expert_linear({out.name}.data, {weight.name}.data, {indices.name}.data, {x.name}.data, "
            f"{tokens}, {selected}, {weight.shape[0]}, {channels}, {inner}, {per_expert});",
            [weight, indices, x],
        )
        self.expert_contractions += 1
        return out

    def loop_einsum(self, meta, labels, output, sizes, reduction, values) -> Value:
        loop_var = {label: f"o{i}" for i, label in enumerate(output)}
        loop_var.update({label: f"r{i}" for i, label in enumerate(reduction)})
        factors = []
        for label, value in zip(labels, values):
            terms = [f"{loop_var[letter]} * {stride}" for letter, size, stride in zip(label, value.shape, contiguous_strides(value.shape)) if size != 1]
            factors.append(f"{value.name}[{' + '.join(terms) or '0'}]")
        out = self.allocate(tuple(meta.shape), meta.dtype)
        self.record(loop_nest(out, tuple(sizes[label] for label in reduction), " * ".join(factors)), values)
        return out

    def matrix(self, meta, labels, output, sizes, reduction, values) -> Optional[Value]:
        found = matrix_axes(labels, output, reduction)
        if found is None:
            return None
        batch_axes, row_axis, column_axis, inner_axis = found
        out_strides = dict(zip(output, contiguous_strides(tuple(meta.shape))))
        rows, columns, inner = sizes[row_axis], sizes[column_axis], sizes[inner_axis]
        row_stride = out_strides[row_axis]
        if out_strides[column_axis] != 1 or max(rows, columns, inner, row_stride) >= 2**31:
            return None
        layouts = []
        for label, value in zip(labels, values):
            layouts.append(dict(zip(label, value.view.strides if value.view else contiguous_strides(value.shape))))
            for letter in {row_axis, column_axis, inner_axis} & set(label):
                if value.shape[label.index(letter)] != sizes[letter]:
                    return None
        left, right = layouts
        if not (left[inner_axis] == 1 or left[row_axis] == 1):
            return None
        if not (right[column_axis] == 1 or right[inner_axis] == 1):
            return None
        trans_a, trans_b = left[inner_axis] != 1, right[column_axis] != 1
        lda = left[inner_axis if trans_a else row_axis]
        ldb = right[column_axis if trans_b else inner_axis]
        if lda < sizes[row_axis if trans_a else inner_axis] or ldb < sizes[inner_axis if trans_b else column_axis]:
            return None
        if max(lda, ldb) >= 2**31:
            raise ValueError("Matrix strides exceed the BLAS integer range")
        operands = [value.root if value.view else self.materialize(value) for value in values]
        out = self.allocate(tuple(meta.shape), meta.dtype)
        offsets = []
        for label, value, layout in zip(labels, values, layouts):
            terms = [str(value.view.offset if value.view else 0)]
            terms += [f"b{i} * {layout[letter]}" for i, letter in enumerate(batch_axes) if value.shape[label.index(letter)] != 1]
            offsets.append(" + ".join(terms))
        destination = " + ".join(f"b{i} * {out_strides[letter]}" for i, letter in enumerate(batch_axes)) or "0"
        code = "\n".join(f"for (size_t b{i} = 0; b{i} < {sizes[letter]}; ++b{i})" for i, letter in enumerate(batch_axes))
        code += (
            f"\ngemm({out.name}.data + {destination}, {operands[0].name}.data + {offsets[0]}, "
            f"{operands[1].name}.data + {offsets[1]}, {rows}, {columns}, {inner}, {lda}, {ldb}, {row_stride}, "
            f"{str(trans_a).lower()}, {str(trans_b).lower()});"
        )
        self.record(code, operands)
        self.matrix_contractions += 1
        return out

    # -- output ----------------------------------------------------------------------------------------
    def render(self, line: Union[str, Value]) -> str:
        if isinstance(line, str):
            return line
        ctype = CTYPES[line.dtype]
        if line.name in self.output_buffers:
            pointer = f"outputs[{self.output_buffers[line.name]}]"
        else:
            pointer = f"workspace.data() + {self.allocations[line.name].offset}"
        return f"auto {line.name} = view<{ctype}, {dims(line.shape)}>(reinterpret_cast<{ctype}*>({pointer}));"

    def generate(self, inputs, outputs, stats) -> GeneratedCode:
        flags = ["-DCHROMA_CBLAS"] if self.blas else []
        stats = dict(stats, expert_contractions=self.expert_contractions, backend="cpu", math_library="cblas" if self.blas else "portable")
        body = "\n".join(self.render(line) for line in self.lines)
        source = TEMPLATE.format(weight_bytes=stats["weight_bytes"], workspace_bytes=stats["workspace_bytes"], body=body)
        if self.extensions:
            source = '#include "codegen/cpu/extensions.h"\n' + source
        return GeneratedCode({"model.cc": source}, "model.cc", flags, stats, inputs, outputs, self.weights)


# C ABI around the generated program; the oracle runner binds it with ctypes.
TEMPLATE = """#include "codegen/cpu/kernels.h"
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
using namespace chroma;
namespace {{
struct ModelProgram {{
    Buffer weights{{{weight_bytes}}};
    Buffer workspace{{{workspace_bytes}}};
    explicit ModelProgram(const char* path) {{ read_weights(path, weights.data(), weights.size()); }}
    void run(const void* const* inputs, void* const* outputs) {{
{body}
    }}
}};
int fail(int status, const char* message, char* error, size_t length) {{
    if (error && length) {{
        std::strncpy(error, message, length - 1);
        error[length - 1] = 0;
    }}
    return status;
}}
}}  // namespace
extern "C" {{
__attribute__((visibility("default"))) int oracle_create(const char* weights, void** handle, char* error, size_t length) {{
    try {{
        *handle = new ModelProgram(weights);
        return 0;
    }} catch (const std::exception& e) {{
        return fail(2, e.what(), error, length);
    }}
}}
__attribute__((visibility("default"))) int oracle_run(void* handle, const void* const* inputs, void* const* outputs, char* error, size_t length) {{
    try {{
        static_cast<ModelProgram*>(handle)->run(inputs, outputs);
        return 0;
    }} catch (const std::out_of_range& e) {{
        return fail(1, e.what(), error, length);
    }} catch (const std::exception& e) {{
        return fail(2, e.what(), error, length);
    }}
}}
__attribute__((visibility("default"))) void oracle_destroy(void* handle) {{ delete static_cast<ModelProgram*>(handle); }}
}}
"""
