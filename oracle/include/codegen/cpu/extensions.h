// ORACLE - test infrastructure only. Kernels for operators this build adds to the reference's table
// (the reference's CPU backend, chroma/_src/codegen/cpu/kernels.h, has no counterpart). Included by a
// generated program only when it uses one, so programs without them still compile against the
// reference's own headers.
#pragma once

#include "codegen/cpu/kernels.h"
#include <cmath>
#include <limits>

namespace chroma {

// log(sum(exp(x))) along Axis with torch's definition (aten/src/ATen/native/ReduceOps.cpp logsumexp):
// m = the maximum along the axis, replaced by 0 when it is infinite; result = log(sum(exp(x - m))) + m.
// The sum is a float accumulated in index order, like the reference softmax's (kernels.h:125-151); the
// result is converted to T once. A NaN element makes the sum NaN, a +inf element makes it +inf, and a
// line of -inf sums to 0, whose log is -inf.
template <int Axis, class T, auto SO, Expression E> void logsumexp(TensorView<T, SO> out, E x) {
    constexpr auto S = E::shape;
    constexpr size_t width = static_cast<size_t>(S[Axis]);
    constexpr size_t inner = inner_size<S, Axis>();
    constexpr size_t lines = numel(S) / width;
    static_assert(numel(SO) == lines, "logsumexp removes one axis");
    for (size_t line = 0; line < lines; ++line) {
        const size_t first = line / inner * width * inner + line % inner;
        float peak = -std::numeric_limits<float>::infinity();
        for (size_t k = 0; k < width; ++k) {
            peak = std::max(peak, float(x[first + k * inner]));
        }
        const float shift = std::isinf(peak) ? 0.0f : peak;
        float total = 0;
        for (size_t k = 0; k < width; ++k) {
            total += std::exp(float(x[first + k * inner]) - shift);
        }
        out.data[line] = T(std::log(total) + shift);
    }
}

}  // namespace chroma
