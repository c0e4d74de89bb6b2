// ORACLE (test infrastructure only): lazily evaluated tensor expressions of the CPU restatement.
// An expression has a static ``shape``, a ``value_type`` and ``operator[](flat index)``. Composition
// rules follow chroma/_src/codegen/cpu/expressions.h:8-122: binary operations broadcast, ``reindex``
// maps a flat index through per-dimension strides plus an offset, ``gather`` selects rows by an int64
// index (negative indices wrap only when allowed) and throws std::out_of_range otherwise, and
// ``evaluate`` writes every element in order.
#pragma once

#include "core/tensor.h"
#include <functional>
#include <stdexcept>
#include <type_traits>
#include <utility>

namespace chroma {
template <class E>
concept Expression = requires(const E& e, size_t i) {
    E::shape;
    typename E::value_type;
    e[i];
};

template <class T> struct Scalar {
    using value_type = T;
    static constexpr auto shape = dims<>;
    T value;
    T operator[](size_t) const { return value; }
};

template <Expression E, class F> struct Unary {
    using value_type = std::invoke_result_t<F, typename E::value_type>;
    static constexpr auto shape = E::shape;
    E input;
    F op;
    value_type operator[](size_t i) const { return op(input[i]); }
};

template <Expression E, class F> Unary<E, F> unary(E input, F op) { return {input, op}; }

template <class T, Expression E> auto astype(E input) {
    return unary(input, [](auto value) { return static_cast<T>(value); });
}

template <Expression A, Expression B, class F> struct Binary {
    using value_type = std::invoke_result_t<F, typename A::value_type, typename B::value_type>;
    static constexpr auto shape = broadcast_shape<A::shape, B::shape>();
    A lhs;
    B rhs;
    F op;
    value_type operator[](size_t i) const {
        return op(lhs[broadcast_index<A::shape, shape>(i)], rhs[broadcast_index<B::shape, shape>(i)]);
    }
};

template <Expression A, Expression B, class F> Binary<A, B, F> binary(A lhs, B rhs, F op) { return {lhs, rhs, op}; }
template <Expression A, Expression B> auto operator+(A lhs, B rhs) { return binary(lhs, rhs, std::plus<>{}); }
template <Expression A, Expression B> auto operator-(A lhs, B rhs) { return binary(lhs, rhs, std::minus<>{}); }
template <Expression A, Expression B> auto operator*(A lhs, B rhs) { return binary(lhs, rhs, std::multiplies<>{}); }
template <Expression A, Expression B> auto operator/(A lhs, B rhs) { return binary(lhs, rhs, std::divides<>{}); }

// Element i of the result reads input[Offset + sum_d coordinate_d(i) * Strides[d]].
template <auto Extents, auto Strides, size_t Offset, Expression E> struct Reindex {
    using value_type = typename E::value_type;
    static constexpr auto shape = Extents;
    E input;
    value_type operator[](size_t i) const {
        size_t source = Offset;
        size_t rest = i;
        for (size_t d = Extents.size(); d-- > 0;) {
            const size_t extent = static_cast<size_t>(Extents[d]);
            source += rest % extent * static_cast<size_t>(Strides[d]);
            rest /= extent;
        }
        return input[source];
    }
};

template <auto Extents, auto Strides, size_t Offset = 0, Expression E> Reindex<Extents, Strides, Offset, E> reindex(E input) {
    return {input};
}

template <auto Extents, Expression E> struct Reshape {
    using value_type = typename E::value_type;
    static constexpr auto shape = Extents;
    static_assert(numel(Extents) == numel(E::shape), "reshape keeps the element count");
    E input;
    value_type operator[](size_t i) const { return input[i]; }
};

template <auto Extents, Expression E> Reshape<Extents, E> reshape(E input) { return {input}; }

template <auto Extents, Expression E, Expression I, bool AllowNegative> struct Gather {
    using value_type = typename E::value_type;
    static constexpr auto shape = Extents;
    static constexpr size_t rows = static_cast<size_t>(E::shape[0]);
    static constexpr size_t row_size = numel(E::shape) / rows;
    E input;
    I indices;
    value_type operator[](size_t i) const {
        int64_t row = indices[i / row_size];
        if (AllowNegative && row < 0) {
            row += static_cast<int64_t>(rows);
        }
        if (row < 0 || row >= static_cast<int64_t>(rows)) {
            throw std::out_of_range("Tensor idx out of range");
        }
        return input[static_cast<size_t>(row) * row_size + i % row_size];
    }
};

template <auto Extents, bool AllowNegative = true, Expression E, Expression I>
Gather<Extents, E, I, AllowNegative> gather(E input, I indices) {
    return {input, indices};
}

template <class T, auto Extents, Expression E> void evaluate(TensorView<T, Extents> out, E expression) {
    static_assert(Extents == E::shape, "evaluate: shape mismatch");
    constexpr size_t count = numel(Extents);
    for (size_t i = 0; i < count; ++i) {
        out.data[i] = expression[i];
    }
}
}  // namespace chroma
