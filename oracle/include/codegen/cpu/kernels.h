// ORACLE (test infrastructure only): the CPU restatement's whole-tensor kernels.
// Numerics follow chroma/_src/codegen/cpu/kernels.h:24-193 step for step: float accumulation in index
// order, bias added after the product for float linears and inside the float sum for bfloat16 ones,
// RMSNorm as x * (1 / sqrt(sum(x^2) / n + eps)) * w, a two-pass softmax that divides in the last pass,
// top-k through the standard library's partial_sort / nth_element with the same comparator and NaN rule,
// and concatenation by block copies. Function names and template parameters match the reference so
// the same generated program compiles against either header set.
#pragma once

#include "codegen/cpu/expressions.h"
#include <algorithm>
#include <array>
#include <cmath>
#include <limits>

#if defined(CHROMA_CBLAS)
// BLAS mode links NumPy's bundled OpenBLAS (64-bit integer interface, "scipy_" symbol prefix).
extern "C" {
void scipy_cblas_sgemm64_(int order, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha, const float* a,
                          int64_t lda, const float* b, int64_t ldb, float beta, float* c, int64_t ldc);
void scipy_cblas_sgemv64_(int order, int trans, int64_t m, int64_t n, float alpha, const float* a, int64_t lda,
                          const float* x, int64_t incx, float beta, float* y, int64_t incy);
}
namespace chroma::blas {
constexpr int row_major = 101, no_trans = 111, trans = 112;
}
#endif

namespace chroma {
// Number of elements after Axis in a contiguous tensor of shape S: the stride along Axis.
template <auto S, int Axis> consteval size_t inner_size() {
    size_t count = 1;
    for (size_t d = static_cast<size_t>(Axis) + 1; d < S.size(); ++d) {
        count *= static_cast<size_t>(S[d]);
    }
    return count;
}

template <class T>
void gemm(T* out, const T* a, const T* b, int rows, int columns, int inner, int lda, int ldb, int ldc, bool trans_a,
          bool trans_b) {
#if defined(CHROMA_CBLAS)
    if constexpr (std::is_same_v<T, float>) {
        scipy_cblas_sgemm64_(blas::row_major, trans_a ? blas::trans : blas::no_trans, trans_b ? blas::trans : blas::no_trans,
                             rows, columns, inner, 1.0f, a, lda, b, ldb, 0.0f, out, ldc);
        return;
    }
#endif
    for (int i = 0; i < rows; ++i) {
        for (int j = 0; j < columns; ++j) {
            float sum = 0;
            for (int k = 0; k < inner; ++k) {
                const size_t left = trans_a ? size_t(k) * lda + i : size_t(i) * lda + k;
                const size_t right = trans_b ? size_t(j) * ldb + k : size_t(k) * ldb + j;
                sum += float(a[left]) * float(b[right]);
            }
            out[size_t(i) * ldc + j] = sum;
        }
    }
}

inline void linear(float* out, const float* input, const float* weight, const float* bias, int rows, int columns,
                   int inner) {
#if defined(CHROMA_CBLAS)
    scipy_cblas_sgemm64_(blas::row_major, blas::no_trans, blas::trans, rows, columns, inner, 1.0f, input, inner, weight,
                         inner, 0.0f, out, columns);
#else
    gemm(out, input, weight, rows, columns, inner, inner, inner, columns, false, true);
#endif
    if (bias != nullptr) {
        for (int i = 0; i < rows; ++i) {
            float* row = out + size_t(i) * columns;
            for (int j = 0; j < columns; ++j) {
                row[j] += bias[j];
            }
        }
    }
}

inline void linear(bfloat16_t* out, const bfloat16_t* input, const bfloat16_t* weight, const bfloat16_t* bias,
                   int rows, int columns, int inner) {
    for (int i = 0; i < rows; ++i) {
        for (int j = 0; j < columns; ++j) {
            float sum = 0;
            for (int k = 0; k < inner; ++k) {
                sum += float(input[size_t(i) * inner + k]) * float(weight[size_t(j) * inner + k]);
            }
            out[size_t(i) * columns + j] = sum + (bias != nullptr ? float(bias[j]) : 0.0f);
        }
    }
}

// out[b, e, :] = weight[indices[b, e]] @ input[b or (b, e), :]; an index outside [-experts, experts)
// throws, a negative one wraps.
template <class T>
void expert_linear(T* out, const T* weight, const int64_t* indices, const T* input, int tokens, int selected,
                   int experts, int columns, int inner, bool per_expert) {
    for (int b = 0; b < tokens; ++b) {
        for (int e = 0; e < selected; ++e) {
            const size_t slot = size_t(b) * selected + e;
            int64_t expert = indices[slot];
            if (expert < 0) {
                expert += experts;
            }
            if (expert < 0 || expert >= experts) {
                throw std::out_of_range("Expert idx out of range");
            }
            const T* w = weight + size_t(expert) * columns * inner;
            const T* x = input + (per_expert ? slot : size_t(b)) * inner;
            T* y = out + slot * columns;
#if defined(CHROMA_CBLAS)
            if constexpr (std::is_same_v<T, float>) {
                scipy_cblas_sgemv64_(blas::row_major, blas::no_trans, columns, inner, 1.0f, w, inner, x, 1, 0.0f, y, 1);
                continue;
            }
#endif
            linear(y, x, w, nullptr, 1, columns, inner);
        }
    }
}

template <class T, auto S, Expression E, Expression W>
void rmsnorm(TensorView<T, S> out, E x, W weight, float epsilon) {
    constexpr size_t columns = static_cast<size_t>(S.back());
    constexpr size_t rows = numel(S) / columns;
    for (size_t r = 0; r < rows; ++r) {
        const size_t start = r * columns;
        float squares = 0.0f;
        for (size_t j = 0; j < columns; ++j) {
            const float v = x[start + j];
            squares += v * v;
        }
        const float scale = 1.0f / std::sqrt(squares / float(columns) + epsilon);
        for (size_t j = 0; j < columns; ++j) {
            out.data[start + j] = float(x[start + j]) * scale * float(weight[j]);
        }
    }
}

template <bool Upper, int64_t Diagonal, class T, auto S, Expression E> void triangular(TensorView<T, S> out, E x) {
    constexpr size_t columns = static_cast<size_t>(S[S.size() - 1]);
    constexpr size_t rows = static_cast<size_t>(S[S.size() - 2]);
    for (size_t i = 0; i < numel(S); ++i) {
        const int64_t offset = int64_t(i % columns) - int64_t(i / columns % rows);
        const bool keep = Upper ? offset >= Diagonal : offset <= Diagonal;
        out.data[i] = keep ? static_cast<T>(x[i]) : T(0);
    }
}

template <int Axis, class T, auto S, Expression E> void softmax(TensorView<T, S> out, E x) {
    static_assert(S == E::shape, "softmax keeps the shape");
    constexpr size_t width = static_cast<size_t>(S[Axis]);
    constexpr size_t inner = inner_size<S, Axis>();
    constexpr size_t lines = numel(S) / width;
    for (size_t line = 0; line < lines; ++line) {
        const size_t first = line / inner * width * inner + line % inner;
        float peak = -std::numeric_limits<float>::infinity();
        for (size_t k = 0; k < width; ++k) {
            peak = std::max(peak, float(x[first + k * inner]));
        }
        float total = 0;
        for (size_t k = 0; k < width; ++k) {
            const float term = std::exp(float(x[first + k * inner]) - peak);
            if constexpr (std::is_same_v<T, float>) {
                out.data[first + k * inner] = term;
            }
            total += term;
        }
        for (size_t k = 0; k < width; ++k) {
            if constexpr (std::is_same_v<T, float>) {
                out.data[first + k * inner] /= total;
            } else {
                out.data[first + k * inner] = std::exp(float(x[first + k * inner]) - peak) / total;
            }
        }
    }
}

template <int Axis, bool Largest, bool Sorted, class T, auto S, Expression E>
void topk(TensorView<T, S> values, TensorView<int64_t, S> indices, E x) {
    constexpr size_t width = static_cast<size_t>(E::shape[Axis]);
    constexpr size_t k = static_cast<size_t>(S[Axis]);
    constexpr size_t inner = inner_size<S, Axis>();
    static_assert(k <= width, "top-k selects at most the axis");
    // NaN outranks every number when selecting the largest and loses to every number otherwise.
    auto before = [](const std::pair<float, int64_t>& a, const std::pair<float, int64_t>& b) {
        if constexpr (Largest) {
            return (std::isnan(a.first) && !std::isnan(b.first)) || a.first > b.first;
        } else {
            return (!std::isnan(a.first) && std::isnan(b.first)) || a.first < b.first;
        }
    };
    std::array<std::pair<float, int64_t>, width> candidates;
    for (size_t line = 0; line < numel(S) / k; ++line) {
        const size_t source = line / inner * width * inner + line % inner;
        const size_t target = line / inner * k * inner + line % inner;
        for (size_t j = 0; j < width; ++j) {
            candidates[j] = {x[source + j * inner], static_cast<int64_t>(j)};
        }
        if constexpr (k * 64 <= width) {
            std::partial_sort(candidates.begin(), candidates.begin() + k, candidates.end(), before);
        } else {
            std::nth_element(candidates.begin(), candidates.begin() + k - 1, candidates.end(), before);
            if constexpr (Sorted) {
                std::sort(candidates.begin(), candidates.begin() + k - 1, before);
            }
        }
        for (size_t j = 0; j < k; ++j) {
            values.data[target + j * inner] = candidates[j].first;
            indices.data[target + j * inner] = candidates[j].second;
        }
    }
}

template <int Axis, size_t Start, class T, auto S, Expression E> void concat_part(TensorView<T, S> out, E x) {
    constexpr size_t inner = inner_size<S, Axis>();
    constexpr size_t block = static_cast<size_t>(E::shape[Axis]) * inner;
    constexpr size_t out_block = static_cast<size_t>(S[Axis]) * inner;
    for (size_t i = 0; i < numel(E::shape); ++i) {
        out.data[i / block * out_block + Start * inner + i % block] = x[i];
    }
}
}  // namespace chroma
