// ORACLE (test infrastructure only): compile-time shapes and broadcasting for the CPU restatement.
// Semantics of chroma/_src/core/layout.h:8-50: ``dims<...>`` is a constexpr std::array of extents,
// broadcasting right-aligns shapes and a size-1 extent repeats.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>

namespace chroma {
template <int64_t... Extents>
inline constexpr std::array<int64_t, sizeof...(Extents)> dims{Extents...};

template <class Shape> constexpr size_t numel(const Shape& shape) {
    size_t count = 1;
    for (auto extent : shape) {
        count *= static_cast<size_t>(extent);
    }
    return count;
}

template <auto A, auto B> consteval auto broadcast_shape() {
    constexpr size_t rank = A.size() < B.size() ? B.size() : A.size();
    std::array<int64_t, rank> shape{};
    for (size_t d = 0; d < rank; ++d) {
        const size_t from_end = rank - 1 - d;
        const int64_t a = from_end < A.size() ? A[A.size() - 1 - from_end] : 1;
        const int64_t b = from_end < B.size() ? B[B.size() - 1 - from_end] : 1;
        if (a != 1 && b != 1 && a != b) {
            throw "broadcast: incompatible extents";
        }
        shape[d] = a == 1 ? b : a;
    }
    return shape;
}

// Flat index into a tensor of shape From for flat index ``i`` of the broadcast result shape To.
template <auto From, auto To> inline size_t broadcast_index(size_t i) {
    if constexpr (From.size() == To.size()) {
        if constexpr (From == To) {
            return i;
        }
    }
    {
        constexpr size_t pad = To.size() - From.size();
        size_t offset = 0;
        size_t stride = 1;
        for (size_t d = To.size(); d-- > 0;) {
            const size_t coordinate = i % static_cast<size_t>(To[d]);
            i /= static_cast<size_t>(To[d]);
            if (d >= pad) {
                const size_t extent = static_cast<size_t>(From[d - pad]);
                offset += extent == 1 ? 0 : coordinate * stride;
                stride *= extent;
            }
        }
        return offset;
    }
}
}  // namespace chroma
