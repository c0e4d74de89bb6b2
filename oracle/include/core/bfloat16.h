// ORACLE (test infrastructure only): bfloat16 storage type of the CPU restatement.
// Round-to-nearest-even from float, every NaN -> 0x7fc0, widening by a 16-bit shift; the rule of
// chroma/_src/core/bfloat16.h:7-17. Type and member names match it so generated oracle code compiles
// against either header set.
#pragma once

#include <cstdint>
#include <cstring>

namespace chroma {
struct bfloat16_t {
    uint16_t bits;

    bfloat16_t() = default;
    constexpr bfloat16_t(float value) : bits(round(value)) {}
    constexpr operator float() const { return widen(bits); }

    static constexpr uint16_t round(float value) {
        const uint32_t word = __builtin_bit_cast(uint32_t, value);
        if ((word & 0x7fffffffu) > 0x7f800000u) {
            return 0x7fc0;
        }
        const uint32_t bias = 0x7fffu + ((word >> 16) & 1u);
        return static_cast<uint16_t>((word + bias) >> 16);
    }
    static constexpr float widen(uint16_t bits) { return __builtin_bit_cast(float, uint32_t{bits} << 16); }
};
static_assert(sizeof(bfloat16_t) == 2, "bfloat16_t is two bytes");
}  // namespace chroma
