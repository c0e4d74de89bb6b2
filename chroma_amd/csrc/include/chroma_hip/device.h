// Device-side building blocks shared by every generated gfx950 kernel of the hip backend:
// bfloat16 storage rounding, checked gather indices, the transcendental functions used by fused
// elementwise chains, and wave64 / workgroup reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace chroma {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------------
// bfloat16: round to nearest even, every NaN becomes 0x7fc0, widening is a 16-bit shift. Bit-for-bit
// the host rule (chroma/_src/core/bfloat16.h:7-17).
__device__ __forceinline__ float bf16_to_f32(uint16_t bits) { return __uint_as_float(uint32_t(bits) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float value) {
    const uint32_t word = __float_as_uint(value);
    if ((word & 0x7fffffffu) > 0x7f800000u) {
        return 0x7fc0;
    }
    return uint16_t((word + 0x7fffu + ((word >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float round_bf16(float value) { return bf16_to_f32(f32_to_bf16(value)); }

// ---------------------------------------------------------------------------------------------
// Gather row index with the reference's bounds rule (chroma/_src/codegen/cuda/runtime.h:18-32):
// an index outside [0, count) - or outside [-count, count) when negative indices are allowed - raises
// the program's error word and reads row 0 instead.
__device__ __forceinline__ uint64_t checked_index(int64_t value, uint64_t count, bool negative, unsigned int* error) {
    if (value >= 0) {
        if (uint64_t(value) < count) {
            return uint64_t(value);
        }
    } else if (negative) {
        const uint64_t distance = uint64_t(-(value + 1)) + 1;
        if (distance <= count) {
            return count - distance;
        }
    }
    atomicOr(error, 1u);
    return 0;
}

// ---------------------------------------------------------------------------------------------
// Transcendentals for fused chains. These use the hardware exp2 / reciprocal units instead of the
// correctly-rounded library routines, which cost 3-5x the instructions and would make bandwidth-bound
// chains compute-bound. Error bounds (relative, fp32):
//   exp(x):      <= 1.2e-7 + 6e-8 * |x|   (argument rounding of x*log2(e), then v_exp_f32's 1 ulp)
//   sigmoid(x):  <= 3e-7
//   tanh(x):     <= 3e-7 absolute for |x| >= 0.05; below that an odd Taylor polynomial, <= 1e-9 relative
// All propagate NaN and saturate correctly at +-inf; results below ~1e-38 may flush to zero.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float fast_sigmoid(float x) { return fast_rcp(1.0f + fast_exp(-x)); }

__device__ __forceinline__ float fast_tanh(float x) {
    const float magnitude = __builtin_fabsf(x);
    const float square = x * x;
    const float series = x * __builtin_fmaf(square, __builtin_fmaf(square, 0.133333333f, -0.333333333f), 1.0f);
    // 1 - 2 / (exp(2|x|) + 1), sign restored: exact limits at +-inf, NaN passes through.
    const float wide = 1.0f - 2.0f * fast_rcp(fast_exp(2.0f * magnitude) + 1.0f);
    const float signed_wide = __builtin_copysignf(wide, x);
    return magnitude < 0.05f ? series : signed_wide;
}

__device__ __forceinline__ float fast_silu(float x) { return x * fast_sigmoid(x); }

// ---------------------------------------------------------------------------------------------
// Streaming (non-temporal) vector stores for results no later instruction of the same kernel reads.
typedef float float2_nt __attribute__((ext_vector_type(2)));
typedef float float4_nt __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_streaming4(float* p, float a, float b, float c, float d) {
    __builtin_nontemporal_store(float4_nt{a, b, c, d}, reinterpret_cast<float4_nt*>(p));
}

__device__ __forceinline__ void store_streaming2(float* p, float a, float b) {
    __builtin_nontemporal_store(float2_nt{a, b}, reinterpret_cast<float2_nt*>(p));
}

// Streaming (non-temporal) vector loads for operands a kernel reads once: they are not kept in L2 or the
// last-level cache, which leaves those to the data that is reused.
typedef unsigned int uint2_nt __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float4_nt load_streaming4(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const float4_nt*>(p));
}

__device__ __forceinline__ float2_nt load_streaming2(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const float2_nt*>(p));
}

typedef unsigned int uint4_nt __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4_nt load_streaming_bf16x8(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint4_nt*>(p));
}

__device__ __forceinline__ uint2_nt load_streaming_bf16x4(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint2_nt*>(p));
}

__device__ __forceinline__ uint32_t load_streaming_bf16x2(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// ---------------------------------------------------------------------------------------------
// Wave64 reductions (butterfly over all 64 lanes; every lane receives the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        v += __shfl_xor(v, offset, kWave);
    }
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        v = __builtin_fmaxf(v, __shfl_xor(v, offset, kWave));
    }
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        const uint32_t lo = __shfl_xor(uint32_t(v), offset, kWave);
        const uint32_t hi = __shfl_xor(uint32_t(v >> 32), offset, kWave);
        const uint64_t other = (uint64_t(hi) << 32) | lo;
        v = other > v ? other : v;
    }
    return v;
}

// Workgroup reductions for Waves wave64 waves; ``scratch`` holds at least Waves floats of LDS.
template <int Waves> __device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    if constexpr (Waves > 1) {
        const int wave = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0) {
            scratch[wave] = v;
        }
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < Waves; ++w) {
            total += scratch[w];
        }
        __syncthreads();
        v = total;
    }
    return v;
}

template <int Waves> __device__ __forceinline__ float block_max(float v, float* scratch) {
    v = wave_max(v);
    if constexpr (Waves > 1) {
        const int wave = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0) {
            scratch[wave] = v;
        }
        __syncthreads();
        float best = scratch[0];
#pragma unroll
        for (int w = 1; w < Waves; ++w) {
            best = __builtin_fmaxf(best, scratch[w]);
        }
        __syncthreads();
        v = best;
    }
    return v;
}

// Top-k selection key: larger key = selected earlier. ``largest`` ranks NaN above every number,
// smallest-first ranks it below; ties go to the lower index (the low 32 bits hold ~index).
__device__ __forceinline__ uint64_t topk_key(float value, uint32_t index, bool largest) {
    const float canonical = value + 0.0f;  // -0 and +0 tie, as they compare equal
    const uint32_t bits = __float_as_uint(canonical);
    uint32_t order = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    const bool nan = __builtin_isnan(value);
    if (largest) {
        order = nan ? 0xffffffffu : order;
    } else {
        order = nan ? 0u : ~order;
    }
    return (uint64_t(order) << 32) | uint64_t(0xffffffffu - index);
}

}  // namespace chroma
