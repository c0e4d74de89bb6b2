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

// The same rounding for intermediate values on gfx950's v_cvt_pk_bf16_f32 (round to nearest even, like
// f32_to_bf16 for every value but NaN, which stays a NaN with another payload): one conversion and one
// shift instead of five integer operations. Stored results keep f32_to_bf16, whose NaN is always 0x7fc0.
__device__ __forceinline__ float round_bf16_fast(float value) { return float(__bf16(value)); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two intermediate values rounded the same way with one v_cvt_pk_bf16_f32, then widened back.
__device__ __forceinline__ void round_bf16_pair(float& x, float& y) {
    const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x, y}, bf16x2_t));
    x = __uint_as_float(w << 16);
    y = __uint_as_float(w & 0xffff0000u);
}

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
// Words that one workgroup hands to another within a kernel. A device-scope store writes through the
// XCD's L2 (``global_store ... sc1``) and a device-scope load does not take a stale L2 line, so once the
// storing thread's stores are complete (s_waitcnt vmcnt(0)) a later device-scope load in any workgroup
// sees them, without the whole-L2 write-back and invalidate of a device-scope fence. The handoff itself
// (a ticket) is a device-scope atomic taken after the stores complete.
template <class T> __device__ __forceinline__ void store_device(T* p, T v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
template <class T> __device__ __forceinline__ T load_device(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void device_stores_complete() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---------------------------------------------------------------------------------------------
// Cooperative row kernels (chroma_coop_*): P workgroups share each row of a wide row reduction, each
// keeping its part of the row in registers between the row's statistics and its normalisation, so the row
// is read from HBM once. Per row ("round") every part publishes N floats (its partial statistics) as 64-bit
// words, the float's bits and the round's tag (round + 1) side by side, each written by one device-scope
// atomic store, so a reader that sees the tag sees the float with it. The kernels publish round r before
// they wait for round r - 1 (so a round's exchange overlaps a whole row of work), so a part can run ahead:
// it publishes round r + 1 once it has read round r - 1, but round r + 2 only after it has read round r,
// which needs every part to have published r; a part can therefore publish round r + 4 only after every
// part has read round r (each reads round r before publishing r + 2). Rounds cycle through four slot sets,
// and a reader never takes a word of another round: tags are unique within a launch, and the last part of
// a group to finish the kernel returns the group's words to zero (the runtime zeroes the workspace at
// load and after a wait that gave up). The consumer requests the words before its next row's loads
// (vector loads complete in order, so it does not wait behind them) and checks the tags with a wave vote;
// it polls again only while a part is behind. The waits need all of the kernel's workgroups resident at
// once: the code generator launches at most one per compute unit, and the runtime refuses to load a
// cooperative grid the device cannot hold. A wait is bounded: after kCoopSpinLimit polls it sets
// kCoopTimeout in the error word and the kernel ends (the runtime then raises), so it cannot hang.
constexpr uint32_t kCoopDepartWord = 128;   // error-region words 128..191: per-group departure counters
constexpr uint32_t kCoopGroups = 64;
constexpr uint32_t kCoopTimeout = 2u;       // error-word bit of a cooperative wait that gave up
constexpr uint32_t kCoopSpinLimit = 1u << 21;

// Publish this part's N floats for ``round``: lanes 0 .. N - 1 of the first wave store one word each.
template <int P, int N>
__device__ __forceinline__ void coop_publish(unsigned long long* slots, uint32_t part, uint32_t round, const float (&mine)[N]) {
    static_assert(N >= 1 && N <= 2, "one or two floats per part");
    const uint32_t lane = threadIdx.x;
    if (lane < uint32_t(N)) {
        const float value = (N == 1 || lane == 0) ? mine[0] : mine[N - 1];
        const unsigned long long word = (static_cast<unsigned long long>(round + 1u) << 32) | __float_as_uint(value);
        store_device(slots + (round & 3u) * uint32_t(P * N) + part * uint32_t(N) + lane, word);
    }
}

// Request the words of ``round`` (lane i of the first wave: word i of the round's set), to be checked by
// ``coop_wait``; call before the next row's loads.
template <int P, int N>
__device__ __forceinline__ unsigned long long coop_peek(const unsigned long long* slots, uint32_t round) {
    static_assert(P * N <= 64, "one word per lane of a wave");
    const uint32_t lane = threadIdx.x;
    return lane < uint32_t(P * N) ? load_device(slots + (round & 3u) * uint32_t(P * N) + lane) : 0ull;
}

// Wait until every part's words of ``round`` carry its tag (polling again from ``word``, the lane's peeked
// word) and give every thread the floats in part order; false (and kCoopTimeout in the error word) if the
// wait gave up.
template <int P, int N>
__device__ __forceinline__ bool coop_wait(const unsigned long long* slots, uint32_t round, unsigned long long word, float (&all)[P][N],
                                          unsigned int* error) {
    __shared__ float shared_all[P * N];
    __shared__ int shared_ok;
    if (threadIdx.x < kWave) {
        const uint32_t lane = threadIdx.x;
        const unsigned int tag = round + 1u;
        uint32_t polls = 0;
        bool arrived = true;
        while (!__all(lane >= uint32_t(P * N) || uint32_t(word >> 32) == tag)) {
            if (++polls > kCoopSpinLimit) {
                arrived = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            word = coop_peek<P, N>(slots, round);
        }
        if (lane < uint32_t(P * N)) {
            shared_all[lane] = __uint_as_float(uint32_t(word));
        }
        if (lane == 0) {
            shared_ok = arrived;
            if (!arrived) {
                atomicOr(error, kCoopTimeout);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < P; ++q) {
#pragma unroll
        for (int n = 0; n < N; ++n) {
            all[q][n] = shared_all[q * N + n];
        }
    }
    const bool ok = shared_ok != 0;
    __syncthreads();  // shared_all is rewritten by the next round
    return ok;
}

// End of a cooperative kernel for one workgroup: the last part of the group to leave (every part has read
// every round by then) returns the group's words and its departure counter to zero for the next launch.
template <int P, int N>
__device__ __forceinline__ void coop_depart(unsigned long long* slots, unsigned int* depart) {
    __shared__ int last;
    __syncthreads();
    if (threadIdx.x == 0) {
        last = atomicAdd(depart, 1u) == uint32_t(P - 1);
    }
    __syncthreads();
    if (last) {
        for (uint32_t i = threadIdx.x; i < uint32_t(4 * P * N); i += blockDim.x) {
            store_device(slots + i, 0ull);
        }
        if (threadIdx.x == 0) {
            atomicExch(depart, 0u);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Reads ``bytes`` (a multiple of 16) at ``p`` and discards them: a weight stream of the next launch is then
// served from the memory-side cache (MALL) instead of HBM. A matrix-core product's copy ring has a few
// stages in flight, so with cold weights every stage waits for an HBM round trip (C5's QKV product: 81 us
// cold, 66 us warm); the read-ahead itself streams at HBM rate. Grid-stride, 16 bytes per thread per trip.
__device__ __forceinline__ void prefetch_bytes(const void* __restrict__ p, size_t bytes) {
    const uint4* v = static_cast<const uint4*>(p);
    const size_t count = bytes / 16u;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x) {
        const uint4 word = v[i];
        __asm__ volatile("" ::"v"(word.x), "v"(word.y), "v"(word.z), "v"(word.w));
    }
}

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
// Wave64 reductions; every lane receives the result. Within each 16-lane row the partners come from DPP
// (quad_perm [1,0,3,2] and [2,3,0,1], then row_half_mirror and row_mirror), so the exchange is folded
// into the add or max itself (``v_add_f32_dpp``) instead of a separate permute through the LDS
// crossbar; across rows gfx950's ``v_permlane16_swap`` and ``v_permlane32_swap`` exchange whole rows and
// half-waves in registers. Each step combines two equal-sized partial results, and both partners
// combine the same two values, so all 64 lanes end with bit-identical results.
template <int Control> __device__ __forceinline__ float dpp_partner(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Control, 0xF, 0xF, true));
}

template <class Op> __device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = op(v, dpp_partner<0xB1>(v));   // quad_perm [1,0,3,2]: lane ^ 1
    v = op(v, dpp_partner<0x4E>(v));   // quad_perm [2,3,0,1]: lane ^ 2
    v = op(v, dpp_partner<0x141>(v));  // row_half_mirror: the other quad of each 8 lanes
    v = op(v, dpp_partner<0x140>(v));  // row_mirror: the other half of each 16-lane row
    const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(rows[0]), __uint_as_float(rows[1]));  // rows 0+1 and 2+3
    const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(halves[0]), __uint_as_float(halves[1]));  // lanes 0-31 + 32-63
}

// Workgroup barrier that publishes LDS only: the fences are restricted to the local address space, so
// the wait before the barrier is lgkmcnt(0) and global loads still in flight (a weight stream requested
// ahead of a staging prologue) are not waited for. For code whose threads exchange data through LDS only.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float wave_sum(float v) {
    return wave_reduce(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_max(float v) {
    return wave_reduce(v, [](float a, float b) { return __builtin_fmaxf(a, b); });
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
