// Matrix kernels of the hip backend (the replacement for the reference's cuBLAS Sgemm path,
// chroma/_src/codegen/cuda/runtime.h:175-181): Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]), row-major,
// float32 or bfloat16 storage, float32 accumulation, bias added to the finished sum.
#pragma once

#include "device.h"

namespace chroma {

template <class T> struct Vec4;
template <> struct Vec4<float> {
    static __device__ __forceinline__ float4 load(const float* p) { return *reinterpret_cast<const float4*>(p); }
};
template <> struct Vec4<uint16_t> {
    static __device__ __forceinline__ float4 load(const uint16_t* p) {
        const uint2 raw = *reinterpret_cast<const uint2*>(p);
        return float4{bf16_to_f32(uint16_t(raw.x & 0xffffu)), bf16_to_f32(uint16_t(raw.x >> 16)),
                      bf16_to_f32(uint16_t(raw.y & 0xffffu)), bf16_to_f32(uint16_t(raw.y >> 16))};
    }
};

template <class T> __device__ __forceinline__ float load1(const T* p);
template <> __device__ __forceinline__ float load1<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float load1<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

template <class T> __device__ __forceinline__ void store1(T* p, float v);
template <> __device__ __forceinline__ void store1<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void store1<uint16_t>(uint16_t* p, float v) { *p = f32_to_bf16(v); }

__device__ __forceinline__ float dot4(float acc, float4 a, float4 b) {
    acc = __builtin_fmaf(a.x, b.x, acc);
    acc = __builtin_fmaf(a.y, b.y, acc);
    acc = __builtin_fmaf(a.z, b.z, acc);
    acc = __builtin_fmaf(a.w, b.w, acc);
    return acc;
}

// Skinny product for few rows of X (M <= 16): memory-bound on W, which is streamed once with 128-bit
// loads. A wave covers 64 / LPR rows of W at a time; LPR lanes split K in 4-element pieces, each lane
// holding its slice of every X row in registers when that fits. Partial sums meet through a
// butterfly over the LPR lanes; the first lane of each row group adds the bias and stores.
// ``wave`` / ``waves`` enumerate the waves cooperating on this product.
template <int M, int K, int LPR, class T>
__device__ __forceinline__ void dot_rows(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                         T* __restrict__ out, uint32_t out_stride, uint32_t rows, uint32_t wave,
                                         uint32_t waves) {
    constexpr int G = kWave / LPR;
    constexpr int STEPS = K / (4 * LPR);
    static_assert(K % (4 * LPR) == 0, "K must split into 4-element pieces per lane");
    constexpr bool CACHE_X = STEPS * M <= 16;
    constexpr int UNROLL = STEPS >= 4 ? 1 : (STEPS >= 2 ? 2 : 4);
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t group = lane / LPR;
    const uint32_t sub = lane % LPR;

    float4 xr[CACHE_X ? STEPS : 1][CACHE_X ? M : 1];
    if constexpr (CACHE_X) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                xr[s][m] = Vec4<T>::load(x + size_t(m) * K + (s * LPR + sub) * 4);
            }
        }
    }
    for (uint32_t base = wave * G * UNROLL; base < rows; base += waves * G * UNROLL) {
        float acc[UNROLL][M];
        float4 wv[UNROLL][STEPS];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint32_t row = base + u * G + group;
            const uint32_t safe = row < rows ? row : rows - 1;
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                wv[u][s] = Vec4<T>::load(w + size_t(safe) * K + (s * LPR + sub) * 4);
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float a = 0.0f;
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    const float4 xv = CACHE_X ? xr[CACHE_X ? s : 0][CACHE_X ? m : 0]
                                              : Vec4<T>::load(x + size_t(m) * K + (s * LPR + sub) * 4);
                    a = dot4(a, wv[u][s], xv);
                }
                acc[u][m] = a;
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
#pragma unroll
                for (int offset = LPR / 2; offset > 0; offset >>= 1) {
                    acc[u][m] += __shfl_xor(acc[u][m], offset, kWave);
                }
            }
            const uint32_t row = base + u * G + group;
            if (sub == 0 && row < rows) {
                const float b = bias ? load1<T>(bias + row) : 0.0f;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    store1<T>(out + size_t(m) * out_stride + row, acc[u][m] + b);
                }
            }
        }
    }
}

template <int M, int K, int LPR, class T>
__device__ __forceinline__ void skinny_linear(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                              T* __restrict__ out, uint32_t n) {
    const uint32_t waves_per_block = blockDim.x / kWave;
    const uint32_t wave = blockIdx.x * waves_per_block + threadIdx.x / kWave;
    dot_rows<M, K, LPR, T>(x, w, bias, out, n, n, wave, gridDim.x * waves_per_block);
}

// Selected-expert products: out[slot, :] = W[expert(slot)] . x[token or slot]^T for every (token, slot)
// pair, reading the chosen expert's [C, K] slab in place (the reference's expert_linear,
// chroma/_src/codegen/cpu/kernels.h:76-99). Indices wrap when negative; an index outside
// [-experts, experts) raises the error word and reads expert 0. grid.y enumerates the slots.
template <int K, int LPR, class T, bool PER_SLOT_INPUT>
__device__ __forceinline__ void expert_linear(const T* __restrict__ w, const int64_t* __restrict__ indices,
                                              const T* __restrict__ x, T* __restrict__ out, uint32_t selected,
                                              uint32_t experts, uint32_t channels, uint32_t blocks_per_slot,
                                              unsigned int* error) {
    const uint32_t slot = blockIdx.y;
    const uint32_t token = slot / selected;
    const uint64_t expert = checked_index(indices[slot], experts, true, error);
    const T* slab = w + expert * uint64_t(channels) * K;
    const T* row = x + uint64_t(PER_SLOT_INPUT ? slot : token) * K;
    const uint32_t waves_per_block = blockDim.x / kWave;
    const uint32_t wave = blockIdx.x * waves_per_block + threadIdx.x / kWave;
    dot_rows<1, K, LPR, T>(row, slab, nullptr, out + uint64_t(slot) * channels, channels, channels, wave,
                           blocks_per_slot * waves_per_block);
}

// General product for larger M: 64 x 64 output tiles, K staged through LDS 16 at a time, each of the
// 256 threads accumulating a 4 x 4 block in registers.
template <class T>
__device__ __forceinline__ void tiled_linear(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                             T* __restrict__ out, uint32_t m_total, uint32_t n_total, uint32_t k_total) {
    __shared__ float xs[16][64 + 4];
    __shared__ float ws[16][64 + 4];
    const uint32_t n0 = blockIdx.x * 64u;
    const uint32_t m0 = blockIdx.y * 64u;
    const uint32_t tx = threadIdx.x % 16u;
    const uint32_t ty = threadIdx.x / 16u;
    float acc[4][4] = {};
    for (uint32_t k0 = 0; k0 < k_total; k0 += 16u) {
#pragma unroll
        for (uint32_t i = threadIdx.x; i < 1024u; i += 256u) {
            const uint32_t r = i / 16u, c = i % 16u;
            const uint32_t gk = k0 + c;
            const uint32_t gm = m0 + r, gn = n0 + r;
            xs[c][r] = (gm < m_total && gk < k_total) ? load1<T>(x + size_t(gm) * k_total + gk) : 0.0f;
            ws[c][r] = (gn < n_total && gk < k_total) ? load1<T>(w + size_t(gn) * k_total + gk) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t kk = 0; kk < 16u; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = xs[kk][ty * 4 + i];
                b[i] = ws[kk][tx * 4 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t gm = m0 + ty * 4 + i;
        if (gm >= m_total) {
            continue;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t gn = n0 + tx * 4 + j;
            if (gn < n_total) {
                const float b = bias ? load1<T>(bias + gn) : 0.0f;
                store1<T>(out + size_t(gm) * n_total + gn, acc[i][j] + b);
            }
        }
    }
}

}  // namespace chroma
