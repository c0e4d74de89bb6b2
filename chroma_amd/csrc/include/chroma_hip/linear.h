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

// ---------------------------------------------------------------------------------------------
// Matrix-core product for bfloat16: Y[M, N] = X[M, K] . W[N, K]^T (+ bias), float32 accumulation in
// the MFMA accumulators, one bfloat16 rounding of (sum + bias) at the end - the reference's bf16 linear
// numerics (chroma/_src/codegen/cpu/kernels.h:63-74) with a different summation order.
//
// Workgroup: 256 threads = 4 waves, a 128 x 128 output tile, K staged through LDS 32 at a time
// (rows padded by 8 elements against bank conflicts), double-buffered: the next K slice is loaded from
// HBM into registers while the current one feeds the matrix cores. Each wave owns a 64 x 64 quadrant
// as 4 x 4 tiles of v_mfma_f32_16x16x32_bf16. Operand layout of that instruction on gfx950: lane l
// supplies A[row l % 16][k 8 * (l / 16) .. + 7] and B[k 8 * (l / 16) .. + 7][column l % 16]; it receives
// D[rows 4 * (l / 16) .. + 3][column l % 16]. K must be a multiple of 8 (16-byte rows).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void mfma_linear_bf16(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                 const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
                                                 uint32_t m_total, uint32_t n_total, uint32_t k_total) {
    constexpr int BM = 128, BN = 128, BK = 32, PAD = 8, LD = BK + PAD;
    __shared__ __attribute__((aligned(16))) uint16_t as[2][BM * LD];
    __shared__ __attribute__((aligned(16))) uint16_t bs[2][BN * LD];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % 64u, wave = tid / 64u;
    const uint32_t wm = wave / 2u, wn = wave % 2u;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    // Global -> register staging: 512 chunks of 8 elements per operand tile, two per thread.
    uint4 ra[2], rb[2];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t chunk = tid + i * 256u;
            const uint32_t row = chunk / 4u, kc = (chunk % 4u) * 8u;
            const uint32_t gk = k0 + kc;
            const uint32_t gm = m0 + row, gn = n0 + row;
            ra[i] = (gm < m_total && gk < k_total) ? *reinterpret_cast<const uint4*>(x + size_t(gm) * k_total + gk) : uint4{0, 0, 0, 0};
            rb[i] = (gn < n_total && gk < k_total) ? *reinterpret_cast<const uint4*>(w + size_t(gn) * k_total + gk) : uint4{0, 0, 0, 0};
        }
    };
    auto stash = [&](int buffer) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t chunk = tid + i * 256u;
            const uint32_t row = chunk / 4u, kc = (chunk % 4u) * 8u;
            *reinterpret_cast<uint4*>(&as[buffer][row * LD + kc]) = ra[i];
            *reinterpret_cast<uint4*>(&bs[buffer][row * LD + kc]) = rb[i];
        }
    };

    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    const uint32_t steps = (k_total + BK - 1) / BK;
    fetch(0);
    stash(0);
    __syncthreads();
    for (uint32_t step = 0; step < steps; ++step) {
        const int buffer = step & 1;
        if (step + 1 < steps) {
            fetch((step + 1) * BK);
        }
        bf16x8_t a[4], b[4];
        const uint32_t koff = (lane / 16u) * 8u;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t arow = wm * 64u + t * 16u + lane % 16u;
            const uint32_t brow = wn * 64u + t * 16u + lane % 16u;
            a[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&as[buffer][arow * LD + koff]));
            b[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&bs[buffer][brow * LD + koff]));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
        if (step + 1 < steps) {
            stash(buffer ^ 1);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t gn = n0 + wn * 64u + j * 16u + lane % 16u;
            if (gn >= n_total) {
                continue;
            }
            const float b = bias ? bf16_to_f32(bias[gn]) : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm * 64u + i * 16u + (lane / 16u) * 4u + r;
                if (gm < m_total) {
                    out[size_t(gm) * n_total + gn] = f32_to_bf16(acc[i][j][r] + b);
                }
            }
        }
    }
}

// Matrix-core product for float32 (v_mfma_f32_16x16x4_f32): same tiling as the bfloat16 kernel with K
// staged 16 at a time; lane l supplies A[row l % 16][k l / 16] and B[k l / 16][column l % 16] of each
// 4-deep step. K must be a multiple of 4 (16-byte rows). The bias is added to the finished sum, as the
// reference's float linear does after its GEMM (chroma/_src/codegen/cpu/kernels.h:46-61).
__device__ __forceinline__ void mfma_linear_f32(const float* __restrict__ x, const float* __restrict__ w,
                                                const float* __restrict__ bias, float* __restrict__ out,
                                                uint32_t m_total, uint32_t n_total, uint32_t k_total) {
    constexpr int BM = 128, BN = 128, BK = 16, PAD = 4, LD = BK + PAD;
    __shared__ __attribute__((aligned(16))) float as[2][BM * LD];
    __shared__ __attribute__((aligned(16))) float bs[2][BN * LD];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % 64u, wave = tid / 64u;
    const uint32_t wm = wave / 2u, wn = wave % 2u;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    float4 ra[2], rb[2];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t chunk = tid + i * 256u;
            const uint32_t row = chunk / 4u, kc = (chunk % 4u) * 4u;
            const uint32_t gk = k0 + kc;
            const uint32_t gm = m0 + row, gn = n0 + row;
            ra[i] = (gm < m_total && gk < k_total) ? *reinterpret_cast<const float4*>(x + size_t(gm) * k_total + gk) : float4{0, 0, 0, 0};
            rb[i] = (gn < n_total && gk < k_total) ? *reinterpret_cast<const float4*>(w + size_t(gn) * k_total + gk) : float4{0, 0, 0, 0};
        }
    };
    auto stash = [&](int buffer) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t chunk = tid + i * 256u;
            const uint32_t row = chunk / 4u, kc = (chunk % 4u) * 4u;
            *reinterpret_cast<float4*>(&as[buffer][row * LD + kc]) = ra[i];
            *reinterpret_cast<float4*>(&bs[buffer][row * LD + kc]) = rb[i];
        }
    };

    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    const uint32_t steps = (k_total + BK - 1) / BK;
    fetch(0);
    stash(0);
    __syncthreads();
    for (uint32_t step = 0; step < steps; ++step) {
        const int buffer = step & 1;
        if (step + 1 < steps) {
            fetch((step + 1) * BK);
        }
#pragma unroll
        for (int s = 0; s < BK / 4; ++s) {
            const uint32_t k = s * 4u + lane / 16u;
            float a[4], b[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                a[t] = as[buffer][(wm * 64u + t * 16u + lane % 16u) * LD + k];
                b[t] = bs[buffer][(wn * 64u + t * 16u + lane % 16u) * LD + k];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (step + 1 < steps) {
            stash(buffer ^ 1);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t gn = n0 + wn * 64u + j * 16u + lane % 16u;
            if (gn >= n_total) {
                continue;
            }
            const float b = bias ? bias[gn] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm * 64u + i * 16u + (lane / 16u) * 4u + r;
                if (gm < m_total) {
                    out[size_t(gm) * n_total + gn] = acc[i][j][r] + b;
                }
            }
        }
    }
}

}  // namespace chroma
