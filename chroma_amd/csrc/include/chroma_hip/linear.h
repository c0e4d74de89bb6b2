// Matrix kernels of the hip backend (the replacement for the reference's cuBLAS Sgemm path,
// chroma/_src/codegen/cuda/runtime.h:175-181): Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]), row-major,
// float32 or bfloat16 storage, float32 accumulation, bias added to the finished sum.
#pragma once

#include <type_traits>
#include <utility>

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

// The storage value of v (rounded to bfloat16 for uint16_t storage) and its widening back to float.
template <class T> __device__ __forceinline__ T storage_of(float v);
template <> __device__ __forceinline__ float storage_of<float>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t storage_of<uint16_t>(float v) { return f32_to_bf16(v); }
template <class T> __device__ __forceinline__ float widen_of(T v);
template <> __device__ __forceinline__ float widen_of<float>(float v) { return v; }
template <> __device__ __forceinline__ float widen_of<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

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

// Streaming products for few rows of X: Y[m, n] = X[m, :] . W[n, :] (+ bias[n]) with every byte of W read
// once through 16-byte non-temporal loads (the weight read is the whole cost of these products). LPR
// lanes share one row of W, each holding PER_LANE 16-byte chunks; a wave covers 64 / LPR rows per step
// and ROWS steps at once, and every chunk of those rows is requested before any arithmetic, so about
// PER_LANE * ROWS * 1 KiB per wave is in flight. X is widened to float in LDS (``xs``, M * K floats) when
// the caller provides it, else read through the cache. Partial sums meet through a butterfly over the
// LPR lanes; the first lane of each row adds the bias and stores.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

template <class T> struct Chunk16;
template <> struct Chunk16<float> {
    static constexpr int N = 4;
    static __device__ __forceinline__ u32x4_t load(const float* p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)); }
    static __device__ __forceinline__ float get(const u32x4_t& c, int e) { return __uint_as_float(c[e]); }
};
template <> struct Chunk16<uint16_t> {
    static constexpr int N = 8;
    static __device__ __forceinline__ u32x4_t load(const uint16_t* p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)); }
    static __device__ __forceinline__ float get(const u32x4_t& c, int e) {
        return __uint_as_float((e & 1) ? (c[e / 2] & 0xffff0000u) : (c[e / 2] << 16));
    }
};

// One step of ``stream_rows`` for one lane: its 16-byte chunks of ROWS rows of W, all requested before
// any arithmetic. A kernel may request its first step before its prologue (see ``stream_linear_fetch``),
// so the weight read overlaps the evaluation of X into LDS.
// A row of CHUNKS 16-byte chunks need not split evenly over the LPR lanes (RAGGED): the last of a lane's
// PER_LANE chunks is then past the row's end for some lanes, which load another chunk of the same row
// instead and leave it out of the arithmetic (``live``).
template <int K, int LPR, int ROWS, class T>
struct StreamStep {
    static constexpr int N = Chunk16<T>::N;
    static constexpr int CHUNKS = K / N;
    static constexpr int PER_LANE = (CHUNKS + LPR - 1) / LPR;
    static constexpr bool RAGGED = CHUNKS % LPR != 0;
    static constexpr int G = kWave / LPR;
    static_assert(K % N == 0, "rows must split into 16-byte chunks");
    u32x4_t chunks[ROWS][PER_LANE];

    // whether chunk c of this lane (sub = lane % LPR) lies in the row
    static __device__ __forceinline__ bool live(int c, uint32_t sub) { return !RAGGED || c + 1 < PER_LANE || c * LPR + sub < uint32_t(CHUNKS); }

    __device__ __forceinline__ void fetch(const T* __restrict__ w, uint32_t base, uint32_t rows) {
        const uint32_t lane = threadIdx.x % kWave;
        const uint32_t group = lane / LPR, sub = lane % LPR;
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint32_t row = base + r * G + group;
            const uint32_t safe = row < rows ? row : rows - 1;
#pragma unroll
            for (int c = 0; c < PER_LANE; ++c) {
                const uint32_t chunk = live(c, sub) ? c * LPR + sub : sub;
                chunks[r][c] = Chunk16<T>::load(w + size_t(safe) * K + chunk * N);
            }
        }
    }
};

template <int M, int K, int LPR, int ROWS, bool STAGED, bool PREFETCHED, class T>
__device__ __forceinline__ void stream_rows(const T* __restrict__ x, const float* xs, const T* __restrict__ w, const T* __restrict__ bias,
                                            T* __restrict__ out, uint32_t out_stride, uint32_t rows, uint32_t wave, uint32_t waves,
                                            StreamStep<K, LPR, ROWS, T>* first) {
    using C = Chunk16<T>;
    using Step = StreamStep<K, LPR, ROWS, T>;
    constexpr int PER_LANE = Step::PER_LANE;
    constexpr int G = Step::G;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t group = lane / LPR;
    const uint32_t sub = lane % LPR;
    auto xv = [&](int m, uint32_t k) -> float {
        if constexpr (STAGED) {
            return xs[m * K + k];
        } else {
            return load1<T>(x + size_t(m) * K + k);
        }
    };
    uint32_t base = wave * G * ROWS;
    if (base >= rows) {
        return;
    }
    Step local;
    Step& step = PREFETCHED ? *first : local;  // the prefetched step is used (and refilled) in place
    if constexpr (!PREFETCHED) {
        step.fetch(w, base, rows);
    }
    for (;;) {
        // Keep X's values from being hoisted out of this loop: they would take K registers per lane
        // (LDS or cache reads are cheap to repeat; registers are needed for the chunks in flight).
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            float acc[M];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                acc[m] = 0.0f;
            }
#pragma unroll
            for (int c = 0; c < PER_LANE; ++c) {
                if (!Step::live(c, sub)) {
                    continue;  // past the row's end (ragged rows only)
                }
                const uint32_t k0 = (c * LPR + sub) * C::N;
#pragma unroll
                for (int e = 0; e < C::N; ++e) {
                    const float wv = C::get(step.chunks[r][c], e);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        acc[m] += wv * xv(m, k0 + e);
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
#pragma unroll
                for (int offset = LPR / 2; offset > 0; offset >>= 1) {
                    acc[m] += __shfl_xor(acc[m], offset, kWave);
                }
            }
            const uint32_t row = base + r * G + group;
            if (sub == 0 && row < rows) {
                const float b = bias ? load1<T>(bias + row) : 0.0f;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    store1<T>(out + size_t(m) * out_stride + row, acc[m] + b);
                }
            }
        }
        base += waves * G * ROWS;
        if (base >= rows) {
            break;
        }
        step.fetch(w, base, rows);
    }
}

// Y = X . W^T (+ bias) for M <= 16 rows of X through ``stream_rows``; with STAGED, ``xs`` is an LDS array of
// M * K floats that already holds X (the caller's generated code widens X, or evaluates the fused
// expression X stands for, into it and synchronizes). With ``first``, this wave's first step was
// requested by ``stream_linear_fetch`` before the prologue.
template <int K, int LPR, int ROWS, class T>
__device__ __forceinline__ void stream_linear_fetch(StreamStep<K, LPR, ROWS, T>& first, const T* __restrict__ w, uint32_t n) {
    const uint32_t wave = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    const uint32_t base = wave * StreamStep<K, LPR, ROWS, T>::G * ROWS;
    if (base < n) {
        first.fetch(w, base, n);
    }
}

template <int M, int K, int LPR, int ROWS, bool STAGED, class T>
__device__ __forceinline__ void stream_linear(const T* __restrict__ x, const float* xs, const T* __restrict__ w, const T* __restrict__ bias,
                                              T* __restrict__ out, uint32_t n) {
    const uint32_t waves_per_block = blockDim.x / kWave;
    const uint32_t wave = blockIdx.x * waves_per_block + threadIdx.x / kWave;
    stream_rows<M, K, LPR, ROWS, STAGED, false, T>(x, xs, w, bias, out, n, n, wave, gridDim.x * waves_per_block, nullptr);
}

// (The prefetched step is passed by reference and never compared with null: a private-memory address
// in a comparison keeps the step out of registers.)
template <int M, int K, int LPR, int ROWS, bool STAGED, class T>
__device__ __forceinline__ void stream_linear(const T* __restrict__ x, const float* xs, const T* __restrict__ w, const T* __restrict__ bias,
                                              T* __restrict__ out, uint32_t n, StreamStep<K, LPR, ROWS, T>& first) {
    const uint32_t waves_per_block = blockDim.x / kWave;
    const uint32_t wave = blockIdx.x * waves_per_block + threadIdx.x / kWave;
    stream_rows<M, K, LPR, ROWS, STAGED, true, T>(x, xs, w, bias, out, n, n, wave, gridDim.x * waves_per_block, &first);
}

// The same product by one workgroup alone (its waves split the rows of W), as the epilogue of a kernel
// that has just produced X in LDS; ``stream_block_fetch`` requests each wave's first step early.
template <int K, int LPR, int ROWS, class T>
// The waves of the grid.z parts of one workgroup position share W's rows: wave w of part p is wave
// p * (waves per workgroup) + w of gridDim.z * (waves per workgroup).
__device__ __forceinline__ void stream_block_fetch(StreamStep<K, LPR, ROWS, T>& first, const T* __restrict__ w, uint32_t n) {
    const uint32_t wave = blockIdx.z * (blockDim.x / kWave) + threadIdx.x / kWave;
    const uint32_t base = wave * StreamStep<K, LPR, ROWS, T>::G * ROWS;
    if (base < n) {
        first.fetch(w, base, n);
    }
}

template <int M, int K, int LPR, int ROWS, bool STAGED, class T>
__device__ __forceinline__ void stream_block_linear(const T* __restrict__ x, const float* xs, const T* __restrict__ w, const T* __restrict__ bias,
                                                    T* __restrict__ out, uint32_t n, StreamStep<K, LPR, ROWS, T>& first) {
    const uint32_t per_block = blockDim.x / kWave;
    stream_rows<M, K, LPR, ROWS, STAGED, true, T>(x, xs, w, bias, out, n, n, blockIdx.z * per_block + threadIdx.x / kWave,
                                                  gridDim.z * per_block, &first);
}

// Selected-expert products through ``stream_rows``: out[slot, :] = W[expert(slot)] . x[token or slot]^T,
// reading the chosen expert's [C, K] slab in place (the reference's expert_linear,
// chroma/_src/codegen/cpu/kernels.h:76-99). Indices wrap when negative; an index outside
// [-experts, experts) raises the error word and reads expert 0. grid.y enumerates the slots.
// With STAGED, ``xs`` already holds this slot's input row (K floats, written by the caller); with
// ``first``, this wave's first step of the slab was requested by ``stream_expert_fetch``.
template <int K, int LPR, int ROWS, class T>
__device__ __forceinline__ void stream_expert_fetch(StreamStep<K, LPR, ROWS, T>& first, const T* __restrict__ w, const int64_t* __restrict__ indices,
                                                    uint32_t experts, uint32_t channels, unsigned int* error) {
    const uint64_t expert = checked_index(indices[blockIdx.y], experts, true, error);
    const uint32_t wave = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    const uint32_t base = wave * StreamStep<K, LPR, ROWS, T>::G * ROWS;
    if (base < channels) {
        first.fetch(w + expert * uint64_t(channels) * K, base, channels);
    }
}

template <int K, int LPR, int ROWS, bool STAGED, class T, bool PER_SLOT_INPUT, bool PREFETCHED = false>
__device__ __forceinline__ void stream_expert_rows(const T* __restrict__ w, const int64_t* __restrict__ indices, const T* __restrict__ x,
                                                   const float* xs, T* __restrict__ out, uint32_t selected, uint32_t experts, uint32_t channels,
                                                   uint32_t blocks_per_slot, unsigned int* error, StreamStep<K, LPR, ROWS, T>* first) {
    const uint32_t slot = blockIdx.y;
    const uint32_t token = slot / selected;
    const uint64_t expert = checked_index(indices[slot], experts, true, error);
    const T* slab = w + expert * uint64_t(channels) * K;
    const T* row = STAGED ? x : x + uint64_t(PER_SLOT_INPUT ? slot : token) * K;
    const uint32_t waves_per_block = blockDim.x / kWave;
    const uint32_t wave = blockIdx.x * waves_per_block + threadIdx.x / kWave;
    stream_rows<1, K, LPR, ROWS, STAGED, PREFETCHED, T>(row, xs, slab, nullptr, out + uint64_t(slot) * channels, channels, channels, wave,
                                                        blocks_per_slot * waves_per_block, first);
}

// The same product for a slot whose expert index the kernel has just selected itself (``routed_expert_stream``):
// ``chosen`` is that index, checked like a stored one.
template <int K, int LPR, int ROWS, class T>
__device__ __forceinline__ void stream_expert_chosen(const T* __restrict__ w, int64_t chosen, const float* xs, T* __restrict__ out,
                                                     uint32_t experts, uint32_t channels, uint32_t blocks_per_slot, unsigned int* error) {
    const uint32_t slot = blockIdx.y;
    const uint64_t expert = checked_index(chosen, experts, true, error);
    const uint32_t waves_per_block = blockDim.x / kWave;
    const uint32_t wave = blockIdx.x * waves_per_block + threadIdx.x / kWave;
    stream_rows<1, K, LPR, ROWS, true, false, T>(nullptr, xs, w + expert * uint64_t(channels) * K, nullptr, out + uint64_t(slot) * channels, channels,
                                                 channels, wave, blocks_per_slot * waves_per_block, nullptr);
}

template <int K, int LPR, int ROWS, bool STAGED, class T, bool PER_SLOT_INPUT>
__device__ __forceinline__ void stream_expert_linear(const T* __restrict__ w, const int64_t* __restrict__ indices, const T* __restrict__ x,
                                                     const float* xs, T* __restrict__ out, uint32_t selected, uint32_t experts, uint32_t channels,
                                                     uint32_t blocks_per_slot, unsigned int* error) {
    stream_expert_rows<K, LPR, ROWS, STAGED, T, PER_SLOT_INPUT, false>(w, indices, x, xs, out, selected, experts, channels, blocks_per_slot, error,
                                                                       nullptr);
}

template <int K, int LPR, int ROWS, bool STAGED, class T, bool PER_SLOT_INPUT>
__device__ __forceinline__ void stream_expert_linear(const T* __restrict__ w, const int64_t* __restrict__ indices, const T* __restrict__ x,
                                                     const float* xs, T* __restrict__ out, uint32_t selected, uint32_t experts, uint32_t channels,
                                                     uint32_t blocks_per_slot, unsigned int* error, StreamStep<K, LPR, ROWS, T>& first) {
    stream_expert_rows<K, LPR, ROWS, STAGED, T, PER_SLOT_INPUT, true>(w, indices, x, xs, out, selected, experts, channels, blocks_per_slot, error,
                                                                      &first);
}

// Mixture-of-experts router for one token row per workgroup: logits[e] = x . W[e] (+ bias[e])
// for E <= 64 experts, rounded to the storage type and written out; then the reference's top-k (k
// rounds of a wave argmax over keys that rank NaN highest and break ties toward the lower index, sorted,
// chroma/_src/codegen/gpu.py:300-337) writes values and int64 indices; then the softmax of the k chosen
// values (float max, exp, sum, division; rounded) is written too. ``xs`` holds the row (K floats).
//
// The logits are LPR-lane dot products over 16-byte chunks of W (all of a step's chunks requested before
// any arithmetic), 64 / LPR experts per step; LPR == 0 means rows that are not whole chunks (a scalar
// wave-wide loop instead).
template <int E, int K, int LPR, class T>
__device__ __forceinline__ void router_fetch(StreamStep<K, LPR, 1, T>& first, const T* __restrict__ w) {
    const uint32_t e0 = threadIdx.x / kWave * StreamStep<K, LPR, 1, T>::G;
    if (e0 < uint32_t(E)) {
        first.fetch(w, e0, E);
    }
}

// With PREFETCHED (LPR > 0 only), this wave's first step of W was requested into ``first`` by
// ``router_fetch`` before the prologue that stages the row; the step is then used and refilled in place.
//
// With CHOSEN (``routed_expert_stream``), every workgroup of the kernel selects for its row: the chosen
// indices go to ``chosen`` (LDS, k entries, visible to every wave when this returns), and the global
// outputs are written only where ``write`` holds (one workgroup per row).
template <int E, int K, int LPR, bool LARGEST, class T, bool PREFETCHED = false, bool CHOSEN = false>
__device__ __forceinline__ void router_rows(const float* xs, const T* __restrict__ w, const T* __restrict__ bias, T* __restrict__ logits,
                                            T* __restrict__ values, int64_t* __restrict__ indices, T* __restrict__ weights, uint32_t k,
                                            StreamStep<K, (LPR > 0 ? LPR : 1), 1, T>* first, int32_t* chosen_s = nullptr, bool write = true) {
    static_assert(E <= kWave, "one expert per lane");
    static_assert(LPR == 0 || !StreamStep<K, (LPR > 0 ? LPR : 1), 1, T>::RAGGED, "router rows split evenly over their lanes");
    __shared__ float logit_s[E];
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
    if constexpr (LPR > 0) {
        using C = Chunk16<T>;
        using Step = StreamStep<K, LPR, 1, T>;
        constexpr int PER_LANE = Step::PER_LANE;
        constexpr int G = Step::G;
        const uint32_t group = lane / LPR, sub = lane % LPR;
        uint32_t e0 = wave * G;
        if (e0 < uint32_t(E)) {
            Step local;
            Step& step = PREFETCHED ? *first : local;
            if constexpr (!PREFETCHED) {
                step.fetch(w, e0, E);
            }
            for (;;) {
                const uint32_t e = e0 + group;
                float partial = 0.0f;
#pragma unroll
                for (int c = 0; c < PER_LANE; ++c) {
                    if (c % 8 == 0) {
                        // read X from LDS a few chunks at a time (all of it at once would not fit in registers)
                        __asm__ volatile("" ::: "memory");
                    }
#pragma unroll
                    for (int i = 0; i < C::N; ++i) {
                        partial += C::get(step.chunks[0][c], i) * xs[(c * LPR + sub) * C::N + i];
                    }
                }
#pragma unroll
                for (int offset = LPR / 2; offset > 0; offset >>= 1) {
                    partial += __shfl_xor(partial, offset, kWave);
                }
                if (sub == 0 && e < uint32_t(E)) {
                    logit_s[e] = partial;
                }
                e0 += waves * G;
                if (e0 >= uint32_t(E)) {
                    break;
                }
                step.fetch(w, e0, E);
            }
        }
    } else {
        for (uint32_t e = wave; e < uint32_t(E); e += waves) {
            float partial = 0.0f;
            for (uint32_t i = lane; i < uint32_t(K); i += kWave) {
                partial += xs[i] * load1<T>(w + size_t(e) * K + i);
            }
            partial = wave_sum(partial);
            if (lane == 0) {
                logit_s[e] = partial;
            }
        }
    }
    __syncthreads();
    if (wave != 0) {
        if constexpr (CHOSEN) {
            __syncthreads();  // the first wave's selection
        }
        return;  // the first wave selects; without CHOSEN no barrier follows
    }
    const float mine = lane < uint32_t(E) ? logit_s[lane] : 0.0f;
    float logit = 0.0f;
    uint64_t key = 0;
    if (lane < uint32_t(E)) {
        const float b = bias ? load1<T>(bias + lane) : 0.0f;
        const T stored = storage_of<T>(mine + b);
        if (write) {
            logits[lane] = stored;
        }
        logit = widen_of<T>(stored);  // the rounded logit, as stored
        key = topk_key(logit, lane, LARGEST);
    }
    float chosen[E];
    for (uint32_t s = 0; s < k; ++s) {
        const uint64_t top = wave_max_u64(key);
        const uint32_t winner = 0xffffffffu - uint32_t(top);
        chosen[s] = __shfl(logit, int(winner), kWave);
        if (lane == winner) {
            key = 0;
        }
        if (lane == 0) {
            if constexpr (CHOSEN) {
                chosen_s[s] = int32_t(winner);
            }
            if (write) {
                store1<T>(values + s, chosen[s]);
                indices[s] = int64_t(winner);
            }
        }
    }
    if constexpr (CHOSEN) {
        __syncthreads();  // publishes chosen_s to the other waves
        if (!write) {
            return;
        }
    }
    if (lane == 0) {
        float peak = -__builtin_inff();
        for (uint32_t s = 0; s < k; ++s) {
            peak = __builtin_fmaxf(peak, chosen[s]);
        }
        float total = 0.0f;
        for (uint32_t s = 0; s < k; ++s) {
            total += fast_exp(chosen[s] - peak);
        }
        for (uint32_t s = 0; s < k; ++s) {
            store1<T>(weights + s, fast_exp(chosen[s] - peak) / total);
        }
    }
}

template <int E, int K, int LPR, bool LARGEST, class T>
__device__ __forceinline__ void router_row(const float* xs, const T* __restrict__ w, const T* __restrict__ bias, T* __restrict__ logits,
                                           T* __restrict__ values, int64_t* __restrict__ indices, T* __restrict__ weights, uint32_t k) {
    router_rows<E, K, LPR, LARGEST, T, false>(xs, w, bias, logits, values, indices, weights, k, nullptr);
}

// A router whose gate weights are too large for one workgroup's stream (GPT-OSS-20B: 32 x 2880): grid.x
// parts (the first wave of each; the other waves only share the staging prologue, whose row loads are
// then all in flight at once) compute G = 64 / LPR experts' logits of row blockIdx.y (bias added, rounded and
// stored as router_rows stores them, with device-scope stores); each part then waits for its stores to
// complete and takes a ticket from the row's counter, and the part that takes the last ticket selects: it
// reads the row's stored logits with device-scope loads, picks the
// top k with router_rows' ranking and tie rules and writes values, int64 indices and the softmax of the
// values, then resets the counter to 0 for the next launch. No part waits for another. ``counter`` holds
// one word per row (kRouterTickets at most), zero when the kernel starts: the program's error region,
// which the runtime clears at load, past its index-error word.
constexpr uint32_t kRouterTicketWord = 16;  // first word of the tickets in the 64-word error region
constexpr uint32_t kRouterTickets = 48;

template <int E, int K, int LPR, bool LARGEST, class T>
__device__ __forceinline__ void router_split(const float* xs, const T* __restrict__ w, const T* __restrict__ bias, T* __restrict__ logits,
                                             T* __restrict__ values, int64_t* __restrict__ indices, T* __restrict__ weights, uint32_t k,
                                             unsigned int* counter) {
    static_assert(E <= kWave && LPR > 0 && !StreamStep<K, LPR, 1, T>::RAGGED, "one expert per lane, rows split evenly over their lanes");
    using C = Chunk16<T>;
    using Step = StreamStep<K, LPR, 1, T>;
    constexpr int PER_LANE = Step::PER_LANE;
    constexpr int G = Step::G;
    const uint32_t lane = threadIdx.x % kWave, group = lane / LPR, sub = lane % LPR;
    const uint32_t row = blockIdx.y, parts = gridDim.x;
    T* row_logits = logits + size_t(row) * E;
    if (threadIdx.x < kWave) {
        const uint32_t e0 = blockIdx.x * G, e = e0 + group;
        Step step;
        step.fetch(w, e0, E);
        float partial = 0.0f;
#pragma unroll
        for (int c = 0; c < PER_LANE; ++c) {
            if (c % 8 == 0) {
                __asm__ volatile("" ::: "memory");
            }
#pragma unroll
            for (int i = 0; i < C::N; ++i) {
                partial += C::get(step.chunks[0][c], i) * xs[(c * LPR + sub) * C::N + i];
            }
        }
#pragma unroll
        for (int offset = LPR / 2; offset > 0; offset >>= 1) {
            partial += __shfl_xor(partial, offset, kWave);
        }
        if (sub == 0 && e < uint32_t(E)) {
            store_device(row_logits + e, storage_of<T>(partial + (bias ? load1<T>(bias + e) : 0.0f)));
        }
    }
    device_stores_complete();  // this part's logits are visible to device-scope loads before its ticket is taken
    __shared__ unsigned int ticket;
    __syncthreads();
    if (threadIdx.x == 0) {
        ticket = atomicAdd(counter + row, 1u);
    }
    __syncthreads();
    if (ticket != parts - 1 || threadIdx.x >= kWave) {
        return;
    }
    float logit = 0.0f;
    uint64_t key = 0;
    if (lane < uint32_t(E)) {
        logit = widen_of<T>(load_device(row_logits + lane));  // every part's stored, rounded logit
        key = topk_key(logit, lane, LARGEST);
    }
    float chosen[E];
    for (uint32_t s = 0; s < k; ++s) {
        const uint64_t top = wave_max_u64(key);
        const uint32_t winner = 0xffffffffu - uint32_t(top);
        chosen[s] = __shfl(logit, int(winner), kWave);
        if (lane == winner) {
            key = 0;
        }
        if (lane == 0) {
            store1<T>(values + size_t(row) * k + s, chosen[s]);
            indices[size_t(row) * k + s] = int64_t(winner);
        }
    }
    if (lane == 0) {
        float peak = -__builtin_inff();
        for (uint32_t s = 0; s < k; ++s) {
            peak = __builtin_fmaxf(peak, chosen[s]);
        }
        float total = 0.0f;
        for (uint32_t s = 0; s < k; ++s) {
            total += fast_exp(chosen[s] - peak);
        }
        for (uint32_t s = 0; s < k; ++s) {
            store1<T>(weights + size_t(row) * k + s, fast_exp(chosen[s] - peak) / total);
        }
        atomicExch(counter + row, 0u);
    }
}

// A router fused into its first expert product (one kernel instead of two): each workgroup of the expert
// stream (grid.y: slot = token * selected + s) recomputes its token's router from the staged row ``xs``
// (the gate weights are small: E x K), takes expert s of the selection and streams that expert's slab.
// The workgroup at blockIdx.x == 0 of slot s == 0 also writes the router's outputs (logits, values,
// indices, softmax weights) for later readers. Selection, rounding and tie rules are router_rows'.
template <int E, int K, int RLPR, bool LARGEST, int SK, int LPR, int ROWS, class T>
__device__ __forceinline__ void routed_expert_stream(const float* xs, const T* __restrict__ gate, const T* __restrict__ gate_bias,
                                                     T* __restrict__ logits, T* __restrict__ values, int64_t* __restrict__ indices,
                                                     T* __restrict__ weights, uint32_t selected, const T* __restrict__ w, T* __restrict__ out,
                                                     uint32_t experts, uint32_t channels, uint32_t blocks_per_slot, unsigned int* error) {
    __shared__ int32_t chosen_s[E];
    const uint32_t token = blockIdx.y / selected, s = blockIdx.y % selected;
    const bool write = blockIdx.x == 0 && s == 0;
    router_rows<E, K, RLPR, LARGEST, T, false, true>(xs, gate, gate_bias, logits + size_t(token) * E, values + size_t(token) * selected,
                                                     indices + size_t(token) * selected, weights + size_t(token) * selected, selected, nullptr,
                                                     chosen_s, write);
    stream_expert_chosen<SK, LPR, ROWS, T>(w, int64_t(chosen_s[s]), xs, out, experts, channels, blocks_per_slot, error);
}

template <int E, int K, int LPR, bool LARGEST, class T>
__device__ __forceinline__ void router_row(const float* xs, const T* __restrict__ w, const T* __restrict__ bias, T* __restrict__ logits,
                                           T* __restrict__ values, int64_t* __restrict__ indices, T* __restrict__ weights, uint32_t k,
                                           StreamStep<K, LPR, 1, T>& first) {
    router_rows<E, K, LPR, LARGEST, T, true>(xs, w, bias, logits, values, indices, weights, k, &first);
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
// Matrix-core products. C[m, n] = sum_k A[m, k] B[k, n] (+ bias[n]) for one batch entry, float32
// accumulation in the MFMA accumulators and one rounding to the storage type at the store - the
// reference's numerics for float and bfloat16 products (chroma/_src/codegen/cpu/kernels.h:24-74) with a
// different summation order.
//
// A is row-major with unit k stride: A[m, k] at a[m * lda + k]. B is either k-contiguous
// (B[k, n] at b[n * ldb + k], a linear layer's weight) or n-contiguous (B[k, n] at b[k * ldb + n]); C is
// row-major, C[m, n] at c[m * ldc + n]. Row strides and base addresses must keep 16-byte alignment.
//
// Workgroup: 256 threads = 4 waves, a 128 x 128 output tile, K staged through LDS in slices (32 for
// bfloat16, 16 for float), double-buffered so the next slice streams from HBM while the current one
// feeds the matrix cores. LDS rows are padded against bank conflicts. Each wave owns a 64 x 64 quadrant
// as 4 x 4 tiles of v_mfma_f32_16x16x32_bf16 (lane l supplies A[row l % 16][k 8(l / 16) .. +7] and
// B[k 8(l / 16) .. +7][column l % 16]) or v_mfma_f32_16x16x4_f32 (A[l % 16][l / 16], B[l / 16][l % 16]);
// lane l receives D[rows 4(l / 16) .. +3][column l % 16].
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <class T> struct Mfma;
template <> struct Mfma<uint16_t> {
    static constexpr int BK = 32, PAD = 8, CHUNK = 8;  // a 16-byte chunk holds 8 elements
    using Chunk = uint4;
};
template <> struct Mfma<float> {
    static constexpr int BK = 16, PAD = 4, CHUNK = 4;
    using Chunk = float4;
};

// Store a wave's 4 x 4 accumulator tiles (rows m0 + wm 64 .., columns n0 + wn 64 ..), one rounding each.
template <class T>
__device__ __forceinline__ void mfma_store(const f32x4_t (&acc)[4][4], const T* __restrict__ bias, T* __restrict__ c,
                                           uint32_t ldc, uint32_t m_total, uint32_t n_total,
                                           const int32_t* __restrict__ c_rows, uint32_t m0, uint32_t n0) {
    const uint32_t lane = threadIdx.x % 64u, wave = threadIdx.x / 64u;
    const uint32_t wm = wave / 2u, wn = wave % 2u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t gn = n0 + wn * 64u + j * 16u + lane % 16u;
            if (gn >= n_total) {
                continue;
            }
            const float offset = bias ? load1<T>(bias + gn) : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm * 64u + i * 16u + (lane / 16u) * 4u + r;
                if (gm < m_total) {
                    const size_t crow = c_rows ? size_t(c_rows[gm]) : size_t(gm);
                    store1<T>(c + crow * ldc + gn, acc[i][j][r] + offset);
                }
            }
        }
    }
}

// bfloat16 with a k-contiguous B and K a multiple of 64: 64-deep slices, so each slice feeds 32 MFMAs per
// wave between the issue of the next slice's loads and the wait for them (twice the cover of 32-deep
// slices, half the barriers). Every thread moves the same four A rows and four B rows at every slice, so
// their addresses are formed once; rows past the edge of the tile repeat the last valid row (their
// results are never stored), which keeps every load unconditional and in bounds. The MFMA sequence per
// accumulator is the one of the 32-deep path, so both give the same bits.
// LDS placement of 16-byte chunk ``chunk`` (0..7) of tile row ``row`` in the 64-deep path: unpadded
// 128-byte rows with the chunk index XORed by the row's low bits, so the 16 rows one fragment read touches
// and the 8 chunks one row write touches all fall in distinct banks (no LDS bank-conflict cycles on gfx950).
__device__ __forceinline__ uint32_t deep_lds(uint32_t row, uint32_t chunk) { return row * 64u + ((chunk ^ (row & 7u)) * 8u); }

__device__ __forceinline__ void mfma_gemm_deep(const uint16_t* __restrict__ a, uint32_t lda, const uint16_t* __restrict__ b,
                                               uint32_t ldb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ c,
                                               uint32_t ldc, uint32_t m_total, uint32_t n_total, uint32_t k_total,
                                               const int32_t* __restrict__ a_rows, const int32_t* __restrict__ c_rows,
                                               uint32_t m_base, uint32_t n_base) {
    constexpr int BM = 128, BN = 128, BK = 64, LD = 64, CH = 8;
    constexpr int CHUNKS = BM * BK / CH / 256;  // 16-byte chunks per thread and operand per slice
    __shared__ __attribute__((aligned(16))) uint16_t as[2][BM * LD];
    __shared__ __attribute__((aligned(16))) uint16_t bs[2][BN * LD];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % 64u, wave = tid / 64u;
    const uint32_t wm = wave / 2u, wn = wave % 2u;
    const uint32_t m0 = m_base, n0 = n_base;
    if (m0 >= m_total) {
        return;
    }
    const uint32_t kc = (tid % (BK / CH)) * CH;
    const uint16_t* pa[CHUNKS];
    const uint16_t* pb[CHUNKS];
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        const uint32_t row = tid / (BK / CH) + i * (256u / (BK / CH));
        const uint32_t gm = m0 + row < m_total ? m0 + row : m_total - 1u;
        const uint32_t gn = n0 + row < n_total ? n0 + row : n_total - 1u;
        pa[i] = a + (a_rows ? size_t(a_rows[gm]) : size_t(gm)) * lda + kc;
        pb[i] = b + size_t(gn) * ldb + kc;
    }
    uint32_t srow[CHUNKS];
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        srow[i] = deep_lds(tid / (BK / CH) + i * (256u / (BK / CH)), tid % (BK / CH));
    }
    uint4 ra[CHUNKS], rb[CHUNKS];
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        ra[i] = *reinterpret_cast<const uint4*>(pa[i]);
        rb[i] = *reinterpret_cast<const uint4*>(pb[i]);
    }
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        *reinterpret_cast<uint4*>(&as[0][srow[i]]) = ra[i];
        *reinterpret_cast<uint4*>(&bs[0][srow[i]]) = rb[i];
    }
    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    const uint32_t steps = k_total / BK;
    __syncthreads();
    for (uint32_t step = 0; step < steps; ++step) {
        const int buffer = step & 1;
        const bool more = step + 1 < steps;
        const uint32_t k_next = more ? (step + 1) * BK : 0u;  // the last slice re-reads slice 0, unused
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            ra[i] = *reinterpret_cast<const uint4*>(pa[i] + k_next);
            rb[i] = *reinterpret_cast<const uint4*>(pb[i] + k_next);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            bf16x8_t fa[4], fb[4];
            const uint32_t chunk = half * 4u + lane / 16u;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t ia = deep_lds(wm * 64u + t * 16u + lane % 16u, chunk);
                const uint32_t ib = deep_lds(wn * 64u + t * 16u + lane % 16u, chunk);
                fa[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&as[buffer][ia]));
                fb[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&bs[buffer][ib]));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < CHUNKS; ++i) {
                *reinterpret_cast<uint4*>(&as[buffer ^ 1][srow[i]]) = ra[i];
                *reinterpret_cast<uint4*>(&bs[buffer ^ 1][srow[i]]) = rb[i];
            }
        }
        __syncthreads();
    }
    mfma_store<uint16_t>(acc, bias, c, ldc, m_total, n_total, c_rows, m0, n0);
}

// bfloat16 with a k-contiguous B, K a multiple of 64 and 16-byte aligned rows, on kDirectThreads threads
// (8 waves as 4 x 2, each a 32 x 64 part of the 128 x 128 tile). Each 64-deep slice goes from global memory
// straight into LDS (global_load_lds_dwordx4: no staging registers and no LDS store instructions, which
// took a third of the time of the register-staged bodies), double-buffered: the next slice's copies are
// issued at the start of a step and waited for only at its end, and the second half's fragments are read
// while the first half's MFMAs issue. LDS layout as ``deep_lds``: the lane that fills LDS position p of
// a tile row fetches the global chunk p ^ (row & 7). Rows past the tile's edge repeat the last valid row
// (never stored). The MFMA sequence per accumulator is the 64-deep path's.
constexpr uint32_t kDirectThreads = 512;

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

template <class T>
__device__ __forceinline__ void mfma_gemm_direct(const uint16_t* __restrict__ a, uint32_t lda, const uint16_t* __restrict__ b,
                                                 uint32_t ldb, const T* __restrict__ bias, T* __restrict__ c, uint32_t ldc,
                                                 uint32_t m_total, uint32_t n_total, uint32_t k_total, const int32_t* __restrict__ a_rows,
                                                 const int32_t* __restrict__ c_rows, uint32_t m0, uint32_t n0) {
    constexpr int WM = 4, WN = 2, WAVES = WM * WN, BM = 128, BN = 128;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // 16 x 16 tiles per wave: 2 x 4
    constexpr int BLOCKS = BM / 8 / WAVES;                // 8-row (1 KB) blocks each wave copies per operand per slice
    // One LDS array for both operands and both buffers: with two arrays the compiler could not tell the
    // fragment reads from the copies in flight and made every read wait for all of them (vmcnt(0)), so the
    // next slice's copies never overlapped the current slice's MFMAs.
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * (BM + BN) * 64];
    auto as = [&](int buffer) { return lds + buffer * (BM + BN) * 64; };
    auto bs = [&](int buffer) { return lds + buffer * (BM + BN) * 64 + BM * 64; };
    const uint32_t tid = threadIdx.x, lane = tid % 64u, wave = tid / 64u;
    const uint32_t wm = wave / WN, wn = wave % WN;
    if (m0 >= m_total) {
        return;
    }
    const uint16_t* ga[BLOCKS];
    const uint16_t* gb[BLOCKS];
#pragma unroll
    for (int i = 0; i < BLOCKS; ++i) {
        const uint32_t row = (i * WAVES + wave) * 8u + lane / 8u;
        const uint32_t chunk = (lane % 8u) ^ (row & 7u);
        const uint32_t gm = m0 + row < m_total ? m0 + row : m_total - 1u;
        const uint32_t gn = n0 + row < n_total ? n0 + row : n_total - 1u;
        ga[i] = a + (a_rows ? size_t(a_rows[gm]) : size_t(gm)) * lda + chunk * 8u;
        gb[i] = b + size_t(gn) * ldb + chunk * 8u;
    }
    auto copy = [&](int buffer, uint32_t k0) {
#pragma unroll
        for (int i = 0; i < BLOCKS; ++i) {
            __builtin_amdgcn_global_load_lds((global_void*)(ga[i] + k0), (lds_void*)(as(buffer) + (i * WAVES + wave) * 512u), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((global_void*)(gb[i] + k0), (lds_void*)(bs(buffer) + (i * WAVES + wave) * 512u), 16, 0, 0);
        }
    };
    auto fragments = [&](int buffer, int half, bf16x8_t (&fa)[TM], bf16x8_t (&fb)[TN]) {
        const uint32_t chunk = half * 4u + lane / 16u;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            fa[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(as(buffer) + (deep_lds(wm * (BM / WM) + t * 16u + lane % 16u, chunk))));
        }
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            fb[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(bs(buffer) + (deep_lds(wn * (BN / WN) + t * 16u + lane % 16u, chunk))));
        }
    };
    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    const uint32_t steps = k_total / 64u;
    copy(0, 0);
    __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): the first slice is in LDS
    __syncthreads();
    if (m0 + wm * (BM / WM) >= m_total) {
        // every row of this wave's part lies past the tile's edge (a ragged expert tile): it only copies
        // its share of each slice and keeps the workgroup's barriers; the MFMA pipe and LDS reads it leaves
        // free go to the other resident workgroup
        for (uint32_t step = 0; step < steps; ++step) {
            if (step + 1 < steps) {
                copy((step & 1) ^ 1, (step + 1) * 64u);
            }
            __builtin_amdgcn_s_waitcnt(0xF70);
            __syncthreads();
        }
        return;
    }
    bf16x8_t fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    fragments(0, 0, fa0, fb0);
    for (uint32_t step = 0; step < steps; ++step) {
        const int buffer = step & 1;
        const bool more = step + 1 < steps;
        if (more) {
            copy(buffer ^ 1, (step + 1) * 64u);  // the other buffer was last read before the previous barrier
        }
        fragments(buffer, 1, fa1, fb1);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa0[i], fb0[j], acc[i][j], 0, 0, 0);
            }
        }
        // one fragment read of the second half between pairs of the first half's MFMAs
#pragma unroll
        for (int g = 0; g < TM + TN; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa1[i], fb1[j], acc[i][j], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): the next slice has landed
        __syncthreads();
        if (more) {
            fragments(buffer ^ 1, 0, fa0, fb0);
        }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint32_t gn = n0 + wn * (BN / WN) + j * 16u + lane % 16u;
        if (gn >= n_total) {
            continue;
        }
        const float offset = bias ? load1<T>(bias + gn) : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm * (BM / WM) + i * 16u + (lane / 16u) * 4u + r;
                if (gm < m_total) {
                    const size_t crow = c_rows ? size_t(c_rows[gm]) : size_t(gm);
                    store1<T>(c + crow * ldc + gn, acc[i][j][r] + offset);
                }
            }
        }
    }
}

// Compile-time index loops: ``unroll<N>(fn)`` calls fn(integral_constant<int, 0>) ... fn(<N - 1>), so every
// register array below is indexed by constants before any optimisation runs (a runtime-indexed private
// array is placed in memory instead of registers).
template <class Fn, int... I>
__device__ __forceinline__ void unroll_impl(Fn&& fn, std::integer_sequence<int, I...>) {
    (fn(std::integral_constant<int, I>{}), ...);
}
template <int N, class Fn>
__device__ __forceinline__ void unroll(Fn&& fn) {
    unroll_impl(fn, std::make_integer_sequence<int, N>{});
}

// Wide bfloat16 body for large products: a kWideM x kWideN (256 x 192) tile on kWideThreads threads, 4
// waves as 2 x 2, each wave a 128 x 96 part (8 x 6 MFMA tiles, 192 accumulator registers). K advances in
// 32-deep stages copied global -> LDS directly (global_load_lds_dwordx4) into a 5-slot ring (3 stages in
// flight, 140 KiB, one workgroup per CU). A stage's 7 copies per wave are spread one per MFMA row, the
// next stage's fragments are read right after their last use (A fragment i after MFMA row i, B fragments
// during the last row), and stage s refills the slot stage s-1 used: every wave consumed those fragments
// in its stage s-1 MFMAs before the barrier that opens stage s. The larger tile reads 0.29 KB of LDS and
// copies 0.15 KB per MFMA (the 128 x 128 body: 0.75 and 0.25), which the measured LDS and copy throughput
// of a compute unit favour. LDS rows are 64 B; the 16-byte chunk c of row r sits at position
// c ^ wide_swizzle(r), so a fragment read (16 rows x 64 B) touches distinct banks both when 16 lanes share
// a 256-byte bank cycle and when 8 lanes share 128 bytes. MFMA operands are swapped (W fragment first) so a
// lane holds 4 consecutive output columns of one row and stores them as one 8-byte write. Each output
// element accumulates the same 32-deep MFMA sequence as the 64-deep bodies. Requires bfloat16, a
// k-contiguous B, K % 32 = 0 and lda, ldb multiples of 8.
constexpr uint32_t kWideThreads = 256, kWideM = 256, kWideN = 192;

__device__ __forceinline__ uint32_t wide_swizzle(uint32_t row) { return ((row >> 2) ^ (row >> 1)) & 3u; }

// s_waitcnt immediate waiting for at most n outstanding vector-memory operations (lgkm and exp counts free)
constexpr int16_t vmcnt_wait(uint32_t n) { return int16_t((n & 15u) | ((n >> 4) << 14) | 0x70u | 0xF00u); }

// ``mfma_gemm_ring`` is that body for any BM x BN tile on WM x WN waves (each wave BM / WM x BN / WN, in
// 16 x 16 MFMA tiles) with an S-slot ring (S - 2 stages in flight): the dense linears take 256 x 192 on
// 2 x 2 waves with 5 slots (``mfma_gemm_wide``); the expert products take 128-slot x 384- or 320-channel
// tiles on 1 x 4 waves (each wave all 128 slots of a 96- or 80-channel strip), which keeps the 128-slot
// tiles of the ragged per-expert slot counts while reading 0.29-0.32 KB of LDS per MFMA instead of the
// 32 x 64 wave tiles' 0.75 (the expert body was LDS-bound at about a fifth of the matrix-core peak).
//
// ``ring`` is the caller's LDS array of at least ``ring_elements<BM, BN, S>()`` bf16 elements (one array per
// kernel, see grouped_expert_linear). When BM / 16 is not a multiple of the wave count, the A copies of the
// last round go past the tile's row blocks: those copies repeat its last block (the same bytes to the same
// LDS position), so every wave still issues the same number of copies per stage and the vmcnt waits hold.
template <int BM, int BN, int S>
constexpr int ring_elements() {
    return S * (BM + BN) * 32;
}

//
// With an ``epilogue`` (any callable but nullptr) the tile stores nothing itself: for every output row gm of
// the tile (c_rows[gm], or gm) and every 4 consecutive columns n .. n + 3 a lane holds, it calls
// epilogue(row, n, v, tag) with v[r] the float value the plain store would round to bfloat16 (acc + bias)
// and ``tag`` the caller's (the grouped expert products pass the tile's expert).
template <class T, int BM, int BN, int WM, int WN, int S, int L = BM / WM / 16, class Epilogue = std::nullptr_t>
__device__ __forceinline__ void mfma_gemm_ring(const uint16_t* __restrict__ a, uint32_t lda, const uint16_t* __restrict__ b,
                                               uint32_t ldb, const T* __restrict__ bias, T* __restrict__ c, uint32_t ldc,
                                               uint32_t m_total, uint32_t n_total, uint32_t k_total,
                                               const int32_t* __restrict__ a_rows, const int32_t* __restrict__ c_rows, uint32_t m0,
                                               uint32_t n0, uint32_t a_div, uint16_t* ring, Epilogue epilogue = nullptr,
                                               uint32_t tag = 0) {
    static_assert(sizeof(T) == 2, "the ring body takes bfloat16");
    static_assert(S >= 3, "the ring needs a slot being read, one landed and one being filled");
    constexpr int WAVES = WM * WN;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
    constexpr int A_BLOCKS = BM / 16;
    constexpr int CA = (A_BLOCKS + WAVES - 1) / WAVES, CB = BN / 16 / WAVES, PER = CA + CB;  // 1 KB copies per wave per stage
    constexpr int SLOT = (BM + BN) * 32;                                                    // bf16 elements per ring slot
    static_assert(CB * 16 * WAVES == BN, "whole B row blocks per wave");
    static_assert(TM * WM * 16 == BM && TN * WN * 16 == BN, "whole 16 x 16 tiles per wave");
    // L live 16-row tiles per wave (the others hold no row of the tile: no MFMA, fragment read or store);
    // the stage's copies are spread over the live rows' MFMA sequences, copy c in row c % L
    static_assert(L >= 1 && L <= TM && (L == TM || WM == 1), "live row tiles of a one-row-group tile");
    const uint32_t lane = threadIdx.x % 64u, wave = threadIdx.x / 64u;
    const uint32_t wm = wave / WN, wn = wave % WN;
    // copy i moves 16 rows x 64 B: lane -> row block * 16 + lane / 4, LDS position lane % 4
    const uint16_t* src[PER];
    uint32_t dst[PER];
    unroll<PER>([&](auto ic) {
        constexpr int i = ic;
        const uint32_t spread = (i < CA ? i : i - CA) * WAVES + wave;
        const uint32_t block = i < CA && spread >= uint32_t(A_BLOCKS) ? uint32_t(A_BLOCKS - 1) : spread;
        const uint32_t row = block * 16u + lane / 4u;
        const uint32_t chunk = (lane % 4u) ^ wide_swizzle(row);
        if constexpr (i < CA) {
            const uint32_t g = m0 + row < m_total ? m0 + row : m_total - 1u;
            src[i] = a + (a_rows ? size_t(uint32_t(a_rows[g]) / a_div) : size_t(g)) * lda + chunk * 8u;
            dst[i] = block * 512u;
        } else {
            const uint32_t g = n0 + row < n_total ? n0 + row : n_total - 1u;
            src[i] = b + size_t(g) * ldb + chunk * 8u;
            dst[i] = BM * 32u + block * 512u;
        }
    });
    uint32_t oa[L], ob[TN];
    unroll<L>([&](auto t) {
        const uint32_t row = wm * (BM / WM) + t * 16u + lane % 16u;
        oa[t] = row * 32u + (((lane / 16u) ^ wide_swizzle(row)) * 8u);
    });
    unroll<TN>([&](auto t) {
        const uint32_t row = wn * (BN / WN) + t * 16u + lane % 16u;
        ob[t] = BM * 32u + row * 32u + (((lane / 16u) ^ wide_swizzle(row)) * 8u);
    });
    const uint32_t steps = k_total / 32u;
    // stages past the end re-copy the last stage into a slot that is never read again
    auto k_of = [&](uint32_t stage) { return (stage < steps ? stage : steps - 1u) * 32u; };
    auto copy = [&](auto ic, uint32_t slot, uint32_t k0) {
        constexpr int i = ic;
        __builtin_amdgcn_global_load_lds((global_void*)(src[i] + k0), (lds_void*)(ring + slot * SLOT + dst[i]), 16, 0, 0);
    };
    // the copies of live row r (c = r, r + L, ...) and how many there are
    auto copies_of_row = [&](auto rc, uint32_t slot, uint32_t k0) {
        unroll<PER>([&](auto cc) {
            if constexpr (int(cc) % L == int(rc)) copy(cc, slot, k0);
        });
    };
    constexpr auto row_copies = [](int r) { return (PER - r + L - 1) / L; };
    unroll<S - 1>([&](auto st) { unroll<PER>([&](auto i) { copy(i, uint32_t(st), k_of(st)); }); });
    __builtin_amdgcn_s_waitcnt(vmcnt_wait((S - 2) * PER));  // stage 0 landed
    __builtin_amdgcn_s_barrier();
    bf16x8_t fa[L], fb[TN];
    unroll<L>([&](auto t) { fa[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(ring + oa[t])); });
    unroll<TN>([&](auto t) { fb[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(ring + ob[t])); });
    f32x4_t acc[L][TN];
    unroll<L>([&](auto i) { unroll<TN>([&](auto j) { acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}; }); });
    for (uint32_t s = 0; s + 1u < steps; ++s) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_wait((S - 3) * PER));  // stage s+1 landed (s+2 .. s+S-2 may be in flight)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const uint16_t* next = ring + ((s + 1u) % S) * SLOT;
        const uint32_t fill = (s + S - 1u) % S, k_fill = k_of(s + S - 1u);
        unroll<L - 1>([&](auto ic) {
            constexpr int i = ic;
            unroll<TN>([&](auto jc) {
                constexpr int j = jc;
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
                if constexpr (j == TN / 2) copies_of_row(ic, fill, k_fill);
            });
            fa[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(next + oa[i]));
        });
        unroll<TN>([&](auto jc) {
            constexpr int j = jc;
            acc[L - 1][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[L - 1], acc[L - 1][j], 0, 0, 0);
            if constexpr (j == TN / 2) copies_of_row(std::integral_constant<int, L - 1>{}, fill, k_fill);
            fb[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(next + ob[j]));
        });
        fa[L - 1] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(next + oa[L - 1]));
        // issue order: per row, half its MFMAs, its copies, the rest, one fragment read
        unroll<L - 1>([&](auto ic) {
            __builtin_amdgcn_sched_group_barrier(0x008, TN / 2 + 1, 0);
            if constexpr (row_copies(int(ic)) > 0) {
                __builtin_amdgcn_sched_group_barrier(0x020, row_copies(int(ic)), 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, TN - TN / 2 - 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        });
        unroll<TN>([&](auto jc) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if constexpr (int(jc) == TN / 2 && row_copies(L - 1) > 0) {
                __builtin_amdgcn_sched_group_barrier(0x020, row_copies(L - 1), 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        });
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    unroll<L>([&](auto i) {
        unroll<TN>([&](auto j) { acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0); });
    });
    __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));  // re-copies of the last stage land before the workgroup ends
    // lane holds row lane % 16 and columns 4 (lane / 16) .. + 3 of each 16 x 16 tile
    const bool vector_rows = (ldc & 3u) == 0;
    unroll<L>([&](auto i) {
        const uint32_t gm = m0 + wm * (BM / WM) + i * 16u + lane % 16u;
        if (gm < m_total) {
            const uint32_t c_row = c_rows ? uint32_t(c_rows[gm]) : gm;
            T* row = c + size_t(c_row) * ldc;
            unroll<TN>([&](auto j) {
                const uint32_t gn = n0 + wn * (BN / WN) + j * 16u + (lane / 16u) * 4u;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    v[r] = acc[i][j][r] + (bias && gn + r < n_total ? load1<T>(bias + gn + r) : 0.0f);
                }
                if constexpr (!std::is_same_v<Epilogue, std::nullptr_t>) {
                    if (gn + 3u < n_total) {
                        epilogue(c_row, gn, v, tag);
                    }
                } else if (vector_rows && gn + 3u < n_total) {
                    const uint32_t lo = uint32_t(f32_to_bf16(v[0])) | (uint32_t(f32_to_bf16(v[1])) << 16);
                    const uint32_t hi = uint32_t(f32_to_bf16(v[2])) | (uint32_t(f32_to_bf16(v[3])) << 16);
                    *reinterpret_cast<uint2*>(row + gn) = uint2{lo, hi};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (gn + r < n_total) {
                            store1<T>(row + gn + r, v[r]);
                        }
                    }
                }
            });
        }
    });
}

template <class T>
__device__ __forceinline__ void mfma_gemm_wide(const uint16_t* __restrict__ a, uint32_t lda, const uint16_t* __restrict__ b,
                                               uint32_t ldb, const T* __restrict__ bias, T* __restrict__ c, uint32_t ldc,
                                               uint32_t m_total, uint32_t n_total, uint32_t k_total,
                                               const int32_t* __restrict__ a_rows, const int32_t* __restrict__ c_rows, uint32_t m0,
                                               uint32_t n0) {
    __shared__ __attribute__((aligned(1024))) uint16_t ring[ring_elements<kWideM, kWideN, 5>()];
    mfma_gemm_ring<T, kWideM, kWideN, 2, 2, 5>(a, lda, b, ldb, bias, c, ldc, m_total, n_total, k_total, a_rows, c_rows, m0, n0, 1u, ring);
}

template <class T, bool B_K_CONTIGUOUS>
__device__ __forceinline__ void mfma_gemm_sliced(const T* __restrict__ a, uint32_t lda, const T* __restrict__ b, uint32_t ldb,
                                                 const T* __restrict__ bias, T* __restrict__ c, uint32_t ldc, uint32_t m_total,
                                                 uint32_t n_total, uint32_t k_total, const int32_t* __restrict__ a_rows,
                                                 const int32_t* __restrict__ c_rows, uint32_t m_base, uint32_t n_base) {
    using M = Mfma<T>;
    using Chunk = typename M::Chunk;
    constexpr int BM = 128, BN = 128, BK = M::BK, LD = BK + M::PAD, CH = M::CHUNK;
    constexpr int A_CHUNKS = BM * BK / CH / 256;  // 16-byte chunks each thread moves per slice
    __shared__ __attribute__((aligned(16))) T as[2][BM * LD];
    __shared__ __attribute__((aligned(16))) T bs[2][BN * LD];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % 64u, wave = tid / 64u;
    const uint32_t wm = wave / 2u, wn = wave % 2u;
    const uint32_t m0 = m_base, n0 = n_base;

    Chunk ra[A_CHUNKS], rb[A_CHUNKS];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const uint32_t chunk = tid + i * 256u;
            const uint32_t row = chunk / (BK / CH), kc = (chunk % (BK / CH)) * CH;
            const uint32_t gk = k0 + kc, gm = m0 + row;
            const size_t arow = a_rows ? size_t(a_rows[gm < m_total ? gm : 0]) : size_t(gm);
            ra[i] = (gm < m_total && gk < k_total) ? *reinterpret_cast<const Chunk*>(a + arow * lda + gk) : Chunk{};
            if constexpr (B_K_CONTIGUOUS) {
                const uint32_t gn = n0 + row;
                rb[i] = (gn < n_total && gk < k_total) ? *reinterpret_cast<const Chunk*>(b + size_t(gn) * ldb + gk) : Chunk{};
            } else {
                // n-contiguous B: chunk i covers CH consecutive columns of one k row.
                const uint32_t kr = chunk / (BN / CH), nc = (chunk % (BN / CH)) * CH;
                const uint32_t gkr = k0 + kr, gn = n0 + nc;
                rb[i] = (gkr < k_total && gn < n_total) ? *reinterpret_cast<const Chunk*>(b + size_t(gkr) * ldb + gn) : Chunk{};
            }
        }
    };
    auto stash = [&](int buffer) {
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const uint32_t chunk = tid + i * 256u;
            const uint32_t row = chunk / (BK / CH), kc = (chunk % (BK / CH)) * CH;
            *reinterpret_cast<Chunk*>(&as[buffer][row * LD + kc]) = ra[i];
            if constexpr (B_K_CONTIGUOUS) {
                *reinterpret_cast<Chunk*>(&bs[buffer][row * LD + kc]) = rb[i];
            } else {
                const uint32_t kr = chunk / (BN / CH), nc = (chunk % (BN / CH)) * CH;
                const T* values = reinterpret_cast<const T*>(&rb[i]);
#pragma unroll
                for (int e = 0; e < CH; ++e) {
                    bs[buffer][(nc + e) * LD + kr] = values[e];
                }
            }
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
        if constexpr (sizeof(T) == 2) {
            bf16x8_t fa[4], fb[4];
            const uint32_t koff = (lane / 16u) * 8u;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                fa[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&as[buffer][(wm * 64u + t * 16u + lane % 16u) * LD + koff]));
                fb[t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&bs[buffer][(wn * 64u + t * 16u + lane % 16u) * LD + koff]));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int sub = 0; sub < BK / 4; ++sub) {
                const uint32_t k = sub * 4u + lane / 16u;
                float fa[4], fb[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    fa[t] = as[buffer][(wm * 64u + t * 16u + lane % 16u) * LD + k];
                    fb[t] = bs[buffer][(wn * 64u + t * 16u + lane % 16u) * LD + k];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
        if (step + 1 < steps) {
            stash(buffer ^ 1);
        }
        __syncthreads();
    }
    mfma_store<T>(acc, bias, c, ldc, m_total, n_total, c_rows, m0, n0);
}

// PATH 0 takes the 64-deep bfloat16 path whenever its conditions hold; PATH 1 always takes the sliced one;
// PATH 2 is the direct-to-LDS body (kDirectThreads threads), for bfloat16 with a k-contiguous B, K % 64 = 0
// and lda, ldb multiples of 8, which the code generator guarantees before it selects it.
template <class T, bool B_K_CONTIGUOUS, int PATH = 0>
__device__ __forceinline__ void mfma_gemm(const T* __restrict__ a, uint32_t lda, const T* __restrict__ b, uint32_t ldb,
                                          const T* __restrict__ bias, T* __restrict__ c, uint32_t ldc, uint32_t m_total,
                                          uint32_t n_total, uint32_t k_total, const int32_t* __restrict__ a_rows,
                                          const int32_t* __restrict__ c_rows, uint32_t m_base, uint32_t n_base) {
    if constexpr (PATH == 2) {
        static_assert(sizeof(T) == 2 && B_K_CONTIGUOUS, "the direct-to-LDS body takes bfloat16 with a k-contiguous B");
        mfma_gemm_direct<T>(a, lda, b, ldb, bias, c, ldc, m_total, n_total, k_total, a_rows, c_rows, m_base, n_base);
        return;
    }
    if constexpr (sizeof(T) == 2 && B_K_CONTIGUOUS && PATH == 0) {
        if (k_total % 64u == 0 && lda % 8u == 0 && ldb % 8u == 0) {
            mfma_gemm_deep(a, lda, b, ldb, bias, c, ldc, m_total, n_total, k_total, a_rows, c_rows, m_base, n_base);
            return;
        }
    }
    if constexpr (PATH != 2) {
        mfma_gemm_sliced<T, B_K_CONTIGUOUS>(a, lda, b, ldb, bias, c, ldc, m_total, n_total, k_total, a_rows, c_rows, m_base, n_base);
    }
}

// XCD-aware tile order. Workgroups are handed to the 8 XCDs (each with its own L2) round-robin by
// workgroup id, so neighbouring ids land on different L2s. A launch of 8 * ceil(tiles / 8) workgroups
// instead gives XCD j the contiguous logical tiles [j * per, (j + 1) * per): tiles that share operand rows
// run on one L2, and each operand tile is fetched from HBM by one XCD instead of by all eight. Returns
// false for the padding workgroups.
__device__ __forceinline__ bool xcd_logical_tile(uint32_t tiles, uint32_t& logical) {
    const uint32_t per = (tiles + 7u) / 8u;
    const uint32_t p = blockIdx.x;
    logical = (p % 8u) * per + p / 8u;
    return p / 8u < per && logical < tiles;
}

// A linear layer on the matrix cores: Y[M, N] = X[M, K] . W[N, K]^T (+ bias). One-dimensional launch of
// 8 * ceil(tiles / 8) workgroups (tiles = ceil(M / 128) * ceil(N / 128)); logical tiles run down groups of
// 8 row tiles before moving to the next column tile, so an XCD's run of tiles covers a compact block of
// X rows and W rows.
template <class T, int PATH = 0>
__device__ __forceinline__ void mfma_linear(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                            T* __restrict__ out, uint32_t m_total, uint32_t n_total, uint32_t k_total) {
    const uint32_t gx = (n_total + 127u) / 128u, gy = (m_total + 127u) / 128u;
    uint32_t logical;
    if (!xcd_logical_tile(gx * gy, logical)) {
        return;
    }
    constexpr uint32_t G = 8;
    const uint32_t group = logical / (G * gx), first = group * G;
    const uint32_t height = gy - first < G ? gy - first : G;
    const uint32_t within = logical - group * G * gx;
    const uint32_t ty = first + within % height, tx = within / height;
    mfma_gemm<T, true, PATH>(x, k_total, w, k_total, bias, out, n_total, m_total, n_total, k_total, nullptr, nullptr, ty * 128u,
                             tx * 128u);
}

// A linear layer on the wide body: Y[M, N] = X[M, K] . W[N, K]^T (+ bias) in kWideM x kWideN tiles, launched
// as 8 * ceil(tiles / 8) workgroups of kWideThreads; logical tiles run down groups of 4 row tiles before
// the next column tile, so an XCD's concurrent tiles share X and W rows in its L2.
template <class T>
__device__ __forceinline__ void mfma_linear_wide(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                                 T* __restrict__ out, uint32_t m_total, uint32_t n_total, uint32_t k_total) {
    const uint32_t gx = (n_total + kWideN - 1u) / kWideN, gy = (m_total + kWideM - 1u) / kWideM;
    uint32_t logical;
    if (!xcd_logical_tile(gx * gy, logical)) {
        return;
    }
    constexpr uint32_t G = 4;
    const uint32_t group = logical / (G * gx), first = group * G;
    const uint32_t height = gy - first < G ? gy - first : G;
    const uint32_t within = logical - group * G * gx;
    const uint32_t ty = first + within % height, tx = within / height;
    mfma_gemm_wide<T>(x, k_total, w, k_total, bias, out, n_total, m_total, n_total, k_total, nullptr, nullptr, ty * kWideM,
                      tx * kWideN);
}

// A linear layer on the ring body in kMidM x kMidN (128 x 192) tiles on 2 x 2 waves (each a 64 x 96 part,
// 24 accumulator tiles) with a 5-slot ring (100 KiB of LDS): the products whose 256 x 192 tiles would leave
// much of the chip idle (C5's output projection, 2048 x 2880 x 4096: 120 wide tiles against 240 of these,
// 78.2 -> 58.2 us in isolation, the 128 x 128 direct body 63.0 us). Launched as 8 * ceil(tiles / 8)
// workgroups of kMidThreads; logical tiles run down groups of 8 row tiles before the next column tile.
constexpr uint32_t kMidThreads = 256, kMidM = 128, kMidN = 192;

template <class T>
__device__ __forceinline__ void mfma_linear_mid(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                                T* __restrict__ out, uint32_t m_total, uint32_t n_total, uint32_t k_total) {
    const uint32_t gx = (n_total + kMidN - 1u) / kMidN, gy = (m_total + kMidM - 1u) / kMidM;
    uint32_t logical;
    if (!xcd_logical_tile(gx * gy, logical)) {
        return;
    }
    constexpr uint32_t G = 8;
    const uint32_t group = logical / (G * gx), first = group * G;
    const uint32_t height = gy - first < G ? gy - first : G;
    const uint32_t within = logical - group * G * gx;
    const uint32_t ty = first + within % height, tx = within / height;
    __shared__ __attribute__((aligned(1024))) uint16_t ring[ring_elements<kMidM, kMidN, 5>()];
    mfma_gemm_ring<T, kMidM, kMidN, 2, 2, 5>(x, k_total, w, k_total, bias, out, n_total, m_total, n_total, k_total, nullptr, nullptr,
                                             ty * kMidM, tx * kMidN, 1u, ring);
}

// Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]) for few columns (N <= 64: a router's gate) and many rows: one
// workgroup of 4 waves per 16 rows of X, the waves splitting K into quarters; the matrix-core operands are
// read straight from global memory (each X row once, W - N x K, small - from L2), 8 k-steps of loads in
// flight per wave; the waves' float partial sums meet in LDS and are added in wave order, the bias added
// to the finished sum and the result rounded once (the numerics of every matrix-core product here).
// bfloat16: v_mfma_f32_16x16x32_bf16 (K % 32 == 0); float: v_mfma_f32_16x16x4f32 (K % 4 == 0). Rows past
// M and columns past N read the last row or column and are not stored.
template <class T, int N>
__device__ __forceinline__ void narrow_linear(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                              T* __restrict__ out, uint32_t m, uint32_t k_total) {
    static_assert(N >= 1 && N <= 64, "few columns");
    constexpr int NT = (N + 15) / 16;
    constexpr bool BF16 = sizeof(T) == 2;
    constexpr uint32_t KS = BF16 ? 32u : 4u;  // k per MFMA
    constexpr int UNROLL = 8;
    __shared__ float partial[4][16][NT * 16];
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, col = lane % 16u, quad = lane / 16u;
    const uint32_t r0 = blockIdx.x * 16u;
    const uint32_t row = r0 + col < m ? r0 + col : m - 1u;
    const uint32_t steps = k_total / KS;
    const uint32_t begin = steps * wave / 4u, end = steps * (wave + 1u) / 4u;
    const T* xr = x + size_t(row) * k_total + (BF16 ? quad * 8u : quad);
    const T* wr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t n = t * 16u + col < uint32_t(N) ? t * 16u + col : uint32_t(N) - 1u;
        wr[t] = w + size_t(n) * k_total + (BF16 ? quad * 8u : quad);
    }
    f32x4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (uint32_t s0 = begin; s0 < end; s0 += UNROLL) {
        if constexpr (BF16) {
            bf16x8_t fa[UNROLL], fb[UNROLL][NT];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint32_t s = s0 + u < end ? s0 + u : end - 1u;
                fa[u] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(xr + s * KS));
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    fb[u][t] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(wr[t] + s * KS));
                }
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                if (s0 + u < end) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[u], fb[u][t], acc[t], 0, 0, 0);
                    }
                }
            }
        } else {
            float fa[UNROLL], fb[UNROLL][NT];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint32_t s = s0 + u < end ? s0 + u : end - 1u;
                fa[u] = xr[s * KS];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    fb[u][t] = wr[t][s * KS];
                }
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                if (s0 + u < end) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[u], fb[u][t], acc[t], 0, 0, 0);
                    }
                }
            }
        }
    }
    // lane holds rows 4 quad .. + 3 of column ``col`` of each 16-column tile
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            partial[wave][quad * 4u + i][t * 16u + col] = acc[t][i];
        }
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < 16u * NT * 16u; e += blockDim.x) {
        const uint32_t r = e / (NT * 16u), c = e % (NT * 16u);
        if (r0 + r < m && c < uint32_t(N)) {
            const float sum = ((partial[0][r][c] + partial[1][r][c]) + partial[2][r][c]) + partial[3][r][c];
            store1<T>(out + size_t(r0 + r) * N + c, sum + (bias ? load1<T>(bias + c) : 0.0f));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Expert-grouped mixture-of-experts products.
//
// ``route_slots`` (one workgroup) turns the [tokens x selected] expert ids into a slot permutation grouped
// by expert and a table of row tiles; ids are checked like every gather (negative ids wrap, an id
// outside [-experts, experts) raises the error word and counts as expert 0). Layout of ``scratch``
// (int32): [0, E) per-expert counts, [E, 2E+1) offsets, [2E+1] tile count, then ``slots`` permutation
// entries, then the tile table as (expert, first row) pairs, ``expert_tile_bound`` of them; then a second
// table, [tile count, (expert, first row) pairs], for taller last tiles. An expert's tiles hold 128 slots
// each while more than ``last`` of its slots remain, then one tile takes the rest: the first table has
// ``last`` = 128 (ceil(count / 128) tiles), the second 160 (a remainder of at most 32 slots rides on the
// expert's last full tile, a 160-slot tile, instead of costing a whole tile of its own).
// ``grouped_expert_linear`` then computes, for every tile, Y[slot, :] = W[e] . X[row(slot)]^T on the
// matrix cores: each expert's [C, K] slab is read once per tile instead of once per slot. Every output
// row is an independent dot product, so the order of slots inside a group changes no result bit.
constexpr uint32_t kTallLastTile = 160;

// Tiles a table can hold: ceil(slots / 128) + experts covers every rule above.
__host__ __device__ constexpr uint32_t expert_tile_bound(uint32_t slots, uint32_t experts) { return (slots + 127u) / 128u + experts; }

// The tile count word of the table for ``last`` (its (expert, first row) pairs follow it, except in the
// first table, whose pairs follow the permutation).
__device__ __forceinline__ uint32_t expert_table_word(uint32_t slots, uint32_t experts, uint32_t last) {
    return last == 128u ? 2u * experts + 1u : 2u * experts + 2u + slots + 2u * expert_tile_bound(slots, experts);
}

__device__ __forceinline__ uint32_t expert_row_tiles(uint32_t count, uint32_t last) {
    return count == 0u ? 0u : 1u + (count > last ? (count - last + 127u) / 128u : 0u);
}

// Slots in the tile of an expert with ``count`` slots that starts at slot ``first`` (a multiple of 128).
__device__ __forceinline__ uint32_t expert_tile_rows(uint32_t count, uint32_t first, uint32_t last) {
    return count - first <= last ? count - first : 128u;
}

// The first kRouteHeld slots of each thread keep their expert in registers between the counting and the
// scattering pass (slots past blockDim x kRouteHeld read their id again). The per-expert counts,
// offsets and both tile tables come from the first wave, 64 experts at a time with wave prefix sums (the
// same entries, in the same places, as a walk over the experts in order).
constexpr uint32_t kRouteHeld = 16;

__device__ __forceinline__ void route_slots(const int64_t* __restrict__ indices, uint32_t slots, uint32_t experts,
                                            int32_t* __restrict__ scratch, unsigned int* error) {
    extern __shared__ int32_t shared_counts[];
    int32_t* counts = scratch;
    int32_t* offsets = scratch + experts;
    int32_t* tile_count = scratch + 2 * experts + 1;
    int32_t* permutation = tile_count + 1;
    int32_t* tiles = permutation + slots;
    for (uint32_t e = threadIdx.x; e < experts; e += blockDim.x) {
        shared_counts[e] = 0;
    }
    __syncthreads();
    uint32_t held[kRouteHeld];
#pragma unroll
    for (uint32_t i = 0; i < kRouteHeld; ++i) {
        const uint32_t t = threadIdx.x + i * blockDim.x;
        held[i] = 0;
        if (t < slots) {
            held[i] = uint32_t(checked_index(indices[t], experts, true, error));
            atomicAdd(&shared_counts[held[i]], 1);
        }
    }
    for (uint32_t t = threadIdx.x + kRouteHeld * blockDim.x; t < slots; t += blockDim.x) {
        atomicAdd(&shared_counts[uint32_t(checked_index(indices[t], experts, true, error))], 1);
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
        const uint32_t lane = threadIdx.x;
        int32_t* tall_count = scratch + expert_table_word(slots, experts, kTallLastTile);
        int32_t* tall = tall_count + 1;
        uint32_t running = 0, tile = 0, tall_tile = 0;  // totals of the experts before this step's 64
        for (uint32_t e0 = 0; e0 < experts; e0 += kWave) {
            const uint32_t e = e0 + lane;
            const uint32_t count = e < experts ? uint32_t(shared_counts[e]) : 0u;
            const uint32_t n = expert_row_tiles(count, 128u), m = expert_row_tiles(count, kTallLastTile);
            uint32_t c_in = count, n_in = n, m_in = m;  // inclusive prefix sums over the lanes
#pragma unroll
            for (int d = 1; d < kWave; d <<= 1) {
                const uint32_t c_up = __shfl_up(c_in, d, kWave), n_up = __shfl_up(n_in, d, kWave), m_up = __shfl_up(m_in, d, kWave);
                if (lane >= uint32_t(d)) {
                    c_in += c_up;
                    n_in += n_up;
                    m_in += m_up;
                }
            }
            if (e < experts) {
                const uint32_t offset = running + c_in - count, first = tile + n_in - n, first_tall = tall_tile + m_in - m;
                counts[e] = int32_t(count);
                offsets[e] = int32_t(offset);
                for (uint32_t t = 0; t < n; ++t) {
                    tiles[2 * (first + t)] = int32_t(e);
                    tiles[2 * (first + t) + 1] = int32_t(128u * t);
                }
                for (uint32_t t = 0; t < m; ++t) {
                    tall[2 * (first_tall + t)] = int32_t(e);
                    tall[2 * (first_tall + t) + 1] = int32_t(128u * t);
                }
                shared_counts[e] = int32_t(offset);  // the scatter's cursor
            }
            running += __shfl(c_in, kWave - 1, kWave);
            tile += __shfl(n_in, kWave - 1, kWave);
            tall_tile += __shfl(m_in, kWave - 1, kWave);
        }
        if (lane == 0) {
            offsets[experts] = int32_t(running);
            *tile_count = int32_t(tile);
            *tall_count = int32_t(tall_tile);
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t i = 0; i < kRouteHeld; ++i) {
        const uint32_t t = threadIdx.x + i * blockDim.x;
        if (t < slots) {
            permutation[atomicAdd(&shared_counts[held[i]], 1)] = int32_t(t);
        }
    }
    for (uint32_t t = threadIdx.x + kRouteHeld * blockDim.x; t < slots; t += blockDim.x) {
        int64_t raw = indices[t];
        raw = raw < 0 ? raw + int64_t(experts) : raw;
        const uint32_t e = (raw < 0 || raw >= int64_t(experts)) ? 0u : uint32_t(raw);
        permutation[atomicAdd(&shared_counts[e], 1)] = int32_t(t);
    }
}

// Logical order of the grouped products: expert by expert, and inside an expert column tile by column
// tile with that expert's row tiles adjacent, so the row tiles that share a slab of W[e] run together and
// an XCD's run of logical tiles reads each slab once. Expert e owns logical tiles
// [gx * first_e, gx * (first_e + n_e)), n_e = ceil(count_e / 128) row tiles starting at tile first_e of the
// routing table (n_e by ``expert_row_tiles`` with the routing's ``last``). Every wave finds (row tile,
// column tile) of ``logical`` with a wave-wide scan of the per-expert counts; ``logical`` < gx * (tile
// count) always has one.
__device__ __forceinline__ void expert_tile_of(const int32_t* __restrict__ counts, uint32_t experts, uint32_t gx,
                                               uint32_t logical, uint32_t& tile, uint32_t& column, uint32_t last) {
    const uint32_t lane = threadIdx.x % kWave;
    uint32_t carry = 0;
    tile = 0;
    column = 0;
    for (uint32_t e0 = 0; e0 < experts; e0 += kWave) {
        const uint32_t e = e0 + lane;
        const uint32_t n = e < experts ? expert_row_tiles(uint32_t(counts[e]), last) : 0u;
        uint32_t inclusive = n;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t up = __shfl_up(inclusive, d, kWave);
            inclusive += lane >= uint32_t(d) ? up : 0u;
        }
        const uint32_t first = carry + inclusive - n;
        const unsigned long long hit = __ballot(n > 0 && gx * first <= logical && logical < gx * (first + n));
        if (hit) {
            const int source = __ffsll(hit) - 1;
            const uint32_t f = __shfl(first, source, kWave), count = __shfl(n, source, kWave);
            const uint32_t r = logical - gx * f;
            column = r / count;
            tile = f + r % count;
            return;
        }
        carry += __shfl(inclusive, kWave - 1, kWave);
    }
}

// Per-slot input rows (``PER_SLOT``: X is [slots, K]) or per-token rows (X is [tokens, K], token = slot /
// selected). ``rows`` receives the A-row of each permuted slot and is filled by each workgroup before its
// product. One-dimensional launch of 8 * ceil(ceil(C / 128) * max tiles / 8) workgroups, mapped to tiles
// in the expert-major, XCD-aware order above; workgroups past gx * (tile count) return at once.
// PATH 3 is the ring body on 128-slot x BN-channel tiles on RWM x RWN waves (64 RWM RWN threads; bfloat16,
// K % 32 = 0, ``channels`` a multiple of BN), and on LAST-slot tiles (LAST = 160, RWM = 1: 10 row blocks of
// 16) for an expert's last tile when the routing was built with ``last`` = LAST; the two bodies share the
// kernel's one LDS array. The other paths take 128 x 128 tiles (LAST = 128).

template <int BN, int LAST = 128>
constexpr int ring_expert_slots() {
    return (LAST + BN) * 64 * 5 <= 150 * 1024 ? 5 : 4;
}

//
// An ``epilogue`` (ring path only) replaces the stores of Y: it is called for every slot of a tile and every
// 4 consecutive channels a lane holds, as mfma_gemm_ring describes, with the tile's expert as its tag (every
// slot of a tile is routed to that expert); ``out`` is then not written.
template <class T, bool PER_SLOT, int PATH = 0, int BN = 128, int RWM = 1, int RWN = 4, int LAST = 128,
          int RS = ring_expert_slots<BN, LAST>(), class Epilogue = std::nullptr_t>
__device__ __forceinline__ void grouped_expert_linear(const T* __restrict__ w, const T* __restrict__ x, T* __restrict__ out,
                                                      const int32_t* __restrict__ scratch, uint32_t slots, uint32_t selected,
                                                      uint32_t experts, uint32_t channels, uint32_t inner, Epilogue epilogue = nullptr) {
    static_assert(PATH == 3 || std::is_same_v<Epilogue, std::nullptr_t>, "epilogues on the ring path only");
    static_assert(PATH == 3 || BN == 128, "only the ring path takes wider channel tiles");
    static_assert(LAST == 128 || (PATH == 3 && LAST == int(kTallLastTile) && RWM == 1), "taller last tiles on the ring path only");
    const int32_t* offsets = scratch + experts;
    const uint32_t table = expert_table_word(slots, experts, LAST);
    const uint32_t tile_count = uint32_t(scratch[table]);
    const int32_t* permutation = scratch + 2 * experts + 2;
    const int32_t* tiles = LAST == 128 ? permutation + slots : scratch + table + 1;
    const uint32_t gx = (channels + BN - 1u) / BN;
    uint32_t logical;
    if (!xcd_logical_tile(gx * tile_count, logical)) {
        return;
    }
    uint32_t tile, column;
    expert_tile_of(scratch, experts, gx, logical, tile, column, LAST);
    const uint32_t expert = uint32_t(tiles[2 * tile]);
    const uint32_t first = uint32_t(tiles[2 * tile + 1]);
    const uint32_t count = uint32_t(offsets[expert + 1] - offsets[expert]);
    const uint32_t rows = expert_tile_rows(count, first, LAST);
    if constexpr (PATH == 3) {
        // the tile's slots are read straight from the permutation in global memory (the A row of a slot is
        // slot / selected for per-token inputs): the ring is then the kernel's only LDS array, and the
        // compiler can tell its fragment reads from the copies in flight (with other LDS arrays in the kernel
        // it made every fragment read wait for all outstanding copies, which serialised the pipeline)
        static_assert(sizeof(T) == 2, "the ring body takes bfloat16");
        const int32_t* slots_of_tile = permutation + offsets[expert] + first;
        __shared__ __attribute__((aligned(1024))) uint16_t ring[ring_elements<LAST, BN, RS>()];
        const T* slab = w + size_t(expert) * channels * inner;
        // the body for the tile's live 16-row blocks: 1, 2, 4 or 8 of a 128-slot tile, all of a taller last tile
        auto body = [&](auto bm, auto live) {
            mfma_gemm_ring<T, int(bm), BN, RWM, RWN, RS, int(live)>(x, inner, slab, inner, nullptr, out, channels, rows, channels, inner,
                                                                     slots_of_tile, slots_of_tile, 0u, column * BN,
                                                                     PER_SLOT ? 1u : selected, ring, epilogue, expert);
        };
        using I = std::integral_constant<int, 128>;
        if constexpr (LAST > 128) {
            if (rows > 128u) {
                body(std::integral_constant<int, LAST>{}, std::integral_constant<int, LAST / 16>{});
                return;
            }
        }
        if constexpr (RWM == 1) {
            if (rows <= 16u) {
                body(I{}, std::integral_constant<int, 1>{});
            } else if (rows <= 32u) {
                body(I{}, std::integral_constant<int, 2>{});
            } else if (rows <= 64u) {
                body(I{}, std::integral_constant<int, 4>{});
            } else {
                body(I{}, std::integral_constant<int, 8>{});
            }
        } else {
            body(I{}, std::integral_constant<int, 128 / RWM / 16>{});
        }
    } else {
        __shared__ int32_t a_rows[128], c_rows[128];
        for (uint32_t r = threadIdx.x; r < 128u; r += blockDim.x) {
            const int32_t slot = r < rows ? permutation[offsets[expert] + first + r] : 0;
            a_rows[r] = PER_SLOT ? slot : slot / int32_t(selected);
            c_rows[r] = slot;
        }
        __syncthreads();
        mfma_gemm<T, true, PATH>(x, inner, w + size_t(expert) * channels * inner, inner, nullptr, out, channels, rows, channels, inner,
                                 a_rows, c_rows, 0u, column * 128u);
    }
}

}  // namespace chroma
