// Fused grouped-query attention with sinks: the replacement for the reference workload's chain
//
//     s   = einsum("qhmd,khmd->hmqk", q, k) * scale + mask          (each step rounded to the storage type)
//     p   = softmax(cat([s, sink], -1), -1)[..., :-1]                (float statistics, p rounded)
//     out = einsum("hmqk,khmd->qhmd", p, v)                          (float accumulation, rounded once)
//
// (chroma/models/gpt_oss.py sdpa, chroma/models/cached.py:38-48, lowered by the reference into two
// contractions, two elementwise steps, a concatenation and a softmax: gpu.py:275-298, :390-424) without
// storing the [heads, queries, keys] scores. Every rounding point of the chain is kept: the scores, the
// scaled scores and the masked scores are rounded to the storage type, the softmax statistics are float,
// each probability is exp(x - max) / sum rounded to the storage type before it meets V, and the output
// sum is float. Two things differ from the reference: the order of the float sums, and, in the
// matrix-core kernels only, the quotient, which is exp(x - max) times the float reciprocal of the sum
// (attention_mfma_bf16: within one ulp of the correctly rounded quotient) or one exp2 whose exponent
// carries log2 of the sum (attention_heads_mfma_bf16: within a few ulps), before the rounding to the
// storage type.
#pragma once

#include "device.h"
#include "linear.h"

namespace chroma {

// Rounding of an intermediate value to the storage type (the values stay in registers or LDS; results
// written to memory go through f32_to_bf16).
template <bool BF16> __device__ __forceinline__ float storage_round(float x) {
    if constexpr (BF16) {
        return round_bf16_fast(x);
    } else {
        return x;
    }
}

// Online (max, sum of exp) update with -inf handled like the reference's two-pass softmax: a row whose
// values are all -inf keeps sum 0.
__device__ __forceinline__ void softmax_stats_add(float& peak, float& total, float x) {
    const float top = __builtin_fmaxf(peak, x);
    total = top == -__builtin_inff() ? 0.0f : total * fast_exp(peak - top) + fast_exp(x - top);
    peak = top;
}

// Merge the statistics (other_peak, other_total) of another set of values into (peak, total).
__device__ __forceinline__ void softmax_stats_merge(float& peak, float& total, float other_peak, float other_total) {
    const float top = __builtin_fmaxf(peak, other_peak);
    total = top == -__builtin_inff() ? 0.0f
                                     : (peak == -__builtin_inff() ? 0.0f : total * fast_exp(peak - top)) +
                                           (other_peak == -__builtin_inff() ? 0.0f : other_total * fast_exp(other_peak - top));
    peak = top;
}

// Scratch of the split-key form for one (query row, key/value head): per split the partial statistics
// [G][2] (max, sum of exp) and the partial sums p . v [G][D].
struct AttentionSplit {
    float* stats;
    float* partial;
    uint32_t splits, split;
};

// One workgroup computes one query row t for all G query heads of one key/value head (the caller fixes t
// and the head inside its loaders) over the keys [begin, end). Loaders: load_q(g, d), load_k(j, d),
// load_v(j, d), load_mask(j, g), load_sink(g) return floats (storage values widened); store(g, d, value)
// writes one rounded result.
//
// PHASE 0 (whole row): pass 1 computes thread-per-key scores and per-thread online statistics, reduced
// over the workgroup with the sink logit folded in; pass 2, per chunk of THREADS keys, writes
// thread-per-key probabilities to LDS, then threads arranged as KL key lanes x DG dimension groups (DS =
// D / DG consecutive dimensions each) accumulate p * v, and the key lanes are summed at the end.
// Long rows split their keys over workgroups: PHASE 1 writes each split's statistics (no sink), PHASE 2
// combines every split's statistics and the sink into the row's, then writes the split's p . v sums;
// ``attention_combine`` adds the splits in order. Every probability is the row's exp(x - max) / sum,
// rounded, in all phases.
template <int PHASE, int D, int G, int THREADS, bool BF16, class LoadQ, class LoadK, class LoadV, class LoadMask, class LoadSink, class Store>
__device__ __forceinline__ void attention_rows(uint32_t begin, uint32_t end, float scale, LoadQ load_q, LoadK load_k, LoadV load_v,
                                               LoadMask load_mask, LoadSink load_sink, Store store, AttentionSplit split) {
    constexpr int WAVES = THREADS / kWave;
    constexpr int DG = D >= 32 ? 8 : (D >= 8 ? D / 4 : 1);  // dimension groups
    constexpr int DS = D / DG;                               // dimensions per thread
    constexpr int KL = THREADS / DG < kWave ? THREADS / DG : kWave;  // key lanes of one group in a wave
    constexpr int SLABS = THREADS / (DG * KL);               // groups of key lanes summed through LDS
    static_assert(D % DG == 0 && THREADS % (DG * KL) == 0 && (KL & (KL - 1)) == 0, "attention_rows shape");
    __shared__ float q_s[G][D];
    __shared__ float p_s[G][THREADS];
    __shared__ float wave_peak[WAVES][G], wave_total[WAVES][G];
    __shared__ float peak_s[G], total_s[G];
    __shared__ float slab_s[SLABS > 1 ? SLABS : 1][G][D];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % kWave, wave = tid / kWave;
    const float neg_inf = -__builtin_inff();
    for (uint32_t i = tid; i < uint32_t(G * D); i += THREADS) {
        q_s[i / D][i % D] = load_q(i / D, i % D);
    }
    __syncthreads();

    // Masked score of key j for every head: s2[g]. The empty asm keeps the compiler from hoisting the
    // G x D query values out of the key loop into registers (they are LDS broadcasts, cheap to re-read).
    auto scores = [&](uint32_t j, float (&s2)[G]) {
        __asm__ volatile("" ::: "memory");
        float kd[D];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            kd[d] = load_k(j, d);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float dot = 0.0f;
#pragma unroll
            for (int d = 0; d < D; ++d) {
                dot += q_s[g][d] * kd[d];
            }
            const float s = storage_round<BF16>(dot);
            const float s1 = storage_round<BF16>(s * scale);
            s2[g] = storage_round<BF16>(s1 + load_mask(j, g));
        }
    };

    // ---- pass 1: statistics (phases 0 and 1)
    if constexpr (PHASE != 2) {
        float peak[G], total[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            peak[g] = neg_inf;
            total[g] = 0.0f;
        }
        for (uint32_t j = begin + tid; j < end; j += THREADS) {
            float s2[G];
            scores(j, s2);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                softmax_stats_add(peak[g], total[g], s2[g]);
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float top = wave_max(peak[g]);
            const float sum = wave_sum(peak[g] == neg_inf ? 0.0f : total[g] * fast_exp(peak[g] - top));
            if (lane == 0) {
                wave_peak[wave][g] = top;
                wave_total[wave][g] = sum;
            }
        }
        __syncthreads();
        if (tid < uint32_t(G)) {
            float top = neg_inf, sum = 0.0f;
            for (int w = 0; w < WAVES; ++w) {
                softmax_stats_merge(top, sum, wave_peak[w][tid], wave_total[w][tid]);
            }
            if constexpr (PHASE == 1) {
                split.stats[(split.split * G + tid) * 2] = top;
                split.stats[(split.split * G + tid) * 2 + 1] = sum;
            } else {
                softmax_stats_add(top, sum, load_sink(tid));
                peak_s[tid] = top;
                total_s[tid] = sum;
            }
        }
        if constexpr (PHASE == 1) {
            return;
        }
    } else {
        if (tid < uint32_t(G)) {
            float top = neg_inf, sum = 0.0f;
            for (uint32_t w = 0; w < split.splits; ++w) {
                softmax_stats_merge(top, sum, split.stats[(w * G + tid) * 2], split.stats[(w * G + tid) * 2 + 1]);
            }
            softmax_stats_add(top, sum, load_sink(tid));
            peak_s[tid] = top;
            total_s[tid] = sum;
        }
    }
    __syncthreads();

    // ---- pass 2: probabilities and p . v
    const uint32_t kl = tid % KL, dg = (tid / KL) % DG, slab = tid / (KL * DG);
    float acc[G][DS];
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < DS; ++e) {
            acc[g][e] = 0.0f;
        }
    }
    for (uint32_t base = begin; base < end; base += THREADS) {
        const uint32_t j = base + tid;
        if (j < end) {
            float s2[G];
            scores(j, s2);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                p_s[g][tid] = storage_round<BF16>(fast_exp(s2[g] - peak_s[g]) / total_s[g]);
            }
        }
        __syncthreads();
        const uint32_t count = end - base < uint32_t(THREADS) ? end - base : uint32_t(THREADS);
        for (uint32_t i = slab * KL + kl; i < count; i += KL * SLABS) {
            float vd[DS];
#pragma unroll
            for (int e = 0; e < DS; ++e) {
                vd[e] = load_v(base + i, dg * DS + e);
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float p = p_s[g][i];
#pragma unroll
                for (int e = 0; e < DS; ++e) {
                    acc[g][e] += p * vd[e];
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < DS; ++e) {
#pragma unroll
            for (int offset = KL / 2; offset > 0; offset >>= 1) {
                acc[g][e] += __shfl_xor(acc[g][e], offset, kWave);
            }
        }
    }
    // Results: phase 0 stores them, phase 2 writes the split's partial sums.
    auto emit = [&](uint32_t g, uint32_t d, float value) {
        if constexpr (PHASE == 2) {
            split.partial[(size_t(split.split) * G + g) * D + d] = value;
        } else {
            store(g, d, value);
        }
    };
    if constexpr (SLABS > 1) {
        if (kl == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
#pragma unroll
                for (int e = 0; e < DS; ++e) {
                    slab_s[slab][g][dg * DS + e] = acc[g][e];
                }
            }
        }
        __syncthreads();
        for (uint32_t i = tid; i < uint32_t(G * D); i += THREADS) {
            float sum = 0.0f;
            for (int w = 0; w < SLABS; ++w) {
                sum += slab_s[w][i / D][i % D];
            }
            emit(i / D, i % D, sum);
        }
    } else if (kl == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int e = 0; e < DS; ++e) {
                emit(g, dg * DS + e, acc[g][e]);
            }
        }
    }
}

// One query row and one key/value head per workgroup with one wave per query head (blockDim.x = 64 G):
// for short key ranges the wave's lanes split the keys and every reduction is a wave butterfly, so the
// workgroup synchronizes only once, after the query rows are staged. Same numerics as attention_rows.
template <int D, int G, bool BF16, class LoadQ, class LoadK, class LoadV, class LoadMask, class LoadSink, class Store>
__device__ __forceinline__ void attention_waves(uint32_t keys, float scale, LoadQ load_q, LoadK load_k, LoadV load_v, LoadMask load_mask,
                                                LoadSink load_sink, Store store) {
    __shared__ float q_s[G][D];
    const uint32_t tid = threadIdx.x, lane = tid % kWave, g = tid / kWave;
    const float neg_inf = -__builtin_inff();
    for (uint32_t i = tid; i < uint32_t(G * D); i += blockDim.x) {
        q_s[i / D][i % D] = load_q(i / D, i % D);
    }
    __syncthreads();
    float q[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        q[d] = q_s[g][d];
    }
    auto score = [&](uint32_t j) -> float {
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            dot += q[d] * load_k(j, d);
        }
        const float s = storage_round<BF16>(dot);
        const float s1 = storage_round<BF16>(s * scale);
        return storage_round<BF16>(s1 + load_mask(j, g));
    };
    // Each lane takes keys lane, lane + 64, ... in that order; U of them per batch, their loads issued
    // together (a batch's keys past the end read the last key and contribute nothing).
    constexpr int U = D <= 16 ? 8 : (D <= 32 ? 4 : 2);
    float peak = neg_inf, total = 0.0f;
    for (uint32_t j0 = lane; j0 < keys; j0 += U * kWave) {
        float s[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = j0 + u * kWave;
            s[u] = score(j < keys ? j : keys - 1);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (j0 + u * kWave < keys) {
                softmax_stats_add(peak, total, s[u]);
            }
        }
    }
#pragma unroll
    for (int offset = 1; offset < kWave; offset <<= 1) {
        softmax_stats_merge(peak, total, __shfl_xor(peak, offset, kWave), __shfl_xor(total, offset, kWave));
    }
    softmax_stats_add(peak, total, load_sink(g));
    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        acc[d] = 0.0f;
    }
    for (uint32_t j0 = lane; j0 < keys; j0 += U * kWave) {
        float p[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = j0 + u * kWave;
            p[u] = storage_round<BF16>(fast_exp(score(j < keys ? j : keys - 1) - peak) / total);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = j0 + u * kWave;
            if (j < keys) {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    acc[d] += p[u] * load_v(j, d);
                }
            }
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
        for (int offset = 1; offset < kWave; offset <<= 1) {
            acc[d] += __shfl_xor(acc[d], offset, kWave);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (lane == uint32_t(d) % kWave) {
            store(g, d, acc[d]);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Split-key attention for a few query rows over long key ranges (decode steps), reading the stored
// key/value rows with 16-byte loads: rows [0, past) come from memory (row j of this key/value head at
// rows + j * stride, elements contiguous and rows 16-byte aligned), rows [past, keys) from an LDS array
// of floats (the new rows, evaluated by the caller). Same numerics as ``attention_rows`` (scores rounded
// at each step, float statistics, probabilities rounded after the division by the row's sum, float
// output sums) with the float sums in another order.
template <class T> struct KeyRows {
    const T* rows;
    uint32_t stride, past;
    const float* fresh;
};

// Sum of v over the LPK consecutive lanes of a key group (LPK a power of two): DPP quad permutations,
// then the half-row and row mirrors (within a group whose quads already agree, a mirror partner holds the
// same quad sum as the xor partner), then permlane swaps across rows and half-waves, so every lane of the
// group holds the same sum, added in the order of an xor butterfly.
template <int LPK> __device__ __forceinline__ float key_group_sum(float v) {
    if constexpr (LPK >= 2) v += dpp_partner<0xB1>(v);   // lane ^ 1
    if constexpr (LPK >= 4) v += dpp_partner<0x4E>(v);   // lane ^ 2
    if constexpr (LPK >= 8) v += dpp_partner<0x141>(v);  // the other quad of each 8 lanes
    if constexpr (LPK >= 16) v += dpp_partner<0x140>(v); // the other half of each 16-lane row
    if constexpr (LPK >= 32) {
        const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(rows[0]) + __uint_as_float(rows[1]);
    }
    if constexpr (LPK >= 64) {
        const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(halves[0]) + __uint_as_float(halves[1]);
    }
    return v;
}

// Sum of v over the lanes of a wave that share lane % FROM (FROM a power of two), added in the order of an
// xor butterfly over the offsets FROM, 2 FROM, .., 32: lanes 8 apart meet through DPP (row_ror:8 within
// 16-lane rows), rows and half-waves through gfx950's permlane swaps; smaller offsets through
// ``__shfl_xor``.
template <int FROM> __device__ __forceinline__ float lane_groups_sum(float v) {
    if constexpr (FROM >= 8) {
        if constexpr (FROM == 8) {
            v += dpp_partner<0x128>(v);  // row_ror:8 = lane ^ 8 within each 16-lane row
        }
        if constexpr (FROM <= 16) {
            const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(rows[0]) + __uint_as_float(rows[1]);
        }
        if constexpr (FROM <= 32) {
            const auto halves = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(halves[0]) + __uint_as_float(halves[1]);
        }
        return v;
    } else {
#pragma unroll
        for (int offset = FROM; offset < kWave; offset <<= 1) {
            v += __shfl_xor(v, offset, kWave);
        }
        return v;
    }
}

// Workgroup: 4 waves over keys [begin, end) of one (query row, key/value head), end - begin <= SPAN. A
// key's D elements are LPK lanes x one 16-byte chunk each (N elements), so a wave takes 64 / LPK
// consecutive keys per load and every load instruction reads whole rows; a thread takes U keys, all
// requested at once. Query heads' dot products meet through the LPK lanes (DPP). PHASE 1 writes the
// masked scores of the keys ([keys][G] at ``scores``) and the split's statistics; PHASE 2 merges every
// split's statistics with the sink (32 lanes per head, each merging every 32nd split, then a butterfly),
// then writes the split's partial p . v sums, and the last split to finish adds the splits in order. Each
// phase requests its stored rows (and phase 2 its scores) before the barrier at which the workgroup
// decides whether the split is live, so that round trip overlaps the mask vote or the statistics merge;
// rows the staging prologue evaluated into LDS are read after that barrier. A split whose mask is -inf
// for every key and head computes nothing and writes no scores (its statistics are (-inf, 0) and its
// partial sums 0: exactly what its keys contribute as long as their rows are finite).
constexpr uint32_t kAttentionTicketWord = 64;  // first word of the decode attentions' tickets in the error region
constexpr uint32_t kAttentionTickets = 64;     // (query row, key/value head) rows with a ticket word

template <int PHASE, int D, int G, bool BF16, class T, int SPAN, class LoadQ, class LoadMask, class LoadSink, class Store>
__device__ __forceinline__ void attention_decode(uint32_t begin, uint32_t end, float scale, LoadQ load_q, KeyRows<T> k_rows,
                                                 KeyRows<T> v_rows, LoadMask load_mask, LoadSink load_sink, AttentionSplit split,
                                                 float* scores, Store store, unsigned int* ticket_word) {
    using C = Chunk16<T>;
    constexpr int N = C::N;
    constexpr int LPK = D / N;
    constexpr int KPW = kWave / LPK;
    constexpr int WAVES = 4;
    constexpr int U = (SPAN + WAVES * KPW - 1) / (WAVES * KPW);
    static_assert(D % N == 0 && LPK <= kWave && (LPK & (LPK - 1)) == 0 && U <= 8, "attention_decode shape");
    __shared__ float q_s[G][D];
    __shared__ float wave_peak[WAVES][G], wave_total[WAVES][G];
    __shared__ float peak_s[G], total_s[G];
    __shared__ float acc_s[WAVES][G][D];
    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t kq = lane / LPK, c = lane % LPK;
    const float neg_inf = -__builtin_inff();

    // A key's chunk: the stored row's 16 bytes, requested unconditionally (a new key requests the last
    // stored row instead, so no load waits inside a branch), widened after the barrier; a new key's
    // values come from the LDS rows the staging prologue evaluated.
    auto key_of = [&](int u) { return begin + uint32_t(u) * WAVES * KPW + wave * KPW + kq; };
    auto request = [&](const KeyRows<T>& source, uint32_t j) -> u32x4_t {
        const uint32_t row = j < source.past ? j : source.past - 1;
        return C::load(source.rows + size_t(row) * source.stride + c * N);
    };
    auto widen = [&](const KeyRows<T>& source, uint32_t j, const u32x4_t& bits, float (&out)[N]) {
        const bool stored = j < source.past;
        const uint32_t at = (stored ? 0u : j - source.past) * D + c * N;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            out[e] = stored ? C::get(bits, e) : source.fresh[at + e];
        }
    };

    if constexpr (PHASE == 1) {
        // Is any key of the split unmasked for any head? The query, the stored key rows and the mask
        // values of this thread's keys (which cover the split) are all requested before the barrier that
        // both publishes the staged queries and answers.
        // Element e of the query in the order (half of D, head, position in the half): a wave's 64
        // elements lie in one half of a head (the two sides of a rotary embedding), so the loader's
        // branch on the half does not diverge.
        constexpr uint32_t HALF = D / 2;
#pragma unroll
        for (uint32_t e = tid; e < uint32_t(G * D); e += WAVES * kWave) {
            const uint32_t half = e / (G * HALF), g = e % (G * HALF) / HALF, d = half * HALF + e % HALF;
            q_s[g][d] = load_q(g, d);
        }
        u32x4_t k_bits[U];
        float mk[U][G];
        bool live = false;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t jj = key_of(u) < end ? key_of(u) : end - 1;
            k_bits[u] = request(k_rows, jj);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                mk[u][g] = load_mask(jj, g);
                live |= key_of(u) < end && mk[u][g] != neg_inf;
            }
        }
        if (!__syncthreads_or(live)) {
            if (tid < uint32_t(G)) {
                split.stats[(split.split * G + tid) * 2] = neg_inf;
                split.stats[(split.split * G + tid) * 2 + 1] = 0.0f;
            }
            return;
        }
        float peak[G], total[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            peak[g] = neg_inf;
            total[g] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = key_of(u);
            float kv[N];
            widen(k_rows, j < end ? j : end - 1, k_bits[u], kv);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float dot = 0.0f;
#pragma unroll
                for (int e = 0; e < N; ++e) {
                    dot += q_s[g][c * N + e] * kv[e];
                }
                dot = key_group_sum<LPK>(dot);
                const float s = storage_round<BF16>(dot);
                const float s1 = storage_round<BF16>(s * scale);
                const float s2 = storage_round<BF16>(s1 + mk[u][g]);
                if (j < end) {
                    softmax_stats_add(peak[g], total[g], s2);
                    if (uint32_t(g % LPK) == c) {
                        scores[size_t(j) * G + g] = s2;
                    }
                }
            }
        }
        // The LPK lanes of a key group hold the same statistics: merge the key groups, then the waves.
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int offset = LPK; offset < kWave; offset <<= 1) {
                softmax_stats_merge(peak[g], total[g], __shfl_xor(peak[g], offset, kWave), __shfl_xor(total[g], offset, kWave));
            }
            if (lane == 0) {
                wave_peak[wave][g] = peak[g];
                wave_total[wave][g] = total[g];
            }
        }
        __syncthreads();
        if (tid < uint32_t(G)) {
            float top = neg_inf, sum = 0.0f;
            for (int w = 0; w < WAVES; ++w) {
                softmax_stats_merge(top, sum, wave_peak[w][tid], wave_total[w][tid]);
            }
            split.stats[(split.split * G + tid) * 2] = top;
            split.stats[(split.split * G + tid) * 2 + 1] = sum;
        }
    } else {
        // The stored value rows and the scores of this thread's keys go out first (a live split reads
        // them; a split without unmasked keys wrote no scores, and its loads are never used).
        u32x4_t v_bits[U];
        float sc[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t jj = key_of(u) < end ? key_of(u) : end - 1;
            v_bits[u] = request(v_rows, jj);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                sc[u][g] = scores[size_t(jj) * G + g];
            }
        }
        // The row's statistics: every split's, then the sink; the split is live if any head's own
        // statistics are.
        static_assert(G * 32 <= WAVES * kWave, "one 32-lane group per query head");
        bool live = false;
        {
            // the first FIRST splits of each lane (and this split's own peak) are requested together
            constexpr int FIRST = 2;
            const uint32_t g = tid / 32u, l = tid % 32u, gg = g < uint32_t(G) ? g : 0u;
            float top = neg_inf, sum = 0.0f;
            float split_peak[FIRST], split_total[FIRST];
#pragma unroll
            for (int i = 0; i < FIRST; ++i) {
                const uint32_t w = l + 32u * i < split.splits ? l + 32u * i : 0u;
                split_peak[i] = split.stats[(w * G + gg) * 2];
                split_total[i] = split.stats[(w * G + gg) * 2 + 1];
            }
            const float own_peak = split.stats[(split.split * G + gg) * 2];
            // a lane past the last split merges (-inf, 0), which changes nothing (the merges stay
            // unconditional so that the loads are not sunk into a branch)
#pragma unroll
            for (int i = 0; i < FIRST; ++i) {
                const bool real = l + 32u * i < split.splits;
                softmax_stats_merge(top, sum, real ? split_peak[i] : neg_inf, real ? split_total[i] : 0.0f);
            }
            if (g < uint32_t(G)) {
                for (uint32_t w = l + 32u * FIRST; w < split.splits; w += 32u) {
                    softmax_stats_merge(top, sum, split.stats[(w * G + g) * 2], split.stats[(w * G + g) * 2 + 1]);
                }
            }
#pragma unroll
            for (int offset = 16; offset > 0; offset >>= 1) {
                softmax_stats_merge(top, sum, __shfl_xor(top, offset, kWave), __shfl_xor(sum, offset, kWave));
            }
            if (g < uint32_t(G) && l == 0) {
                softmax_stats_add(top, sum, load_sink(g));
                peak_s[g] = top;
                total_s[g] = sum;
                live = own_peak != neg_inf;
            }
        }
        float* partial = split.partial + size_t(split.split) * G * D;
        // The last split to finish adds every split's partial sums in split order (``attention_combine``'s
        // sum) and returns the ticket word to 0; the partial sums pass between workgroups through
        // device-scope stores and loads around the ticket.
        auto finish = [&]() {
            device_stores_complete();
            __shared__ unsigned int ticket_s;
            __syncthreads();
            if (tid == 0) {
                ticket_s = atomicAdd(ticket_word, 1u);
            }
            __syncthreads();
            if (ticket_s != split.splits - 1) {
                return;
            }
            constexpr uint32_t BATCH = 64;  // splits whose loads go out together
            for (uint32_t i = tid; i < uint32_t(G * D); i += blockDim.x) {
                float sum = 0.0f;
                for (uint32_t s0 = 0; s0 < split.splits; s0 += BATCH) {
                    float part[BATCH];
#pragma unroll
                    for (uint32_t j = 0; j < BATCH; ++j) {
                        const uint32_t s = s0 + j < split.splits ? s0 + j : split.splits - 1;
                        part[j] = load_device(split.partial + size_t(s) * G * D + i);
                    }
#pragma unroll
                    for (uint32_t j = 0; j < BATCH; ++j) {
                        if (s0 + j < split.splits) {
                            sum += part[j];
                        }
                    }
                }
                store(i / D, i % D, sum);
            }
            if (tid == 0) {
                atomicExch(ticket_word, 0u);
            }
        };
        if (!__syncthreads_or(live)) {
            for (uint32_t i = tid; i < uint32_t(G * D); i += blockDim.x) {
                store_device(partial + i, 0.0f);
            }
            finish();
            return;
        }
        float acc[G][N];
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int e = 0; e < N; ++e) {
                acc[g][e] = 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = key_of(u);
            float vv[N];
            widen(v_rows, j < end ? j : end - 1, v_bits[u], vv);
            if (j < end) {
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = storage_round<BF16>(fast_exp(sc[u][g] - peak_s[g]) / total_s[g]);
#pragma unroll
                    for (int e = 0; e < N; ++e) {
                        acc[g][e] += p * vv[e];
                    }
                }
            }
        }
        // Sum the key groups of the wave, then the waves.
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int e = 0; e < N; ++e) {
                acc[g][e] = lane_groups_sum<LPK>(acc[g][e]);
            }
        }
        if (kq == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
#pragma unroll
                for (int e = 0; e < N; ++e) {
                    acc_s[wave][g][c * N + e] = acc[g][e];
                }
            }
        }
        __syncthreads();
        for (uint32_t i = tid; i < uint32_t(G * D); i += blockDim.x) {
            float sum = 0.0f;
            for (int w = 0; w < WAVES; ++w) {
                sum += acc_s[w][i / D][i % D];
            }
            store_device(partial + i, sum);
        }
        finish();
    }
}

// The split-key result: out(g, d) = sum over splits, in split order, of the partial p . v sums.
template <int D, int G, class Store>
__device__ __forceinline__ void attention_combine(const float* partial, uint32_t splits, Store store) {
    for (uint32_t i = threadIdx.x; i < uint32_t(G * D); i += blockDim.x) {
        float sum = 0.0f;
        for (uint32_t s = 0; s < splits; ++s) {
            sum += partial[size_t(s) * G * D + i];
        }
        store(i / D, i % D, sum);
    }
}

// ---------------------------------------------------------------------------------------------
// Matrix-core attention for long bfloat16 query blocks (the prefill of a cached export): the same
// computation as ``attention_rows`` with the two contractions on v_mfma_f32_16x16x32_bf16.
//
// Workgroup: 4 waves = 64 queries of one head (grid.x: kv_head * group + g, grid.y: query blocks);
// keys in blocks of 32, staged in LDS (K row-major, V transposed). Each wave computes
// S^T[32 keys x 16 queries] = K . Q^T as two 16 x 16 tiles (lane l ends with keys 4(l/16)+r and
// 16+4(l/16)+r of query l%16), so its own accumulators, rounded, become the B operand of
// O^T[D x 16] = V^T . P^T once the 32 keys are ordered as slot 8a+b -> key (b < 4 ? 4a+b : 16+4a+b-4);
// the A operand reads V^T in that order. Pass 1 accumulates (max, sum of exp) per query, pass 2
// recomputes the scores and accumulates p . v. A key block whose mask is -inf for every query of the
// workgroup is skipped in both passes: its probabilities are exactly 0, so skipping it changes no bit as
// long as the skipped K/V rows are finite (a NaN there would have poisoned the reference's sum).
//
// Operands: q [T, KV, G, D] with strides (qt, qh, qg, 1); keys and values as rows [.., KV, D] with row
// strides (past rows [0, past), new rows [past, keys)); mask[t, j] at mask + t*mt + kv*mh + g*mg + j;
// sinks at sinks + kv*sh + g*sg; out [T, KV, G, D] contiguous. Row strides and bases keep 16-byte alignment.
struct AttentionOperands {
    const uint16_t* q;
    uint32_t qt, qh, qg;
    const uint16_t *k_past, *k_new, *v_past, *v_new;
    uint32_t kpj, kph, knj, knh, vpj, vph, vnj, vnh;
    const uint16_t* mask;
    uint32_t mt, mh, mg;
    const uint16_t* sinks;
    uint32_t sh, sg;
    uint16_t* out;
    uint32_t tokens, past, keys, kv_heads, group;
    float scale;
    const uint8_t* live_blocks;  // [query blocks][key blocks]: 0 where the mask is -inf throughout (or nullptr)
};

// live_blocks[qb * key_blocks + kb] for queries [64 qb, 64 qb + 64) and keys [32 kb, 32 kb + 32) of a mask
// shared by every head: 0 when every mask value there is -inf, 2 when every one is +0.0 (the block needs
// no mask reads: adding +0.0 to a score changes no bit), 1 otherwise (grid: query blocks x key blocks).
__device__ __forceinline__ void attention_live_blocks(const uint16_t* __restrict__ mask, uint32_t mt, uint32_t tokens, uint32_t keys,
                                                      uint8_t* __restrict__ live_blocks) {
    const uint32_t qb = blockIdx.x, kb = blockIdx.y;
    bool any = false, zero = true;
    for (uint32_t i = threadIdx.x; i < 64u * 32u; i += blockDim.x) {
        const uint32_t t = qb * 64u + i / 32u, j = kb * 32u + i % 32u;
        if (t < tokens && j < keys) {
            const uint16_t bits = mask[size_t(t) * mt + j];
            any |= bits != 0xff80u;
            zero &= bits == 0u;
        }
    }
    any = __syncthreads_or(any);
    zero = __syncthreads_and(zero);
    if (threadIdx.x == 0) {
        live_blocks[qb * gridDim.y + kb] = any ? (zero ? 2 : 1) : 0;
    }
}

// Longest live-block list a workgroup keeps in LDS (key blocks of 32, so 64K keys); longer key ranges
// scan the table in place.
constexpr uint32_t kLiveListMax = 2048;

template <int D> __device__ __forceinline__ void attention_mfma_bf16(const AttentionOperands& a) {
    static_assert(D % 32 == 0 && D <= 128, "head dimension");
    constexpr int KB = 32, KPAD = D + 8, VPAD = KB + 8;
    constexpr uint32_t CHUNKS = (KB * D / 8 + 255) / 256;  // 16-byte K (and V) chunks each thread stages per block
    __shared__ __attribute__((aligned(16))) uint16_t k_s[KB * KPAD];
    __shared__ __attribute__((aligned(16))) uint16_t v_s[D * VPAD];
    __shared__ uint16_t live_list[kLiveListMax];
    __shared__ uint32_t live_total;
    const uint32_t tid = threadIdx.x, lane = tid % 64u, wave = tid / 64u, quad = lane / 16u, col = lane % 16u;
    // grid (query heads, query blocks), dispatched x fastest: later query blocks see more keys under a causal
    // mask, and every head's are dispatched before any head's earlier ones
    const uint32_t head = blockIdx.x, kv = head / a.group, g = head % a.group;
    const uint32_t query_block = gridDim.y - 1u - blockIdx.y;
    const uint32_t block_q0 = query_block * 64u;
    const uint32_t query = block_q0 + wave * 16u + col;
    const bool live = query < a.tokens;
    const uint32_t qrow = live ? query : a.tokens - 1u;

    bf16x8_t qf[D / 32];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
        qf[ks] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(a.q + size_t(qrow) * a.qt + kv * a.qh + g * a.qg + ks * 32u + quad * 8u));
    }
    const uint16_t* mask_row = a.mask + size_t(qrow) * a.mt + kv * a.mh + g * a.mg;
    const float neg_inf = -__builtin_inff();

    // Every global read below is unconditional, its index clamped into range, and what lies out of range
    // is replaced when the data is consumed: a guarded load would end its own branch with a wait for every
    // outstanding load, the prefetched block's included.
    // Mask words of this lane's 8 scores in key block kb, and their values (-inf past the last key or query).
    auto mask_fetch = [&](uint32_t kb, uint32_t (&raw)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t j = kb * KB + (i < 4 ? quad * 4u + i : 16u + quad * 4u + (i - 4));
            raw[i] = mask_row[j < a.keys ? j : a.keys - 1u];
        }
    };
    auto mask_values = [&](uint32_t kb, const uint32_t (&raw)[8], float (&m)[8], bool zero = false) -> bool {
        bool any = false;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t j = kb * KB + (i < 4 ? quad * 4u + i : 16u + quad * 4u + (i - 4));
            m[i] = (live && j < a.keys) ? (zero ? 0.0f : __uint_as_float(raw[i] << 16)) : neg_inf;
            any |= m[i] != neg_inf;
        }
        return any;
    };
    auto masks = [&](uint32_t kb, float (&m)[8]) -> bool {
        uint32_t raw[8];
        mask_fetch(kb, raw);
        return mask_values(kb, raw, m);
    };
    // Global -> registers: this thread's K (and V) chunks of key block kb; bit i of ``valid`` says whether
    // chunk i is a real key row (``put`` writes zeros for the others).
    auto fetch = [&](uint32_t kb, bool values, uint4 (&rk)[CHUNKS], uint4 (&rv)[CHUNKS], uint32_t& valid) {
        valid = 0;
#pragma unroll
        for (uint32_t i = 0; i < CHUNKS; ++i) {
            const uint32_t c = tid + i * 256u;
            const uint32_t cc = c < uint32_t(KB * D / 8) ? c : 0u;
            const uint32_t r = cc / (D / 8), dc = (cc % (D / 8)) * 8u, j = kb * KB + r;
            const uint32_t jj = j < a.keys ? j : a.keys - 1u;
            const bool old = jj < a.past;
            const size_t kr = old ? size_t(jj) * a.kpj + kv * a.kph : size_t(jj - a.past) * a.knj + kv * a.knh;
            rk[i] = *reinterpret_cast<const uint4*>((old ? a.k_past : a.k_new) + kr + dc);
            if (values) {
                const size_t vr = old ? size_t(jj) * a.vpj + kv * a.vph : size_t(jj - a.past) * a.vnj + kv * a.vnh;
                rv[i] = *reinterpret_cast<const uint4*>((old ? a.v_past : a.v_new) + vr + dc);
            }
            valid |= uint32_t(c < uint32_t(KB * D / 8) && j < a.keys) << i;
        }
    };
    // Registers -> LDS: K row-major, V transposed.
    auto put = [&](bool values, const uint4 (&rk)[CHUNKS], const uint4 (&rv)[CHUNKS], uint32_t valid) {
#pragma unroll
        for (uint32_t i = 0; i < CHUNKS; ++i) {
            const uint32_t c = tid + i * 256u;
            if (c < uint32_t(KB * D / 8)) {
                const uint32_t r = c / (D / 8), dc = (c % (D / 8)) * 8u;
                const bool ok = (valid >> i) & 1u;
                *reinterpret_cast<uint4*>(&k_s[r * KPAD + dc]) = ok ? rk[i] : uint4{0, 0, 0, 0};
                if (values) {
                    const uint4 v = ok ? rv[i] : uint4{0, 0, 0, 0};
                    const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
                    for (int x = 0; x < 8; ++x) {
                        v_s[(dc + x) * VPAD + r] = e[x];
                    }
                }
            }
        }
    };
    // Masked scores s2 of this lane's 8 (key, query) pairs.
    auto scores = [&](const float (&m)[8], float (&s2)[8]) {
        f32x4_t acc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                const bf16x8_t kf = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&k_s[(t * 16u + col) * KPAD + ks * 32u + quad * 8u]));
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], acc[t], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float s = round_bf16_fast(acc[i / 4][i % 4]);
            const float s1 = round_bf16_fast(s * a.scale);
            s2[i] = round_bf16_fast(s1 + m[i]);
        }
    };

    // The key blocks this workgroup visits: from the live-block table, compacted into LDS by wave 0 with a
    // ballot per 64 blocks (in key order); without a table (or past the list's capacity) every block, each
    // checked against its mask values with a workgroup-wide vote.
    const uint32_t blocks = (a.keys + KB - 1) / KB;
    const bool listed = a.live_blocks != nullptr && blocks <= kLiveListMax;
    if (listed) {
        if (wave == 0) {
            const uint8_t* row = a.live_blocks + size_t(query_block) * blocks;
            uint32_t n = 0;
            for (uint32_t base = 0; base < blocks; base += 64u) {
                const uint32_t kb = base + lane;
                const uint8_t state = kb < blocks ? row[kb] : 0;
                const unsigned long long bits = __ballot(state != 0);
                if (state != 0) {
                    live_list[n + uint32_t(__popcll(bits & ((1ull << lane) - 1ull)))] = uint16_t(kb | (state == 2 ? 0x8000u : 0u));
                }
                n += uint32_t(__popcll(bits));
            }
            if (lane == 0) {
                live_total = n;
            }
        }
        __syncthreads();
    }
    const uint32_t visits = listed ? live_total : 0u;

    // One pass over the visited blocks. A listed block's K (and V) chunks and mask values are fetched one
    // block ahead, into registers, while the current block is scored; ``body`` gets the block's mask values.
    auto sweep = [&](bool values, auto&& body) {
        uint4 rk[CHUNKS], rv[CHUNKS];
        uint32_t valid = 0;
        if (listed) {
            // separate loops for the two cases: a join of both inside one loop makes the compiler copy
            // the prefetched registers at the join, which waits for the loads
            // (the fetch after the last block re-reads that block, so no branch joins the prefetched registers)
            // Blocks flagged all-zero read no mask words.
            uint32_t raw[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (visits > 0) {
                const uint32_t first = live_list[0];
                fetch(first & 0x7fffu, values, rk, rv, valid);
                if (!(first & 0x8000u)) {
                    mask_fetch(first, raw);
                }
            }
            for (uint32_t i = 0; i < visits; ++i) {
                const uint32_t entry = live_list[i];
                float m[8];
                mask_values(entry & 0x7fffu, raw, m, (entry & 0x8000u) != 0);
                __syncthreads();  // every wave is done reading the previous block's tiles
                put(values, rk, rv, valid);
                const uint32_t next = live_list[i + 1 < visits ? i + 1 : i];
                fetch(next & 0x7fffu, values, rk, rv, valid);
                if (!(next & 0x8000u)) {
                    mask_fetch(next & 0x7fffu, raw);
                }
                __syncthreads();
                body(m);
            }
        } else {
            for (uint32_t kb = 0; kb < blocks; ++kb) {
                float m[8];
                if (!__syncthreads_or(masks(kb, m))) {
                    continue;
                }
                fetch(kb, values, rk, rv, valid);
                put(values, rk, rv, valid);
                __syncthreads();
                body(m);
            }
        }
    };

    float peak = neg_inf, total = 0.0f;
    sweep(false, [&](const float (&m)[8]) {
        float s2[8];
        scores(m, s2);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            softmax_stats_add(peak, total, s2[i]);
        }
    });
    // Combine the four lane groups that share a query, then fold in the sink.
#pragma unroll
    for (int offset = 16; offset < 64; offset <<= 1) {
        const float other_peak = __shfl_xor(peak, offset, kWave), other_total = __shfl_xor(total, offset, kWave);
        const float top = __builtin_fmaxf(peak, other_peak);
        total = top == neg_inf ? 0.0f
                               : (peak == neg_inf ? 0.0f : total * fast_exp(peak - top)) +
                                     (other_peak == neg_inf ? 0.0f : other_total * fast_exp(other_peak - top));
        peak = top;
    }
    softmax_stats_add(peak, total, bf16_to_f32(a.sinks[kv * a.sh + g * a.sg]));
    const float inverse = 1.0f / total;

    f32x4_t o[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        o[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    sweep(true, [&](const float (&m)[8]) {
        float s2[8];
        scores(m, s2);
        bf16x8_t pf;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pf[i] = __builtin_bit_cast(__bf16, f32_to_bf16(fast_exp(s2[i] - peak) * inverse));
        }
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            const uint16_t* row = &v_s[(dt * 16u + col) * VPAD];
            const uint2 lo = *reinterpret_cast<const uint2*>(row + quad * 4u);
            const uint2 hi = *reinterpret_cast<const uint2*>(row + 16u + quad * 4u);
            const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, uint4{lo.x, lo.y, hi.x, hi.y});
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[dt], 0, 0, 0);
        }
    });
    if (live) {
        uint16_t* dst = a.out + ((size_t(query) * a.kv_heads + kv) * a.group + g) * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            const uint32_t d = dt * 16u + quad * 4u;
            const uint32_t w0 = uint32_t(f32_to_bf16(o[dt][0])) | (uint32_t(f32_to_bf16(o[dt][1])) << 16);
            const uint32_t w1 = uint32_t(f32_to_bf16(o[dt][2])) | (uint32_t(f32_to_bf16(o[dt][3])) << 16);
            *reinterpret_cast<uint2*>(dst + d) = uint2{w0, w1};
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Matrix-core attention for long bfloat16 prefills, one workgroup per (16-query tile, key/value head) and
// one wave per HPW query heads of the group: the K tile, the V^T tile and the mask tile of each 64-key block
// are staged into LDS once and serve all G heads (the head-parallel form stages them once per head). With
// HPW = 2 every K and V^T fragment a wave reads from LDS feeds the products of both its heads, halving the
// LDS reads per score (which bound the one-head form); each head's arithmetic is unchanged, so the results
// are bit-identical. Mask
// shared by every head (mh = mg = 0). Same computation as attention_mfma_bf16 and the reference chain:
// S^T = K . Q^T on v_mfma_f32_16x16x32_bf16, each score rounded to bfloat16, scaled and rounded, masked
// and rounded (gfx950's v_cvt_pk_bf16_f32 rounds two values at once, to nearest even like f32_to_bf16);
// pass 1 accumulates (max, sum of exp) per query in float, pass 2 forms p = exp(s - max) / sum as
// 2^(s log2(e) - max log2(e) - log2(sum)) - one multiply-add and one v_exp_f32, within a few float ulps
// of the quotient, far below the bfloat16 rounding p then gets - and O^T += V^T . P^T; the output is
// rounded once.
// The 64-key blocks a query tile visits come from ``attention_live_tiles`` (blocks whose mask is -inf
// throughout are never read); a visited block's next block is staged into the other LDS buffer while it
// is computed, so each block costs one barrier. Key rows past ``keys`` are zeros with a -inf mask, queries
// past ``tokens`` see only -inf and are not stored.
//
// Two steps of the chain are the identity where their operands allow it, and are then left out:
//  * a block whose mask entries are all +0.0 or -0.0 (every causal block below the diagonal): adding a
//    zero and rounding changes no bfloat16 value (only -0 may become +0, and every later use - a max, a
//    difference with the max, exp - gives the same result for either zero), so the block reads no mask;
//  * a power-of-two scale <= 1 (POW2; 1/8 at head dimension 64): the product of a bfloat16 value and the
//    scale is a bfloat16 value whenever it is a normal float, so its rounding is left out and the scale
//    is applied inside the one fused multiply-add that forms s - max. Below the normal range (|s| <
//    2^-126) the unrounded product may differ from the rounded one in its last bits; every exp it feeds
//    is then exp of a difference below 2^-25 in magnitude or of a difference the tiny term does not change,
//    so the probabilities and the output are the same.
// Scores are kept in "u" units: s = u * cs, with cs the scale when its rounding is left out, else 1
// (u is then the masked score itself); u - max/cs never forms: s - max is fma(u, cs, -max), exact in u*cs.

constexpr uint32_t kLiveTilesMax = 1024;  // 64-key blocks a workgroup lists in LDS (64K keys)

// live_tiles[qt * key_blocks + kb] for queries [16 qt, 16 qt + 16) and keys [64 kb, 64 kb + 64) of a mask
// shared by every head: 0 when every entry there is -inf, 2 when every key of the block is below ``keys``
// and every entry is a zero (+0.0 or -0.0), else 1 (grid: query tiles x key blocks).
__device__ __forceinline__ void attention_live_tiles(const uint16_t* __restrict__ mask, uint32_t mt, uint32_t tokens, uint32_t keys,
                                                     uint8_t* __restrict__ live_tiles) {
    const uint32_t qt = blockIdx.x, kb = blockIdx.y;
    bool any = false, zero = kb * 64u + 64u <= keys;
    for (uint32_t i = threadIdx.x; i < 16u * 64u; i += blockDim.x) {
        const uint32_t t = qt * 16u + i / 64u, j = kb * 64u + i % 64u;
        if (t < tokens && j < keys) {
            const uint16_t bits = mask[size_t(t) * mt + j];
            any |= bits != 0xff80u;
            zero &= (bits & 0x7fffu) == 0u;
        }
    }
    any = __syncthreads_or(any);
    zero = __syncthreads_and(zero);
    if (threadIdx.x == 0) {
        live_tiles[qt * gridDim.y + kb] = any ? (zero ? 2 : 1) : 0;
    }
}

// The same table from one wave per tile and 16-byte loads (12,288 tiles of a C5 mask: 24.6 us with four
// workgroup barriers and 2-byte loads per tile): lane l reads row 16 qt + l / 4 at keys 64 kb + 16 (l % 4)
// .. + 15 as two 16-byte chunks, and the wave meets by ballot. Requires ``mt`` and the mask's element offset
// to be multiples of 8 (launched with 64 threads).
__device__ __forceinline__ void attention_live_tiles_wave(const uint16_t* __restrict__ mask, uint32_t mt, uint32_t tokens, uint32_t keys,
                                                          uint8_t* __restrict__ live_tiles) {
    const uint32_t qt = blockIdx.x, kb = blockIdx.y, lane = threadIdx.x % kWave;
    const uint32_t t = qt * 16u + lane / 4u;
    bool any = false, zero = true;
    if (t < tokens) {
#pragma unroll
        for (uint32_t h = 0; h < 2u; ++h) {
            const uint32_t j = kb * 64u + (lane % 4u) * 16u + h * 8u;
            if (j + 8u <= keys) {
                const uint4 v = *reinterpret_cast<const uint4*>(mask + size_t(t) * mt + j);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t bits = (w[e / 2] >> (16 * (e % 2))) & 0xffffu;
                    any |= bits != 0xff80u;
                    zero &= (bits & 0x7fffu) == 0u;
                }
            } else {
                for (uint32_t e = 0; e < 8u && j + e < keys; ++e) {
                    const uint16_t bits = mask[size_t(t) * mt + j + e];
                    any |= bits != 0xff80u;
                    zero &= (bits & 0x7fffu) == 0u;
                }
            }
        }
    }
    const bool live = __ballot(any) != 0ull;
    const bool zeros = kb * 64u + 64u <= keys && __ballot(!zero) == 0ull;
    if (lane == 0) {
        live_tiles[qt * gridDim.y + kb] = live ? (zeros ? 2 : 1) : 0;
    }
}

template <int D, int G, bool POW2, int HPW = 1> __device__ __forceinline__ void attention_heads_mfma_bf16(const AttentionOperands& a) {
    static_assert(D % 32 == 0 && D <= 128 && G >= 1 && G <= 8, "head dimension and group");
    static_assert((HPW == 1 || HPW == 2) && G % HPW == 0, "one or two query heads per wave");
    constexpr int QT = 16, KB = 64, THREADS = 64 * G / HPW;
    // K rows unpadded, their 16-byte chunk c stored at c ^ ((row / 2) & KSWZ) (KSWZ keeps it inside the
    // row): the 16-byte K fragment reads then hit no bank twice (with 144-byte padded rows they accounted
    // for every SQ_LDS_BANK_CONFLICT cycle of the kernel, 1.1x its LDS-active cycles). V^T rows of 136
    // bytes: a fragment read's 16 lanes (one V^T row each, 8 bytes) land on distinct bank pairs. Full C5
    // layer 196 -> 182 us.
    constexpr int KPAD = D, VPAD = KB + 4, MPAD = KB + 4;
    constexpr uint32_t KSWZ = ((D / 8) & 7) == 0 ? 7u : ((D / 8) & 3) == 0 ? 3u : 1u;
    constexpr int CHUNKS = (KB * D / 8 + THREADS - 1) / THREADS;  // 16-byte K (and V) chunks per thread per block
    constexpr int MASKS = (QT * KB + THREADS - 1) / THREADS;      // mask entries per thread per block
    constexpr uint32_t MASKED = 0x8000u;                           // list entry flag: the block reads its mask
    constexpr float kLog2e = 1.44269504088896341f;
    __shared__ __attribute__((aligned(16))) uint16_t k_s[2][KB * KPAD];
    __shared__ __attribute__((aligned(16))) uint16_t v_s[2][D * VPAD];
    __shared__ __attribute__((aligned(16))) uint16_t m_s[2][QT * MPAD];
    __shared__ uint16_t live_list[kLiveTilesMax];
    __shared__ uint32_t live_total;
    // wave w serves query heads HPW w .. HPW w + HPW - 1 of the group: with two, each K and V^T fragment read
    // from LDS feeds both heads' matrix-core products (the LDS reads per score, which bound the one-head form,
    // are halved)
    const uint32_t tid = threadIdx.x, lane = tid % 64u, wave = tid / 64u, g0 = wave * HPW, quad = lane / 16u, col = lane % 16u;
    // grid (KV heads, query tiles): workgroups are dispatched x fastest, so every head's tile t is dispatched
    // before any head's tile t - 1, and later query tiles (more keys) go first across all heads
    const uint32_t kv = blockIdx.x;
    const uint32_t tile = gridDim.y - 1u - blockIdx.y;
    const uint32_t q0 = tile * QT, query = q0 + col;
    const bool live = query < a.tokens;
    const uint32_t qrow = live ? query : a.tokens - 1u;
    const float neg_inf = -__builtin_inff();

    bf16x8_t qf[HPW][D / 32];
#pragma unroll
    for (int hd = 0; hd < HPW; ++hd) {
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            qf[hd][ks] = __builtin_bit_cast(
                bf16x8_t, *reinterpret_cast<const uint4*>(a.q + size_t(qrow) * a.qt + kv * a.qh + (g0 + hd) * a.qg + ks * 32u + quad * 8u));
        }
    }

    // The 64-key blocks this tile visits, in key order, each with the MASKED flag unless its mask is all
    // zeros: wave 0 compacts its row of the live table with a ballot per 64 blocks; without a table (or
    // past the list's capacity) every block, each reading its mask.
    const uint32_t blocks = (a.keys + KB - 1) / KB;
    const bool listed = a.live_blocks != nullptr && blocks <= kLiveTilesMax;
    if (listed) {
        if (wave == 0) {
            const uint8_t* row = a.live_blocks + size_t(tile) * blocks;
            uint32_t n = 0;
            for (uint32_t base = 0; base < blocks; base += 64u) {
                const uint32_t kb = base + lane;
                const uint32_t state = kb < blocks ? row[kb] : 0u;
                const bool on = state != 0;
                const unsigned long long bits = __ballot(on);
                if (on) {
                    live_list[n + uint32_t(__popcll(bits & ((1ull << lane) - 1ull)))] = uint16_t(kb | (state == 1 ? MASKED : 0u));
                }
                n += uint32_t(__popcll(bits));
            }
            if (lane == 0) {
                live_total = n;
            }
        }
        __syncthreads();
    }
    const uint32_t visits = listed ? live_total : blocks;
    // (block index | MASKED) of visit i; uniform over the workgroup, so every branch on it is scalar
    auto entry_of = [&](uint32_t i) -> uint32_t { return listed ? uint32_t(live_list[i]) : (i | MASKED); };

    // Global -> registers (every load unconditional, its index clamped; what lies out of range is replaced
    // when stored to LDS), then registers -> LDS buffer: K row-major, V transposed, mask [query][key].
    uint4 rk[CHUNKS], rv[CHUNKS];
    uint16_t rm[MASKS];
    auto fetch = [&](uint32_t entry, bool values) {
        const uint32_t kb = entry & ~MASKED;
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const uint32_t c = tid + i * THREADS;
            const uint32_t cc = c < uint32_t(KB * D / 8) ? c : 0u;
            // K: 8 lanes per key row (a row's 16-byte chunks side by side); V: the 64 keys of one 8-column
            // chunk side by side, so the transposed LDS writes of a wave are contiguous (see ``put``)
            const uint32_t r = cc / (D / 8), dc = (cc % (D / 8)) * 8u, j = kb * KB + r;
            const uint32_t jj = j < a.keys ? j : a.keys - 1u;
            const bool old = jj < a.past;
            const size_t kr = old ? size_t(jj) * a.kpj + kv * a.kph : size_t(jj - a.past) * a.knj + kv * a.knh;
            rk[i] = *reinterpret_cast<const uint4*>((old ? a.k_past : a.k_new) + kr + dc);
            if (values) {
                const uint32_t vj = kb * KB + cc % KB, vdc = (cc / KB) * 8u;
                const uint32_t vjj = vj < a.keys ? vj : a.keys - 1u;
                const bool vold = vjj < a.past;
                const size_t vr = vold ? size_t(vjj) * a.vpj + kv * a.vph : size_t(vjj - a.past) * a.vnj + kv * a.vnh;
                rv[i] = *reinterpret_cast<const uint4*>((vold ? a.v_past : a.v_new) + vr + vdc);
            }
        }
        if (entry & MASKED) {
#pragma unroll
            for (int i = 0; i < MASKS; ++i) {
                const uint32_t e = tid + i * THREADS;
                const uint32_t t = q0 + (e / KB) % QT, j = kb * KB + e % KB;
                rm[i] = a.mask[size_t(t < a.tokens ? t : a.tokens - 1u) * a.mt + (j < a.keys ? j : a.keys - 1u)];
            }
        }
    };
    auto put = [&](int buffer, uint32_t entry, bool values) {
        const uint32_t kb = entry & ~MASKED;
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const uint32_t c = tid + i * THREADS;
            if (c < uint32_t(KB * D / 8)) {
                const uint32_t r = c / (D / 8), dc = (c % (D / 8)) * 8u;
                const bool ok = kb * KB + r < a.keys;
                *reinterpret_cast<uint4*>(&k_s[buffer][r * KPAD + (((dc / 8u) ^ ((r >> 1) & KSWZ)) * 8u)]) = ok ? rk[i] : uint4{0, 0, 0, 0};
                if (values) {
                    // lanes hold consecutive keys vr of one chunk: each 2-byte store of a wave covers 128
                    // contiguous bytes of a V^T row (no two lanes in one bank at different addresses)
                    const uint32_t vr = c % KB, vdc = (c / KB) * 8u;
                    const uint4 v = kb * KB + vr < a.keys ? rv[i] : uint4{0, 0, 0, 0};
                    const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
                    for (int x = 0; x < 8; ++x) {
                        v_s[buffer][(vdc + x) * VPAD + vr] = e[x];
                    }
                }
            }
        }
        if (entry & MASKED) {
#pragma unroll
            for (int i = 0; i < MASKS; ++i) {
                const uint32_t e = tid + i * THREADS;
                if (e < uint32_t(QT * KB)) {
                    const uint32_t qr = e / KB, kc = e % KB;
                    const bool ok = q0 + qr < a.tokens && kb * KB + kc < a.keys;
                    m_s[buffer][qr * MPAD + kc] = ok ? rm[i] : uint16_t(0xff80u);
                }
            }
        }
    };
    // Scores of this lane (key 16 t + 4 quad + r of the block, query ``col`` of the tile) for each of the
    // wave's heads, in u units; returns cs (s = u * cs).
    auto scores = [&](int buffer, uint32_t entry, float (&u)[HPW][4][4]) -> float {
        f32x4_t acc[HPW][4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int hd = 0; hd < HPW; ++hd) {
                acc[hd][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                const bf16x8_t kf = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&k_s[buffer][(t * 16u + col) * KPAD + (((ks * 4u + quad) ^ (((t * 16u + col) >> 1) & KSWZ)) * 8u)]));
#pragma unroll
                for (int hd = 0; hd < HPW; ++hd) {
                    acc[hd][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[hd][ks], acc[hd][t], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int hd = 0; hd < HPW; ++hd) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                    u[hd][t][r] = acc[hd][t][r];
                    u[hd][t][r + 1] = acc[hd][t][r + 1];
                    round_bf16_pair(u[hd][t][r], u[hd][t][r + 1]);
                }
            }
        }
        if (POW2 && !(entry & MASKED)) {
            return a.scale;
        }
#pragma unroll
        for (int hd = 0; hd < HPW; ++hd) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                    if constexpr (!POW2) {
                        u[hd][t][r] *= a.scale;
                        u[hd][t][r + 1] *= a.scale;
                        round_bf16_pair(u[hd][t][r], u[hd][t][r + 1]);
                    } else {
                        u[hd][t][r] *= a.scale;  // exact: a power-of-two scale, no rounding (see above)
                        u[hd][t][r + 1] *= a.scale;
                    }
                }
            }
        }
        if (entry & MASKED) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint2 m = *reinterpret_cast<const uint2*>(&m_s[buffer][col * MPAD + t * 16u + quad * 4u]);
#pragma unroll
                for (int hd = 0; hd < HPW; ++hd) {
                    u[hd][t][0] += __uint_as_float(m.x << 16);
                    u[hd][t][1] += __uint_as_float(m.x & 0xffff0000u);
                    u[hd][t][2] += __uint_as_float(m.y << 16);
                    u[hd][t][3] += __uint_as_float(m.y & 0xffff0000u);
                    round_bf16_pair(u[hd][t][0], u[hd][t][1]);
                    round_bf16_pair(u[hd][t][2], u[hd][t][3]);
                }
            }
        }
        return 1.0f;
    };
    // One pass over the visited blocks, the next block staged while the current one is computed.
    auto sweep = [&](bool values, auto&& body) {
        if (visits == 0) {
            return;
        }
        const uint32_t first = entry_of(0);
        uint32_t next = entry_of(visits > 1 ? 1u : 0u);
        fetch(first, values);
        put(0, first, values);
        fetch(next, values);
        __syncthreads();
        uint32_t current = first;
        for (uint32_t i = 0; i < visits; ++i) {
            body(int(i & 1u), current);
            // registers hold block i + 1 (or re-read block i when it is the last, never stored)
            if (i + 1 < visits) {
                put(int((i + 1) & 1u), next, values);
            }
            current = next;
            next = entry_of(i + 2 < visits ? i + 2 : visits - 1u);
            fetch(next, values);
            __syncthreads();
        }
    };

    float peak[HPW], total[HPW];
#pragma unroll
    for (int hd = 0; hd < HPW; ++hd) {
        peak[hd] = neg_inf;
        total[hd] = 0.0f;
    }
    sweep(false, [&](int buffer, uint32_t entry) {
        float u[HPW][4][4];
        const float cs = scores(buffer, entry, u);
#pragma unroll
        for (int hd = 0; hd < HPW; ++hd) {
            float top = neg_inf;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                top = __builtin_fmaxf(top, __builtin_fmaxf(__builtin_fmaxf(u[hd][t][0], u[hd][t][1]), __builtin_fmaxf(u[hd][t][2], u[hd][t][3])));
            }
            top = __builtin_fmaxf(peak[hd], top * cs);  // exact: cs is 1 or a power of two
            if (top != neg_inf) {
                // exp(s - top) = 2^(u * cs * log2(e) - top * log2(e)): one multiply-add per score
                const float scale2 = cs * kLog2e, shift = -top * kLog2e;
                float sum = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        sum += __builtin_amdgcn_exp2f(__builtin_fmaf(u[hd][t][r], scale2, shift));
                    }
                }
                total[hd] = total[hd] * fast_exp(peak[hd] - top) + sum;
                peak[hd] = top;
            }
        }
    });
    // Combine the four lane groups that share a query, then fold in the sink.
    // p = exp(s - peak) / total = 2^(s * log2(e) - (peak * log2(e) + log2(total))): the normalisation
    // rides in the exponent's one multiply-add (v_log_f32 is log2). Only a row whose scores and sink are
    // all -inf has total 0; its probabilities are NaN, as the reference's 0 / 0 is.
    float norm[HPW];
#pragma unroll
    for (int hd = 0; hd < HPW; ++hd) {
#pragma unroll
        for (int offset = 16; offset < 64; offset <<= 1) {
            softmax_stats_merge(peak[hd], total[hd], __shfl_xor(peak[hd], offset, kWave), __shfl_xor(total[hd], offset, kWave));
        }
        softmax_stats_add(peak[hd], total[hd], bf16_to_f32(a.sinks[kv * a.sh + (g0 + hd) * a.sg]));
        norm[hd] = -(peak[hd] * kLog2e + __builtin_amdgcn_logf(total[hd]));
    }

    f32x4_t o[HPW][D / 16];
#pragma unroll
    for (int hd = 0; hd < HPW; ++hd) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            o[hd][dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    sweep(true, [&](int buffer, uint32_t entry) {
        float u[HPW][4][4];
        const float scale2 = scores(buffer, entry, u) * kLog2e;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // keys 32 h + (4 quad + r) and 32 h + 16 + (4 quad + r): this lane's B operand slots 0-3 and 4-7
            bf16x8_t pf[HPW];
#pragma unroll
            for (int hd = 0; hd < HPW; ++hd) {
                float e[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(u[hd][2 * h + i / 4][i % 4], scale2, norm[hd]));
                }
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    const bf16x2_t pair = __builtin_convertvector(f32x2_t{e[i], e[i + 1]}, bf16x2_t);
                    pf[hd][i] = pair[0];
                    pf[hd][i + 1] = pair[1];
                }
            }
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) {
                const uint16_t* row = &v_s[buffer][(dt * 16u + col) * VPAD + h * 32u];
                const uint2 lo = *reinterpret_cast<const uint2*>(row + quad * 4u);
                const uint2 hi = *reinterpret_cast<const uint2*>(row + 16u + quad * 4u);
                const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, uint4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
                for (int hd = 0; hd < HPW; ++hd) {
                    o[hd][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[hd], o[hd][dt], 0, 0, 0);
                }
            }
        }
    });
    if (live) {
#pragma unroll
        for (int hd = 0; hd < HPW; ++hd) {
            uint16_t* dst = a.out + ((size_t(query) * a.kv_heads + kv) * a.group + g0 + hd) * D;
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) {
                const uint32_t d = dt * 16u + quad * 4u;
                const uint32_t w0 = uint32_t(f32_to_bf16(o[hd][dt][0])) | (uint32_t(f32_to_bf16(o[hd][dt][1])) << 16);
                const uint32_t w1 = uint32_t(f32_to_bf16(o[hd][dt][2])) | (uint32_t(f32_to_bf16(o[hd][dt][3])) << 16);
                *reinterpret_cast<uint2*>(dst + d) = uint2{w0, w1};
            }
        }
    }
}

}  // namespace chroma
