// Row top-k selection on device matrices: the k largest (or smallest) values of each row of x [rows, width]
// (float32, or bfloat16 bits) with their int64 column ids, in order. The rule is the reference GPU
// backend's top-k (chroma/_src/codegen/gpu.py:300-337): values descending (ascending for smallest), ties
// to the lower id, NaN above every number for largest and below for smallest.
//
// Two launches. ``rows_topk_chunks``: one wave per chunk of 64 x P elements of a row keeps one 64-bit key
// per element in registers (``topk_key``: the value's order in the high word, ~id in the low word, so
// keys are unique and larger means chosen first) and takes the wave-wide largest key k times, writing
// its chunk's k keys in order (0 once the chunk is exhausted) with their values to scratch.
// ``rows_topk_merge``: one workgroup per row; thread t holds the head of chunk t's sorted list, and k
// rounds of a workgroup-wide maximum pick the row's keys in order. Both are exact integer comparisons,
// so the result is the single-pass selection's bit for bit.
//
// Scratch per call: rows x chunks x k keys (8 bytes) and values (4 bytes).
#include "../../include/chroma_hip.h"
#include "select.h"

#include <hip/hip_runtime.h>

#include <chroma_hip/device.h>

#include <cstdio>
#include <mutex>

namespace {

constexpr uint32_t kMergeThreads = 256;  // one chunk list per merge thread

template <class T> __device__ __forceinline__ float widen(T v);
template <> __device__ __forceinline__ float widen<float>(float v) { return v; }
template <> __device__ __forceinline__ float widen<uint16_t>(uint16_t v) { return chroma::bf16_to_f32(v); }

template <class T> __device__ __forceinline__ T narrow(float v);
template <> __device__ __forceinline__ float narrow<float>(float v) { return v; }
// exact: every value came from a bfloat16
template <> __device__ __forceinline__ uint16_t narrow<uint16_t>(float v) { return uint16_t(__float_as_uint(v) >> 16); }

template <int P, class T>
__global__ void __launch_bounds__(256) rows_topk_chunks(const T* __restrict__ x, uint32_t rows, uint32_t width, uint32_t chunks, uint32_t k,
                                                        int largest, uint64_t* __restrict__ keys, float* __restrict__ vals) {
    const uint32_t w = blockIdx.x * 4u + threadIdx.x / 64u;
    if (w >= rows * chunks) {
        return;  // whole waves leave together
    }
    const uint32_t r = w / chunks, c = w % chunks, lane = threadIdx.x % 64u;
    const uint32_t first = c * 64u * P;
    const T* row = x + size_t(r) * width;
    uint64_t key[P];
    float val[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t j = first + p * 64u + lane;
        const bool in = j < width;
        val[p] = in ? widen<T>(row[j]) : 0.0f;
        key[p] = in ? chroma::topk_key(val[p], j, largest != 0) : 0;
    }
    for (uint32_t s = 0; s < k; ++s) {
        uint64_t best = 0;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            best = key[p] > best ? key[p] : best;
        }
        const uint64_t top = chroma::wave_max_u64(best);
        const size_t at = (size_t(r) * chunks + c) * k + s;
        if (top == 0) {
            if (lane == 0) {
                keys[at] = 0;
                vals[at] = 0.0f;
            }
            continue;
        }
        const uint32_t local = (0xffffffffu - uint32_t(top)) - first;
        if (local % 64u == lane) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                if (uint32_t(p) == local / 64u) {
                    vals[at] = val[p];
                    key[p] = 0;
                }
            }
            keys[at] = top;
        }
    }
}

template <class T>
__global__ void __launch_bounds__(kMergeThreads) rows_topk_merge(const uint64_t* __restrict__ keys, const float* __restrict__ vals,
                                                                uint32_t chunks, uint32_t k, T* __restrict__ values, int64_t* __restrict__ ids) {
    __shared__ uint64_t wave_best[kMergeThreads / 64];
    const uint32_t r = blockIdx.x, t = threadIdx.x;
    const size_t base = (size_t(r) * chunks + t) * k;
    uint32_t head = 0;
    uint64_t key = t < chunks ? keys[base] : 0;
    for (uint32_t s = 0; s < k; ++s) {
        const uint64_t best = chroma::wave_max_u64(key);
        if (t % 64u == 0) {
            wave_best[t / 64u] = best;
        }
        __syncthreads();
        uint64_t top = wave_best[0];
#pragma unroll
        for (uint32_t w = 1; w < kMergeThreads / 64; ++w) {
            top = wave_best[w] > top ? wave_best[w] : top;
        }
        __syncthreads();  // every thread has read this round's maxima
        if (top != 0 && key == top) {  // keys are unique: one thread
            values[size_t(r) * k + s] = narrow<T>(vals[base + head]);
            ids[size_t(r) * k + s] = int64_t(0xffffffffu - uint32_t(top));
            ++head;
            key = head < k ? keys[base + head] : 0;
        }
    }
}

// Elements per lane: the fewest of 1, 2, 4, ..., 32 that leave at most kMergeThreads chunks per row.
int lanes_per_chunk(size_t width) {
    for (int p = 1; p <= 32; p *= 2) {
        if ((width + 64u * p - 1) / (64u * p) <= kMergeThreads) {
            return p;
        }
    }
    return 0;
}

template <class T>
hipError_t launch(const void* x, size_t rows, size_t width, int k, int largest, void* values, int64_t* ids, void* scratch, int p,
                  size_t chunks, hipStream_t stream) {
    uint64_t* keys = static_cast<uint64_t*>(scratch);
    float* vals = reinterpret_cast<float*>(keys + rows * chunks * size_t(k));
    const T* xs = static_cast<const T*>(x);
    const uint32_t groups = uint32_t((rows * chunks + 3) / 4);
    const uint32_t r = uint32_t(rows), w = uint32_t(width), c = uint32_t(chunks), kk = uint32_t(k);
    switch (p) {
        case 1: rows_topk_chunks<1, T><<<groups, 256, 0, stream>>>(xs, r, w, c, kk, largest, keys, vals); break;
        case 2: rows_topk_chunks<2, T><<<groups, 256, 0, stream>>>(xs, r, w, c, kk, largest, keys, vals); break;
        case 4: rows_topk_chunks<4, T><<<groups, 256, 0, stream>>>(xs, r, w, c, kk, largest, keys, vals); break;
        case 8: rows_topk_chunks<8, T><<<groups, 256, 0, stream>>>(xs, r, w, c, kk, largest, keys, vals); break;
        case 16: rows_topk_chunks<16, T><<<groups, 256, 0, stream>>>(xs, r, w, c, kk, largest, keys, vals); break;
        default: rows_topk_chunks<32, T><<<groups, 256, 0, stream>>>(xs, r, w, c, kk, largest, keys, vals); break;
    }
    hipError_t status = hipGetLastError();
    if (status != hipSuccess) {
        return status;
    }
    rows_topk_merge<T><<<r, kMergeThreads, 0, stream>>>(keys, vals, c, kk, static_cast<T*>(values), ids);
    return hipGetLastError();
}

int fail(const char* message, char* error, size_t size) {
    if (error && size) {
        std::snprintf(error, size, "%s", message);
    }
    return CHROMA_HIP_RUNTIME_ERROR;
}

}  // namespace

namespace chroma_select {

size_t workspace_bytes(size_t rows, size_t width, int k) {
    const int p = lanes_per_chunk(width);
    if (!rows || !width || k < 1 || size_t(k) > width || size_t(k) > kMaxK || !p) {
        return 0;
    }
    const size_t chunks = (width + 64u * p - 1) / (64u * p);
    if (rows * chunks > 0x7fffffffu) {
        return 0;  // one wave per chunk must fit the grid and 32-bit wave indices
    }
    return rows * chunks * size_t(k) * (sizeof(uint64_t) + sizeof(float));
}

int launch_rows_topk(const void* x, int dtype, size_t rows, size_t width, int k, int largest, void* values, int64_t* ids, void* scratch,
                     size_t scratch_bytes, hipStream_t stream, char* error, size_t error_size) {
    if (dtype != CHROMA_HIP_FLOAT32 && dtype != CHROMA_HIP_BFLOAT16) {
        return fail("rows_topk: dtype must be CHROMA_HIP_FLOAT32 or CHROMA_HIP_BFLOAT16", error, error_size);
    }
    const size_t need = workspace_bytes(rows, width, k);
    if (!need) {
        return fail("rows_topk: want rows >= 1, 1 <= k <= min(width, 1024) and width <= 524288", error, error_size);
    }
    if (!x || !values || !ids || !scratch) {
        return fail("rows_topk: null device pointer", error, error_size);
    }
    if (scratch_bytes < need) {
        char message[160];
        std::snprintf(message, sizeof(message), "rows_topk: scratch of %zu bytes is smaller than the %zu this selection needs",
                      scratch_bytes, need);
        return fail(message, error, error_size);
    }
    const int p = lanes_per_chunk(width);
    const size_t chunks = (width + 64u * p - 1) / (64u * p);
    const hipError_t status = dtype == CHROMA_HIP_FLOAT32
                                  ? launch<float>(x, rows, width, k, largest, values, ids, scratch, p, chunks, stream)
                                  : launch<uint16_t>(x, rows, width, k, largest, values, ids, scratch, p, chunks, stream);
    if (status != hipSuccess) {
        char message[160];
        std::snprintf(message, sizeof(message), "rows_topk launch: %s", hipGetErrorString(status));
        return fail(message, error, error_size);
    }
    return CHROMA_HIP_OK;
}

}  // namespace chroma_select

namespace {

// Scratch of chroma_hip_rows_topk_static: one copy of this array per GPU, at that GPU's own address, kept
// until the process ends. Its address on a device comes from hipGetSymbolAddress on the first call there;
// the array's name itself is a host-side stand-in that must never reach a kernel or a copy.
constexpr size_t kStaticScratchBytes = CHROMA_HIP_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_address[kMaxDevices] = {};  // per device, null until looked up

int static_scratch(void** address, char* error, size_t error_size) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        return fail("rows_topk_static: no usable current device", error, error_size);
    }
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_address[device]) {
        void* found = nullptr;
        const hipError_t status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
        if (status != hipSuccess || !found) {
            char message[160];
            std::snprintf(message, sizeof(message), "rows_topk_static: hipGetSymbolAddress: %s", hipGetErrorString(status));
            return fail(message, error, error_size);
        }
        scratch_address[device] = found;
    }
    *address = scratch_address[device];
    return CHROMA_HIP_OK;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) size_t chroma_hip_rows_topk_workspace(size_t rows, size_t width, int k) {
    return chroma_select::workspace_bytes(rows, width, k);
}

__attribute__((visibility("default"))) int chroma_hip_rows_topk(const void* x, int dtype, size_t rows, size_t width, int k, int largest,
                                                                void* values, int64_t* ids, void* workspace, size_t workspace_bytes,
                                                                void* stream, char* error, size_t error_size) {
    return chroma_select::launch_rows_topk(x, dtype, rows, width, k, largest, values, ids, workspace, workspace_bytes,
                                           static_cast<hipStream_t>(stream), error, error_size);
}

__attribute__((visibility("default"))) int chroma_hip_rows_topk_static(const void* x, int dtype, size_t rows, size_t width, int k,
                                                                       int largest, void* values, int64_t* ids, void* stream, char* error,
                                                                       size_t error_size) {
    const size_t need = chroma_select::workspace_bytes(rows, width, k);
    if (need > kStaticScratchBytes) {
        char message[200];
        std::snprintf(message, sizeof(message), "rows_topk_static: this selection needs %zu bytes of scratch; the static scratch holds %zu",
                      need, kStaticScratchBytes);
        return fail(message, error, error_size);
    }
    void* address = nullptr;
    const int status = static_scratch(&address, error, error_size);
    if (status != CHROMA_HIP_OK) {
        return status;
    }
    return chroma_select::launch_rows_topk(x, dtype, rows, width, k, largest, values, ids, address, kStaticScratchBytes,
                                           static_cast<hipStream_t>(stream), error, error_size);
}

}  // extern "C"
