// The KV-cached decoder's attention masks built on the device: a multi-step (prefill) call of the
// GPT-OSS-20B-shaped model needs two 2048 x 6144 masks, which took ~8 ms to build in NumPy and a 50 MB
// upload; here one launch writes both from the cache's slot table (the rule of the reference's host
// masks, chroma/_src/decoder.py:116-128).
#include "../../include/chroma_hip.h"
#include "masks.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace {

// One thread per (query t, key j) element of both masks.
template <class T>
__global__ void __launch_bounds__(256) decoder_masks(const int64_t* __restrict__ slots, int64_t context, int64_t position, int64_t steps,
                                                     int64_t window, T blocked, T* __restrict__ full, T* __restrict__ windowed) {
    const int64_t keys = context + steps;
    const int64_t total = steps * keys;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t t = i / keys, j = i % keys;
        const int64_t time = position + t;
        bool in_full, in_window;
        if (j < context) {
            const int64_t kt = slots[j];
            const bool usable = kt >= 0 && kt <= time;
            in_full = usable && kt > time - context;
            in_window = usable && kt > time - window;
        } else {
            const int64_t c = j - context;
            in_full = c <= t && c > t - context;
            in_window = c <= t && c > t - window;
        }
        full[i] = in_full ? T(0) : blocked;
        windowed[i] = in_window ? T(0) : blocked;
    }
}

}  // namespace

namespace chroma_masks {

int launch_decoder_masks(const int64_t* slots, int64_t context, int64_t position, int64_t steps, int64_t window, bool bfloat16,
                         void* full, void* windowed, hipStream_t stream, char* error, size_t error_size) {
    if (context < 1 || steps < 1 || window < 1 || position < 0) {
        std::snprintf(error, error_size, "decoder masks: context %lld, steps %lld, window %lld, position %lld", (long long)context,
                      (long long)steps, (long long)window, (long long)position);
        return CHROMA_HIP_RUNTIME_ERROR;
    }
    const int64_t total = steps * (context + steps);
    const int64_t blocks = (total + 255) / 256;
    const dim3 grid(unsigned(blocks > 8192 ? 8192 : blocks));
    if (bfloat16) {
        hipLaunchKernelGGL(decoder_masks<uint16_t>, grid, dim3(256), 0, stream, slots, context, position, steps, window, uint16_t(0xFF80u),
                           static_cast<uint16_t*>(full), static_cast<uint16_t*>(windowed));
    } else {
        hipLaunchKernelGGL(decoder_masks<uint32_t>, grid, dim3(256), 0, stream, slots, context, position, steps, window, uint32_t(0xFF800000u),
                           static_cast<uint32_t*>(full), static_cast<uint32_t*>(windowed));
    }
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) {
        std::snprintf(error, error_size, "decoder masks launch: %s", hipGetErrorString(status));
        return CHROMA_HIP_RUNTIME_ERROR;
    }
    return CHROMA_HIP_OK;
}

}  // namespace chroma_masks
