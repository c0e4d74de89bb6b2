// Batched device-to-device rectangle copies in one kernel launch: the KV-cached decoder commits each step's
// new key and value rows (up to two runs each, when the rows wrap around the cache) with one launch
// instead of one runtime copy call per rectangle (a runtime 2-D copy costs ~15 us of host time, a kernel
// launch ~1.5 us). grid.y enumerates the rectangles; a rectangle whose addresses, pitches and width are
// 16-byte aligned moves 16-byte chunks, any other one bytes.
#include "../../include/chroma_hip.h"
#include "copy.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace {

struct Rects {
    chroma_copy::Rect rect[chroma_copy::kMaxRects];
};

__global__ void __launch_bounds__(256) copy_rects(Rects rects) {
    const chroma_copy::Rect r = rects.rect[blockIdx.y];
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    const size_t first = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const bool wide = ((reinterpret_cast<uintptr_t>(r.dst) | reinterpret_cast<uintptr_t>(r.src) | r.dst_pitch | r.src_pitch | r.width) & 15u) == 0;
    if (wide) {
        const size_t chunks = r.width / 16u;
        for (size_t i = first; i < chunks * r.height; i += stride) {
            const size_t row = i / chunks, chunk = i % chunks;
            const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const char*>(r.src) + row * r.src_pitch + chunk * 16u);
            *reinterpret_cast<uint4*>(static_cast<char*>(r.dst) + row * r.dst_pitch + chunk * 16u) = v;
        }
    } else {
        for (size_t i = first; i < r.width * r.height; i += stride) {
            const size_t row = i / r.width, column = i % r.width;
            static_cast<char*>(r.dst)[row * r.dst_pitch + column] = static_cast<const char*>(r.src)[row * r.src_pitch + column];
        }
    }
}

}  // namespace

namespace chroma_copy {

int launch_copy_rects(const Rect* rects, int count, hipStream_t stream, char* error, size_t error_size) {
    if (count < 1 || count > kMaxRects) {
        std::snprintf(error, error_size, "copy_2d_batch takes 1 to %d rectangles", kMaxRects);
        return CHROMA_HIP_RUNTIME_ERROR;
    }
    Rects all{};
    size_t most = 1;
    for (int i = 0; i < count; ++i) {
        if (rects[i].dst_pitch < rects[i].width || rects[i].src_pitch < rects[i].width) {
            std::snprintf(error, error_size, "copy_2d_batch pitch smaller than the row width");
            return CHROMA_HIP_RUNTIME_ERROR;
        }
        all.rect[i] = rects[i];
        const size_t units = rects[i].width * rects[i].height;
        most = units > most ? units : most;
    }
    const size_t blocks = (most / 16u + 255u) / 256u;
    const dim3 grid(unsigned(blocks < 1 ? 1 : (blocks > 1024 ? 1024 : blocks)), unsigned(count), 1);
    hipLaunchKernelGGL(copy_rects, grid, dim3(256), 0, stream, all);
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) {
        std::snprintf(error, error_size, "copy_2d_batch launch: %s", hipGetErrorString(status));
        return CHROMA_HIP_RUNTIME_ERROR;
    }
    return CHROMA_HIP_OK;
}

}  // namespace chroma_copy
