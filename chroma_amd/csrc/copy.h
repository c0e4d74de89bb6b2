// Internal interface between the runtime (runtime.cpp) and its batched device copy kernel (copy.hip).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>

namespace chroma_copy {

constexpr int kMaxRects = 4;  // rectangles one launch copies

struct Rect {
    void* dst;
    size_t dst_pitch;
    const void* src;
    size_t src_pitch;
    size_t width;   // bytes per row
    size_t height;  // rows
};

// Queue the copies of ``count`` (1..kMaxRects) device-to-device rectangles on ``stream`` as one kernel
// launch. Returns a CHROMA_HIP_* status and writes a message on failure.
int launch_copy_rects(const Rect* rects, int count, hipStream_t stream, char* error, size_t error_size);

}  // namespace chroma_copy
