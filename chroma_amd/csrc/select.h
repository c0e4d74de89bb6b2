// Internal interface between the runtime (runtime.cpp) and the row selection kernels (select.hip).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace chroma_select {

constexpr size_t kMaxK = 1024;  // largest k a selection takes

// Scratch bytes a selection of the k extreme values of ``rows`` rows of ``width`` elements needs, or 0 when
// the shape is not supported (k outside [1, min(width, kMaxK)], width above 524,288, or no rows).
size_t workspace_bytes(size_t rows, size_t width, int k);

// Queue the selection on ``stream`` (values in x's type, int64 ids, both [rows, k] on the device). Returns a
// CHROMA_HIP_* status and writes a message on failure.
int launch_rows_topk(const void* x, int dtype, size_t rows, size_t width, int k, int largest, void* values, int64_t* ids, void* scratch,
                     size_t scratch_bytes, hipStream_t stream, char* error, size_t error_size);

}  // namespace chroma_select
