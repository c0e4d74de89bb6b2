// Internal interface between the runtime (runtime.cpp) and its decoder-mask kernel (masks.hip).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace chroma_masks {

// Queue, on ``stream``, the two masks [steps, context + steps] of one multi-step decoder call: element
// (t, j) is 0 when key j may be attended by query t and -inf otherwise, in float32 (``bfloat16`` false) or
// bfloat16. Query t sits at time position + t. A cached key j < context holds time slots[j] (negative:
// empty) and may be attended when it is valid, not after the query and inside the window (slots[j] >
// time - window); new key c = j - context, at time position + c, when c <= t and c > t - window. ``full``
// takes window ``context``, ``windowed`` takes ``window``. ``slots`` is device memory. Returns a
// CHROMA_HIP_* status and writes a message on failure.
int launch_decoder_masks(const int64_t* slots, int64_t context, int64_t position, int64_t steps, int64_t window, bool bfloat16,
                         void* full, void* windowed, hipStream_t stream, char* error, size_t error_size);

}  // namespace chroma_masks
