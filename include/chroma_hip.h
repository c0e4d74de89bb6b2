/* C ABI of the hip backend runtime (libchroma_hip.so).
 *
 * The runtime owns one device allocation per program (weights | workspace | error word | input staging |
 * output staging), uploads the weights once, and runs the compiled launch plan with
 * hipModuleLaunchKernel (optionally replayed as a captured hipGraph) on its own stream.
 *
 * Status codes: 0 ok, 1 index error (a gather or expert index was out of range; the program stays usable),
 * 2 runtime error. On a non-zero status ``error`` receives a NUL-terminated message (at most
 * ``error_size`` bytes including the terminator).
 */
#ifndef CHROMA_HIP_H
#define CHROMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CHROMA_HIP_OK 0
#define CHROMA_HIP_INDEX_ERROR 1
#define CHROMA_HIP_RUNTIME_ERROR 2

/* Element types of the selection entry points. */
#define CHROMA_HIP_FLOAT32 0
#define CHROMA_HIP_BFLOAT16 1

/* Load the compiled artifact in ``artifact_dir`` (its model.plan, code object and weights file) on the
 * current device. Replaces the reference's generated ``create_model(const char* weights)`` +
 * ``chroma::cuda::Runner::initialize`` (chroma/_src/codegen/cuda/codegen.py:35-40,
 * chroma/_src/codegen/cuda/runtime.h:116-145). A weights file of the wrong size fails with
 * "Missing weights file or incorrect byte size" (chroma/_src/core/tensor.h:29-33). */
int chroma_hip_create(const char* artifact_dir, void** handle, char* error, size_t error_size);

/* One synchronous call: copy every input from host memory, run the plan, copy every output back.
 * Replaces ``ModelProgram::run(const void* const* inputs, void* const* outputs)`` /
 * ``Runner::run`` (chroma/_src/codegen/cuda/codegen.py:29-33, runtime.h:147-173). Input and output
 * pointers are host buffers with exactly the manifest's byte sizes. A null input pointer (an extension:
 * the reference has no such case) keeps what that input's device staging region already holds, and a
 * null output pointer leaves that output on the device; the KV-cached decoder uses both to keep its
 * cache device-resident. */
int chroma_hip_run(void* handle, const void* const* inputs, void* const* outputs, char* error, size_t error_size);

/* Device name for ``Program.device`` (the reference's ``Runner::device_name``, runtime.h:182). */
const char* chroma_hip_device_name(void* handle);

/* sha256 signature of the tensor specs the plan was compiled for (the reference extension's
 * ``signature`` attribute, chroma/_src/build.py:53-57, checked by program.py:98-99). */
const char* chroma_hip_signature(void* handle);

/* Release every device allocation after the stream drains (runtime.h:94-114). */
void chroma_hip_destroy(void* handle);

/* --- device-resident execution (no counterpart in the reference: benchmarking and callers that keep
 * data on the device between calls) --- */

/* Copy host inputs into the program's input staging regions (no launch). */
int chroma_hip_upload(void* handle, const void* const* inputs, char* error, size_t error_size);

/* Run the plan ``iterations`` times on whatever the staging regions hold, then synchronize and check the
 * error word. If ``milliseconds`` is non-null it receives the total time between hipEvents recorded on
 * the runtime's stream around the launches. */
int chroma_hip_execute(void* handle, int iterations, float* milliseconds, char* error, size_t error_size);

/* Capture ``copies`` back-to-back executions of the plan as one graph and launch it ``iterations``
 * times; ``milliseconds`` (if non-null) receives the total time between hipEvents around those launches
 * (divide by copies x iterations for one execution). Times a plan of one short kernel without the host's
 * per-replay graph launch. */
int chroma_hip_execute_chained(void* handle, int copies, int iterations, float* milliseconds, char* error, size_t error_size);

/* The two attention masks [steps, context + steps] of a multi-step KV-cached decoder call, built on the
 * device into the staging regions of inputs ``full_input`` and ``window_input`` (float32 or bfloat16,
 * ``dtype`` CHROMA_HIP_FLOAT32 / CHROMA_HIP_BFLOAT16) by a kernel queued on the program's stream, so the
 * next resident run (given NULL for those inputs) uses them. ``slots`` (host, ``context`` entries) holds
 * the time of each cache row or a negative value for an empty row; query t sits at position + t. Element
 * (t, j) is 0 where key j is valid, not after the query and inside the window (``context`` for the full
 * mask, ``window`` for the other), -inf elsewhere: the reference decoder's host masks
 * (chroma/_src/decoder.py:116-128), which this replaces for multi-step calls (no counterpart in the
 * reference's C++: its masks are host arrays uploaded every call). */
int chroma_hip_decoder_masks(void* handle, const int64_t* slots, int64_t context, int64_t position, int64_t steps, int64_t window,
                             int dtype, int full_input, int window_input, char* error, size_t error_size);

/* Copy the output staging regions to host buffers. */
int chroma_hip_download(void* handle, void* const* outputs, char* error, size_t error_size);

/* Select plain launches (0) or hipGraph replay of the whole plan (1). Returns the previous mode. */
int chroma_hip_set_graph(void* handle, int enabled);

/* Number of launches in the plan, and the device address of the program's allocation (for tests that
 * inspect device memory through another API). */
int chroma_hip_launch_count(void* handle);
void* chroma_hip_device_base(void* handle);

/* Device addresses of input ``index``'s and output ``index``'s staging regions (null when out of range).
 * They stay valid until ``chroma_hip_destroy``. */
void* chroma_hip_input_pointer(void* handle, int index);
void* chroma_hip_output_pointer(void* handle, int index);

/* Device-to-device copy of ``height`` rows of ``width`` bytes (row pitches ``dst_pitch`` and
 * ``src_pitch``) on the program's stream, complete on return. Both addresses must lie in device memory
 * of the program's device, for example staging regions of two programs; the KV-cached decoder commits
 * new cache rows and hands its cache between its prefill and decode programs with it. */
int chroma_hip_copy_2d(void* handle, void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width, size_t height,
                       char* error, size_t error_size);

/* The same copy, only queued: it runs before the program's later runs and copies, and
 * ``chroma_hip_synchronize`` waits for it (and everything else queued on the program's stream). The
 * decoder commits each step's new cache rows this way and synchronizes only when another program
 * takes the cache over. */
int chroma_hip_copy_2d_queued(void* handle, void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width,
                              size_t height, char* error, size_t error_size);
int chroma_hip_synchronize(void* handle, char* error, size_t error_size);

/* Zero input ``index``'s staging region, queued on the program's stream like
 * ``chroma_hip_copy_2d_queued``. No counterpart in the reference (whose decoder uploads a zeroed host
 * cache): the decoder starts a fresh device-resident KV cache with it instead of uploading zeros. */
int chroma_hip_clear_input(void* handle, int index, char* error, size_t error_size);

/* Up to four queued device-to-device rectangle copies (as ``chroma_hip_copy_2d_queued``) in one kernel
 * launch on the program's stream. No counterpart in the reference: the decoder commits a step's new key
 * and value rows with it (a runtime 2-D copy call costs several times a kernel launch in host time). */
typedef struct chroma_hip_rect {
    void* dst;
    size_t dst_pitch;
    const void* src;
    size_t src_pitch;
    size_t width;  /* bytes per row */
    size_t height; /* rows */
} chroma_hip_rect;
int chroma_hip_copy_2d_batch_queued(void* handle, const chroma_hip_rect* rects, int count, char* error, size_t error_size);

/* Page-locked host memory for arrays that programs read and write: copies to and from it go straight to
 * the DMA engines, while other host arrays above 256 KiB move through two pinned staging slots of the
 * program. ``chroma_hip_host_free`` takes only pointers from ``chroma_hip_host_alloc``. No counterpart
 * in the reference (its runtime copies pageable arrays, cuda/runtime.h:147-173); ``Program`` returns
 * fresh outputs in such memory. */
int chroma_hip_host_alloc(size_t bytes, void** pointer, char* error, size_t error_size);
void chroma_hip_host_free(void* pointer);

/* --- row selection (top-k over rows of a device matrix) ---
 * The device counterpart of the reference's GPU top-k family (chroma/_src/codegen/gpu.py:300-337) over
 * whole vocabulary rows, for callers that pick tokens from logits on the device (the reference's chat
 * script sorts the downloaded row instead, scripts/chat.py:82-98): the ``k`` largest (``largest`` != 0)
 * or smallest values of each row of ``x`` [rows, width] (CHROMA_HIP_FLOAT32, or CHROMA_HIP_BFLOAT16
 * bits) into ``values`` [rows, k] (x's type) and ``ids`` [rows, k] (int64), in order, ties to the lower
 * id, NaN above every number for largest and below for smallest. 1 <= k <= min(width, 1024) and width <=
 * 524,288. */

/* Scratch bytes ``chroma_hip_rows_topk`` needs for this shape, or 0 when the shape is not supported. */
size_t chroma_hip_rows_topk_workspace(size_t rows, size_t width, int k);

/* Queue the selection on ``stream`` (a hipStream_t; null for the null stream) and return: x, values, ids
 * and ``workspace`` (at least chroma_hip_rows_topk_workspace bytes) are device memory of the current
 * device, and the caller synchronizes the stream before reading the results or reusing the workspace. */
int chroma_hip_rows_topk(const void* x, int dtype, size_t rows, size_t width, int k, int largest, void* values, int64_t* ids,
                         void* workspace, size_t workspace_bytes, void* stream, char* error, size_t error_size);

/* ``chroma_hip_rows_topk`` without a workspace: the scratch is a static device array of
 * CHROMA_HIP_STATIC_SCRATCH_BYTES per GPU (looked up on the first call on each device and kept until the
 * process ends), so the call allocates nothing. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). A selection needing more scratch than the array holds (chroma_hip_rows_topk_workspace) is
 * rejected with a message. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams, or two threads) race and must be serialized by the caller. */
#define CHROMA_HIP_STATIC_SCRATCH_BYTES ((size_t)4 << 20)
int chroma_hip_rows_topk_static(const void* x, int dtype, size_t rows, size_t width, int k, int largest, void* values, int64_t* ids,
                                void* stream, char* error, size_t error_size);

/* ``chroma_hip_run`` followed, on the program's stream and under the same single synchronization, by the
 * selection of the ``k`` largest values of each of the ``rows`` rows of output ``output_index`` (``width``
 * elements of ``dtype`` each, which must be that output's byte size): ``values`` and ``ids`` are host
 * buffers of rows x k elements. That output itself is downloaded only if ``outputs[output_index]`` is
 * non-null. The selection's device scratch is allocated by the program on first use and kept. The
 * KV-cached decoder's ``greedy`` / ``append_top`` use it to return a token instead of a vocabulary row. */
int chroma_hip_run_top(void* handle, const void* const* inputs, void* const* outputs, int output_index, int dtype, size_t rows,
                       size_t width, int k, void* values, int64_t* ids, char* error, size_t error_size);

#ifdef __cplusplus
}
#endif

#endif /* CHROMA_HIP_H */
