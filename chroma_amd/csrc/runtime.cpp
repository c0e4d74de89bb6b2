// Host runtime of the hip backend: the C ABI declared in include/chroma_hip.h.
//
// A program is one hipMalloc'd allocation laid out by the compiler (weights | workspace | error word |
// inputs | outputs), one non-blocking stream, the code object's kernels and a launch list whose
// arguments are pre-resolved device pointers. ``run`` uploads inputs, launches every kernel (or replays
// the captured hipGraph), downloads the error word and the outputs, and synchronizes once.
#include "../../include/chroma_hip.h"
#include "copy.h"
#include "masks.h"
#include "select.h"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <algorithm>
#include <array>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace {

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct IndexError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void check(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        throw HipError(std::string(what) + ": " + hipGetErrorString(status));
    }
}

class DeviceGuard {
public:
    explicit DeviceGuard(int device) {
        check(hipGetDevice(&previous_), "hipGetDevice");
        if (previous_ != device) {
            check(hipSetDevice(device), "hipSetDevice");
        }
        device_ = device;
    }
    ~DeviceGuard() {
        if (previous_ != device_) {
            hipSetDevice(previous_);
        }
    }

private:
    int previous_ = 0;
    int device_ = 0;
};

struct Region {
    size_t offset = 0;
    size_t bytes = 0;
};

// Host transfers. Copies of at most kDirectBytes, and copies to or from pinned blocks handed out by
// chroma_hip_host_alloc, are queued on the stream as they are. Larger copies of pageable memory move
// through two pinned staging slots of kStagingSlot bytes: the CPU copy into or out of one slot overlaps
// the DMA of the other (HIP's own pageable path reaches about a third of the link's pinned rate).
constexpr size_t kDirectBytes = size_t(256) << 10;
constexpr size_t kErrorRegion = 1024;  // bytes the plan reserves at its error offset
constexpr size_t kStagingSlot = size_t(2) << 20;

std::mutex pinned_mutex;
std::map<uintptr_t, size_t> pinned_blocks;  // start -> bytes of each block from chroma_hip_host_alloc

bool is_pinned(const void* pointer, size_t bytes) {
    std::lock_guard<std::mutex> lock(pinned_mutex);
    const uintptr_t start = reinterpret_cast<uintptr_t>(pointer);
    auto block = pinned_blocks.upper_bound(start);
    if (block == pinned_blocks.begin()) {
        return false;
    }
    --block;
    return start >= block->first && start + bytes <= block->first + block->second;
}

struct Launch {
    std::string kernel;
    unsigned grid[3] = {1, 1, 1};
    unsigned block = 1;
    unsigned shared = 0;
    std::vector<size_t> offsets;
    hipFunction_t function = nullptr;
    std::vector<void*> pointers;  // device pointers, one per kernel parameter
    std::vector<void*> arguments;  // addresses of ``pointers`` entries, as hipModuleLaunchKernel wants
};

struct Plan {
    std::string signature, code_object, weights_file;
    size_t arena = 0, weight_bytes = 0, error = 0;
    std::vector<Region> inputs, outputs;
    std::vector<Launch> launches;
};

Plan read_plan(const std::string& path) {
    std::ifstream stream(path);
    if (!stream) {
        throw std::runtime_error("Cannot open the launch plan " + path);
    }
    Plan plan;
    std::string line;
    std::getline(stream, line);
    if (line != "chroma-hip-plan 2") {  // version 2: the error region is 1 KiB (version 1 plans reserved 256 B)
        throw std::runtime_error("Unsupported launch plan version in " + path);
    }
    while (std::getline(stream, line)) {
        std::istringstream fields(line);
        std::string key;
        fields >> key;
        if (key == "signature") {
            fields >> plan.signature;
        } else if (key == "code_object") {
            fields >> plan.code_object;
        } else if (key == "weights_file") {
            fields >> plan.weights_file;
        } else if (key == "arena") {
            fields >> plan.arena;
        } else if (key == "weights") {
            fields >> plan.weight_bytes;
        } else if (key == "error") {
            fields >> plan.error;
        } else if (key == "input" || key == "output") {
            size_t index = 0;
            Region region;
            fields >> index >> region.offset >> region.bytes;
            auto& list = key == "input" ? plan.inputs : plan.outputs;
            if (index != list.size()) {
                throw std::runtime_error("Launch plan regions out of order");
            }
            list.push_back(region);
        } else if (key == "launch") {
            Launch launch;
            size_t count = 0;
            fields >> launch.kernel >> launch.grid[0] >> launch.grid[1] >> launch.grid[2] >> launch.block >> launch.shared >> count;
            launch.offsets.resize(count);
            for (auto& offset : launch.offsets) {
                fields >> offset;
            }
            if (!fields) {
                throw std::runtime_error("Malformed launch line: " + line);
            }
            plan.launches.push_back(std::move(launch));
        } else if (!key.empty()) {
            throw std::runtime_error("Unknown launch plan entry: " + key);
        }
    }
    // Every region the runtime copies to or from, and every kernel argument, must lie inside the one
    // allocation, so a stale or edited plan cannot make a copy or a launch reach outside it.
    auto inside = [&](size_t offset, size_t bytes) { return offset <= plan.arena && bytes <= plan.arena - offset; };
    for (const auto& launch : plan.launches) {
        for (size_t offset : launch.offsets) {
            if (offset >= plan.arena) {
                throw std::runtime_error("Launch plan argument outside the program allocation");
            }
        }
    }
    for (const auto* list : {&plan.inputs, &plan.outputs}) {
        for (const auto& region : *list) {
            if (!inside(region.offset, region.bytes)) {
                throw std::runtime_error("Launch plan input or output region outside the program allocation");
            }
        }
    }
    if (!inside(plan.error, kErrorRegion) || !inside(0, plan.weight_bytes)) {
        throw std::runtime_error("Launch plan error region or weights outside the program allocation");
    }
    return plan;
}

// Byte size of a file, or -1 when it cannot be opened.
long file_size(const std::string& path) {
    std::FILE* file = std::fopen(path.c_str(), "rb");
    if (!file) {
        return -1;
    }
    long size = -1;
    if (std::fseek(file, 0, SEEK_END) == 0) {
        size = std::ftell(file);
    }
    std::fclose(file);
    return size;
}

class Program {
public:
    Program(const std::string& directory) {
        plan_ = read_plan(directory + "/model.plan");
        // Checked before anything is allocated: a wrong weights file is the common load failure.
        const long weights = file_size(directory + "/" + plan_.weights_file);
        if (weights < 0 || static_cast<size_t>(weights) != plan_.weight_bytes) {
            throw std::runtime_error("Missing weights file or incorrect byte size");
        }
        check(hipGetDevice(&device_), "hipGetDevice");
        try {
            hipDeviceProp_t properties{};
            check(hipGetDeviceProperties(&properties, device_), "hipGetDeviceProperties");
            name_ = std::string(properties.name) + " (" + properties.gcnArchName + ")";
            check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreateWithFlags");
            check(hipEventCreate(&start_), "hipEventCreate");
            check(hipEventCreate(&stop_), "hipEventCreate");
            check(hipHostMalloc(reinterpret_cast<void**>(&error_host_), sizeof(unsigned), hipHostMallocDefault), "hipHostMalloc");
            check(hipMalloc(&base_, plan_.arena ? plan_.arena : 1), "hipMalloc program allocation");
            // The whole error region starts at zero: word 0 is the index-error flag, words 16-63 the per-row
            // tickets of split routers (chroma::router_split) and words 64-127 those of split-key decode
            // attentions (chroma::attention_decode); both return them to zero.
            check(hipMemset(static_cast<char*>(base_) + plan_.error, 0, kErrorRegion), "Clear error region");
            // The workspace starts at zero too: cooperative kernels exchange tagged words there and return
            // them to zero themselves (every other workspace buffer is written before it is read).
            check(hipMemset(static_cast<char*>(base_) + plan_.weight_bytes, 0, plan_.error - plan_.weight_bytes), "Clear workspace");
            upload_weights(directory + "/" + plan_.weights_file);
            check(hipModuleLoad(&module_, (directory + "/" + plan_.code_object).c_str()), "hipModuleLoad");
            std::map<std::string, hipFunction_t> functions;
            for (auto& launch : plan_.launches) {
                auto found = functions.find(launch.kernel);
                if (found == functions.end()) {
                    hipFunction_t function = nullptr;
                    check(hipModuleGetFunction(&function, module_, launch.kernel.c_str()), "hipModuleGetFunction");
                    found = functions.emplace(launch.kernel, function).first;
                }
                launch.function = found->second;
                if (launch.kernel.rfind("chroma_coop_", 0) == 0) {
                    check_co_resident(launch);
                }
                launch.pointers.resize(launch.offsets.size());
                launch.arguments.resize(launch.offsets.size());
                for (size_t i = 0; i < launch.offsets.size(); ++i) {
                    launch.pointers[i] = static_cast<char*>(base_) + launch.offsets[i];
                    launch.arguments[i] = &launch.pointers[i];
                }
            }
        } catch (...) {
            release();  // a constructor that throws runs no destructor
            throw;
        }
        // The whole plan replays as one captured hipGraph unless CHROMA_HIP_GRAPH=0 (a plan of one kernel is
        // launched directly either way: see launch_all).
        const char* graph = std::getenv("CHROMA_HIP_GRAPH");
        use_graph_ = graph == nullptr || std::strcmp(graph, "0") != 0;
    }

    ~Program() { release(); }

    // Frees whatever exists so far (every handle starts null) after the stream has drained. Never throws:
    // it runs from the destructor and from a failed constructor.
    void release() noexcept {
        if (device_ < 0) {
            return;
        }
        int previous = device_;
        hipGetDevice(&previous);
        hipSetDevice(device_);
        if (stream_) {
            hipStreamSynchronize(stream_);
        }
        if (graph_exec_) {
            hipGraphExecDestroy(graph_exec_);
        }
        if (graph_) {
            hipGraphDestroy(graph_);
        }
        drop_select_graph();
        if (module_) {
            hipModuleUnload(module_);
        }
        if (base_) {
            hipFree(base_);
        }
        if (select_) {
            hipFree(select_);
        }
        if (select_host_) {
            hipHostFree(select_host_);
        }
        if (error_host_) {
            hipHostFree(error_host_);
        }
        if (slots_) {
            hipFree(slots_);
        }
        if (slots_host_) {
            hipHostFree(slots_host_);
        }
        if (slots_copied_) {
            hipEventDestroy(slots_copied_);
        }
        for (int slot = 0; slot < 2; ++slot) {
            if (staging_[slot]) {
                hipHostFree(staging_[slot]);
            }
            if (staged_[slot]) {
                hipEventDestroy(staged_[slot]);
            }
            staging_[slot] = nullptr;
            staged_[slot] = nullptr;
        }
        if (start_) {
            hipEventDestroy(start_);
        }
        if (stop_) {
            hipEventDestroy(stop_);
        }
        if (stream_) {
            hipStreamDestroy(stream_);
        }
        graph_exec_ = nullptr;
        graph_ = nullptr;
        select_exec_ = nullptr;
        select_graph_ = nullptr;
        module_ = nullptr;
        base_ = nullptr;
        select_ = nullptr;
        select_bytes_ = 0;
        select_host_ = nullptr;
        select_host_bytes_ = 0;
        slots_ = nullptr;
        slots_host_ = nullptr;
        slots_capacity_ = 0;
        slots_copied_ = nullptr;
        error_host_ = nullptr;
        start_ = stop_ = nullptr;
        stream_ = nullptr;
        if (previous != device_) {
            hipSetDevice(previous);
        }
        device_ = -1;
    }

    const std::string& name() const { return name_; }
    const std::string& signature() const { return plan_.signature; }
    int launch_count() const { return static_cast<int>(plan_.launches.size()); }
    void* base() const { return base_; }

    int set_graph(int enabled) {
        const int previous = use_graph_ ? 1 : 0;
        use_graph_ = enabled != 0;
        return previous;
    }

    void run(const void* const* inputs, void* const* outputs) {
        DeviceGuard guard(device_);
        try {
            upload(inputs);
            launch_all();
            check(hipMemcpyAsync(error_host_, static_cast<char*>(base_) + plan_.error, sizeof(unsigned), hipMemcpyDeviceToHost, stream_),
                  "Read index error");
            download(outputs);
            check(hipStreamSynchronize(stream_), "HIP execution");
            raise_index_error();
        } catch (const HipError&) {
            hipStreamSynchronize(stream_);  // host arrays must outlive every queued copy
            throw;
        }
    }

    // ``run`` with a row selection over output ``index`` queued after the plan: only the k values and ids
    // of each row come back (and the outputs whose host pointers are non-null), after one synchronization.
    void run_top(const void* const* inputs, void* const* outputs, int index, int dtype, size_t rows, size_t width, int k, void* values,
                 int64_t* ids) {
        DeviceGuard guard(device_);
        if (index < 0 || size_t(index) >= plan_.outputs.size()) {
            throw std::runtime_error("run_top: output index out of range");
        }
        if (dtype != CHROMA_HIP_FLOAT32 && dtype != CHROMA_HIP_BFLOAT16) {
            throw std::runtime_error("run_top: dtype must be CHROMA_HIP_FLOAT32 or CHROMA_HIP_BFLOAT16");
        }
        const size_t item = dtype == CHROMA_HIP_FLOAT32 ? 4 : 2;
        if (rows * width * item != plan_.outputs[index].bytes) {
            throw std::runtime_error("run_top: rows x width elements do not match the output's byte size");
        }
        const size_t scratch = chroma_select::workspace_bytes(rows, width, k);
        if (!scratch) {
            throw std::runtime_error("run_top: want 1 <= k <= min(width, 1024) and width <= 524288");
        }
        auto align = [](size_t n) { return (n + 255) / 256 * 256; };
        const size_t value_bytes = rows * size_t(k) * item, id_bytes = rows * size_t(k) * sizeof(int64_t);
        // ids then values, adjacent, so one copy brings both back
        const size_t result_bytes = id_bytes + value_bytes;
        const size_t need = align(scratch) + result_bytes;
        if (need > select_bytes_ || result_bytes > select_host_bytes_) {
            check(hipStreamSynchronize(stream_), "Selection scratch");
            if (select_) {
                check(hipFree(select_), "hipFree selection scratch");
                select_ = nullptr;
                select_bytes_ = 0;
            }
            if (select_host_) {
                check(hipHostFree(select_host_), "hipHostFree selection results");
                select_host_ = nullptr;
                select_host_bytes_ = 0;
            }
            drop_select_graph();
            check(hipMalloc(&select_, need), "hipMalloc selection scratch");
            select_bytes_ = need;
            check(hipHostMalloc(&select_host_, result_bytes, hipHostMallocDefault), "hipHostMalloc selection results");
            select_host_bytes_ = result_bytes;
        }
        char* base = static_cast<char*>(select_);
        int64_t* device_ids = reinterpret_cast<int64_t*>(base + align(scratch));
        void* device_values = base + align(scratch) + id_bytes;
        try {
            upload(inputs);
            const std::array<size_t, 6> key{size_t(index), size_t(dtype), rows, width, size_t(k), reinterpret_cast<size_t>(select_)};
            launch_all_then(key, [&]() {
                char message[256] = {0};
                if (chroma_select::launch_rows_topk(static_cast<char*>(base_) + plan_.outputs[index].offset, dtype, rows, width, k, 1,
                                                    device_values, device_ids, select_, scratch, stream_, message, sizeof(message))) {
                    throw HipError(message);
                }
            });
            check(hipMemcpyAsync(error_host_, static_cast<char*>(base_) + plan_.error, sizeof(unsigned), hipMemcpyDeviceToHost, stream_),
                  "Read index error");
            check(hipMemcpyAsync(select_host_, device_ids, result_bytes, hipMemcpyDeviceToHost, stream_), "Download selection");
            download(outputs);
            check(hipStreamSynchronize(stream_), "HIP execution");
            std::memcpy(ids, select_host_, id_bytes);
            std::memcpy(values, static_cast<char*>(select_host_) + id_bytes, value_bytes);
            raise_index_error();
        } catch (const HipError&) {
            hipStreamSynchronize(stream_);
            throw;
        }
    }

    // A null input pointer leaves that input's staging region as it is (device-resident data from an
    // earlier upload or device copy); a null output pointer skips that output's download.
    // Consecutive inputs whose host arrays sit in one page-locked block at the same distances as their
    // staging regions go up as one copy (the gaps are padding on both sides).
    void upload(const void* const* inputs) {
        DeviceGuard guard(device_);
        // Inputs in staging order; a run of adjacent given inputs whose host arrays lie at the same distances
        // as their staging regions (a page-locked mirror of the staging) goes up as one copy.
        const size_t count = plan_.inputs.size();
        std::vector<size_t> order(count);
        for (size_t i = 0; i < count; ++i) {
            order[i] = i;
        }
        std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return plan_.inputs[a].offset < plan_.inputs[b].offset; });
        for (size_t n = 0; n < count;) {
            const size_t i = order[n];
            if (!plan_.inputs[i].bytes || !inputs[i]) {
                ++n;
                continue;
            }
            const char* first = static_cast<const char*>(inputs[i]);
            const size_t start = plan_.inputs[i].offset;
            size_t end = n + 1;
            while (end < count && plan_.inputs[order[end]].bytes && inputs[order[end]] &&
                   static_cast<const char*>(inputs[order[end]]) - first == std::ptrdiff_t(plan_.inputs[order[end]].offset - start)) {
                ++end;
            }
            const size_t last = order[end - 1];
            const size_t span = plan_.inputs[last].offset + plan_.inputs[last].bytes - start;
            if (end - n > 1 && is_pinned(first, span)) {
                to_device(static_cast<char*>(base_) + start, first, span);
            } else {
                for (size_t k = n; k < end; ++k) {
                    to_device(static_cast<char*>(base_) + plan_.inputs[order[k]].offset, inputs[order[k]], plan_.inputs[order[k]].bytes);
                }
            }
            n = end;
        }
    }

    // Pageable destinations hold their data when this returns; pinned and small ones once the stream
    // has drained (finish_download).
    void download(void* const* outputs) {
        DeviceGuard guard(device_);
        for (size_t i = 0; i < plan_.outputs.size(); ++i) {
            if (plan_.outputs[i].bytes && outputs[i]) {
                to_host(outputs[i], static_cast<char*>(base_) + plan_.outputs[i].offset, plan_.outputs[i].bytes);
            }
        }
    }

    void finish_download() { check(hipStreamSynchronize(stream_), "Download output"); }

    void* input_pointer(size_t index) const {
        return index < plan_.inputs.size() ? static_cast<char*>(base_) + plan_.inputs[index].offset : nullptr;
    }
    void* output_pointer(size_t index) const {
        return index < plan_.outputs.size() ? static_cast<char*>(base_) + plan_.outputs[index].offset : nullptr;
    }

    // Device-to-device rectangle copy on this program's stream (``height`` rows of ``width`` bytes),
    // finished before returning unless ``queued`` (then ordered before this program's later work).
    void copy_2d(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width, size_t height, bool queued) {
        DeviceGuard guard(device_);
        if (!width || !height) {
            return;
        }
        if (dst_pitch < width || src_pitch < width) {
            throw std::runtime_error("copy_2d pitch smaller than the row width");
        }
        check(hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, width, height, hipMemcpyDeviceToDevice, stream_), "hipMemcpy2DAsync");
        if (!queued) {
            check(hipStreamSynchronize(stream_), "Device copy");
        }
    }

    // Queued zero fill of input ``index``'s staging region (never part of a captured graph).
    void clear_input(size_t index) {
        DeviceGuard guard(device_);
        if (index >= plan_.inputs.size()) {
            throw std::runtime_error("clear_input: no such input");
        }
        if (plan_.inputs[index].bytes) {
            check(hipMemsetAsync(input_pointer(index), 0, plan_.inputs[index].bytes, stream_), "hipMemsetAsync");
        }
    }

    // Queued rectangle copies in one kernel launch (copy.hip).
    void copy_2d_batch(const chroma_hip_rect* rects, int count) {
        DeviceGuard guard(device_);
        if (count < 1 || count > chroma_copy::kMaxRects) {
            throw std::runtime_error("copy_2d_batch takes 1 to 4 rectangles");
        }
        chroma_copy::Rect copies[chroma_copy::kMaxRects];
        int used = 0;
        for (int i = 0; i < count; ++i) {
            if (rects[i].width && rects[i].height) {
                copies[used++] = chroma_copy::Rect{rects[i].dst, rects[i].dst_pitch, rects[i].src, rects[i].src_pitch, rects[i].width, rects[i].height};
            }
        }
        if (!used) {
            return;
        }
        char message[256] = {0};
        if (chroma_copy::launch_copy_rects(copies, used, stream_, message, sizeof(message))) {
            throw std::runtime_error(message);
        }
    }

    // The two attention masks of a multi-step decoder call, written by a kernel queued on this program's
    // stream straight into the staging regions of inputs ``full_input`` and ``window_input`` (so the next
    // resident run, given None for them, uses them): the slot table goes up (through a pinned copy), and
    // chroma_masks builds both masks from it.
    void decoder_masks(const int64_t* slots, int64_t context, int64_t position, int64_t steps, int64_t window, bool bfloat16,
                       size_t full_input, size_t window_input) {
        DeviceGuard guard(device_);
        if (full_input >= plan_.inputs.size() || window_input >= plan_.inputs.size() || context < 1 || steps < 1) {
            throw std::runtime_error("decoder_masks: no such inputs or an empty call");
        }
        const size_t bytes = size_t(steps) * size_t(context + steps) * (bfloat16 ? 2u : 4u);
        if (plan_.inputs[full_input].bytes != bytes || plan_.inputs[window_input].bytes != bytes) {
            throw std::runtime_error("decoder_masks: the mask inputs are not [steps, context + steps] of that dtype");
        }
        if (slots_copied_ == nullptr) {
            check(hipEventCreateWithFlags(&slots_copied_, hipEventDisableTiming), "decoder_masks hipEventCreate");
        } else {
            // the previous call's upload out of the pinned table has finished before the table is rewritten
            // (the device table itself is only rewritten by a copy queued after the kernels that read it)
            check(hipEventSynchronize(slots_copied_), "decoder_masks");
        }
        if (slots_capacity_ < size_t(context)) {
            check(hipStreamSynchronize(stream_), "decoder_masks");  // the old device table is no longer read
            if (slots_) {
                hipFree(slots_);
                slots_ = nullptr;
            }
            if (slots_host_) {
                hipHostFree(slots_host_);
                slots_host_ = nullptr;
            }
            slots_capacity_ = 0;
            check(hipMalloc(reinterpret_cast<void**>(&slots_), size_t(context) * sizeof(int64_t)), "decoder_masks hipMalloc");
            check(hipHostMalloc(reinterpret_cast<void**>(&slots_host_), size_t(context) * sizeof(int64_t), hipHostMallocDefault),
                  "decoder_masks hipHostMalloc");
            slots_capacity_ = size_t(context);
        }
        std::memcpy(slots_host_, slots, size_t(context) * sizeof(int64_t));
        check(hipMemcpyAsync(slots_, slots_host_, size_t(context) * sizeof(int64_t), hipMemcpyHostToDevice, stream_), "decoder_masks upload");
        check(hipEventRecord(slots_copied_, stream_), "decoder_masks hipEventRecord");
        char message[256] = {0};
        if (chroma_masks::launch_decoder_masks(slots_, context, position, steps, window, bfloat16, input_pointer(full_input),
                                               input_pointer(window_input), stream_, message, sizeof(message))) {
            throw std::runtime_error(message);
        }
    }

    void synchronize() {
        DeviceGuard guard(device_);
        check(hipStreamSynchronize(stream_), "Synchronize");
    }

    float execute(int iterations, bool timed) {
        DeviceGuard guard(device_);
        if (timed) {
            check(hipEventRecord(start_, stream_), "hipEventRecord");
        }
        for (int i = 0; i < iterations; ++i) {
            launch_all();
        }
        float milliseconds = 0.0f;
        if (timed) {
            check(hipEventRecord(stop_, stream_), "hipEventRecord");
        }
        check(hipMemcpyAsync(error_host_, static_cast<char*>(base_) + plan_.error, sizeof(unsigned), hipMemcpyDeviceToHost, stream_),
              "Read index error");
        check(hipStreamSynchronize(stream_), "HIP execution");
        if (timed) {
            check(hipEventElapsedTime(&milliseconds, start_, stop_), "hipEventElapsedTime");
        }
        raise_index_error();
        return milliseconds;
    }

    // ``copies`` back-to-back executions of the plan captured as one graph, launched ``iterations`` times
    // between hipEvents: the per-execution time without the host's per-replay graph launch, so a plan of
    // one short kernel is timed by its kernel and the dispatch barrier in front of it. Returns the total.
    float execute_chained(int copies, int iterations) {
        DeviceGuard guard(device_);
        if (copies < 1 || iterations < 1 || plan_.launches.empty()) {
            throw std::runtime_error("execute_chained needs a plan and positive counts");
        }
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            for (int i = 0; i < copies; ++i) {
                launch_direct();
            }
        } catch (...) {
            hipStreamEndCapture(stream_, &graph);
            if (graph) {
                hipGraphDestroy(graph);
            }
            throw;
        }
        check(hipStreamEndCapture(stream_, &graph), "hipStreamEndCapture");
        std::unique_ptr<std::remove_pointer_t<hipGraph_t>, hipError_t (*)(hipGraph_t)> graph_owner(graph, hipGraphDestroy);
        check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
        std::unique_ptr<std::remove_pointer_t<hipGraphExec_t>, hipError_t (*)(hipGraphExec_t)> exec_owner(exec, hipGraphExecDestroy);
        check(hipGraphLaunch(exec, stream_), "hipGraphLaunch");  // warm-up
        check(hipEventRecord(start_, stream_), "hipEventRecord");
        for (int i = 0; i < iterations; ++i) {
            check(hipGraphLaunch(exec, stream_), "hipGraphLaunch");
        }
        check(hipEventRecord(stop_, stream_), "hipEventRecord");
        check(hipMemcpyAsync(error_host_, static_cast<char*>(base_) + plan_.error, sizeof(unsigned), hipMemcpyDeviceToHost, stream_),
              "Read index error");
        check(hipStreamSynchronize(stream_), "HIP execution");
        float milliseconds = 0.0f;
        check(hipEventElapsedTime(&milliseconds, start_, stop_), "hipEventElapsedTime");
        raise_index_error();
        return milliseconds;
    }

private:
    void ensure_staging() {
        for (int slot = 0; slot < 2; ++slot) {
            if (!staged_[slot]) {
                check(hipEventCreateWithFlags(&staged_[slot], hipEventDisableTiming), "hipEventCreateWithFlags");
            }
            if (!staging_[slot]) {
                check(hipHostMalloc(&staging_[slot], kStagingSlot, hipHostMallocDefault), "hipHostMalloc staging");
            }
        }
    }

    void to_device(void* device, const void* host, size_t bytes) {
        if (bytes <= kDirectBytes || is_pinned(host, bytes)) {
            check(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, stream_), "Upload input");
            return;
        }
        ensure_staging();
        for (size_t at = 0, chunk = 0; at < bytes; at += kStagingSlot, ++chunk) {
            const int slot = int(chunk % 2);
            const size_t n = std::min(kStagingSlot, bytes - at);
            check(hipEventSynchronize(staged_[slot]), "Upload input");  // the slot's last DMA has finished
            std::memcpy(staging_[slot], static_cast<const char*>(host) + at, n);
            check(hipMemcpyAsync(static_cast<char*>(device) + at, staging_[slot], n, hipMemcpyHostToDevice, stream_), "Upload input");
            check(hipEventRecord(staged_[slot], stream_), "Upload input");
        }
    }

    void to_host(void* host, const void* device, size_t bytes) {
        if (bytes <= kDirectBytes || is_pinned(host, bytes)) {
            check(hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost, stream_), "Download output");
            return;
        }
        ensure_staging();
        const size_t chunks = (bytes + kStagingSlot - 1) / kStagingSlot;
        auto drain = [&](size_t chunk) {
            const int slot = int(chunk % 2);
            const size_t at = chunk * kStagingSlot;
            check(hipEventSynchronize(staged_[slot]), "Download output");
            std::memcpy(static_cast<char*>(host) + at, staging_[slot], std::min(kStagingSlot, bytes - at));
        };
        for (size_t chunk = 0; chunk < chunks; ++chunk) {
            const int slot = int(chunk % 2);
            if (chunk >= 2) {
                drain(chunk - 2);  // frees the slot while the DMA of chunk - 1 runs
            }
            const size_t at = chunk * kStagingSlot;
            check(hipMemcpyAsync(staging_[slot], static_cast<const char*>(device) + at, std::min(kStagingSlot, bytes - at),
                                 hipMemcpyDeviceToHost, stream_),
                  "Download output");
            check(hipEventRecord(staged_[slot], stream_), "Download output");
        }
        for (size_t chunk = chunks >= 2 ? chunks - 2 : 0; chunk < chunks; ++chunk) {
            drain(chunk);
        }
    }

    // A cooperative kernel (chroma_coop_*) has its workgroups wait for each other, which needs every one of
    // them resident at once: refuse to load a program whose cooperative grid this device cannot hold (its
    // waits are bounded and would end in an error rather than a hang, but the result would be lost).
    void check_co_resident(const Launch& launch) {
        int per_cu = 0, cus = 0;
        check(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, launch.function, int(launch.block), launch.shared),
              "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
        check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_), "hipDeviceGetAttribute");
        const size_t grid = size_t(launch.grid[0]) * launch.grid[1] * launch.grid[2];
        if (size_t(per_cu) * size_t(cus) < grid) {
            throw std::runtime_error("Cooperative kernel " + launch.kernel + " needs " + std::to_string(grid) +
                                     " co-resident workgroups; this device holds " + std::to_string(per_cu * cus));
        }
    }

    void raise_index_error() {
        if (*error_host_) {
            const unsigned word = *error_host_;
            *error_host_ = 0;
            // the whole error region: the index word and the in-kernel handoff tickets (words 16-255), which
            // every launch returns to zero itself; clearing them here too (outside any captured graph, after
            // the stream has drained) leaves nothing for a later launch to inherit
            check(hipMemsetAsync(static_cast<char*>(base_) + plan_.error, 0, kErrorRegion, stream_), "Clear index error");
            check(hipStreamSynchronize(stream_), "Clear index error");
            if (word & 2u) {
                // words a cooperative kernel left behind would match a later launch's tags
                check(hipMemsetAsync(static_cast<char*>(base_) + plan_.weight_bytes, 0, plan_.error - plan_.weight_bytes, stream_),
                      "Clear workspace");
                check(hipStreamSynchronize(stream_), "Clear workspace");
                throw std::runtime_error("Cooperative workgroups timed out waiting for each other");
            }
            throw IndexError("Tensor index out of range");
        }
    }

    void launch_direct() {
        for (auto& launch : plan_.launches) {
            check(hipModuleLaunchKernel(launch.function, launch.grid[0], launch.grid[1], launch.grid[2], launch.block, 1, 1,
                                        launch.shared, stream_, launch.arguments.data(), nullptr),
                  "hipModuleLaunchKernel");
        }
    }

    void drop_select_graph() noexcept {
        if (select_exec_) {
            hipGraphExecDestroy(select_exec_);
        }
        if (select_graph_) {
            hipGraphDestroy(select_graph_);
        }
        select_exec_ = nullptr;
        select_graph_ = nullptr;
    }

    // The plan followed by ``select`` (queued on the stream). With graphs on, both replay as one captured
    // graph, kept for the selection ``key`` it was captured with (so a greedy decode step is one graph
    // launch: the selection's kernels cost neither host-side launches nor a plain-stream gap).
    template <class Select> void launch_all_then(const std::array<size_t, 6>& key, Select select) {
        if (!use_graph_ || plan_.launches.empty()) {
            launch_direct();
            select();
            return;
        }
        if (!select_exec_ || select_key_ != key) {
            drop_select_graph();
            check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            try {
                launch_direct();
                select();
            } catch (...) {
                hipGraph_t broken = nullptr;
                hipStreamEndCapture(stream_, &broken);
                if (broken) {
                    hipGraphDestroy(broken);
                }
                throw;
            }
            check(hipStreamEndCapture(stream_, &select_graph_), "hipStreamEndCapture");
            check(hipGraphInstantiate(&select_exec_, select_graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
            select_key_ = key;
        }
        check(hipGraphLaunch(select_exec_, stream_), "hipGraphLaunch");
    }

    void launch_all() {
        // A plan of one kernel gains nothing from a graph: replaying a one-node graph cost ~5 us more per
        // execution than the direct launch on MI355X (the C2 kernel: 274 against 270 us per execution).
        if (!use_graph_ || plan_.launches.size() <= 1) {
            launch_direct();
            return;
        }
        if (!graph_exec_) {
            check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            try {
                launch_direct();
            } catch (...) {
                hipGraph_t broken = nullptr;
                hipStreamEndCapture(stream_, &broken);
                if (broken) {
                    hipGraphDestroy(broken);
                }
                throw;
            }
            check(hipStreamEndCapture(stream_, &graph_), "hipStreamEndCapture");
            check(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
        }
        check(hipGraphLaunch(graph_exec_, stream_), "hipGraphLaunch");
    }

    void upload_weights(const std::string& path) {
        std::FILE* file = std::fopen(path.c_str(), "rb");
        long size = -1;
        if (file && std::fseek(file, 0, SEEK_END) == 0) {
            size = std::ftell(file);
        }
        if (!file || size < 0 || static_cast<size_t>(size) != plan_.weight_bytes) {
            if (file) {
                std::fclose(file);
            }
            throw std::runtime_error("Missing weights file or incorrect byte size");
        }
        std::rewind(file);
        // Stream through a pinned staging buffer so large weight files never need a host copy of their size.
        const size_t chunk = size_t(64) << 20;
        char* staging = nullptr;
        check(hipHostMalloc(reinterpret_cast<void**>(&staging), chunk, hipHostMallocDefault), "hipHostMalloc");
        std::unique_ptr<char, hipError_t (*)(void*)> owner(staging, hipHostFree);
        for (size_t done = 0; done < plan_.weight_bytes;) {
            const size_t bytes = std::min(chunk, plan_.weight_bytes - done);
            if (std::fread(staging, 1, bytes, file) != bytes) {
                std::fclose(file);
                throw std::runtime_error("Cannot read weights");
            }
            check(hipMemcpy(static_cast<char*>(base_) + done, staging, bytes, hipMemcpyHostToDevice), "Upload weights");
            done += bytes;
        }
        std::fclose(file);
    }

    Plan plan_;
    int device_ = -1;
    std::string name_;
    hipStream_t stream_ = nullptr;
    hipEvent_t start_ = nullptr, stop_ = nullptr;
    void* base_ = nullptr;
    unsigned* error_host_ = nullptr;
    hipModule_t module_ = nullptr;
    bool use_graph_ = false;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t graph_exec_ = nullptr;
    void* staging_[2] = {nullptr, nullptr};  // pinned slots for pageable host transfers (allocated on first use)
    int64_t* slots_ = nullptr;       // decoder_masks: the cache's slot table on the device (allocated on first use)
    int64_t* slots_host_ = nullptr;  // and its pinned copy (the caller's array may be gone before the copy ends)
    size_t slots_capacity_ = 0;      // entries both hold
    hipEvent_t slots_copied_ = nullptr;  // recorded after each upload out of slots_host_
    void* select_ = nullptr;  // run_top's selection scratch and device results (allocated on first use)
    size_t select_bytes_ = 0;
    void* select_host_ = nullptr;  // pinned landing area of run_top's ids and values
    size_t select_host_bytes_ = 0;
    // run_top's plan and selection captured as one graph, for the selection it was captured with
    hipGraph_t select_graph_ = nullptr;
    hipGraphExec_t select_exec_ = nullptr;
    std::array<size_t, 6> select_key_{};
    hipEvent_t staged_[2] = {nullptr, nullptr};
};

int fail(int status, const char* message, char* error, size_t size) {
    if (error && size) {
        std::snprintf(error, size, "%s", message);
    }
    return status;
}

template <class F> int guarded(char* error, size_t size, F body) {
    try {
        body();
        return CHROMA_HIP_OK;
    } catch (const IndexError& e) {
        return fail(CHROMA_HIP_INDEX_ERROR, e.what(), error, size);
    } catch (const std::exception& e) {
        return fail(CHROMA_HIP_RUNTIME_ERROR, e.what(), error, size);
    } catch (...) {
        return fail(CHROMA_HIP_RUNTIME_ERROR, "unknown error", error, size);
    }
}

Program* program(void* handle) { return static_cast<Program*>(handle); }

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int chroma_hip_create(const char* artifact_dir, void** handle, char* error, size_t error_size) {
    return guarded(error, error_size, [&] {
        *handle = nullptr;
        *handle = new Program(artifact_dir);
    });
}

__attribute__((visibility("default"))) int chroma_hip_run(void* handle, const void* const* inputs, void* const* outputs, char* error,
                                                          size_t error_size) {
    return guarded(error, error_size, [&] { program(handle)->run(inputs, outputs); });
}

__attribute__((visibility("default"))) int chroma_hip_run_top(void* handle, const void* const* inputs, void* const* outputs, int output_index,
                                                              int dtype, size_t rows, size_t width, int k, void* values, int64_t* ids,
                                                              char* error, size_t error_size) {
    return guarded(error, error_size, [&] { program(handle)->run_top(inputs, outputs, output_index, dtype, rows, width, k, values, ids); });
}

__attribute__((visibility("default"))) const char* chroma_hip_device_name(void* handle) { return program(handle)->name().c_str(); }

__attribute__((visibility("default"))) const char* chroma_hip_signature(void* handle) { return program(handle)->signature().c_str(); }

__attribute__((visibility("default"))) void chroma_hip_destroy(void* handle) { delete program(handle); }

__attribute__((visibility("default"))) int chroma_hip_upload(void* handle, const void* const* inputs, char* error, size_t error_size) {
    return guarded(error, error_size, [&] {
        program(handle)->upload(inputs);
        program(handle)->finish_download();
    });
}

__attribute__((visibility("default"))) int chroma_hip_execute(void* handle, int iterations, float* milliseconds, char* error,
                                                              size_t error_size) {
    return guarded(error, error_size, [&] {
        const float elapsed = program(handle)->execute(iterations, milliseconds != nullptr);
        if (milliseconds) {
            *milliseconds = elapsed;
        }
    });
}

__attribute__((visibility("default"))) int chroma_hip_execute_chained(void* handle, int copies, int iterations, float* milliseconds,
                                                                      char* error, size_t error_size) {
    return guarded(error, error_size, [&] {
        const float elapsed = program(handle)->execute_chained(copies, iterations);
        if (milliseconds) {
            *milliseconds = elapsed;
        }
    });
}

__attribute__((visibility("default"))) int chroma_hip_download(void* handle, void* const* outputs, char* error, size_t error_size) {
    return guarded(error, error_size, [&] {
        program(handle)->download(outputs);
        program(handle)->finish_download();
    });
}

__attribute__((visibility("default"))) int chroma_hip_set_graph(void* handle, int enabled) { return program(handle)->set_graph(enabled); }

__attribute__((visibility("default"))) int chroma_hip_launch_count(void* handle) { return program(handle)->launch_count(); }

__attribute__((visibility("default"))) void* chroma_hip_device_base(void* handle) { return program(handle)->base(); }

__attribute__((visibility("default"))) int chroma_hip_decoder_masks(void* handle, const int64_t* slots, int64_t context, int64_t position,
                                                                    int64_t steps, int64_t window, int dtype, int full_input,
                                                                    int window_input, char* error, size_t error_size) {
    return guarded(error, error_size, [&] {
        if (dtype != CHROMA_HIP_FLOAT32 && dtype != CHROMA_HIP_BFLOAT16) {
            throw std::runtime_error("decoder_masks: float32 or bfloat16 masks");
        }
        if (full_input < 0 || window_input < 0) {
            throw std::runtime_error("decoder_masks: negative input index");
        }
        program(handle)->decoder_masks(slots, context, position, steps, window, dtype == CHROMA_HIP_BFLOAT16, size_t(full_input),
                                       size_t(window_input));
    });
}

__attribute__((visibility("default"))) void* chroma_hip_input_pointer(void* handle, int index) {
    return index < 0 ? nullptr : program(handle)->input_pointer(size_t(index));
}

__attribute__((visibility("default"))) void* chroma_hip_output_pointer(void* handle, int index) {
    return index < 0 ? nullptr : program(handle)->output_pointer(size_t(index));
}

__attribute__((visibility("default"))) int chroma_hip_host_alloc(size_t bytes, void** pointer, char* error, size_t error_size) {
    return guarded(error, error_size, [&] {
        *pointer = nullptr;
        check(hipHostMalloc(pointer, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc");
        std::lock_guard<std::mutex> lock(pinned_mutex);
        pinned_blocks[reinterpret_cast<uintptr_t>(*pointer)] = bytes;
    });
}

__attribute__((visibility("default"))) void chroma_hip_host_free(void* pointer) {
    if (!pointer) {
        return;
    }
    {
        std::lock_guard<std::mutex> lock(pinned_mutex);
        pinned_blocks.erase(reinterpret_cast<uintptr_t>(pointer));
    }
    hipHostFree(pointer);
}

__attribute__((visibility("default"))) int chroma_hip_copy_2d(void* handle, void* dst, size_t dst_pitch, const void* src, size_t src_pitch,
                                                              size_t width, size_t height, char* error, size_t error_size) {
    return guarded(error, error_size, [&] { program(handle)->copy_2d(dst, dst_pitch, src, src_pitch, width, height, false); });
}

__attribute__((visibility("default"))) int chroma_hip_copy_2d_batch_queued(void* handle, const chroma_hip_rect* rects, int count, char* error,
                                                                            size_t error_size) {
    return guarded(error, error_size, [&] { program(handle)->copy_2d_batch(rects, count); });
}

__attribute__((visibility("default"))) int chroma_hip_copy_2d_queued(void* handle, void* dst, size_t dst_pitch, const void* src, size_t src_pitch,
                                                                     size_t width, size_t height, char* error, size_t error_size) {
    return guarded(error, error_size, [&] { program(handle)->copy_2d(dst, dst_pitch, src, src_pitch, width, height, true); });
}

__attribute__((visibility("default"))) int chroma_hip_clear_input(void* handle, int index, char* error, size_t error_size) {
    return guarded(error, error_size, [&] {
        if (index < 0) {
            throw std::runtime_error("clear_input: negative input index");
        }
        program(handle)->clear_input(size_t(index));
    });
}

__attribute__((visibility("default"))) int chroma_hip_synchronize(void* handle, char* error, size_t error_size) {
    return guarded(error, error_size, [&] { program(handle)->synchronize(); });
}
}
