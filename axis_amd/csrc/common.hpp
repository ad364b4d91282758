// Shared runtime pieces of libaxis_hip: the device handle, the stream-ordered caching allocator,
// error reporting and launch helpers.  Compiled for gfx950 only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>
#include <map>
#include <vector>
#include <string>
#include <unordered_map>

#include "../../include/axis_hip.h"
#include "finish.hpp"

struct axis_device_s {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    // Free blocks by rounded size.  All launches share one stream, so a block released after its
    // last use was enqueued can serve any later launch without a host wait.
    std::multimap<size_t, void *> free_blocks;
    std::unordered_map<void *, size_t> live;
    // Large blocks start at a rotating 4 KiB offset into their driver allocation (raw base kept
    // here): buffers a power of two apart alias onto the same HBM channels when streamed together.
    std::unordered_map<void *, void *> raw;
    unsigned skew_next = 0;
    size_t in_use = 0;
    size_t cached = 0;
    int multiprocessors = 256;
    // Device::cuda_bf16 (backend.rs:274-283): matrix products take bf16-rounded operands and
    // accumulate in fp32; everything else stays fp32.
    bool bf16_matmul = false;
    // Short split-K products over few tiles run their slices in one block's waves (gemm.hip,
    // gemm_fold_kernel); AXIS_GEMM_UNFOLDED set at creation keeps them as separate slices plus a
    // sum launch (the same bits, for comparison).
    bool fold_splits = true;
    // launch timing (axis_timing_*): event pairs and work per family
    bool timing = false;
    struct Timed {
        hipEvent_t start, stop;
        double work;
    };
    std::map<std::string, std::vector<Timed>> timed;
    std::vector<hipEvent_t> spare_events;
    // This GPU's copy of the allocation-free product's scratch array (gemm.hip), bound at create,
    // and the event that orders its users: every handle on this GPU shares both, so each call
    // waits for the previous call's last launch (from any handle) before reusing the array.
    float *static_scratch = nullptr;
    hipEvent_t static_scratch_done = nullptr;
    // Deferred finishing sums (axis_finish_defer): while on, the last sum of a weight or bias
    // gradient is recorded here instead of launched, and the scratch block it reads is held, until
    // one batched launch (axis_finish_flush) runs every recorded sum.
    bool deferring = false;
    std::vector<axis::FinishTask> deferred;
    std::vector<void *> deferred_blocks;
    size_t deferred_bytes = 0;  // held by deferred_blocks; a batch is launched past kMaxDeferredBytes
};

struct axis_plan_s {
    int32_t *offsets = nullptr;       // groups + 1
    int32_t *left = nullptr;          // count
    int32_t *right = nullptr;         // count, or null
    int32_t *chunk_offsets = nullptr; // chunks + 1: absolute bounds into left/right
    int32_t *chunk_group = nullptr;   // groups + 1: first chunk of each group
    int64_t groups = 0;
    int64_t count = 0;
    int64_t chunks = 0;
};

namespace axis {

constexpr int kGroupedChunk = 512;  // runtime/backend.rs:27 (GROUPED_CHUNK)

int fail(int code, const std::string &message);
int hip_fail(hipError_t error, const char *what);
int enter(axis_device device);  // validates the handle and makes its GPU current
int launch_status(const char *kernel);
int alloc(axis_device device, size_t bytes, void **out);
void release(axis_device device, void *ptr);
int bind_static_scratch(axis_device device);  // gemm.hip

// RAII scratch block from the device's caching allocator (returned on scope exit; stream order
// makes the reuse safe).
struct Scratch {
    axis_device device = nullptr;
    void *ptr = nullptr;
    Scratch() = default;
    Scratch(const Scratch &) = delete;
    Scratch &operator=(const Scratch &) = delete;
    ~Scratch() {
        if (ptr) release(device, ptr);
    }
    int get(axis_device d, size_t bytes) {
        device = d;
        return alloc(d, bytes, &ptr);
    }
    template <class T> T *as() const { return static_cast<T *>(ptr); }
    void *take() {  // the caller now owns the block
        void *p = ptr;
        ptr = nullptr;
        return p;
    }
};

// Records a finishing sum on a deferring handle and takes `held` (the block the sum reads) until
// the batched launch has been enqueued (finish.hip).  A full batch is launched first.
int defer_finish(axis_device device, const FinishTask &task, Scratch &held);
// Launches every recorded sum in one kernel and returns their blocks to the allocator.
int flush_finish(axis_device device);

// A buffer an entry reads or writes: its first byte and extent (1 when the entry reads it through
// strides, so only a pending output that holds its first byte is seen).
struct Span {
    const void *ptr;
    int64_t bytes;
};
// Launches the recorded sums when one of them writes into a span (finish.hip).
int finish_overlapping(axis_device device, std::initializer_list<Span> spans);
// Every kernel entry passes its buffers here before it launches: a pending finishing sum that
// writes one of them runs first, so no entry reads (or overwrites) a gradient whose last sum is
// still deferred.  Free when nothing is pending.
inline int guard(axis_device device, std::initializer_list<Span> spans) {
    return device->deferred.empty() ? AXIS_OK : finish_overlapping(device, spans);
}

inline unsigned blocks_for(int64_t work, int per_block, int64_t cap = 1 << 20) {
    int64_t b = (work + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return static_cast<unsigned>(b);
}

// Brackets one launch of a timed family with events on the device's stream (no-op unless
// timing is enabled).
struct TimedLaunch {
    axis_device device;
    const char *family;
    double work;
    hipEvent_t start = nullptr;
    TimedLaunch(axis_device d, const char *f, double w);
    ~TimedLaunch();
};

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace axis

#define AXIS_ENTER(dev)                                  \
    do {                                                 \
        int axis_enter_status = axis::enter(dev);        \
        if (axis_enter_status) return axis_enter_status; \
    } while (0)

#define AXIS_REQUIRE(cond, msg)                                         \
    do {                                                                \
        if (!(cond)) return axis::fail(AXIS_ERROR_INVALID, (msg));     \
    } while (0)

#define AXIS_GUARD(dev, ...)                                                   \
    do {                                                                       \
        if (int axis_guard_status = axis::guard((dev), {__VA_ARGS__})) return axis_guard_status; \
    } while (0)

#define AXIS_HIP(call)                                       \
    do {                                                     \
        hipError_t axis_hip_error = (call);                  \
        if (axis_hip_error != hipSuccess)                    \
            return axis::hip_fail(axis_hip_error, #call);    \
    } while (0)
