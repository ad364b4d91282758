// Device handle, caching allocator, host<->device copies, CSR plan upload
// (runtime/backend.rs:203-392, :1449-1475, :1542-1597).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace {
thread_local std::string g_last_error;
constexpr size_t kGranule = 512;
// Blocks of at least 1 MiB are placed at (n mod 16) * 4 KiB into a slightly larger driver
// allocation, n counting such blocks: streams that would otherwise sit a power of two apart
// (equal-sized tensors allocated back to back) then spread over the HBM channels.  Measured on
// MI355X: four 16 MiB Adam streams run at 5.4 TB/s unskewed and 6.0 TB/s skewed.
constexpr size_t kSkewMin = size_t(1) << 20;
constexpr size_t kSkewStep = 4096;
constexpr size_t kSkewSlots = 16;
}  // namespace

namespace axis {

int fail(int code, const std::string &message) {
    g_last_error = message;
    return code;
}

int hip_fail(hipError_t error, const char *what) {
    return fail(error == hipErrorOutOfMemory ? AXIS_ERROR_MEMORY : AXIS_ERROR_HIP,
                std::string(what) + ": " + hipGetErrorString(error));
}

int enter(axis_device device) {
    if (!device) return fail(AXIS_ERROR_INVALID, "null axis_device");
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess || current != device->ordinal) {
        AXIS_HIP(hipSetDevice(device->ordinal));
    }
    return AXIS_OK;
}

int launch_status(const char *kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, kernel);
    return AXIS_OK;
}

// Returns a block to the driver (its raw base when the block was skewed).
void driver_free(axis_device device, void *ptr) {
    auto r = device->raw.find(ptr);
    if (r != device->raw.end()) {
        (void)hipFree(r->second);
        device->raw.erase(r);
    } else {
        (void)hipFree(ptr);
    }
}

void drop_cache(axis_device device) {
    for (auto &kv : device->free_blocks) driver_free(device, kv.second);
    device->free_blocks.clear();
    device->cached = 0;
}

int alloc(axis_device device, size_t bytes, void **out) {
    size_t size = std::max<size_t>(kGranule, (bytes + kGranule - 1) / kGranule * kGranule);
    auto it = device->free_blocks.find(size);
    if (it != device->free_blocks.end()) {
        *out = it->second;
        device->free_blocks.erase(it);
        device->cached -= size;
    } else {
        const bool skew = size >= kSkewMin;
        const size_t offset = skew ? (size_t)(device->skew_next++ % kSkewSlots) * kSkewStep : 0;
        const size_t request = skew ? size + (kSkewSlots - 1) * kSkewStep : size;
        void *ptr = nullptr;
        hipError_t e = hipMalloc(&ptr, request);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            // Give the cache back to the driver and try once more.
            AXIS_HIP(hipStreamSynchronize(device->stream));
            drop_cache(device);
            e = hipMalloc(&ptr, request);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                return fail(AXIS_ERROR_MEMORY, "hipMalloc of " + std::to_string(request) +
                                                   " bytes failed: " + hipGetErrorString(e));
            }
        }
        *out = static_cast<char *>(ptr) + offset;
        if (skew) device->raw[*out] = ptr;
    }
    device->live[*out] = size;
    device->in_use += size;
    return AXIS_OK;
}

void release(axis_device device, void *ptr) {
    auto it = device->live.find(ptr);
    if (it == device->live.end()) return;
    device->free_blocks.emplace(it->second, ptr);
    device->cached += it->second;
    device->in_use -= it->second;
    device->live.erase(it);
}

namespace {
hipEvent_t take_event(axis_device device) {
    if (!device->spare_events.empty()) {
        hipEvent_t e = device->spare_events.back();
        device->spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
}  // namespace

TimedLaunch::TimedLaunch(axis_device d, const char *f, double w) : device(d), family(f), work(w) {
    if (!device || !device->timing) return;
    start = take_event(device);
    if (start) (void)hipEventRecord(start, device->stream);
}

TimedLaunch::~TimedLaunch() {
    if (!start) return;
    hipEvent_t stop = take_event(device);
    if (!stop) return;
    (void)hipEventRecord(stop, device->stream);
    device->timed[family].push_back({start, stop, work});
}

}  // namespace axis

namespace {

__global__ void fill_kernel(float *__restrict__ out, float value, int64_t len) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < len; i += stride) out[i] = value;
}

}  // namespace

extern "C" {

const char *axis_last_error(void) { return g_last_error.c_str(); }

const char *axis_version(void) { return "axis_hip 0.1.0 (gfx950, fp32 MFMA)"; }

int axis_device_create(int ordinal, axis_device *out) {
    if (!out) return axis::fail(AXIS_ERROR_INVALID, "null output handle");
    int count = 0;
    AXIS_HIP(hipGetDeviceCount(&count));
    if (ordinal < 0 || ordinal >= count)
        return axis::fail(AXIS_ERROR_INVALID, "device ordinal " + std::to_string(ordinal) +
                                                  " out of range (" + std::to_string(count) +
                                                  " devices)");
    AXIS_HIP(hipSetDevice(ordinal));
    hipDeviceProp_t prop;
    AXIS_HIP(hipGetDeviceProperties(&prop, ordinal));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return axis::fail(AXIS_ERROR_INVALID, std::string("libaxis_hip is built for gfx950; device is ") +
                                                  prop.gcnArchName);
    auto *device = new axis_device_s();
    device->ordinal = ordinal;
    device->multiprocessors = prop.multiProcessorCount;
    device->fold_splits = std::getenv("AXIS_GEMM_UNFOLDED") == nullptr;
    hipError_t e = hipStreamCreateWithFlags(&device->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete device;
        return axis::hip_fail(e, "hipStreamCreateWithFlags");
    }
    if (int st = axis::bind_static_scratch(device)) {
        (void)hipStreamDestroy(device->stream);
        delete device;
        return st;
    }
    *out = device;
    return AXIS_OK;
}

int axis_device_create_bf16(int ordinal, axis_device *out) {
    if (int st = axis_device_create(ordinal, out)) return st;
    (*out)->bf16_matmul = true;
    return AXIS_OK;
}

int axis_device_bf16_matmul(axis_device device, int *enabled) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(enabled, "null output");
    *enabled = device->bf16_matmul ? 1 : 0;
    return AXIS_OK;
}

int axis_device_destroy(axis_device device) {
    AXIS_ENTER(device);
    AXIS_HIP(hipStreamSynchronize(device->stream));
    axis::drop_cache(device);
    for (auto &kv : device->live) axis::driver_free(device, kv.first);
    for (auto &kv : device->timed)
        for (auto &t : kv.second) {
            (void)hipEventDestroy(t.start);
            (void)hipEventDestroy(t.stop);
        }
    for (hipEvent_t e : device->spare_events) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(device->stream);
    delete device;
    return AXIS_OK;
}

int axis_device_synchronize(axis_device device) {
    AXIS_ENTER(device);
    if (int st = axis::flush_finish(device)) return st;
    AXIS_HIP(hipStreamSynchronize(device->stream));
    return AXIS_OK;
}

int axis_device_stream(axis_device device, void **stream) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(stream, "null stream output");
    *stream = device->stream;
    return AXIS_OK;
}

int axis_alloc(axis_device device, size_t bytes, void **out) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(out, "null output pointer");
    return axis::alloc(device, bytes, out);
}

int axis_free(axis_device device, void *ptr) {
    AXIS_ENTER(device);
    if (!ptr) return AXIS_OK;
    auto it = device->live.find(ptr);
    AXIS_REQUIRE(it != device->live.end(), "axis_free of a pointer this device did not allocate");
    // a deferred sum still to write here runs first (its block is then free to reuse)
    if (int st = axis_finish_before_read(device, ptr, it->second)) return st;
    axis::release(device, ptr);
    return AXIS_OK;
}

int axis_memory_stats(axis_device device, size_t *in_use, size_t *cached) {
    AXIS_ENTER(device);
    if (in_use) *in_use = device->in_use;
    if (cached) *cached = device->cached;
    return AXIS_OK;
}

int axis_empty_cache(axis_device device) {
    AXIS_ENTER(device);
    AXIS_HIP(hipStreamSynchronize(device->stream));
    axis::drop_cache(device);
    return AXIS_OK;
}

int axis_upload(axis_device device, void *dst, const void *src, size_t bytes) {
    AXIS_ENTER(device);
    if (bytes == 0) return AXIS_OK;
    AXIS_REQUIRE(dst && src, "null upload pointer");
    if (int st = axis_finish_before_read(device, dst, bytes)) return st;  // a pending sum writes there first
    AXIS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, device->stream));
    // Pageable sources are staged by the runtime; wait so the caller may reuse `src` at once.
    AXIS_HIP(hipStreamSynchronize(device->stream));
    return AXIS_OK;
}

int axis_read(axis_device device, void *dst, const void *src, size_t bytes) {
    AXIS_ENTER(device);
    if (bytes == 0) return AXIS_OK;
    AXIS_REQUIRE(dst && src, "null read pointer");
    if (int st = axis_finish_before_read(device, src, bytes)) return st;
    AXIS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, device->stream));
    AXIS_HIP(hipStreamSynchronize(device->stream));
    return AXIS_OK;
}

int axis_copy(axis_device device, void *dst, const void *src, size_t bytes) {
    AXIS_ENTER(device);
    if (bytes == 0) return AXIS_OK;
    AXIS_REQUIRE(dst && src, "null copy pointer");
    if (int st = axis_finish_before_read(device, src, bytes)) return st;
    if (int st = axis_finish_before_read(device, dst, bytes)) return st;
    AXIS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, device->stream));
    return AXIS_OK;
}

int axis_fill(axis_device device, float *out, float value, int64_t len) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(len >= 0, "negative length");
    if (len == 0) return AXIS_OK;
    AXIS_REQUIRE(out, "null output");
    if (int st = axis_finish_before_read(device, out, (size_t)len * sizeof(float))) return st;
    fill_kernel<<<axis::blocks_for(len, 256, 8192), 256, 0, device->stream>>>(out, value, len);
    return axis::launch_status("fill_kernel");
}

int axis_timing_enable(axis_device device, int enabled) {
    AXIS_ENTER(device);
    device->timing = enabled != 0;
    return AXIS_OK;
}

int axis_timing_reset(axis_device device) {
    AXIS_ENTER(device);
    AXIS_HIP(hipStreamSynchronize(device->stream));
    for (auto &kv : device->timed)
        for (auto &t : kv.second) {
            device->spare_events.push_back(t.start);
            device->spare_events.push_back(t.stop);
        }
    device->timed.clear();
    return AXIS_OK;
}

int axis_timing_read(axis_device device, const char *family, int64_t *launches, double *milliseconds,
                     double *work) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(family, "null timing family");
    AXIS_HIP(hipStreamSynchronize(device->stream));
    int64_t n = 0;
    double ms = 0.0, w = 0.0;
    auto it = device->timed.find(family);
    if (it != device->timed.end()) {
        for (auto &t : it->second) {
            float elapsed = 0.0f;
            AXIS_HIP(hipEventElapsedTime(&elapsed, t.start, t.stop));
            ms += elapsed;
            w += t.work;
            ++n;
        }
    }
    if (launches) *launches = n;
    if (milliseconds) *milliseconds = ms;
    if (work) *work = w;
    return AXIS_OK;
}

int axis_plan_create(axis_device device, const int32_t *offsets, const int32_t *left,
                     const int32_t *right, int64_t groups, int uncapped, axis_plan *out) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(out && offsets, "null plan argument");
    AXIS_REQUIRE(groups >= 1, "plan needs at least one group");
    AXIS_REQUIRE(offsets[0] == 0, "plan offsets must start at 0");
    for (int64_t g = 0; g < groups; ++g)
        AXIS_REQUIRE(offsets[g + 1] >= offsets[g], "plan offsets must be nondecreasing");
    int64_t count = offsets[groups];
    if (!uncapped)
        AXIS_REQUIRE(count >= 1 && count <= 16777216,
                     "index plan must have 1..=16777216 contributions (experimental backend limit)");
    AXIS_REQUIRE(count == 0 || left, "null plan indices");
    // chunked_offsets (runtime/backend.rs:37-50): split each group's range at 512 contributions.
    std::vector<int32_t> chunk_offsets{offsets[0]};
    std::vector<int32_t> chunk_group{0};
    for (int64_t g = 0; g < groups; ++g) {
        int32_t cursor = offsets[g], end = offsets[g + 1];
        while (cursor < end) {
            cursor = std::min(cursor + axis::kGroupedChunk, end);
            chunk_offsets.push_back(cursor);
        }
        chunk_group.push_back(static_cast<int32_t>(chunk_offsets.size()) - 1);
    }
    auto *plan = new axis_plan_s();
    plan->groups = groups;
    plan->count = count;
    plan->chunks = static_cast<int64_t>(chunk_offsets.size()) - 1;
    auto upload = [&](int32_t **dst, const int32_t *src, size_t n) -> int {
        if (n == 0) return AXIS_OK;
        int status = axis::alloc(device, n * sizeof(int32_t), reinterpret_cast<void **>(dst));
        if (status) return status;
        AXIS_HIP(hipMemcpyAsync(*dst, src, n * sizeof(int32_t), hipMemcpyHostToDevice,
                                device->stream));
        return AXIS_OK;
    };
    int status = upload(&plan->offsets, offsets, groups + 1);
    if (!status) status = upload(&plan->left, left, count);
    if (!status && right) status = upload(&plan->right, right, count);
    if (!status) status = upload(&plan->chunk_offsets, chunk_offsets.data(), chunk_offsets.size());
    if (!status) status = upload(&plan->chunk_group, chunk_group.data(), chunk_group.size());
    if (!status) {
        hipError_t e = hipStreamSynchronize(device->stream);
        if (e != hipSuccess) status = axis::hip_fail(e, "plan upload");
    }
    if (status) {
        axis_plan_destroy(device, plan);
        return status;
    }
    *out = plan;
    return AXIS_OK;
}

int axis_plan_destroy(axis_device device, axis_plan plan) {
    AXIS_ENTER(device);
    if (!plan) return AXIS_OK;
    for (int32_t *p : {plan->offsets, plan->left, plan->right, plan->chunk_offsets, plan->chunk_group})
        if (p) axis::release(device, p);
    delete plan;
    return AXIS_OK;
}

}  // extern "C"
