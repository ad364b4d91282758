// Deferred finishing sums: one launch for the last sums of several weight and bias gradients.
//
// The products and fused scatters that produce a layer's weight or bias gradient end with a short
// sum over partial results (split-K slices, per-block column partials).  Each is a few
// microseconds of work and a launch of its own.  While a handle defers them, those sums are
// recorded with the blocks they read held; the batched kernel below then runs every recorded sum
// in one launch, block b of the grid taking a block's share of one task, through the same device
// routines (finish.hpp) as the single-task kernels, so every output has the bits it would have
// had.  A caller that reads one of these outputs first asks for it with axis_finish_before_read.
#include <algorithm>

#include "common.hpp"

namespace {

constexpr int kMaxFinish = 24;  // tasks per launch (the batch travels as a kernel argument)
// Scratch a batch may hold before it is launched: each deferred sum keeps its partial block (up to
// 64 MiB of split slices) until the batch runs, so a deep, wide backward would otherwise hold
// every layer's partials at once.
constexpr size_t kMaxDeferredBytes = size_t(256) << 20;

struct FinishBatch {
    axis::FinishTask task[kMaxFinish];
    int32_t count;
};

// 256 threads.  Kind 0 (split sums): as split_sum_kernel, 64 outputs per block, wave g adding the
// slices of lane group g; kind 2 as split_sum4_kernel, 256 outputs per block.  Kind 1 (column
// block sums): 16 columns per block, thread t summing row
// range t / 16 of column t % 16 -- the ranges and their order of column_block_sum_kernel, whose
// 16-wave blocks hold the long-lived, latency-bound blocks of short sums back in a shared launch.
__global__ void __launch_bounds__(256) finish_batch_kernel(FinishBatch b) {
    __shared__ float lds[16][64];
    int32_t local = (int32_t)blockIdx.x;
    int t = 0;
    while (t + 1 < b.count && local >= b.task[t].blocks) local -= b.task[t++].blocks;
    const axis::FinishTask &k = b.task[t];
    if (k.kind == 2) {
        __shared__ axis::finish_floatx4 acc[4][64];
        const int lane = threadIdx.x & 63, group = threadIdx.x >> 6;
        const int64_t i4 = ((int64_t)local * 64 + lane) * 4;
        acc[group][lane] = axis::split_sum_part4(k.partial, i4, k.len, (int32_t)k.count, k.stride, group);
        __syncthreads();
        if (group == 0 && i4 < k.len) {
            axis::split_sum_store4(k.out_a, i4, acc[0][lane], acc[1][lane], acc[2][lane], acc[3][lane], k.bias, k.n,
                                   k.d, k.alpha, k.beta, k.perm_c, k.perm_taps);
        }
    } else if (k.kind == 0) {
        const int lane = threadIdx.x & 63, group = threadIdx.x >> 6;
        const int64_t i = (int64_t)local * 64 + lane;
        lds[group][lane] = axis::split_sum_part(k.partial, i, k.len, (int32_t)k.count, k.stride, group);
        __syncthreads();
        if (group == 0 && i < k.len)
            axis::split_sum_store(k.out_a, i, lds[0][lane], lds[1][lane], lds[2][lane], lds[3][lane], k.bias, k.n,
                                  k.d, k.alpha, k.beta, k.perm_c, k.perm_taps);
    } else {
        const int col = threadIdx.x & 15, range = threadIdx.x >> 4;
        const int64_t e = (int64_t)local * 16 + col;
        lds[range][col] = axis::column_block_part(k.partial, k.count, k.len, k.stride, e, range);
        __syncthreads();
        if (range == 0 && e < k.len) axis::column_block_store(&lds[0][col], e, k.split, k.out_a, k.out_b);
    }
}

bool overlaps(const axis::FinishTask &t, const char *lo, const char *hi) {
    auto hit = [&](const float *out, int64_t floats) {
        const char *a = reinterpret_cast<const char *>(out);
        return out && a < hi && lo < a + floats * (int64_t)sizeof(float);
    };
    if (t.kind != 1) return hit(t.out_a, t.len);
    const int64_t below = std::min(t.split, t.len);
    return hit(t.out_a, below) || hit(t.out_b, t.len - below);
}

}  // namespace

namespace axis {

int flush_finish(axis_device device) {
    if (device->deferred.empty()) return AXIS_OK;
    FinishBatch b{};
    int64_t blocks = 0;
    bool products = false;
    for (size_t i = 0; i < device->deferred.size(); ++i) {
        b.task[i] = device->deferred[i];
        blocks += b.task[i].blocks;
        products = products || b.task[i].kind != 1;
    }
    b.count = (int32_t)device->deferred.size();
    int status = AXIS_OK;
    {
        // The split sums finish products of the "gemm" timing family (no work of their own).
        TimedLaunch timed(products ? device : nullptr, "gemm", 0.0);
        finish_batch_kernel<<<(unsigned)blocks, 256, 0, device->stream>>>(b);
        status = launch_status("finish_batch_kernel");
    }
    // Stream order: later launches that reuse these blocks run after the batch has read them.
    for (void *p : device->deferred_blocks) release(device, p);
    device->deferred.clear();
    device->deferred_blocks.clear();
    device->deferred_bytes = 0;
    return status;
}

int finish_overlapping(axis_device device, std::initializer_list<Span> spans) {
    for (const Span &sp : spans) {
        if (!sp.ptr || sp.bytes <= 0) continue;
        const char *lo = static_cast<const char *>(sp.ptr);
        for (const FinishTask &t : device->deferred)
            if (overlaps(t, lo, lo + sp.bytes)) return flush_finish(device);
    }
    return AXIS_OK;
}

int defer_finish(axis_device device, const FinishTask &task, Scratch &held) {
    if (task.blocks < 1 || (int64_t)task.blocks > (int64_t)INT32_MAX / 2)
        return fail(AXIS_ERROR_INVALID, "finishing sum too large to defer");
    int64_t blocks = task.blocks;
    for (const FinishTask &t : device->deferred) blocks += t.blocks;
    if (device->deferred.size() == (size_t)kMaxFinish || blocks > (int64_t)INT32_MAX / 2)
        if (int st = flush_finish(device)) return st;
    device->deferred.push_back(task);
    if (held.ptr) {
        auto it = device->live.find(held.ptr);
        device->deferred_bytes += it == device->live.end() ? 0 : it->second;
        device->deferred_blocks.push_back(held.take());
    }
    if (device->deferred_bytes > kMaxDeferredBytes) return flush_finish(device);
    return AXIS_OK;
}

}  // namespace axis

extern "C" {

int axis_finish_defer(axis_device device, int enabled) {
    AXIS_ENTER(device);
    if (!enabled) {
        device->deferring = false;
        return axis::flush_finish(device);
    }
    device->deferring = true;
    return AXIS_OK;
}

int axis_finish_flush(axis_device device) {
    AXIS_ENTER(device);
    return axis::flush_finish(device);
}

int axis_finish_pending(axis_device device, int64_t *tasks) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(tasks, "null output");
    *tasks = (int64_t)device->deferred.size();
    return AXIS_OK;
}

int axis_finish_before_read(axis_device device, const void *ptr, size_t bytes) {
    AXIS_ENTER(device);
    if (device->deferred.empty() || !ptr || bytes == 0) return AXIS_OK;
    const char *lo = static_cast<const char *>(ptr);
    for (const axis::FinishTask &t : device->deferred)
        if (overlaps(t, lo, lo + bytes)) return axis::flush_finish(device);
    return AXIS_OK;
}

}  // extern "C"
