// Second stage of the reference's chunked column sum (Device::grouped over the align reverse
// plan, backend.rs:1089-1125 with chunked_offsets :37-50): out[c] = scale * (((0 + p0) + p1) + ...)
// over the chunk partials p_q = partial[q][c], in chunk order.
#pragma once

#include "common.hpp"
#include "finish.hpp"

namespace axis {

typedef float floatx4_cs __attribute__((ext_vector_type(4)));
constexpr int kCombineStage = 4096;

// One block per column.  The block stages the column's chunk partials through LDS (parallel,
// coalesced across chunks of the same column block) and one lane adds them in chunk order.
__global__ static void __launch_bounds__(256) column_combine_kernel(const float *__restrict__ partial,
                                                                    int64_t chunks, int64_t width,
                                                                    float scale, float *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) float staged[kCombineStage];
    const int64_t c = blockIdx.x;
    float sum = 0.0f;
    for (int64_t base = 0; base < chunks; base += kCombineStage) {
        const int n = (int)(chunks - base < kCombineStage ? chunks - base : kCombineStage);
        for (int i = threadIdx.x; i < n; i += 256) staged[i] = partial[(base + i) * width + c];
        __syncthreads();
        if (threadIdx.x == 0) {
            const floatx4_cs *v = reinterpret_cast<const floatx4_cs *>(staged);
            int i = 0;
            for (; i + 4 <= n; i += 4) {
                const floatx4_cs q = v[i / 4];
                sum = sum + q[0];
                sum = sum + q[1];
                sum = sum + q[2];
                sum = sum + q[3];
            }
            for (; i < n; ++i) sum = sum + staged[i];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[c] = sum * scale;
}

// Sum over the rows of partial[rows][width] (row pitch `pitch`) in a fixed association: the 16
// waves of a block take consecutive row ranges of ceil(rows / 16), each summed in row order, and
// the 16 range sums are added in range order (column_block_part / column_block_store).  Used for
// per-block partials of this library's own fused kernels (not a reference summation order).  One
// block per 64 columns (a lane per column, so every row read is coalesced); columns below `split`
// go to out_a[e], the rest to out_b[e - split] (skipped when out_b is null).
__global__ static void __launch_bounds__(1024) column_block_sum_kernel(const float *__restrict__ partial,
                                                                       int64_t rows, int64_t width, int64_t pitch,
                                                                       int64_t split, float *__restrict__ out_a,
                                                                       float *__restrict__ out_b) {
    __shared__ float range_sum[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    range_sum[wave][lane] = column_block_part(partial, rows, width, pitch, e, wave);
    __syncthreads();
    if (wave == 0 && e < width) column_block_store(&range_sum[0][lane], e, split, out_a, out_b);
}

// The column block sum of `partial` (held by `owner`), launched now, or recorded with `owner`'s
// block held when the handle defers finishing sums (the outputs are then final gradients).
inline int column_block_sum(axis_device device, Scratch &owner, int64_t rows, int64_t width, int64_t pitch,
                            int64_t split, float *out_a, float *out_b) {
    const float *partial = owner.as<float>();
    if (device->deferring) {
        FinishTask t{};
        t.partial = partial;
        t.out_a = out_a;
        t.out_b = out_b;
        t.len = width;
        t.count = rows;
        t.stride = pitch;
        t.split = split;
        t.kind = 1;
        t.blocks = (int32_t)((width + 15) / 16);
        return defer_finish(device, t, owner);
    }
    column_block_sum_kernel<<<(unsigned)((width + 63) / 64), 1024, 0, device->stream>>>(partial, rows, width, pitch,
                                                                                      split, out_a, out_b);
    return launch_status("column_block_sum_kernel");
}

}  // namespace axis
