// Second stage of the reference's chunked column sum (Device::grouped over the align reverse
// plan, backend.rs:1089-1125 with chunked_offsets :37-50): out[c] = scale * (((0 + p0) + p1) + ...)
// over the chunk partials p_q = partial[q][c], in chunk order.
#pragma once

#include "common.hpp"

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
// the 16 range sums are added in range order.  Used for per-block partials of this library's own
// fused kernels (not a reference summation order).  One block per 64 columns (a lane per column,
// so every row read is coalesced); columns below `split` go to out_a[e], the rest to
// out_b[e - split] (skipped when out_b is null).
__global__ static void __launch_bounds__(1024) column_block_sum_kernel(const float *__restrict__ partial,
                                                                       int64_t rows, int64_t width, int64_t pitch,
                                                                       int64_t split, float *__restrict__ out_a,
                                                                       float *__restrict__ out_b) {
    __shared__ float range_sum[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    const int64_t span = (rows + 15) / 16;
    const int64_t r0 = wave * span;
    const int64_t r1 = r0 + span < rows ? r0 + span : rows;
    float s = 0.0f;
    if (e < width) {
        constexpr int kBatch = 64;  // loads in flight per lane: the range takes few round trips
        int64_t r = r0;
        for (; r + kBatch <= r1; r += kBatch) {
            float v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) v[u] = partial[(r + u) * pitch + e];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) s = s + v[u];
        }
        for (; r < r1; ++r) s = s + partial[r * pitch + e];
    }
    range_sum[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && e < width) {
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; ++w) total = total + range_sum[w][lane];
        if (e < split)
            out_a[e] = total;
        else if (out_b)
            out_b[e - split] = total;
    }
}

inline int column_block_sum(hipStream_t stream, const float *partial, int64_t rows, int64_t width, int64_t pitch,
                            int64_t split, float *out_a, float *out_b) {
    column_block_sum_kernel<<<(unsigned)((width + 63) / 64), 1024, 0, stream>>>(partial, rows, width, pitch, split,
                                                                              out_a, out_b);
    return launch_status("column_block_sum_kernel");
}

}  // namespace axis
