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

}  // namespace axis
