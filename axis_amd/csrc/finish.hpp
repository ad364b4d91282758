// Finishing sums of this library's products and fused scatters, shared by their own kernels
// (split_sum_kernel in gemm.hip, column_block_sum_kernel in column_sum.hpp) and by the batched
// launch that runs deferred ones (finish.hip): one device routine per sum, so a sum gives the
// same bits whichever kernel runs it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace axis {

// + bias[col], then beta * d + alpha * v.  Each product and the sum round separately, as the
// separate scale / scale / add operations they replace.
__device__ __forceinline__ float finish_value(const float *bias, const float *d, float alpha, float beta,
                                              float v, int64_t idx, int64_t col) {
#pragma clang fp contract(off)
    if (bias) v = v + bias[col];
    if (d) {
        const float t1 = beta * d[idx];
        const float t2 = alpha * v;
        v = t1 + t2;
    }
    return v;
}

// One pending sum.  kind 0: out_a[i] = finish(sum over `count` slices partial[k * stride + i]) for
// i < len (slice association of split_sum_part below), written at the permuted position when
// perm_c is set; kind 2: the same, four outputs per lane (split_sum_part4).  kind 1: column e < len of partial[count][pitch = stride] summed over its rows
// (association of column_block_part below), to out_a[e] below `split`, else out_b[e - split].
struct FinishTask {
    const float *partial;
    float *out_a;
    float *out_b;
    const float *bias;
    const float *d;
    int64_t len;
    int64_t count;
    int64_t stride;
    int64_t split;
    int64_t n;
    float alpha, beta;
    int32_t perm_c, perm_taps;
    int32_t kind;
    int32_t blocks;  // blocks of the batched launch: 64 outputs (kind 0), 16 columns (kind 1), 256 outputs (kind 2)
};

// Split sums: lane group g (of 4) adds slices g, g + 4, g + 8, ... in order; the four group sums
// are then added in group order -- a fixed association for a given slice count.  Up to eight of a
// lane's slice values are loaded before the first of them is added (one memory round trip per
// eight slices instead of one per slice); the adds keep slice order.
__device__ __forceinline__ float split_sum_part(const float *__restrict__ partial, int64_t i, int64_t len,
                                                int32_t splits, int64_t split_stride, int group) {
    constexpr int kAhead = 8;
    float s = 0.f;
    if (i < len)
        for (int32_t k0 = group; k0 < splits; k0 += 4 * kAhead) {
            float v[kAhead];
#pragma unroll
            for (int u = 0; u < kAhead; ++u)
                v[u] = k0 + 4 * u < splits ? partial[(int64_t)(k0 + 4 * u) * split_stride + i] : 0.f;
#pragma unroll
            for (int u = 0; u < kAhead; ++u)
                if (k0 + 4 * u < splits) s += v[u];
        }
    return s;
}

typedef float finish_floatx4 __attribute__((ext_vector_type(4)));

// The same sums for four consecutive outputs i4 .. i4 + 3 per lane (len % 4 == 0 and 16-byte
// aligned slices): one 16-byte load per slice, each output's adds in the same order.
__device__ __forceinline__ finish_floatx4 split_sum_part4(const float *__restrict__ partial, int64_t i4, int64_t len,
                                                          int32_t splits, int64_t split_stride, int group) {
    constexpr int kAhead = 8;
    finish_floatx4 s = {0.f, 0.f, 0.f, 0.f};
    if (i4 < len)
        for (int32_t k0 = group; k0 < splits; k0 += 4 * kAhead) {
            finish_floatx4 v[kAhead];
#pragma unroll
            for (int u = 0; u < kAhead; ++u)
                v[u] = k0 + 4 * u < splits
                           ? *reinterpret_cast<const finish_floatx4 *>(partial + (int64_t)(k0 + 4 * u) * split_stride + i4)
                           : finish_floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < kAhead; ++u)
                if (k0 + 4 * u < splits) s += v[u];
        }
    return s;
}

__device__ __forceinline__ void split_sum_store(float *__restrict__ out, int64_t i, float g0, float g1, float g2,
                                                float g3, const float *__restrict__ bias, int64_t n,
                                                const float *__restrict__ d, float alpha, float beta,
                                                int32_t perm_c, int32_t perm_taps) {
    const float total = ((g0 + g1) + g2) + g3;
    int64_t at = i;
    if (perm_c) {  // row (pos, c) -> c * taps + pos
        const int64_t row = i / n, col = i - row * n;
        at = ((row % perm_c) * perm_taps + row / perm_c) * n + col;
    }
    out[at] = finish_value(bias, d, alpha, beta, total, i, i % n);
}

// split_sum_store for outputs i4 .. i4 + 3 (group sums g0..g3 per output): one 16-byte store when
// the outputs are not permuted.
__device__ __forceinline__ void split_sum_store4(float *__restrict__ out, int64_t i4, finish_floatx4 g0,
                                                 finish_floatx4 g1, finish_floatx4 g2, finish_floatx4 g3,
                                                 const float *__restrict__ bias, int64_t n,
                                                 const float *__restrict__ d, float alpha, float beta,
                                                 int32_t perm_c, int32_t perm_taps) {
    if (perm_c) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            split_sum_store(out, i4 + e, g0[e], g1[e], g2[e], g3[e], bias, n, d, alpha, beta, perm_c, perm_taps);
        return;
    }
    finish_floatx4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        v[e] = finish_value(bias, d, alpha, beta, ((g0[e] + g1[e]) + g2[e]) + g3[e], i4 + e, (i4 + e) % n);
    *reinterpret_cast<finish_floatx4 *>(out + i4) = v;
}

// Column block sums: 16 consecutive row ranges of ceil(rows / 16) (range w = `wave`), each summed in
// row order; the 16 range sums are then added in range order.
__device__ __forceinline__ float column_block_part(const float *__restrict__ partial, int64_t rows, int64_t width,
                                                   int64_t pitch, int64_t e, int wave) {
    const int64_t span = (rows + 15) / 16;
    const int64_t r0 = wave * span;
    const int64_t r1 = r0 + span < rows ? r0 + span : rows;
    float s = 0.0f;
    if (e < width) {
        // 64 loads in flight per lane, the rest of the range 16 at a time: few round trips
        constexpr int kBatch = 64, kTail = 16;
        int64_t r = r0;
        for (; r + kBatch <= r1; r += kBatch) {
            float v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) v[u] = partial[(r + u) * pitch + e];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) s = s + v[u];
        }
        for (; r < r1; r += kTail) {
            float v[kTail];
#pragma unroll
            for (int u = 0; u < kTail; ++u) v[u] = r + u < r1 ? partial[(r + u) * pitch + e] : 0.0f;
#pragma unroll
            for (int u = 0; u < kTail; ++u)
                if (r + u < r1) s = s + v[u];
        }
    }
    return s;
}

// range_sum: the 16 range sums of this lane's column, range w at range_sum[w * 64].
__device__ __forceinline__ void column_block_store(const float *range_sum, int64_t e, int64_t split,
                                                   float *__restrict__ out_a, float *__restrict__ out_b) {
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; ++w) total = total + range_sum[w * 64];
    if (e < split)
        out_a[e] = total;
    else if (out_b)
        out_b[e - split] = total;
}

}  // namespace axis
