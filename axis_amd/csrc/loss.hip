// Softmax and categorical cross-entropy (runtime/backend.rs:829-932, kernels :2424-2543).
// One 256-lane block per row; row maxima and sums are wavefront shuffles plus a 4-entry LDS
// combine.  The reference reduces with a cuTile tile reduction (softmax) or a sequential loop (CE
// forward), neither of which fixes a tree order a GPU can reproduce, so these agree with it to
// fp32 tolerance; the CE gradient is exact given the probabilities.
#include <algorithm>
#include <cfloat>

#include <cmath>

#include "column_sum.hpp"
#include "common.hpp"

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ float block_max(float v, float *scratch) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < kWaves; ++w) r = fmaxf(r, scratch[w]);
    return r;
}
__device__ float block_sum(float v, float *scratch) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.0f;
    for (int w = 0; w < kWaves; ++w) r += scratch[w];
    return r;
}

// probability (optional) and loss (optional) of one row.  CACHE > 0 (width <= CACHE * kBlock): a
// lane's logits, targets and exponentials stay in registers, so the row is read from memory once
// instead of once per pass; each lane still visits its elements j, j + kBlock, ... in order, so
// every sum is the same as the uncached loops'.
template <int CACHE>
__global__ void __launch_bounds__(kBlock) softmax_ce_kernel(const float *__restrict__ logits,
                                                            const float *__restrict__ targets,
                                                            float *__restrict__ probability,
                                                            float *__restrict__ loss, int64_t width) {
    __shared__ float scratch[kWaves];
    const float *z = logits + (int64_t)blockIdx.x * width;
    if constexpr (CACHE > 0) {
        float zc[CACHE], yc[CACHE];
#pragma unroll
        for (int u = 0; u < CACHE; ++u) {
            const int64_t j = threadIdx.x + (int64_t)u * kBlock;
            zc[u] = j < width ? z[j] : -INFINITY;
            yc[u] = loss && j < width ? targets[(int64_t)blockIdx.x * width + j] : 0.0f;
        }
        float m = -INFINITY;
#pragma unroll
        for (int u = 0; u < CACHE; ++u)
            if (threadIdx.x + (int64_t)u * kBlock < width) m = fmaxf(m, zc[u]);
        m = block_max(m, scratch);
        float s = 0.0f, e[CACHE];
#pragma unroll
        for (int u = 0; u < CACHE; ++u) {
            e[u] = 0.0f;
            if (threadIdx.x + (int64_t)u * kBlock < width) {
                e[u] = expf(zc[u] - m);
                s += e[u];
            }
        }
        s = block_sum(s, scratch);
        if (probability) {
            float *p = probability + (int64_t)blockIdx.x * width;
#pragma unroll
            for (int u = 0; u < CACHE; ++u) {
                const int64_t j = threadIdx.x + (int64_t)u * kBlock;
                if (j < width) p[j] = e[u] / s;
            }
        }
        if (loss) {
            const float log_normalizer = m + logf(s);
            float l = 0.0f;
#pragma unroll
            for (int u = 0; u < CACHE; ++u)
                if (threadIdx.x + (int64_t)u * kBlock < width) l += yc[u] * (log_normalizer - zc[u]);
            l = block_sum(l, scratch);
            if (threadIdx.x == 0) loss[blockIdx.x] = l;
        }
        return;
    }
    float m = -INFINITY;
    for (int64_t j = threadIdx.x; j < width; j += kBlock) m = fmaxf(m, z[j]);
    m = block_max(m, scratch);
    float s = 0.0f;
    for (int64_t j = threadIdx.x; j < width; j += kBlock) s += expf(z[j] - m);
    s = block_sum(s, scratch);
    if (probability) {
        float *p = probability + (int64_t)blockIdx.x * width;
        for (int64_t j = threadIdx.x; j < width; j += kBlock) p[j] = expf(z[j] - m) / s;
    }
    if (loss) {
        const float *y = targets + (int64_t)blockIdx.x * width;
        const float log_normalizer = m + logf(s);
        float l = 0.0f;
        for (int64_t j = threadIdx.x; j < width; j += kBlock) l += y[j] * (log_normalizer - z[j]);
        l = block_sum(l, scratch);
        if (threadIdx.x == 0) loss[blockIdx.x] = l;
    }
}

int launch_softmax_ce(hipStream_t stream, const float *logits, const float *targets, float *probability,
                      float *loss, int64_t rows, int64_t width) {
    if (width <= 4 * kBlock)
        softmax_ce_kernel<4><<<(unsigned)rows, kBlock, 0, stream>>>(logits, targets, probability, loss, width);
    else if (width <= 16 * kBlock)
        softmax_ce_kernel<16><<<(unsigned)rows, kBlock, 0, stream>>>(logits, targets, probability, loss, width);
    else
        softmax_ce_kernel<0><<<(unsigned)rows, kBlock, 0, stream>>>(logits, targets, probability, loss, width);
    return axis::launch_status("softmax_ce_kernel");
}

__global__ void __launch_bounds__(kBlock) softmax_backward_kernel(const float *__restrict__ gradient,
                                                                  const float *__restrict__ probability,
                                                                  float *__restrict__ out,
                                                                  int64_t width) {
    __shared__ float scratch[kWaves];
    const int64_t base = (int64_t)blockIdx.x * width;
    float d = 0.0f;
    for (int64_t j = threadIdx.x; j < width; j += kBlock) d += gradient[base + j] * probability[base + j];
    d = block_sum(d, scratch);
    for (int64_t j = threadIdx.x; j < width; j += kBlock)
        out[base + j] = probability[base + j] * (gradient[base + j] - d);
}

// mean_factor != 0: the row gradient is gradient[0] * mean_factor for every row -- the value the
// backward of a mean over the rows (a broadcast times the factor) would have stored.
__global__ void __launch_bounds__(kBlock) ce_backward_kernel(const float *__restrict__ gradient,
                                                             const float *__restrict__ probability,
                                                             const float *__restrict__ targets,
                                                             float *__restrict__ out, int64_t rows,
                                                             int64_t width, float mean_factor) {
    const int64_t total = rows * width;
    const float g_all = mean_factor != 0.0f ? gradient[0] * mean_factor : 0.0f;
    for (int64_t p = (int64_t)blockIdx.x * kBlock + threadIdx.x; p < total;
         p += (int64_t)gridDim.x * kBlock)
        out[p] = (mean_factor != 0.0f ? g_all : gradient[p / width]) * (probability[p] - targets[p]);
}

// The mean cross-entropy backward with the bias gradient of the logits' producer: block (16
// columns, 512-row chunk) computes its chunk's gradient values (as ce_backward_kernel), writes them
// and stages them in LDS; one lane per column then adds the chunk's rows in row order -- the
// column sums of axis_bias_gradient (chunk partials combined in chunk order when rows > 512).
constexpr int kBiasCols = 8;
constexpr int kBiasChunk = axis::kGroupedChunk;
__global__ void __launch_bounds__(kBlock) ce_backward_mean_bias_kernel(
    const float *__restrict__ gradient, float mean_factor, const float *__restrict__ probability,
    const float *__restrict__ targets, float *__restrict__ out, float *__restrict__ partial,
    float *__restrict__ d_bias, int64_t rows, int64_t width, int64_t chunks) {
    constexpr int kPasses = kBiasChunk * kBiasCols / kBlock;
    constexpr int kRowsPerPass = kBlock / kBiasCols;
    __shared__ float staged[kBiasChunk][kBiasCols + 1];
    const int tid = threadIdx.x;
    const int cl = tid % kBiasCols;
    const int64_t c = (int64_t)blockIdx.x * kBiasCols + cl;
    const float g = gradient[0] * mean_factor;
    for (int64_t q = blockIdx.y; q < chunks; q += gridDim.y) {
        const int64_t r0 = q * kBiasChunk;
        const int n_rows = (int)(r0 + kBiasChunk < rows ? kBiasChunk : rows - r0);
        float v[kPasses];
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
            const int r = u * kRowsPerPass + tid / kBiasCols;
            v[u] = 0.0f;
            if (r < n_rows && c < width) {
                const int64_t p = (r0 + r) * width + c;
                v[u] = g * (probability[p] - targets[p]);
                out[p] = v[u];
            }
        }
        __syncthreads();  // the previous chunk's sums have read the stage
#pragma unroll
        for (int u = 0; u < kPasses; ++u) staged[u * kRowsPerPass + tid / kBiasCols][cl] = v[u];
        __syncthreads();
        if (tid < kBiasCols && c < width) {
            float sum = 0.0f;
            for (int r = 0; r < n_rows; ++r) sum = sum + staged[r][tid];
            if (chunks == 1)
                d_bias[c] = 0.0f + sum;
            else
                partial[q * width + c] = sum;
        }
    }
}

int check_rows(const void *a, const void *out, int64_t rows, int64_t width) {
    AXIS_REQUIRE(a && out, "null softmax/cross-entropy buffer");
    AXIS_REQUIRE(rows >= 1 && width >= 1, "softmax/cross-entropy extents must be positive");
    AXIS_REQUIRE(rows <= INT32_MAX, "too many rows for one launch");
    return AXIS_OK;
}

}  // namespace

extern "C" {

int axis_softmax(axis_device device, const float *a, float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * rows * width}, {out, 4 * rows * width});
    if (int s = check_rows(a, out, rows, width)) return s;
    return launch_softmax_ce(device->stream, a, nullptr, out, nullptr, rows, width);
}

int axis_softmax_backward(axis_device device, const float *gradient, const float *probability,
                          float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * rows * width}, {probability, 4 * rows * width}, {out, 4 * rows * width});
    if (int s = check_rows(gradient, out, rows, width)) return s;
    AXIS_REQUIRE(probability, "null probability");
    softmax_backward_kernel<<<(unsigned)rows, kBlock, 0, device->stream>>>(gradient, probability, out,
                                                                            width);
    return axis::launch_status("softmax_backward_kernel");
}

int axis_categorical_cross_entropy(axis_device device, const float *logits, const float *targets,
                                   float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {logits, 4 * rows * width}, {targets, 4 * rows * width}, {out, 4 * rows});
    if (int s = check_rows(logits, out, rows, width)) return s;
    AXIS_REQUIRE(targets, "null targets");
    return launch_softmax_ce(device->stream, logits, targets, nullptr, out, rows, width);
}

int axis_categorical_cross_entropy_backward(axis_device device, const float *gradient,
                                            const float *probability, const float *targets,
                                            float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * rows}, {probability, 4 * rows * width}, {targets, 4 * rows * width}, {out, 4 * rows * width});
    if (int s = check_rows(gradient, out, rows, width)) return s;
    AXIS_REQUIRE(probability && targets, "null probability/targets");
    ce_backward_kernel<<<axis::blocks_for(rows * width, kBlock, 16384), kBlock, 0, device->stream>>>(
        gradient, probability, targets, out, rows, width, 0.0f);
    return axis::launch_status("ce_backward_kernel");
}

int axis_categorical_cross_entropy_backward_mean(axis_device device, const float *gradient, float factor,
                                                 const float *probability, const float *targets, float *out,
                                                 float *d_bias, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4}, {probability, 4 * rows * width}, {targets, 4 * rows * width}, {out, 4 * rows * width}, {d_bias, 4 * width});
    if (int s = check_rows(gradient, out, rows, width)) return s;
    AXIS_REQUIRE(probability && targets, "null probability/targets");
    AXIS_REQUIRE(factor != 0.0f && std::isfinite(factor), "mean factor must be finite and nonzero");
    if (!d_bias) {
        ce_backward_kernel<<<axis::blocks_for(rows * width, kBlock, 16384), kBlock, 0, device->stream>>>(
            gradient, probability, targets, out, rows, width, factor);
        return axis::launch_status("ce_backward_kernel");
    }
    const int64_t chunks = (rows + kBiasChunk - 1) / kBiasChunk;
    axis::Scratch partial;
    if (chunks > 1)
        if (int s = partial.get(device, sizeof(float) * (size_t)(chunks * width))) return s;
    const dim3 grid((unsigned)((width + kBiasCols - 1) / kBiasCols), (unsigned)std::min<int64_t>(chunks, 65535));
    ce_backward_mean_bias_kernel<<<grid, kBlock, 0, device->stream>>>(gradient, factor, probability, targets, out,
                                                                    partial.as<float>(), d_bias, rows, width,
                                                                    chunks);
    if (int s = axis::launch_status("ce_backward_mean_bias_kernel")) return s;
    if (chunks == 1) return AXIS_OK;
    axis::column_combine_kernel<<<(unsigned)width, 256, 0, device->stream>>>(partial.as<float>(), chunks, width,
                                                                           1.0f, d_bias);
    return axis::launch_status("column_combine_kernel");
}

int axis_softmax_cross_entropy(axis_device device, const float *logits, const float *targets,
                               float *probability, float *loss, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {logits, 4 * rows * width}, {targets, 4 * rows * width}, {probability, 4 * rows * width}, {loss, 4 * rows});
    if (int s = check_rows(logits, probability, rows, width)) return s;
    AXIS_REQUIRE(targets && loss, "null targets/loss");
    return launch_softmax_ce(device->stream, logits, targets, probability, loss, rows, width);
}

}  // extern "C"
