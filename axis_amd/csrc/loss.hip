// Softmax and categorical cross-entropy (runtime/backend.rs:829-932, kernels :2424-2543).
// One 256-lane block per row; row maxima and sums are wavefront shuffles plus a 4-entry LDS
// combine.  The reference reduces with a cuTile tile reduction (softmax) or a sequential loop (CE
// forward), neither of which fixes a tree order a GPU can reproduce, so these agree with it to
// fp32 tolerance; the CE gradient is exact given the probabilities.
#include <cfloat>

#include <cmath>

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

// probability (optional) and loss (optional) of one row.
__global__ void __launch_bounds__(kBlock) softmax_ce_kernel(const float *__restrict__ logits,
                                                            const float *__restrict__ targets,
                                                            float *__restrict__ probability,
                                                            float *__restrict__ loss, int64_t width) {
    __shared__ float scratch[kWaves];
    const float *z = logits + (int64_t)blockIdx.x * width;
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
    if (int s = check_rows(a, out, rows, width)) return s;
    softmax_ce_kernel<<<(unsigned)rows, kBlock, 0, device->stream>>>(a, nullptr, out, nullptr, width);
    return axis::launch_status("softmax_ce_kernel");
}

int axis_softmax_backward(axis_device device, const float *gradient, const float *probability,
                          float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    if (int s = check_rows(gradient, out, rows, width)) return s;
    AXIS_REQUIRE(probability, "null probability");
    softmax_backward_kernel<<<(unsigned)rows, kBlock, 0, device->stream>>>(gradient, probability, out,
                                                                            width);
    return axis::launch_status("softmax_backward_kernel");
}

int axis_categorical_cross_entropy(axis_device device, const float *logits, const float *targets,
                                   float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    if (int s = check_rows(logits, out, rows, width)) return s;
    AXIS_REQUIRE(targets, "null targets");
    softmax_ce_kernel<<<(unsigned)rows, kBlock, 0, device->stream>>>(logits, targets, nullptr, out,
                                                                      width);
    return axis::launch_status("softmax_ce_kernel");
}

int axis_categorical_cross_entropy_backward(axis_device device, const float *gradient,
                                            const float *probability, const float *targets,
                                            float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    if (int s = check_rows(gradient, out, rows, width)) return s;
    AXIS_REQUIRE(probability && targets, "null probability/targets");
    ce_backward_kernel<<<axis::blocks_for(rows * width, kBlock, 16384), kBlock, 0, device->stream>>>(
        gradient, probability, targets, out, rows, width, 0.0f);
    return axis::launch_status("ce_backward_kernel");
}

int axis_categorical_cross_entropy_backward_mean(axis_device device, const float *gradient, float factor,
                                                 const float *probability, const float *targets, float *out,
                                                 int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    if (int s = check_rows(gradient, out, rows, width)) return s;
    AXIS_REQUIRE(probability && targets, "null probability/targets");
    AXIS_REQUIRE(factor != 0.0f && std::isfinite(factor), "mean factor must be finite and nonzero");
    ce_backward_kernel<<<axis::blocks_for(rows * width, kBlock, 16384), kBlock, 0, device->stream>>>(
        gradient, probability, targets, out, rows, width, factor);
    return axis::launch_status("ce_backward_kernel");
}

int axis_softmax_cross_entropy(axis_device device, const float *logits, const float *targets,
                               float *probability, float *loss, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    if (int s = check_rows(logits, probability, rows, width)) return s;
    AXIS_REQUIRE(targets && loss, "null targets/loss");
    softmax_ce_kernel<<<(unsigned)rows, kBlock, 0, device->stream>>>(logits, targets, probability,
                                                                      loss, width);
    return axis::launch_status("softmax_ce_kernel");
}

}  // extern "C"
