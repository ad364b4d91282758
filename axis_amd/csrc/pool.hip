// Max pooling over channel-innermost activations: the forward of the reference's
// -min(-unfold(x, fill=-inf)) (model/convolution.rs:1357-1370, Tensor::min tensor.rs:2880-2946,
// grouped_minimum backend.rs:3019-3056) in one pass, emitting the window-local winner as a byte,
// and its backward (Rule::Minimum gather + mask, then unfold's col2im, tensor.rs:5679-5683 and
// backend.rs:1795-1889).
//
// Lanes run along the channel axis (4 channels per lane when the channel extent allows), so
// every load and store is unit-stride across the wave; index decode is 32-bit multiply-high.
// Non-overlapping windows (stride == kernel, no padding, exact tiling) take a scatter-form
// backward -- one lane per output writes its window -- which equals the gather sum exactly: each
// input receives exactly one term, written as 0.0f + g like the sum the reference starts at +0.0.
#include <algorithm>
#include <cfloat>

#include "column_sum.hpp"
#include "common.hpp"
#include "fastdiv.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr uint8_t kNoWinner = 255;

struct PoolArgs {
    int32_t channels, height, width, out_h, out_w;
    int32_t ky, kx, sy, sx, py, px;
    uint32_t total;          // lanes in the launch (vectors of VEC channels)
    FastDiv cvec, ow, oh;    // decode of an output-vector index
    FastDiv iw, ih;          // decode of an input-vector index
    FastDiv sy_div, sx_div;
    // Pooled gradient given as [outer, channels] times g_factor, the same at every pooled position
    // (the backward of a mean over the pooled height and width); otherwise one value per position.
    bool g_broadcast;
    float g_factor;
};

template <int VEC>
struct Vec {
    float v[VEC];
};

template <int VEC>
__device__ __forceinline__ void load_vec(const float *p, float (&v)[VEC]) {
    if constexpr (VEC == 4) {
        const floatx4 x = *reinterpret_cast<const floatx4 *>(p);
        v[0] = x[0], v[1] = x[1], v[2] = x[2], v[3] = x[3];
    } else {
        v[0] = p[0];
    }
}

// The pooled gradient of output vector t (batch o, channel c): gradient[t], or, broadcast,
// gradient[o][c] * g_factor -- the value the mean's backward (a broadcast times the factor) stores.
template <int VEC>
__device__ __forceinline__ void load_gradient(const float *gradient, uint32_t t, uint32_t o, int32_t c,
                                              const PoolArgs &a, float (&g)[VEC]) {
    if (a.g_broadcast) {
        load_vec<VEC>(gradient + (int64_t)o * a.channels + c, g);
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = g[e] * a.g_factor;
    } else {
        load_vec<VEC>(gradient + (int64_t)t * VEC, g);
    }
}

template <int VEC>
__device__ __forceinline__ void store_vec(float *p, const float (&v)[VEC]) {
    if constexpr (VEC == 4) {
        floatx4 x = {v[0], v[1], v[2], v[3]};
        *reinterpret_cast<floatx4 *>(p) = x;
    } else {
        p[0] = v[0];
    }
}

template <int VEC>
__global__ void __launch_bounds__(256) max_pool2d_kernel(const float *__restrict__ in,
                                                         float *__restrict__ out,
                                                         uint8_t *__restrict__ argmax, PoolArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= a.total) return;
    const uint32_t cv = a.cvec.mod(t);
    uint32_t rest = a.cvec.div(t);
    const int32_t ox = (int32_t)a.ow.mod(rest);
    rest = a.ow.div(rest);
    const int32_t oy = (int32_t)a.oh.mod(rest);
    const uint32_t o = a.oh.div(rest);
    const int32_t c = (int32_t)cv * VEC;
    const float *base = in + (int64_t)o * a.height * a.width * a.channels + c;
    float best[VEC];
    int winner[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) best[e] = -INFINITY, winner[e] = kNoWinner;
    for (int32_t ky = 0; ky < a.ky; ++ky) {
        const int32_t iy = oy * a.sy + ky - a.py;
        if (iy < 0 || iy >= a.height) continue;
        for (int32_t kx = 0; kx < a.kx; ++kx) {
            const int32_t ix = ox * a.sx + kx - a.px;
            if (ix < 0 || ix >= a.width) continue;
            float v[VEC];
            load_vec<VEC>(base + ((int64_t)iy * a.width + ix) * a.channels, v);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                // first strictly greater finite value in window order (ky major, kx minor)
                if (v[e] >= -FLT_MAX && v[e] <= FLT_MAX && v[e] > best[e]) {
                    best[e] = v[e];
                    winner[e] = ky * a.kx + kx;
                }
            }
        }
    }
    float r[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) r[e] = winner[e] == kNoWinner ? __builtin_nanf("") : best[e];
    store_vec<VEC>(out + (int64_t)t * VEC, r);
#pragma unroll
    for (int e = 0; e < VEC; ++e) argmax[(int64_t)t * VEC + e] = (uint8_t)winner[e];
}

// Non-overlapping windows: one lane per output vector writes its whole window.
template <int VEC>
__global__ void __launch_bounds__(256) max_pool2d_backward_tiled_kernel(
    const float *__restrict__ gradient, const uint8_t *__restrict__ argmax, float *__restrict__ out,
    PoolArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= a.total) return;
    const uint32_t cv = a.cvec.mod(t);
    uint32_t rest = a.cvec.div(t);
    const int32_t ox = (int32_t)a.ow.mod(rest);
    rest = a.ow.div(rest);
    const int32_t oy = (int32_t)a.oh.mod(rest);
    const uint32_t o = a.oh.div(rest);
    const int32_t c = (int32_t)cv * VEC;
    float g[VEC];
    int w[VEC];
    load_vec<VEC>(gradient + (int64_t)t * VEC, g);
#pragma unroll
    for (int e = 0; e < VEC; ++e) w[e] = argmax[(int64_t)t * VEC + e];
    float *base = out + (int64_t)o * a.height * a.width * a.channels + c;
    for (int32_t ky = 0; ky < a.ky; ++ky) {
        const int32_t iy = oy * a.ky + ky;
        for (int32_t kx = 0; kx < a.kx; ++kx) {
            const int32_t ix = ox * a.kx + kx;
            const int k = ky * a.kx + kx;
            float r[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) r[e] = w[e] == k ? 0.0f + g[e] : 0.0f;
            store_vec<VEC>(base + ((int64_t)iy * a.width + ix) * a.channels, r);
        }
    }
}

// ReLU -> non-overlapping max pool, backward in one scatter: the winner of each window receives
// 0.0f + g when the pooled value (the ReLU output at the winner) is positive; every other input
// position receives 0 -- the pool's scatter followed by the ReLU mask, element for element.
template <int VEC>
__global__ void __launch_bounds__(256) relu_pool_backward_kernel(
    const float *__restrict__ gradient, const float *__restrict__ pooled,
    const uint8_t *__restrict__ argmax, float *__restrict__ out, PoolArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= a.total) return;
    const uint32_t cv = a.cvec.mod(t);
    uint32_t rest = a.cvec.div(t);
    const int32_t ox = (int32_t)a.ow.mod(rest);
    rest = a.ow.div(rest);
    const int32_t oy = (int32_t)a.oh.mod(rest);
    const uint32_t o = a.oh.div(rest);
    const int32_t c = (int32_t)cv * VEC;
    float g[VEC], y[VEC];
    int w[VEC];
    load_gradient<VEC>(gradient, t, o, c, a, g);
    load_vec<VEC>(pooled + (int64_t)t * VEC, y);
#pragma unroll
    for (int e = 0; e < VEC; ++e) w[e] = y[e] > 0.0f ? (int)argmax[(int64_t)t * VEC + e] : -1;
    float *base = out + (int64_t)o * a.height * a.width * a.channels + c;
    for (int32_t ky = 0; ky < a.ky; ++ky) {
        const int32_t iy = oy * a.ky + ky;
        for (int32_t kx = 0; kx < a.kx; ++kx) {
            const int32_t ix = ox * a.kx + kx;
            const int k = ky * a.kx + kx;
            float r[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) r[e] = w[e] == k ? 0.0f + g[e] : 0.0f;
            store_vec<VEC>(base + ((int64_t)iy * a.width + ix) * a.channels, r);
        }
    }
}

// The same scatter with the bias gradient folded in.  A block walks a contiguous range of pooled
// vectors with stride 256, so a lane keeps one channel vector (256 is a multiple of the vector
// count per pixel) and sums the terms it writes; a fixed-order block reduction leaves one partial
// per block and channel, summed afterwards in a fixed order (axis::column_block_sum).  The
// association differs from the reference's 512-row chunks (fp32 tolerance, not bit equality) but
// is the same on every run.
// BC: the pooled gradient is a mean's broadcast (a.g_broadcast), fixed per instance so the loop
// carries no branch on it.
template <int VEC, bool BC>
__global__ void __launch_bounds__(256) relu_pool_backward_bias_kernel(
    const float *__restrict__ gradient, const float *__restrict__ pooled,
    const uint8_t *__restrict__ argmax, float *__restrict__ out, float *__restrict__ partial,
    uint32_t span, PoolArgs a) {
    a.g_broadcast = BC;
    __shared__ float lane_sum[256][VEC];
    const uint32_t begin = blockIdx.x * span;
    const uint32_t end = begin + span < a.total ? begin + span : a.total;
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
    // Two vectors per lane per pass (t and t + 256): both vectors' loads are in flight before the
    // first stores; the bias terms are still added in t order.
    for (uint32_t t0 = begin + threadIdx.x; t0 < end; t0 += 512u) {
        const int pair = t0 + 256u < end ? 2 : 1;
        float g[2][VEC], y[2][VEC];
        uint32_t wb[2];
        uint32_t o[2];
        int32_t oy[2], ox[2], c[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t t = h < pair ? t0 + 256u * h : t0;  // a missing second vector repeats the first's loads
            const uint32_t cv = a.cvec.mod(t);
            uint32_t rest = a.cvec.div(t);
            ox[h] = (int32_t)a.ow.mod(rest);
            rest = a.ow.div(rest);
            oy[h] = (int32_t)a.oh.mod(rest);
            o[h] = a.oh.div(rest);
            c[h] = (int32_t)cv * VEC;
            load_gradient<VEC>(gradient, t, o[h], c[h], a, g[h]);
            load_vec<VEC>(pooled + (int64_t)t * VEC, y[h]);
            // the vector's winner bytes in one load (4-byte aligned when VEC == 4)
            wb[h] = VEC == 4 ? *reinterpret_cast<const uint32_t *>(argmax + (int64_t)t * VEC) : argmax[t];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (h >= pair) break;
            int w[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                w[e] = y[h][e] > 0.0f ? (int)((wb[h] >> (8 * e)) & 0xffu) : -1;
                acc[e] += (w[e] >= 0 && w[e] < a.ky * a.kx) ? 0.0f + g[h][e] : 0.0f;
            }
            float *base = out + (int64_t)o[h] * a.height * a.width * a.channels + c[h];
            for (int32_t ky = 0; ky < a.ky; ++ky) {
                const int32_t iy = oy[h] * a.ky + ky;
                for (int32_t kx = 0; kx < a.kx; ++kx) {
                    const int32_t ix = ox[h] * a.kx + kx;
                    const int k = ky * a.kx + kx;
                    float r[VEC];
#pragma unroll
                    for (int e = 0; e < VEC; ++e) r[e] = w[e] == k ? 0.0f + g[h][e] : 0.0f;
                    store_vec<VEC>(base + ((int64_t)iy * a.width + ix) * a.channels, r);
                }
            }
        }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) lane_sum[threadIdx.x][e] = acc[e];
    __syncthreads();
    const int per_pixel = a.channels / VEC;  // lanes l, l + per_pixel, ... share a channel vector
    for (int c = threadIdx.x; c < a.channels; c += 256) {
        const int cv = c / VEC, e = c % VEC;
        float sum = 0.0f;
        for (int l = cv; l < 256; l += per_pixel) sum += lane_sum[l][e];
        partial[(int64_t)blockIdx.x * a.channels + c] = sum;
    }
}

// Bias-gradient chunks of the same d_pre without reading it: partial[q][c] sums rows
// [512q, 512q + 512) of the [outer*height*width, channels] view in row order, where a row holds
// 0.0f + g exactly at its window's positive winner and +0.0 elsewhere -- the values the scatter
// writes, added in the plain column sum's order.  Each row's window is read unconditionally (the
// window tensors are a quarter of d_pre and stay in cache) so the loads of consecutive rows are
// independent and overlap.
__global__ void __launch_bounds__(256) relu_pool_bias_chunk_kernel(
    const float *__restrict__ gradient, const float *__restrict__ pooled,
    const uint8_t *__restrict__ argmax, float *__restrict__ partial, int64_t rows, int64_t pairs,
    PoolArgs a) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= pairs) return;
    const int64_t q = t / a.channels;
    const int32_t c = (int32_t)(t - q * a.channels);
    const int64_t r0 = q * axis::kGroupedChunk;
    const int32_t count = (int32_t)(r0 + axis::kGroupedChunk < rows ? axis::kGroupedChunk : rows - r0);
    int32_t x = (int32_t)(r0 % a.width);
    int64_t rest = r0 / a.width;
    int32_t y = (int32_t)(rest % a.height);
    int64_t o = rest / a.height;
    int32_t py = y / a.ky, ky = y - py * a.ky;
    int32_t px = x / a.kx, kx = x - px * a.kx;
    // window offset of the current row (in elements of the pooled tensors) and its position code
    int64_t wbase = ((o * a.out_h + py) * a.out_w) * a.channels + c;
    float sum = 0.0f;
#pragma unroll 8
    for (int32_t i = 0; i < count; ++i) {
        const int64_t w = wbase + (int64_t)px * a.channels;
        const int k = ky * a.kx + kx;
        const uint8_t win = argmax[w];
        const float v = pooled[w];
        const float g = a.g_broadcast ? gradient[o * a.channels + c] * a.g_factor : gradient[w];
        sum = sum + ((win == k && v > 0.0f) ? 0.0f + g : 0.0f);
        if (++kx == a.kx) kx = 0, ++px;
        if (++x == a.width) {
            x = 0, px = 0, kx = 0;
            if (++ky == a.ky) ky = 0, wbase += (int64_t)a.out_w * a.channels;
            if (++y == a.height) y = 0, ++o;  // o: the row's image, for a broadcast gradient
        }
    }
    partial[q * a.channels + c] = sum;
}

// General windows: one lane per input vector gathers the windows it won, ky major, kx minor.
template <int VEC>
__global__ void __launch_bounds__(256) max_pool2d_backward_kernel(const float *__restrict__ gradient,
                                                                  const uint8_t *__restrict__ argmax,
                                                                  float *__restrict__ out, PoolArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= a.total) return;
    const uint32_t cv = a.cvec.mod(t);
    uint32_t rest = a.cvec.div(t);
    const int32_t ix = (int32_t)a.iw.mod(rest);
    rest = a.iw.div(rest);
    const int32_t iy = (int32_t)a.ih.mod(rest);
    const uint32_t o = a.ih.div(rest);
    const int32_t c = (int32_t)cv * VEC;
    const int64_t obase = (int64_t)o * a.out_h * a.out_w * a.channels + c;
    float sum[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) sum[e] = 0.0f;
    for (int32_t ky = 0; ky < a.ky; ++ky) {
        const int32_t padded_y = iy + a.py - ky;
        if (padded_y < 0) continue;
        const int32_t oy = (int32_t)a.sy_div.div((uint32_t)padded_y);
        if (oy * a.sy != padded_y || oy >= a.out_h) continue;
        for (int32_t kx = 0; kx < a.kx; ++kx) {
            const int32_t padded_x = ix + a.px - kx;
            if (padded_x < 0) continue;
            const int32_t ox = (int32_t)a.sx_div.div((uint32_t)padded_x);
            if (ox * a.sx != padded_x || ox >= a.out_w) continue;
            const int64_t wpos = obase + ((int64_t)oy * a.out_w + ox) * a.channels;
            const int k = ky * a.kx + kx;
            float g[VEC];
            load_vec<VEC>(gradient + wpos, g);
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                if (argmax[wpos + e] == k) sum[e] += g[e];
        }
    }
    store_vec<VEC>(out + (int64_t)t * VEC, sum);
}

int pool_args(int64_t outer, int32_t height, int32_t width, int64_t channels, const int32_t *kernel,
              const int32_t *stride, const int32_t *padding, PoolArgs *a) {
    AXIS_REQUIRE(kernel && stride && padding, "null pool geometry");
    AXIS_REQUIRE(outer >= 1 && height >= 1 && width >= 1 && channels >= 1,
                 "pool extents must be positive");
    AXIS_REQUIRE(kernel[0] >= 1 && kernel[1] >= 1 && stride[0] >= 1 && stride[1] >= 1,
                 "pool kernel and stride must be positive");
    AXIS_REQUIRE(kernel[0] * kernel[1] < 255, "pool window must have fewer than 255 positions");
    AXIS_REQUIRE(padding[0] >= 0 && padding[1] >= 0 && 2 * padding[0] <= kernel[0] &&
                     2 * padding[1] <= kernel[1],
                 "pool padding must be at most half the kernel extent");
    AXIS_REQUIRE(height + 2 * padding[0] >= kernel[0] && width + 2 * padding[1] >= kernel[1],
                 "pool kernel exceeds the padded spatial extent");
    AXIS_REQUIRE(outer * height * width * channels <= INT32_MAX, "pool input exceeds the 32-bit index range");
    AXIS_REQUIRE(channels <= INT32_MAX, "too many channels");
    a->channels = (int32_t)channels;
    a->height = height;
    a->width = width;
    a->out_h = (height + 2 * padding[0] - kernel[0]) / stride[0] + 1;
    a->out_w = (width + 2 * padding[1] - kernel[1]) / stride[1] + 1;
    a->ky = kernel[0];
    a->kx = kernel[1];
    a->sy = stride[0];
    a->sx = stride[1];
    a->py = padding[0];
    a->px = padding[1];
    a->ow = FastDiv((uint32_t)a->out_w);
    a->oh = FastDiv((uint32_t)a->out_h);
    a->iw = FastDiv((uint32_t)width);
    a->ih = FastDiv((uint32_t)height);
    a->sy_div = FastDiv((uint32_t)stride[0]);
    a->sx_div = FastDiv((uint32_t)stride[1]);
    return AXIS_OK;
}

int relu_pool_backward(axis_device device, const float *gradient, bool broadcast, float factor, const float *pooled,
                       const uint8_t *argmax, float *d_pre, float *d_bias, int64_t outer, int32_t height,
                       int32_t width, int32_t channels, const int32_t pool[2]);

}  // namespace

extern "C" {

int axis_max_pool2d(axis_device device, const float *input, float *out, uint8_t *argmax,
                    int64_t outer, int32_t height, int32_t width, int64_t channels,
                    const int32_t kernel[2], const int32_t stride[2], const int32_t padding[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {input, 4 * outer * height * width * channels}, {out, 1}, {argmax, 1});
    AXIS_REQUIRE(input && out && argmax, "null max_pool2d buffer");
    PoolArgs a{};
    if (int s = pool_args(outer, height, width, channels, kernel, stride, padding, &a)) return s;
    const bool vec = channels % 4 == 0 && axis::aligned16(input) && axis::aligned16(out) &&
                     (reinterpret_cast<uintptr_t>(argmax) & 3u) == 0;
    const int v = vec ? 4 : 1;
    a.cvec = FastDiv((uint32_t)(channels / v));
    a.total = (uint32_t)(outer * a.out_h * a.out_w * (channels / v));
    if (vec)
        max_pool2d_kernel<4><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0, device->stream>>>(
            input, out, argmax, a);
    else
        max_pool2d_kernel<1><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0, device->stream>>>(
            input, out, argmax, a);
    return axis::launch_status("max_pool2d_kernel");
}

int axis_max_pool2d_backward(axis_device device, const float *gradient, const uint8_t *argmax,
                             float *out, int64_t outer, int32_t height, int32_t width,
                             int64_t channels, const int32_t kernel[2], const int32_t stride[2],
                             const int32_t padding[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 1}, {argmax, 1}, {out, 4 * outer * height * width * channels});
    AXIS_REQUIRE(gradient && argmax && out, "null max_pool2d_backward buffer");
    PoolArgs a{};
    if (int s = pool_args(outer, height, width, channels, kernel, stride, padding, &a)) return s;
    const bool vec = channels % 4 == 0 && axis::aligned16(gradient) && axis::aligned16(out) &&
                     (reinterpret_cast<uintptr_t>(argmax) & 3u) == 0;
    const int v = vec ? 4 : 1;
    a.cvec = FastDiv((uint32_t)(channels / v));
    const bool tiled = stride[0] == kernel[0] && stride[1] == kernel[1] && padding[0] == 0 &&
                       padding[1] == 0 && height % kernel[0] == 0 && width % kernel[1] == 0;
    if (tiled) {
        a.total = (uint32_t)(outer * a.out_h * a.out_w * (channels / v));
        if (vec)
            max_pool2d_backward_tiled_kernel<4><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0,
                                                  device->stream>>>(gradient, argmax, out, a);
        else
            max_pool2d_backward_tiled_kernel<1><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0,
                                                  device->stream>>>(gradient, argmax, out, a);
        return axis::launch_status("max_pool2d_backward_tiled_kernel");
    }
    a.total = (uint32_t)(outer * height * width * (channels / v));
    if (vec)
        max_pool2d_backward_kernel<4><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0,
                                        device->stream>>>(gradient, argmax, out, a);
    else
        max_pool2d_backward_kernel<1><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0,
                                        device->stream>>>(gradient, argmax, out, a);
    return axis::launch_status("max_pool2d_backward_kernel");
}

int axis_relu_pool_backward(axis_device device, const float *gradient, const float *pooled,
                            const uint8_t *argmax, float *d_pre, float *d_bias, int64_t outer,
                            int32_t height, int32_t width, int32_t channels, const int32_t pool[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 1}, {pooled, 1}, {argmax, 1}, {d_pre, 4 * outer * height * width * channels}, {d_bias, 4 * (int64_t)channels});
    return relu_pool_backward(device, gradient, false, 1.0f, pooled, argmax, d_pre, d_bias, outer, height, width,
                              channels, pool);
}

int axis_relu_pool_backward_mean(axis_device device, const float *gradient, float factor, const float *pooled,
                                 const uint8_t *argmax, float *d_pre, float *d_bias, int64_t outer,
                                 int32_t height, int32_t width, int32_t channels, const int32_t pool[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 1}, {pooled, 1}, {argmax, 1}, {d_pre, 4 * outer * height * width * channels}, {d_bias, 4 * (int64_t)channels});
    return relu_pool_backward(device, gradient, true, factor, pooled, argmax, d_pre, d_bias, outer, height, width,
                              channels, pool);
}

}  // extern "C"

namespace {

int relu_pool_backward(axis_device device, const float *gradient, bool broadcast, float factor, const float *pooled,
                       const uint8_t *argmax, float *d_pre, float *d_bias, int64_t outer, int32_t height,
                       int32_t width, int32_t channels, const int32_t pool[2]) {
    AXIS_REQUIRE(gradient && pooled && argmax && d_pre && pool, "null relu_pool_backward buffer");
    const int32_t zero[2] = {0, 0};
    PoolArgs a{};
    if (int s = pool_args(outer, height, width, channels, pool, pool, zero, &a)) return s;
    a.g_broadcast = broadcast;
    a.g_factor = factor;
    AXIS_REQUIRE(height % pool[0] == 0 && width % pool[1] == 0,
                 "relu_pool_backward needs windows that tile the input exactly");
    const bool vec = channels % 4 == 0 && axis::aligned16(gradient) && axis::aligned16(pooled) &&
                     axis::aligned16(d_pre) && (reinterpret_cast<uintptr_t>(argmax) & 3u) == 0;
    // the broadcast gradient's rows are [channels]: vector loads need no more alignment than that
    const int v = vec ? 4 : 1;
    a.cvec = FastDiv((uint32_t)(channels / v));
    a.total = (uint32_t)(outer * a.out_h * a.out_w * (channels / v));
    if (d_bias && 256 % (channels / v) == 0) {
        // bias folded into the scatter: blocks of whole 256-vector strides, one partial each
        const int64_t blocks = std::min<int64_t>((a.total + 255) / 256, (int64_t)device->multiprocessors * 8);
        const uint32_t span = (uint32_t)(((a.total + blocks - 1) / blocks + 255) / 256 * 256);
        const int32_t nb = (int32_t)((a.total + span - 1) / span);
        axis::Scratch partial;
        if (int s = partial.get(device, sizeof(float) * (size_t)nb * (size_t)channels)) return s;
        float *part = partial.as<float>();
        if (vec && a.g_broadcast)
            relu_pool_backward_bias_kernel<4, true><<<nb, 256, 0, device->stream>>>(gradient, pooled, argmax, d_pre,
                                                                                  part, span, a);
        else if (vec)
            relu_pool_backward_bias_kernel<4, false><<<nb, 256, 0, device->stream>>>(gradient, pooled, argmax, d_pre,
                                                                                   part, span, a);
        else if (a.g_broadcast)
            relu_pool_backward_bias_kernel<1, true><<<nb, 256, 0, device->stream>>>(gradient, pooled, argmax, d_pre,
                                                                                  part, span, a);
        else
            relu_pool_backward_bias_kernel<1, false><<<nb, 256, 0, device->stream>>>(gradient, pooled, argmax, d_pre,
                                                                                   part, span, a);
        if (int s = axis::launch_status("relu_pool_backward_bias_kernel")) return s;
        return axis::column_block_sum(device, partial, nb, channels, channels, channels, d_bias, nullptr);
    }
    if (vec)
        relu_pool_backward_kernel<4><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0, device->stream>>>(
            gradient, pooled, argmax, d_pre, a);
    else
        relu_pool_backward_kernel<1><<<axis::blocks_for(a.total, 256, INT32_MAX), 256, 0, device->stream>>>(
            gradient, pooled, argmax, d_pre, a);
    if (int s = axis::launch_status("relu_pool_backward_kernel")) return s;
    if (!d_bias) return AXIS_OK;
    const int64_t rows = outer * height * width;
    const int64_t chunks = (rows + axis::kGroupedChunk - 1) / axis::kGroupedChunk;
    const int64_t pairs = chunks * channels;
    axis::Scratch partial;
    if (int s = partial.get(device, sizeof(float) * (size_t)pairs)) return s;
    relu_pool_bias_chunk_kernel<<<axis::blocks_for(pairs, 256, INT32_MAX), 256, 0, device->stream>>>(
        gradient, pooled, argmax, partial.as<float>(), rows, pairs, a);
    if (int s = axis::launch_status("relu_pool_bias_chunk_kernel")) return s;
    axis::column_combine_kernel<<<(unsigned)channels, 256, 0, device->stream>>>(partial.as<float>(), chunks,
                                                                              channels, 1.0f, d_bias);
    return axis::launch_status("column_combine_kernel");
}

}  // namespace
