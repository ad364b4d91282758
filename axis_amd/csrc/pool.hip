// Max pooling over channel-innermost activations: the forward of the reference's
// -min(-unfold(x, fill=-inf)) (model/convolution.rs:1357-1370, Tensor::min tensor.rs:2880-2946,
// grouped_minimum backend.rs:3019-3056) in one pass, emitting the window-local winner as a byte,
// and its backward (Rule::Minimum gather + mask, then unfold's col2im, tensor.rs:5679-5683 and
// backend.rs:1795-1889) as one gather pass per input element.
//
// Lanes run along the channel axis, so every load and store is unit-stride across the wave.
#include <cfloat>

#include "common.hpp"

namespace {

constexpr uint8_t kNoWinner = 255;

struct PoolArgs {
    int64_t outer, channels;
    int32_t height, width, out_h, out_w;
    int32_t ky, kx, sy, sx, py, px;
};

__global__ void __launch_bounds__(256) max_pool2d_kernel(const float *__restrict__ in,
                                                         float *__restrict__ out,
                                                         uint8_t *__restrict__ argmax, PoolArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = a.outer * a.out_h * a.out_w * a.channels;
    if (idx >= total) return;
    const int64_t c = idx % a.channels;
    int64_t rest = idx / a.channels;
    const int32_t ox = (int32_t)(rest % a.out_w);
    rest /= a.out_w;
    const int32_t oy = (int32_t)(rest % a.out_h);
    const int64_t o = rest / a.out_h;
    const float *base = in + o * a.height * a.width * a.channels + c;
    float best = -INFINITY;
    int winner = kNoWinner;
    for (int32_t ky = 0; ky < a.ky; ++ky) {
        const int32_t iy = oy * a.sy + ky - a.py;
        if (iy < 0 || iy >= a.height) continue;
        for (int32_t kx = 0; kx < a.kx; ++kx) {
            const int32_t ix = ox * a.sx + kx - a.px;
            if (ix < 0 || ix >= a.width) continue;
            const float v = base[((int64_t)iy * a.width + ix) * a.channels];
            // first strictly greater finite value in window order (ky major, kx minor)
            if (v >= -FLT_MAX && v <= FLT_MAX && v > best) {
                best = v;
                winner = ky * a.kx + kx;
            }
        }
    }
    out[idx] = winner == kNoWinner ? __builtin_nanf("") : best;
    argmax[idx] = (uint8_t)winner;
}

__global__ void __launch_bounds__(256) max_pool2d_backward_kernel(const float *__restrict__ gradient,
                                                                  const uint8_t *__restrict__ argmax,
                                                                  float *__restrict__ out, PoolArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = a.outer * a.height * a.width * a.channels;
    if (idx >= total) return;
    const int64_t c = idx % a.channels;
    int64_t rest = idx / a.channels;
    const int32_t ix = (int32_t)(rest % a.width);
    rest /= a.width;
    const int32_t iy = (int32_t)(rest % a.height);
    const int64_t o = rest / a.height;
    const int64_t obase = o * a.out_h * a.out_w * a.channels + c;
    float sum = 0.0f;
    for (int32_t ky = 0; ky < a.ky; ++ky) {
        const int32_t padded_y = iy + a.py - ky;
        if (padded_y < 0 || padded_y % a.sy != 0) continue;
        const int32_t oy = padded_y / a.sy;
        if (oy >= a.out_h) continue;
        for (int32_t kx = 0; kx < a.kx; ++kx) {
            const int32_t padded_x = ix + a.px - kx;
            if (padded_x < 0 || padded_x % a.sx != 0) continue;
            const int32_t ox = padded_x / a.sx;
            if (ox >= a.out_w) continue;
            const int64_t w = obase + ((int64_t)oy * a.out_w + ox) * a.channels;
            if (argmax[w] == ky * a.kx + kx) sum += gradient[w];
        }
    }
    out[idx] = sum;
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
    a->outer = outer;
    a->channels = channels;
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
    return AXIS_OK;
}

}  // namespace

extern "C" {

int axis_max_pool2d(axis_device device, const float *input, float *out, uint8_t *argmax,
                    int64_t outer, int32_t height, int32_t width, int64_t channels,
                    const int32_t kernel[2], const int32_t stride[2], const int32_t padding[2]) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(input && out && argmax, "null max_pool2d buffer");
    PoolArgs a{};
    if (int s = pool_args(outer, height, width, channels, kernel, stride, padding, &a)) return s;
    const int64_t total = outer * a.out_h * a.out_w * channels;
    max_pool2d_kernel<<<axis::blocks_for(total, 256, INT32_MAX), 256, 0, device->stream>>>(
        input, out, argmax, a);
    return axis::launch_status("max_pool2d_kernel");
}

int axis_max_pool2d_backward(axis_device device, const float *gradient, const uint8_t *argmax,
                             float *out, int64_t outer, int32_t height, int32_t width,
                             int64_t channels, const int32_t kernel[2], const int32_t stride[2],
                             const int32_t padding[2]) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(gradient && argmax && out, "null max_pool2d_backward buffer");
    PoolArgs a{};
    if (int s = pool_args(outer, height, width, channels, kernel, stride, padding, &a)) return s;
    const int64_t total = outer * (int64_t)height * width * channels;
    max_pool2d_backward_kernel<<<axis::blocks_for(total, 256, INT32_MAX), 256, 0, device->stream>>>(
        gradient, argmax, out, a);
    return axis::launch_status("max_pool2d_backward_kernel");
}

}  // extern "C"
