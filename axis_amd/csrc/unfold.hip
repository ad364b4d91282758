// im2col (unfold2d) and gather-form col2im (unfold2d_backward) on the reference's rank-generic
// UnfoldSpec (runtime/backend.rs:1127-1253, kernels :1604-1689 and :1795-1889).
//
// One lane per output (im2col) or per input element (col2im), like the reference, but every
// per-dimension divide is a precomputed multiply-high (fastdiv.hpp) and all index arithmetic is
// 32-bit (the tensor layer bounds both lengths below 2^31).  col2im keeps the reference's
// summation order -- ky outer, kx inner, starting from +0.0 -- so its result is bit-identical to
// a sequential restatement, and it needs no atomics.
#include <algorithm>

#include "common.hpp"
#include "fastdiv.hpp"

namespace {

struct UnfoldDims {
    int32_t rank;
    FastDiv stride[8];   // divisor giving the coordinate's place value
    FastDiv extent[8];
    int32_t other[8];    // stride on the far side (input stride for im2col, output for col2im)
    int32_t role[8];
};

struct UnfoldArgs {
    UnfoldDims dims;
    FastDiv kx_div, ky_div;  // patch decode (kernel width, kernel height)
    FastDiv sy_div, sx_div;  // col2im stride tests
    int32_t len;
    int32_t channels_per_group;
    int32_t kernel_y, kernel_x, stride_y, stride_x, padding_y, padding_x;
    int32_t height, width;                 // input spatial (im2col) / output spatial (col2im)
    int32_t s0, s1, s2, s3;                // im2col: channel, y, x input strides; col2im: y, x, group, patch
    float fill;
};

__global__ void __launch_bounds__(256) unfold2d_kernel(const float *__restrict__ input,
                                                       float *__restrict__ out, UnfoldArgs a) {
    const uint32_t o = blockIdx.x * 256u + threadIdx.x;
    if (o >= (uint32_t)a.len) return;
    int32_t input_index = 0, oy = 0, ox = 0, group = 0, patch = 0;
    for (int d = 0; d < a.dims.rank; ++d) {
        const int32_t coordinate = (int32_t)a.dims.extent[d].mod(a.dims.stride[d].div(o));
        switch (a.dims.role[d]) {
        case 0: input_index += coordinate * a.dims.other[d]; break;
        case 1: oy = coordinate; break;
        case 2: ox = coordinate; break;
        case 3: group = coordinate; break;
        default: patch = coordinate; break;
        }
    }
    const uint32_t rest = a.kx_div.div((uint32_t)patch);
    const int32_t kx = patch - (int32_t)rest * a.kernel_x;
    const uint32_t cig = a.ky_div.div(rest);
    const int32_t ky = (int32_t)rest - (int32_t)cig * a.kernel_y;
    const int32_t channel = group * a.channels_per_group + (int32_t)cig;
    const int32_t iy = oy * a.stride_y + ky - a.padding_y;
    const int32_t ix = ox * a.stride_x + kx - a.padding_x;
    const bool valid = iy >= 0 && iy < a.height && ix >= 0 && ix < a.width;
    out[o] = valid ? input[input_index + channel * a.s0 + iy * a.s1 + ix * a.s2] : a.fill;
}

__global__ void __launch_bounds__(256) unfold2d_backward_kernel(const float *__restrict__ gradient,
                                                                float *__restrict__ out,
                                                                UnfoldArgs a) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= (uint32_t)a.len) return;
    int32_t output_base = 0, channel = 0, iy = 0, ix = 0;
    for (int d = 0; d < a.dims.rank; ++d) {
        const int32_t coordinate = (int32_t)a.dims.extent[d].mod(a.dims.stride[d].div(i));
        switch (a.dims.role[d]) {
        case 0: output_base += coordinate * a.dims.other[d]; break;
        case 1: channel = coordinate; break;
        case 2: iy = coordinate; break;
        default: ix = coordinate; break;
        }
    }
    const int32_t group = channel / a.channels_per_group;
    const int32_t channel_in_group = channel - group * a.channels_per_group;
    float sum = 0.0f;
    for (int32_t ky = 0; ky < a.kernel_y; ++ky) {
        const int32_t padded_y = iy + (a.padding_y - ky);
        if (padded_y < 0) continue;
        const int32_t oy = (int32_t)a.sy_div.div((uint32_t)padded_y);
        if (oy * a.stride_y != padded_y || oy >= a.height) continue;
        for (int32_t kx = 0; kx < a.kernel_x; ++kx) {
            const int32_t padded_x = ix + (a.padding_x - kx);
            if (padded_x < 0) continue;
            const int32_t ox = (int32_t)a.sx_div.div((uint32_t)padded_x);
            if (ox * a.stride_x != padded_x || ox >= a.width) continue;
            const int32_t patch = (channel_in_group * a.kernel_y + ky) * a.kernel_x + kx;
            sum += gradient[output_base + oy * a.s0 + ox * a.s1 + group * a.s2 + patch * a.s3];
        }
    }
    out[i] = sum;
}

// Patches of a channel-innermost input laid out [rows = batch*oh*ow][patch = (c, ky, kx)] (the
// convolution case with one group): a block stages the kh*kw*channels window values of `rows`
// output pixels in LDS, read with lanes along the channel axis (unit stride), then writes each
// pixel's patch row contiguously.  Same values as unfold2d_kernel, position for position.
struct Im2colArgs {
    int32_t rows, channels, window, patch;  // patch = channels * window
    int32_t out_h, out_w, height, width;
    int32_t kernel_x, stride_y, stride_x, padding_y, padding_x;
    int32_t rows_per_block;
    int64_t batch_stride, y_stride, x_stride;  // input strides (channel stride is 1)
    FastDiv c_div, window_div, ow_div, oh_div, kx_div, patch_div;
    float fill;
};

__global__ void __launch_bounds__(256) im2col_channels_last_kernel(const float *__restrict__ input,
                                                                   float *__restrict__ out,
                                                                   Im2colArgs a) {
    extern __shared__ float tile[];  // [rows_per_block][window][channels + 1]
    const int32_t pitch = a.channels + 1;
    const int32_t row0 = blockIdx.x * a.rows_per_block;
    const int32_t rows = min(a.rows_per_block, a.rows - row0);
    const uint32_t staged = (uint32_t)(rows * a.window * a.channels);
    for (uint32_t idx = threadIdx.x; idx < staged; idx += 256) {
        const uint32_t c = a.c_div.mod(idx);
        const uint32_t rest = a.c_div.div(idx);
        const uint32_t pos = a.window_div.mod(rest);
        const uint32_t r = a.window_div.div(rest);
        const uint32_t pixel = (uint32_t)row0 + r;
        const int32_t ox = (int32_t)a.ow_div.mod(pixel);
        const uint32_t rest2 = a.ow_div.div(pixel);
        const int32_t oy = (int32_t)a.oh_div.mod(rest2);
        const int64_t b = a.oh_div.div(rest2);
        const int32_t kx = (int32_t)a.kx_div.mod(pos);
        const int32_t ky = (int32_t)a.kx_div.div(pos);
        const int32_t iy = oy * a.stride_y + ky - a.padding_y;
        const int32_t ix = ox * a.stride_x + kx - a.padding_x;
        const bool valid = iy >= 0 && iy < a.height && ix >= 0 && ix < a.width;
        tile[(r * a.window + pos) * pitch + c] =
            valid ? input[b * a.batch_stride + iy * a.y_stride + ix * a.x_stride + c] : a.fill;
    }
    __syncthreads();
    const uint32_t written = (uint32_t)(rows * a.patch);
    float *dst = out + (int64_t)row0 * a.patch;
    for (uint32_t idx = threadIdx.x; idx < written; idx += 256) {
        const uint32_t k = a.patch_div.mod(idx);
        const uint32_t r = a.patch_div.div(idx);
        const uint32_t pos = a.window_div.mod(k);
        const uint32_t c = a.window_div.div(k);
        dst[idx] = tile[(r * a.window + pos) * pitch + c];
    }
}

// Recognise the convolution layout of unfold_spec's output: one group, patch innermost, then
// ox, oy and at most one other (batch) dimension, over a channel-innermost input.
bool channels_last_im2col(const axis_unfold_spec *s, Im2colArgs *a) {
    const int32_t kh = s->kernel[0], kw = s->kernel[1];
    const int32_t oh = s->output_spatial[0], ow = s->output_spatial[1];
    int32_t channels = -1;
    for (int d = 0; d < s->input_rank; ++d)
        if (s->backward_metadata[4 * d + 3] == 1) channels = s->backward_metadata[4 * d];
    if (channels < 1 || s->channels_per_group != channels || s->input_special_strides[0] != 1)
        return false;
    const int64_t patch = (int64_t)channels * kh * kw;
    int64_t batch = 1, batch_stride = 0;
    int others = 0;
    for (int d = 0; d < s->output_rank; ++d) {
        const int32_t *md = s->forward_metadata + 4 * d;
        switch (md[3]) {
        case 0:
            if (++others > 1 || md[1] != patch * ow * oh) return false;
            batch = md[0];
            batch_stride = md[2];
            break;
        case 1: if (md[1] != patch * ow) return false; break;
        case 2: if (md[1] != patch) return false; break;
        case 3: if (md[0] != 1) return false; break;
        default: if (md[1] != 1 || md[0] != patch) return false; break;
        }
    }
    const int64_t rows = batch * oh * ow;
    if (rows * patch != s->output_len || rows > INT32_MAX) return false;
    int rows_per_block = (int)std::max<int64_t>(1, 4096 / patch);
    while (rows_per_block > 1 && (int64_t)rows_per_block * kh * kw * (channels + 1) * 4 > 48 * 1024)
        --rows_per_block;
    if ((int64_t)rows_per_block * kh * kw * (channels + 1) * 4 > 64 * 1024) return false;
    a->rows = (int32_t)rows;
    a->channels = channels;
    a->window = kh * kw;
    a->patch = (int32_t)patch;
    a->out_h = oh;
    a->out_w = ow;
    a->height = s->input_spatial[0];
    a->width = s->input_spatial[1];
    a->kernel_x = kw;
    a->stride_y = s->stride[0];
    a->stride_x = s->stride[1];
    a->padding_y = s->padding[0];
    a->padding_x = s->padding[1];
    a->rows_per_block = rows_per_block;
    a->batch_stride = batch_stride;
    a->y_stride = s->input_special_strides[1];
    a->x_stride = s->input_special_strides[2];
    a->c_div = FastDiv((uint32_t)channels);
    a->window_div = FastDiv((uint32_t)(kh * kw));
    a->ow_div = FastDiv((uint32_t)ow);
    a->oh_div = FastDiv((uint32_t)oh);
    a->kx_div = FastDiv((uint32_t)kw);
    a->patch_div = FastDiv((uint32_t)patch);
    a->fill = s->fill;
    return true;
}

int validate(const axis_unfold_spec *s) {
    AXIS_REQUIRE(s, "null unfold spec");
    AXIS_REQUIRE(s->spatial_rank == 2, "unfold supports exactly two spatial axes on this backend");
    AXIS_REQUIRE(s->input_len >= 1 && s->output_len >= 1, "unfold lengths must be positive");
    AXIS_REQUIRE(s->input_len <= INT32_MAX - 255 && s->output_len <= INT32_MAX - 255,
                 "unfold tensor is too large for 32-bit index arithmetic");
    AXIS_REQUIRE(s->input_rank >= 1 && s->input_rank <= 8 && s->output_rank >= 1 &&
                     s->output_rank <= 8,
                 "unfold rank must be 1..8");
    AXIS_REQUIRE(s->kernel[0] >= 1 && s->kernel[1] >= 1 && s->stride[0] >= 1 && s->stride[1] >= 1 &&
                     s->padding[0] >= 0 && s->padding[1] >= 0 && s->channels_per_group >= 1,
                 "unfold kernel/stride must be positive and padding nonnegative");
    int64_t in_len = 1, out_len = 1;
    for (int d = 0; d < s->output_rank; ++d) {
        const int32_t *md = s->forward_metadata + 4 * d;
        AXIS_REQUIRE(md[0] >= 1 && md[1] >= 1 && md[3] >= 0 && md[3] <= 4, "bad forward metadata");
        out_len *= md[0];
    }
    for (int d = 0; d < s->input_rank; ++d) {
        const int32_t *md = s->backward_metadata + 4 * d;
        AXIS_REQUIRE(md[0] >= 1 && md[1] >= 1 && md[3] >= 0 && md[3] <= 3, "bad backward metadata");
        in_len *= md[0];
    }
    AXIS_REQUIRE(in_len == s->input_len && out_len == s->output_len,
                 "unfold metadata extents disagree with the spec lengths");
    return AXIS_OK;
}

UnfoldArgs common_args(const axis_unfold_spec *s) {
    UnfoldArgs a{};
    a.kx_div = FastDiv((uint32_t)s->kernel[1]);
    a.ky_div = FastDiv((uint32_t)s->kernel[0]);
    a.sy_div = FastDiv((uint32_t)s->stride[0]);
    a.sx_div = FastDiv((uint32_t)s->stride[1]);
    a.channels_per_group = s->channels_per_group;
    a.kernel_y = s->kernel[0];
    a.kernel_x = s->kernel[1];
    a.stride_y = s->stride[0];
    a.stride_x = s->stride[1];
    a.padding_y = s->padding[0];
    a.padding_x = s->padding[1];
    a.fill = s->fill;
    return a;
}

}  // namespace

extern "C" {

int axis_unfold(axis_device device, const float *input, float *out, const axis_unfold_spec *spec) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {input, spec ? 4 * spec->input_len : 1}, {out, spec ? 4 * spec->output_len : 1});
    if (int st = validate(spec)) return st;
    AXIS_REQUIRE(input && out, "null unfold buffer");
    Im2colArgs fast{};
    if (channels_last_im2col(spec, &fast)) {
        const unsigned blocks = (unsigned)((fast.rows + fast.rows_per_block - 1) / fast.rows_per_block);
        const size_t lds = (size_t)fast.rows_per_block * fast.window * (fast.channels + 1) * sizeof(float);
        im2col_channels_last_kernel<<<blocks, 256, lds, device->stream>>>(input, out, fast);
        return axis::launch_status("im2col_channels_last_kernel");
    }
    UnfoldArgs a = common_args(spec);
    a.dims.rank = spec->output_rank;
    for (int d = 0; d < spec->output_rank; ++d) {
        const int32_t *md = spec->forward_metadata + 4 * d;
        a.dims.extent[d] = FastDiv((uint32_t)md[0]);
        a.dims.stride[d] = FastDiv((uint32_t)md[1]);
        a.dims.other[d] = md[2];
        a.dims.role[d] = md[3];
    }
    a.len = (int32_t)spec->output_len;
    a.height = spec->input_spatial[0];
    a.width = spec->input_spatial[1];
    a.s0 = spec->input_special_strides[0];
    a.s1 = spec->input_special_strides[1];
    a.s2 = spec->input_special_strides[2];
    unfold2d_kernel<<<axis::blocks_for(a.len, 256, INT32_MAX), 256, 0, device->stream>>>(input, out, a);
    return axis::launch_status("unfold2d_kernel");
}

int axis_unfold_backward(axis_device device, const float *gradient, float *out,
                         const axis_unfold_spec *spec) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, spec ? 4 * spec->output_len : 1}, {out, spec ? 4 * spec->input_len : 1});
    if (int st = validate(spec)) return st;
    AXIS_REQUIRE(gradient && out, "null unfold_backward buffer");
    UnfoldArgs a = common_args(spec);
    a.dims.rank = spec->input_rank;
    for (int d = 0; d < spec->input_rank; ++d) {
        const int32_t *md = spec->backward_metadata + 4 * d;
        a.dims.extent[d] = FastDiv((uint32_t)md[0]);
        a.dims.stride[d] = FastDiv((uint32_t)md[1]);
        a.dims.other[d] = md[2];
        a.dims.role[d] = md[3];
    }
    a.len = (int32_t)spec->input_len;
    a.height = spec->output_spatial[0];
    a.width = spec->output_spatial[1];
    a.s0 = spec->output_special_strides[0];
    a.s1 = spec->output_special_strides[1];
    a.s2 = spec->output_special_strides[3];
    a.s3 = spec->output_special_strides[4];
    unfold2d_backward_kernel<<<axis::blocks_for(a.len, 256, INT32_MAX), 256, 0, device->stream>>>(
        gradient, out, a);
    return axis::launch_status("unfold2d_backward_kernel");
}

}  // extern "C"
