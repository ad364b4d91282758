// Short-reduction convolution kernels (conv_small.hip), used by the convolution entries of
// gemm.hip when a layer's whole patch reduction fits one short MFMA pass.
#pragma once

#include <cstdint>

#include "../../include/axis_hip.h"

namespace axis {

struct SmallConvShape {
    int64_t batch;
    int32_t height, width, channels, out_channels, kh, kw, sy, sx, py, px, out_h, out_w;
};

// stride 1, channels <= 4, channels * kh * kw <= 31, padding < kernel, and the staged band fits
// the prefetch registers and LDS.
bool small_conv_applies(const SmallConvShape &s);

// Convolution + bias into out [batch, out_h, out_w, n] (pooled == null), or bias + ReLU + 2x2
// max pool into pooled / argmax [batch, out_h/2, out_w/2, n] (out_h, out_w even).  input is read
// through ld {batch, channel, row, column}; weight is [(c, ky, kx), n].
int small_conv_forward(axis_device device, const SmallConvShape &s, const float *input, const int64_t ld[4],
                       const float *weight, const float *bias, float *out, float *pooled, uint8_t *argmax);

// Weight gradient [(c, ky, kx), n] and bias gradient [n] (or null) of conv -> ReLU -> 2x2 max pool
// from the pooled gradient, pooled values and winner bytes.
int small_conv_pool_backward_weight(axis_device device, const SmallConvShape &s, const float *input,
                                    const int64_t ld[4], const float *gradient, const float *pooled,
                                    const uint8_t *argmax, float *d_weight, float *d_bias);

}  // namespace axis
