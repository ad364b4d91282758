// bf16 matrix-core path of the dense products on a bf16 device (gemm_bf16.hip), used by gemm.hip's
// dense matmul family when the device rounds product operands to bf16: the reference's
// matmul_bf16 and its two backward kernels (runtime/backend.rs:2209-2312), which convert fp32
// operand tiles to bf16 and accumulate their products in fp32.
//
// Each operand is first staged as bf16 rows [batch][rows][kp] whose reduction index is contiguous
// and zero-padded to kp (a multiple of kBf16Depth); the product kernel then feeds
// v_mfma_f32_16x16x32_bf16 from those rows.  Products of bf16 values are exact in fp32, so the
// result equals the fp32 product of the rounded operands up to the order of the fp32 sums.
#pragma once

#include <cstdint>

#include "../../include/axis_hip.h"

namespace axis {

constexpr int kBf16Depth = 64;  // reduction depth of one LDS stage of the product kernel

// Operand element (t, r) of batch b sits at base[b * s_b + t * s_t + r * s_r].
struct Bf16Source {
    const float *base;
    int64_t s_b, s_t, s_r;
};

// Rounds elements (t < rows, r < k) of each batch to bf16 (nearest, ties to even) into
// dst[b][t][r] (batch stride rows * kp), writing zeros for k <= r < kp.
int stage_bf16(axis_device device, const Bf16Source &src, int64_t batch, int64_t rows, int64_t k, int64_t kp,
               uint16_t *dst);

struct Bf16Gemm {
    const uint16_t *x, *y;     // staged X [m][kp] and Y [n][kp] per batch
    int64_t x_batch, y_batch;  // element strides between batches of the staged operands (0 = shared)
    float *c;                  // output, or reduction slices when splits > 1
    const float *bias, *d;     // + bias[col]; beta * d + alpha * v (whole sums only)
    float alpha, beta;
    int64_t m, n, kp;
    int64_t c_batch, c_split, k_chunk;
    int32_t splits;
};

struct Bf16Tile {
    int rows, cols;  // output rows (of X) and columns (of Y) per block
};

// Output tile for a device with `cus` compute units and a reduction padded to kp: 256 x 256 when
// the output has at least one per CU and they waste at most 1/8 of their area past its edges; else
// 128 x 128 unless the output has too few of them to fill the chip and the reduction is too short
// to be split into slices (under 8 stages), then 64 x 64.
Bf16Tile bf16_gemm_tile(int64_t m, int64_t n, int64_t batch, int64_t kp, int64_t cus);

// Whether bf16_gemm takes this product: its loads address one tile's staged rows with 32-bit
// byte offsets, so (tile rows + 1) * kp * 2 must stay below 2^31 (reductions up to about 8.3M).
// Callers decide before staging anything; a product that does not fit runs on the fp32 matrix
// cores with its operands rounded to bf16 as they are staged in LDS (the same values).
bool bf16_gemm_fits(int64_t m, int64_t n, int64_t batch, int64_t kp, int64_t cus);

// C[b][i][j] = sum_r X[b][i][r] Y[b][j][r] with `tile` from bf16_gemm_tile; slice s of a split
// reduction covers r in [s * k_chunk, (s + 1) * k_chunk) and lands at c + s * c_split.
int bf16_gemm(axis_device device, const Bf16Gemm &g, int64_t batch, Bf16Tile tile);

}  // namespace axis
