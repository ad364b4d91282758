// Convolutions whose whole patch reduction fits one short MFMA pass (channels * kh * kw <= 31,
// stride 1): the first layer of an image network, e.g. 3 channels under a 3x3 kernel (27 terms).
// The reference lowers them like every other convolution (convolution.rs:211-235: unfold ->
// contract -> merge -> + bias; backward through Rule::MatmulRight, tensor.rs:5650-5680); with so
// short a reduction the general implicit GEMM spends most of its time padding the reduction to its
// 32-deep tiles and staging operands, so these kernels keep the whole reduction resident instead:
//
// * A block owns a band of pooling windows (R window rows x S window columns of one image) and
//   stages the input rows the band reads, halo included, in LDS as planes [channel][row][column]
//   with zeros outside the image.  Tap (c, ky, kx) of a pixel is then one LDS word at a fixed
//   offset from the pixel, and the reduction runs in the reference's patch order (c, ky, kx).
// * Pixels are numbered window-major (pixel 4w + 2*ky + kx is position (ky, kx) of window w), so
//   the four consecutive rows a lane holds in each register group of a 32x32 MFMA block are one
//   whole 2x2 window: bias, ReLU and the max pool (first strictly greater finite value, ky major)
//   run in registers, and only pooled values and winner bytes reach HBM.
// * The weight gradient of such a layer is computed straight from the pooled gradient, the
//   pooled values and the winner bytes: the full-resolution pre-activation gradient (ReLU and
//   pool backward) exists only in LDS, one band at a time.  Each 16x16x4 MFMA step reduces over
//   the four pixels of one window.  A plane of ones in the staged input makes row `channels*kh*kw`
//   of the product the bias gradient (the column sum of the same values).
#include <cfloat>

#include "column_sum.hpp"
#include "common.hpp"
#include "conv_small.hpp"
#include "fastdiv.hpp"
#include "pool_rule.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

struct SmallConvArgs {
    const float *x;
    int64_t ld_b;
    int32_t ld_c, ld_h, ld_w;
    int32_t height, width, c_in, kh, kw, py, px;
    int32_t out_h, out_w, n;
    int32_t k;                   // c_in * kh * kw
    int32_t win_rows, win_cols;  // ceil(out_h / 2), ceil(out_w / 2)
    int32_t band_r, band_s;      // windows per band: R rows x S columns
    int32_t bands_y, bands_x;    // bands per image along rows / columns
    int32_t bands;
    int32_t strip_h, strip_w, plane;  // staged rows (2R + kh - 1), columns (2S + kw - 1)
    FastDiv s_div, bx_div, by_div, strip_w_div;
    const float *w;     // [(c, ky, kx), n]
    const float *bias;  // [n] or null
    float *out;         // plain output [batch, out_h, out_w, n]
    float *pooled;      // pooled output [batch, out_h/2, out_w/2, n]
    uint8_t *argmax;
    bool wide;          // outputs allow paired 8-byte stores (and 2-byte winner stores)
    bool vec;           // gradient tensors allow 16-byte loads (n % 4 == 0, aligned)
};

struct Band {
    uint32_t img;
    int32_t wr0, wc0;  // first window row / column
};

__device__ __forceinline__ Band decode_band(const SmallConvArgs &a, uint32_t band) {
    Band b;
    const uint32_t q = a.bx_div.div(band);
    b.wc0 = (int32_t)(band - q * (uint32_t)a.bands_x) * a.band_s;
    b.img = a.by_div.div(q);
    b.wr0 = (int32_t)(q - b.img * (uint32_t)a.bands_y) * a.band_r;
    return b;
}

// Staging of planes 0..c_in-1 of a band's input rows: strip[c][r][col] = x[img, 2*wr0 - py + r,
// 2*wc0 - px + col, c], zero outside the image.  A band holds at most 512 cells (rows x columns)
// of at most 4 channels, so each thread carries two cells of the next band in registers while the
// current band computes.
struct StripRegs {
    float v[2][4];
};

__device__ __forceinline__ void load_strip(const SmallConvArgs &a, const Band &b, int tid, StripRegs &r) {
    const int32_t iy0 = 2 * b.wr0 - a.py, ix0 = 2 * b.wc0 - a.px;
    const int32_t cells = a.strip_h * a.strip_w;
    const float *img = a.x + (int64_t)b.img * a.ld_b;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t t = tid + 256 * i;
        const int32_t row = (int32_t)a.strip_w_div.div((uint32_t)t);
        const int32_t iy = iy0 + row, ix = ix0 + t - row * a.strip_w;
        const bool ok = t < cells && (uint32_t)iy < (uint32_t)a.height && (uint32_t)ix < (uint32_t)a.width;
        const float *src = img + (ok ? (int64_t)iy * a.ld_h + (int64_t)ix * a.ld_w : 0);
#pragma unroll
        for (int c = 0; c < 4; ++c) r.v[i][c] = (ok && c < a.c_in) ? src[(int64_t)c * a.ld_c] : 0.0f;
    }
}

__device__ __forceinline__ void store_strip(const SmallConvArgs &a, float *strip, int tid, const StripRegs &r) {
    const int32_t cells = a.strip_h * a.strip_w;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t t = tid + 256 * i;
        if (t < cells) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (c < a.c_in) strip[c * a.plane + t] = r.v[i][c];
        }
    }
}

// LDS offset of patch term k = (c, ky, kx) from its pixel; term a.k reads plane `at_k` and the
// terms past it plane `past_k`.
__device__ __forceinline__ int32_t term_offset(const SmallConvArgs &a, int32_t k, int32_t at_k, int32_t past_k) {
    if (k == a.k) return at_k * a.plane;
    if (k > a.k) return past_k * a.plane;
    const int32_t taps = a.kh * a.kw;
    const int32_t c = k / taps;
    const int32_t t = k - c * taps;
    const int32_t ky = t / a.kw;
    return c * a.plane + ky * a.strip_w + (t - ky * a.kw);
}

// Forward: KP k-pairs of v_mfma_f32_32x32x2_f32 per pixel tile (2*KP >= k + 1), 32 pixels (8
// windows) by 64 output channels per wave.  Term k of the reduction is the bias: a plane of ones
// in the staged input times a weight row holding the bias, so the products come out biased.
// POOL: ReLU + 2x2 max pool in registers; otherwise the plain convolution + bias.
template <int KP, bool POOL>
__global__ void __launch_bounds__(256, 4) small_conv_forward_kernel(SmallConvArgs a) {
    extern __shared__ float strip[];  // planes 0..c_in-1: input; plane c_in: zeros; c_in + 1: ones
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, half = lane >> 5;
    const int32_t col0 = (int32_t)blockIdx.y * 64;

    // MFMA B operand of k-pair j: W[2j + half][col0 + 2*l32 + b] (column block b holds the odd /
    // even columns, so a lane's two columns are adjacent in the output), the bias at term k.
    // A operand: LDS offset of term 2j + half from the pixel.
    float wreg[KP][2];
    int32_t off[KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) {
        const int32_t k = 2 * j + half;
        off[j] = term_offset(a, k, a.c_in + 1, a.c_in);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int32_t n = col0 + 2 * l32 + b;
            float w = 0.0f;
            if (n < a.n && k < a.k) w = a.w[(int64_t)k * a.n + n];
            if (n < a.n && k == a.k && a.bias != nullptr) w = a.bias[n];
            wreg[j][b] = w;
        }
    }
    bool col_ok[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) col_ok[b] = col0 + 2 * l32 + b < a.n;
    const bool paired = a.wide && col_ok[1];
    for (int32_t t = tid; t < a.plane; t += 256) {
        strip[a.c_in * a.plane + t] = 0.0f;
        strip[(a.c_in + 1) * a.plane + t] = 1.0f;
    }

    const int32_t band_windows = a.band_r * a.band_s;
    const int32_t tiles = band_windows / 8;  // band_s is a multiple of 8: whole tiles per band row
    const int64_t pool_step = 2 * (int64_t)a.n;  // output elements between windows 2 columns apart
    // staged cell of row l32's pixel relative to its tile's first window
    const int32_t lane_px = ((l32 >> 1) & 1) * a.strip_w + 2 * (l32 >> 2) + (l32 & 1);
    StripRegs pre;
    if (blockIdx.x < (uint32_t)a.bands) load_strip(a, decode_band(a, blockIdx.x), tid, pre);
    for (uint32_t band = blockIdx.x; band < (uint32_t)a.bands; band += gridDim.x) {
        const Band bd = decode_band(a, band);
        __syncthreads();  // the previous band's reads are done
        store_strip(a, strip, tid, pre);
        if (band + gridDim.x < (uint32_t)a.bands) load_strip(a, decode_band(a, band + gridDim.x), tid, pre);
        __syncthreads();
        for (int32_t tile = wave; tile < tiles; tile += 4) {
            // Row i = l32: window tile*8 + i/4, position i%4 = (ky, kx) of the window.  The tile's
            // windows sit in window row wr, columns c0 .. c0 + 7 of the band.
            const int32_t wr = (int32_t)a.s_div.div((uint32_t)(tile * 8));
            const int32_t c0 = tile * 8 - wr * a.band_s;
            const float *px0 = strip + (2 * wr * a.strip_w + 2 * c0) + lane_px;
            floatx16 acc[2];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
            // every A operand of the tile is read before the MFMA chain starts (one LDS wait, not
            // one per k-pair)
            float av[KP];
#pragma unroll
            for (int j = 0; j < KP; ++j) av[j] = px0[off[j]];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < KP; ++j)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j], wreg[j][b], acc[b], 0, 0, 0);
            if (!col_ok[0]) continue;
            // Accumulator register v: row i = 8*(v/4) + 4*half + v%4, i.e. window
            // tile*8 + 2*(v/4) + half, position v%4.
            const int32_t c_first = c0 + half;
            if (bd.wr0 + wr >= a.win_rows) continue;
            if constexpr (POOL) {
                // pooled element of the lane's first window; the others follow 2 columns apart
                const int64_t o_first =
                    (((int64_t)bd.img * a.win_rows + bd.wr0 + wr) * a.win_cols + bd.wc0 + c_first) * a.n + col0 +
                    2 * l32;
                float *pooled_at = a.pooled + o_first;
                uint8_t *argmax_at = a.argmax + o_first;
#pragma unroll
                for (int q = 0; q < 4; ++q, pooled_at += pool_step, argmax_at += pool_step) {
                    if (bd.wc0 + c_first + 2 * q >= a.win_cols) continue;
                    float best[2];
                    int winner[2];
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        float y[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) y[e] = acc[b][4 * q + e];
                        relu_pool_window4(y, best[b], winner[b]);
                    }
                    if (paired) {
                        *reinterpret_cast<float2 *>(pooled_at) = make_float2(best[0], best[1]);
                        *reinterpret_cast<uint16_t *>(argmax_at) = (uint16_t)(winner[0] | (winner[1] << 8));
                    } else {
#pragma unroll
                        for (int b = 0; b < 2; ++b) {
                            if (!col_ok[b]) continue;
                            pooled_at[b] = best[b];
                            argmax_at[b] = (uint8_t)winner[b];
                        }
                    }
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int32_t wc = c_first + 2 * q;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int32_t y = 2 * (bd.wr0 + wr) + (e >> 1), x = 2 * (bd.wc0 + wc) + (e & 1);
                        if (y >= a.out_h || x >= a.out_w) continue;
                        const int64_t o = (((int64_t)bd.img * a.out_h + y) * a.out_w + x) * a.n + col0 + 2 * l32;
                        const float v0 = acc[0][4 * q + e], v1 = acc[1][4 * q + e];
                        if (paired) {
                            *reinterpret_cast<float2 *>(a.out + o) = make_float2(v0, v1);
                        } else {
                            a.out[o] = v0;
                            if (col_ok[1]) a.out[o + 1] = v1;
                        }
                    }
                }
            }
        }
    }
}

// Weight and bias gradient through ReLU -> 2x2 max pool: per band, the pre-activation gradient of
// the band's windows is expanded into LDS as dy[window][position][64 columns] (0.0f + g at the
// window's winner when the pooled value is positive, else 0 -- the values axis_relu_pool_backward
// writes), then C^T[n][t] += sum over the window's 4 pixels of dy[p][n] * X[p][t] on
// v_mfma_f32_16x16x4_f32 (A = dy^T: lane -> (n = l%16, p = l/16); B = X: lane -> (p = l/16,
// t = l%16)).  Term t = k is the ones plane: the bias gradient.  Each block writes its partial
// C^T as [32 terms][n]; partials are summed in block order afterwards.  Columns of position p
// are stored XOR 16p, so the four position groups of a wave read different LDS banks.
struct GradRegs {
    floatx4 g[2], p[2];
    uint32_t w[2];
};

__device__ __forceinline__ void load_grad(const SmallConvArgs &a, const Band &bd, int tid, int32_t col0,
                                          const float *__restrict__ g, const float *__restrict__ pooled,
                                          const uint8_t *__restrict__ argmax, GradRegs &r) {
    const int32_t band_windows = a.band_r * a.band_s;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t t = tid + 256 * i;
        const int32_t wi = t >> 4, c4 = (t & 15) * 4;
        const int32_t wr = (int32_t)a.s_div.div((uint32_t)wi);
        const int32_t wc = wi - wr * a.band_s;
        const bool win_ok = wi < band_windows && bd.wr0 + wr < a.win_rows && bd.wc0 + wc < a.win_cols;
        const int64_t pix = ((int64_t)bd.img * a.win_rows + bd.wr0 + wr) * a.win_cols + bd.wc0 + wc;
        const int64_t base = pix * a.n + col0 + c4;
        r.g[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        r.p[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        r.w[i] = 0xffffffffu;
        if (win_ok && a.vec && col0 + c4 < a.n) {
            r.g[i] = *reinterpret_cast<const floatx4 *>(g + base);
            r.p[i] = *reinterpret_cast<const floatx4 *>(pooled + base);
            r.w[i] = *reinterpret_cast<const uint32_t *>(argmax + base);
        } else if (win_ok && !a.vec) {
            uint32_t packed = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool ok = col0 + c4 + e < a.n;
                r.g[i][e] = ok ? g[base + e] : 0.0f;
                r.p[i][e] = ok ? pooled[base + e] : 0.0f;
                packed |= (uint32_t)(ok ? argmax[base + e] : 255) << (8 * e);
            }
            r.w[i] = packed;
        }
    }
}

__device__ __forceinline__ void store_grad(const SmallConvArgs &a, float *dy, int tid, const GradRegs &r) {
    const int32_t band_windows = a.band_r * a.band_s;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t t = tid + 256 * i;
        const int32_t wi = t >> 4, c4 = (t & 15) * 4;
        if (wi >= band_windows) continue;
        // position of each element's winner when its pooled value is positive (else none), and
        // 0 + g, the value the scatter writes there
        uint32_t sel[4];
        float gz[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sel[e] = r.p[i][e] > 0.0f ? (r.w[i] >> (8 * e)) & 0xffu : 0xffu;
            gz[e] = 0.0f + r.g[i][e];
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            floatx4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = sel[e] == (uint32_t)p ? gz[e] : 0.0f;
            *reinterpret_cast<floatx4 *>(dy + (wi * 4 + p) * 64 + (c4 ^ (16 * p))) = o;
        }
    }
}

__global__ void __launch_bounds__(256, 4) small_conv_pool_wgrad_kernel(SmallConvArgs a, const float *__restrict__ g,
                                                                         const float *__restrict__ pooled,
                                                                         const uint8_t *__restrict__ argmax,
                                                                         float *__restrict__ partial) {
    extern __shared__ float lds[];
    float *const strip = lds;                                   // planes 0..c_in-1: input; c_in: ones
    float *const dy = lds + ((a.c_in + 1) * a.plane + 3) / 4 * 4;  // [window][4][64]
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nl = lane & 15, pos = lane >> 4;
    const int32_t col0 = (int32_t)blockIdx.y * 64;
    // staged cells of the lane's two terms at position pos of a window, from the window's first
    // cell; and the lane's gradient column in each column block (XOR-swizzled by position)
    const int32_t lane_px = (pos >> 1) * a.strip_w + (pos & 1);
    const int32_t xoff[2] = {lane_px + term_offset(a, nl, a.c_in, a.c_in),
                             lane_px + term_offset(a, nl + 16, a.c_in, a.c_in)};
    int32_t doff[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) doff[nb] = pos * 64 + 16 * (nb ^ pos) + nl;
    for (int32_t t = tid; t < a.plane; t += 256) strip[a.c_in * a.plane + t] = 1.0f;

    floatx4 acc[4][2];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[nb][kb][v] = 0.0f;

    const int32_t band_windows = a.band_r * a.band_s;
    StripRegs pre;
    GradRegs gpre;
    if (blockIdx.x < (uint32_t)a.bands) {
        const Band first = decode_band(a, blockIdx.x);
        load_strip(a, first, tid, pre);
        load_grad(a, first, tid, col0, g, pooled, argmax, gpre);
    }
    for (uint32_t band = blockIdx.x; band < (uint32_t)a.bands; band += gridDim.x) {
        __syncthreads();
        store_strip(a, strip, tid, pre);
        store_grad(a, dy, tid, gpre);
        if (band + gridDim.x < (uint32_t)a.bands) {
            const Band next = decode_band(a, band + gridDim.x);
            load_strip(a, next, tid, pre);
            load_grad(a, next, tid, col0, g, pooled, argmax, gpre);
        }
        __syncthreads();
        // Windows wi and wi + 4 per pass (band_windows is a multiple of 8): both windows' operands
        // are read before their 16 MFMAs issue.
        for (int32_t wi = wave; wi < band_windows; wi += 8) {
            float x[2][2], d[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int32_t w = wi + 4 * h;
                const int32_t wr = (int32_t)a.s_div.div((uint32_t)w);
                const int32_t wc = w - wr * a.band_s;
                const float *pw = strip + 2 * wr * a.strip_w + 2 * wc;
                x[h][0] = pw[xoff[0]];
                x[h][1] = pw[xoff[1]];
                const float *dyw = dy + w * 256;
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) d[h][nb] = dyw[doff[nb]];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) {
                    acc[nb][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(d[h][nb], x[h][0], acc[nb][0], 0, 0, 0);
                    acc[nb][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(d[h][nb], x[h][1], acc[nb][1], 0, 0, 0);
                }
        }
    }
    // The four waves' sums meet in LDS ([wave][term][64 columns], over the gradient expansion) and
    // are added in wave order.  D register v of lane l: column 4*(l/16) + v (+16 nb), term l%16
    // (+16 kb).
    __syncthreads();
    float *const red = dy;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[(wave * 32 + nl + 16 * kb) * 64 + 16 * nb + 4 * pos + v] = acc[nb][kb][v];
    __syncthreads();
    float *dst = partial + (int64_t)blockIdx.x * 32 * a.n;
    for (int32_t e = tid; e < 32 * 64; e += 256) {
        const int32_t t = e >> 6, col = col0 + (e & 63);
        const float sum = ((red[e] + red[2048 + e]) + red[4096 + e]) + red[6144 + e];
        if (col < a.n) dst[(int64_t)t * a.n + col] = sum;
    }
}

// Windows per band: S columns (a multiple of 8, at most 32; windows past the image are skipped)
// by R rows, R * S <= cap, with at most 512 staged cells (rows x columns), the capacity of the
// threads' prefetch registers.
void band_shape(SmallConvArgs &a, int64_t batch, int32_t cap) {
    auto cells = [&](int32_t r, int32_t s) { return (2 * r + a.kh - 1) * (2 * s + a.kw - 1); };
    a.band_s = (a.win_cols + 7) / 8 * 8;
    if (a.band_s > 32) a.band_s = 32;
    while (a.band_s > 8 && cells(1, a.band_s) > 512) a.band_s -= 8;
    a.band_r = cap / a.band_s;
    if (a.band_r < 1) a.band_r = 1;
    if (a.band_r > a.win_rows) a.band_r = a.win_rows;
    while (a.band_r > 1 && cells(a.band_r, a.band_s) > 512) --a.band_r;
    a.bands_x = (a.win_cols + a.band_s - 1) / a.band_s;
    a.bands_y = (a.win_rows + a.band_r - 1) / a.band_r;
    a.bands = (int32_t)(batch * a.bands_x * a.bands_y);
    a.strip_h = 2 * a.band_r + a.kh - 1;
    a.strip_w = 2 * a.band_s + a.kw - 1;
    a.plane = a.strip_h * a.strip_w;
    a.s_div = FastDiv((uint32_t)a.band_s);
    a.bx_div = FastDiv((uint32_t)a.bands_x);
    a.by_div = FastDiv((uint32_t)a.bands_y);
    a.strip_w_div = FastDiv((uint32_t)a.strip_w);
}

int make_args(const axis::SmallConvShape &s, const float *input, const int64_t ld[4], const float *weight,
              const float *bias, int32_t cap, SmallConvArgs &a) {
    a = SmallConvArgs{};
    a.x = input;
    if (ld) {
        a.ld_b = ld[0];
        a.ld_c = (int32_t)ld[1];
        a.ld_h = (int32_t)ld[2];
        a.ld_w = (int32_t)ld[3];
    }
    a.height = s.height;
    a.width = s.width;
    a.c_in = s.channels;
    a.kh = s.kh;
    a.kw = s.kw;
    a.py = s.py;
    a.px = s.px;
    a.out_h = s.out_h;
    a.out_w = s.out_w;
    a.n = s.out_channels;
    a.k = s.channels * s.kh * s.kw;
    a.win_rows = (s.out_h + 1) / 2;
    a.win_cols = (s.out_w + 1) / 2;
    a.w = weight;
    a.bias = bias;
    band_shape(a, s.batch, cap);
    return AXIS_OK;
}

// Staged planes: the input's channels plus `extra` constant planes.
size_t strip_bytes(const SmallConvArgs &a, int extra) {
    return sizeof(float) * (size_t)(((a.c_in + extra) * a.plane + 3) / 4 * 4);
}

// The weight gradient's expansion [window][4][64], also the four waves' [32][64] sums at the end.
size_t gradient_bytes(const SmallConvArgs &a) {
    const size_t expansion = (size_t)a.band_r * a.band_s * 4 * 64;
    return sizeof(float) * (expansion > 4 * 32 * 64 ? expansion : 4 * 32 * 64);
}

unsigned persistent_blocks(axis_device device, int64_t bands, int64_t columns) {
    const int64_t slots = (int64_t)device->multiprocessors * 4 / (columns > 0 ? columns : 1);
    int64_t per = (bands + (slots > 0 ? slots : 1) - 1) / (slots > 0 ? slots : 1);
    if (per < 1) per = 1;
    return (unsigned)((bands + per - 1) / per);
}

template <bool POOL>
int launch_forward(axis_device device, const SmallConvArgs &a) {
    const int kp = (a.k + 2) / 2;  // the k terms and the bias term
    const unsigned columns = (unsigned)((a.n + 63) / 64);
    dim3 grid(persistent_blocks(device, a.bands, columns), columns);
    const size_t lds = strip_bytes(a, 2);
    hipStream_t st = device->stream;
#define AXIS_SMALL_FWD(KPV)                                                      \
    if (kp <= KPV) {                                                             \
        small_conv_forward_kernel<KPV, POOL><<<grid, 256, lds, st>>>(a);         \
        return axis::launch_status("small_conv_forward_kernel");                 \
    }
    AXIS_SMALL_FWD(2)
    AXIS_SMALL_FWD(4)
    AXIS_SMALL_FWD(6)
    AXIS_SMALL_FWD(8)
    AXIS_SMALL_FWD(10)
    AXIS_SMALL_FWD(12)
    AXIS_SMALL_FWD(14)
    AXIS_SMALL_FWD(16)
#undef AXIS_SMALL_FWD
    return axis::fail(AXIS_ERROR_INVALID, "small convolution reduction too long");
}

}  // namespace

namespace axis {

bool small_conv_applies(const SmallConvShape &s) {
    if (s.sy != 1 || s.sx != 1 || s.out_h < 1 || s.out_w < 1) return false;
    if ((int64_t)s.channels * s.kh * s.kw > 31 || s.channels > 4) return false;
    if (s.py > s.kh - 1 || s.px > s.kw - 1) return false;
    if (s.batch * ((s.out_h + 1) / 2) * ((s.out_w + 1) / 2) >= INT32_MAX) return false;
    // four blocks per CU: the staged band (and the backward's gradient expansion) within 40 KiB
    SmallConvArgs fwd, bwd;
    make_args(s, nullptr, nullptr, nullptr, nullptr, 64, fwd);
    make_args(s, nullptr, nullptr, nullptr, nullptr, 32, bwd);
    const size_t limit = 40 * 1024;
    return fwd.plane <= 512 && bwd.plane <= 512 && strip_bytes(fwd, 2) <= limit &&
           strip_bytes(bwd, 1) + gradient_bytes(bwd) <= limit;
}

int small_conv_forward(axis_device device, const SmallConvShape &s, const float *input, const int64_t ld[4],
                       const float *weight, const float *bias, float *out, float *pooled, uint8_t *argmax) {
    SmallConvArgs a;
    if (int st = make_args(s, input, ld, weight, bias, 64, a)) return st;
    a.out = out;
    a.pooled = pooled;
    a.argmax = argmax;
    a.wide = (a.n & 1) == 0 && (pooled ? (reinterpret_cast<uintptr_t>(pooled) & 7) == 0 &&
                                              (reinterpret_cast<uintptr_t>(argmax) & 1) == 0
                                        : (reinterpret_cast<uintptr_t>(out) & 7) == 0);
    TimedLaunch timed(device, "gemm", 2.0 * (double)s.batch * s.out_h * s.out_w * s.out_channels * a.k);
    return pooled ? launch_forward<true>(device, a) : launch_forward<false>(device, a);
}

int small_conv_pool_backward_weight(axis_device device, const SmallConvShape &s, const float *input,
                                    const int64_t ld[4], const float *gradient, const float *pooled,
                                    const uint8_t *argmax, float *d_weight, float *d_bias) {
    SmallConvArgs a;
    if (int st = make_args(s, input, ld, nullptr, nullptr, 32, a)) return st;
    a.vec = (a.n & 3) == 0 && aligned16(gradient) && aligned16(pooled) &&
            (reinterpret_cast<uintptr_t>(argmax) & 3) == 0;
    const unsigned columns = (unsigned)((a.n + 63) / 64);
    const unsigned blocks = persistent_blocks(device, a.bands, columns);
    Scratch partial;
    if (int st = partial.get(device, sizeof(float) * (size_t)blocks * 32 * (size_t)a.n)) return st;
    const size_t lds = strip_bytes(a, 1) + gradient_bytes(a);
    {
        TimedLaunch timed(device, "gemm", 2.0 * (double)s.batch * s.out_h * s.out_w * s.out_channels * a.k);
        small_conv_pool_wgrad_kernel<<<dim3(blocks, columns), 256, lds, device->stream>>>(a, gradient, pooled, argmax,
                                                                                          partial.as<float>());
        if (int st = launch_status("small_conv_pool_wgrad_kernel")) return st;
    }
    // d_weight[t][n] (t < k) and d_bias[n] (t = k) = the sum over blocks of partial[block][t][n]
    const int64_t outputs = (int64_t)(a.k + (d_bias ? 1 : 0)) * a.n;
    return column_block_sum(device, partial, blocks, outputs, 32 * (int64_t)a.n, (int64_t)a.k * a.n, d_weight,
                            d_bias);
}

}  // namespace axis
