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

typedef float floatx2 __attribute__((ext_vector_type(2)));
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

// ---------------------------------------------------------------------------------------------
// Fixed-geometry instances.  For the usual first layer (1 or 3 channels under a 3x3 kernel, images
// whose windows span at least 25 columns, whole 64-column groups of outputs) the patch shape and the
// band shape (32 window columns) are compile-time constants, so that:
// * the next band's input cells stream straight into a second LDS buffer (buffer_load ... lds, one
//   4-byte cell per lane; cells outside the image are loads past the resource's record count and
//   land as 0), with no prefetch registers and no LDS store pass;
// * every LDS operand read is a base register plus an immediate offset;
// * the forward's max pool runs on the bit patterns of the pre-activations (a signed integer
//   compare orders positive floats like the float compare and puts every negative value, -0 and
//   negative NaN below +0), with one check per tile for +inf or positive NaN, which take the exact
//   scan instead;
// * the weight gradient selects each MFMA operand from the band's pooled gradient, pooled values
//   and winner bytes in registers (g at the window's winner when the pooled value is positive,
//   else 0) instead of expanding the pre-activation gradient in LDS.
// Both instances make the same MFMA calls in the same order as the generic kernels above.

constexpr uint32_t kOutside = 0x80000000u;  // a buffer offset past the record count: loads 0, stores drop

__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
    return reinterpret_cast<T *>(uniform_u64(reinterpret_cast<uint64_t>(p)));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
}

typedef __attribute__((address_space(3))) void *lds_void;
typedef __attribute__((address_space(3))) float lds_float;

// C channels under a KH x KW kernel; bands of BR x 32 windows.  Staged rows are SW cells apart and
// planes PP cells apart (both at least the band's extent), chosen per kernel so that one operand
// read of a wave meets no LDS bank conflict.
template <int C, int KH, int KW, int BR, int SW_, int PP>
struct Fixed {
    static constexpr int BS = 32;                     // window columns per band
    static constexpr int WIDTH = 2 * BS + KW - 1;     // staged columns
    static constexpr int SW = SW_;                    // row pitch
    static constexpr int SH = 2 * BR + KH - 1;        // staged rows
    static constexpr int CELLS = SW * SH;             // cells of a plane, row padding included
    static constexpr int CHUNKS = (CELLS + 63) / 64;  // 64-cell wave loads per plane
    static constexpr int PLANE = PP;                  // plane pitch
    static constexpr int K = C * KH * KW;             // patch terms; term K is the bias
    static constexpr int LOADS = C * CHUNKS;          // wave loads per band
    static constexpr int SLOTS = (LOADS + 3) / 4;     // wave loads per wave
    static constexpr int XBUF = (C + 1) * PLANE;      // input planes and the ones plane
    static_assert(SW >= WIDTH && PLANE >= 64 * CHUNKS, "pitches cover the band");
    // LDS offset of patch term k = (c, ky, kx) from its pixel's cell; terms from K on read the
    // ones plane
    static constexpr int off(int k) {
        return k >= K ? C * PLANE : (k / (KH * KW)) * PLANE + (k % (KH * KW)) / KW * SW + k % KW;
    }
};

// The staging of a band's input planes: wave load q = wave + 4 s moves cells 64 (q % CHUNKS) ..
// + 63 of plane q / CHUNKS (lane i: cell 64 (q % CHUNKS) + i), so each wave load fills 256
// consecutive LDS bytes; the row padding (columns WIDTH .. SW - 1) loads 0.  A cell's offset from
// the band's corner is fixed; its row and column are recomputed per band (a multiply-shift by the
// constant row pitch) for the image-bounds test.
template <class F>
struct StripStream {
    uint32_t rel[F::SLOTS];  // byte offset of the cell from the band's corner (row 0, column 0)
    int wave, lane;

    __device__ __forceinline__ void init(const SmallConvArgs &a, int tid) {
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        lane = tid & 63;
#pragma unroll
        for (int s = 0; s < F::SLOTS; ++s) {
            const int q = wave + 4 * s;
            const int t = 64 * (q % F::CHUNKS) + lane;
            const int r = t / F::SW, c = t - r * F::SW;
            rel[s] = (uint32_t)((r * a.ld_h + c * a.ld_w + q / F::CHUNKS * a.ld_c) * 4);
        }
    }

    __device__ __forceinline__ void load(const SmallConvArgs &a, const Band &b, float *buf) const {
        const int32_t iy0 = 2 * b.wr0 - a.py, ix0 = 2 * b.wc0 - a.px;
        const __amdgpu_buffer_rsrc_t rsrc = rsrc_of(uniform_ptr(a.x + (int64_t)b.img * a.ld_b));
        const int32_t corner = (iy0 * a.ld_h + ix0 * a.ld_w) * 4;  // negative inside the padding
#pragma unroll
        for (int s = 0; s < F::SLOTS; ++s) {
            const int q = wave + 4 * s;
            if (q < F::LOADS) {
                const uint32_t t = 64u * (uint32_t)(q % F::CHUNKS) + (uint32_t)lane;
                const uint32_t r = t / F::SW, c = t - r * F::SW;
                const bool in = t < (uint32_t)F::CELLS && c < (uint32_t)F::WIDTH &&
                                (uint32_t)(iy0 + (int32_t)r) < (uint32_t)a.height &&
                                (uint32_t)(ix0 + (int32_t)c) < (uint32_t)a.width;
                const uint32_t off = in ? (uint32_t)corner + rel[s] : kOutside;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rsrc, (lds_void)(buf + q / F::CHUNKS * F::PLANE + 64 * (q % F::CHUNKS)), 4, off, 0, 0, 0);
            }
        }
    }
};

// Term pairs (2j, 2j + 1) of the forward's k-pairs: the lane half that reads term 2j + 1 reads it
// delta[j] cells past term 2j.  Lanes keep one base register per distinct delta: pair j reads
// through the base of pair first[j], the first pair with the same delta.
template <class F, int KP>
struct PairTable {
    int delta[KP], first[KP];
    constexpr PairTable() : delta{}, first{} {
        for (int j = 0; j < KP; ++j) delta[j] = F::off(2 * j + 1) - F::off(2 * j);
        for (int j = 0; j < KP; ++j) {
            int i = 0;
            while (delta[i] != delta[j]) ++i;
            first[j] = i;
        }
    }
};

// Forward with ReLU + 2x2 max pool (the POOL form of small_conv_forward_kernel) over bands of 2 x 32
// windows: wave w computes tiles (window row 0 and 1, window columns 8w .. 8w + 7) of each band.
template <int C, int KH, int KW>
__global__ void __launch_bounds__(256, 4) small_conv_pool_forward_fixed_kernel(SmallConvArgs a) {
    // rows 80 cells apart (16 banks): a tile's two pixel rows fill the 32 banks of a half-wave read
    using F = Fixed<C, KH, KW, 2, 80, 512>;
    constexpr int KP = (F::K + 2) / 2;  // the K terms and the bias
    constexpr PairTable<F, KP> pairs{};
    __shared__ float lds[2 * F::XBUF];
    const int tid = threadIdx.x, lane = tid & 63;
    const int l32 = lane & 31, half = lane >> 5;
    const int32_t col0 = (int32_t)blockIdx.y * 64;

    // MFMA B operand of k-pair j: W[2j + half][col0 + 2 l32 + b], the bias at term K, 0 past it
    float wreg[KP][2];
#pragma unroll
    for (int j = 0; j < KP; ++j) {
        const int32_t k = 2 * j + half;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int32_t n = col0 + 2 * l32 + b;
            float w = 0.0f;
            if (k < F::K) w = a.w[(int64_t)k * a.n + n];
            if (k == F::K && a.bias != nullptr) w = a.bias[n];
            wreg[j][b] = w;
        }
    }
    for (int32_t t = tid; t < F::PLANE; t += 256) {
        lds[C * F::PLANE + t] = 1.0f;
        lds[F::XBUF + C * F::PLANE + t] = 1.0f;
    }
    StripStream<F> stream;
    stream.init(a, tid);
    const int wave = stream.wave;
    // the lane's pixel cell: window l32 / 4 of the wave's tile, position (l32 / 2 % 2, l32 % 2)
    const int32_t lane_cell = ((l32 >> 1) & 1) * F::SW + 2 * (l32 >> 2) + (l32 & 1) + 16 * wave;
    // pooled element of the lane's first window (2q + half, q = 0) from the tile's first window
    // at column col0
    const int32_t lane_out = half * a.n + 2 * l32;
    const uint32_t bands = (uint32_t)a.bands;

    uint32_t band = blockIdx.x;
    if (band < bands) stream.load(a, decode_band(a, band), lds);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    auto run = [&](uint32_t bnd, auto parity) {
        constexpr int P = decltype(parity)::value;
        const Band bd = decode_band(a, bnd);
        if (bnd + gridDim.x < bands) stream.load(a, decode_band(a, bnd + gridDim.x), lds + (P ^ 1) * F::XBUF);
        const float *px = lds + P * F::XBUF + lane_cell;
        const float *pd[KP];
#pragma unroll
        for (int j = 0; j < KP; ++j)
            if (pairs.first[j] == j) pd[j] = px + (half ? pairs.delta[j] : 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {  // the wave's tile in window row i of the band
            if (bd.wr0 + i >= a.win_rows) break;
            float av[KP];
#pragma unroll
            for (int j = 0; j < KP; ++j) av[j] = pd[pairs.first[j]][2 * i * F::SW + F::off(2 * j)];
            __builtin_amdgcn_sched_barrier(0);
            floatx16 acc[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[0], wreg[0][b], floatx16{}, 0, 0, 0);
#pragma unroll
            for (int j = 1; j < KP; ++j)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j], wreg[j][b], acc[b], 0, 0, 0);
            // Register group q of block b: window 2q + half of the tile, positions 0..3.  The
            // largest bit pattern of each window; +inf or a positive NaN anywhere in the wave's
            // windows sends the tile to the exact scan.
            int32_t top[2][4];
            int32_t most = INT32_MIN;
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int32_t y0 = __float_as_int(acc[b][4 * q]), y1 = __float_as_int(acc[b][4 * q + 1]);
                    const int32_t y2 = __float_as_int(acc[b][4 * q + 2]), y3 = __float_as_int(acc[b][4 * q + 3]);
                    top[b][q] = max(max(max(y0, y1), y2), y3);
                    most = max(most, top[b][q]);
                }
            // pooled values of window pair q (block b: window 2q + half, columns col0 + 2 l32 + b)
            // and their winner bytes; the tile's first window is window row wr0 + i, column
            // wc0 + 8 wave, and `room` windows of the lane's half-row lie inside the image
            const int64_t first =
                (((int64_t)bd.img * a.win_rows + bd.wr0 + i) * a.win_cols + bd.wc0 + 8 * wave) * a.n + col0;
            const int32_t room = a.win_cols - bd.wc0 - 8 * wave - half;
            // streaming (non-temporal) stores: measured 2 us faster per launch than plain ones here
            auto put = [&](int q, const float best[2], const int winner[2]) {
                if (2 * q >= room) return;
                __builtin_nontemporal_store(floatx2{best[0], best[1]},
                                            reinterpret_cast<floatx2 *>(a.pooled + first + 2 * q * a.n + lane_out));
                __builtin_nontemporal_store((uint16_t)(winner[0] | (winner[1] << 8)),
                                            reinterpret_cast<uint16_t *>(a.argmax + first + 2 * q * a.n + lane_out));
            };
            if (__builtin_amdgcn_ballot_w64(most >= 0x7f800000) == 0) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float best[2];
                    int winner[2];
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        const int32_t m = top[b][q];
                        best[b] = __int_as_float(m > 0 ? m : 0);
                        int w = __float_as_int(acc[b][4 * q + 2]) == m ? 2 : 3;
                        w = __float_as_int(acc[b][4 * q + 1]) == m ? 1 : w;
                        winner[b] = (m <= 0 || __float_as_int(acc[b][4 * q]) == m) ? 0 : w;
                    }
                    put(q, best, winner);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float best[2];
                    int winner[2];
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        float y[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) y[e] = acc[b][4 * q + e];
                        relu_pool_window4(y, best[b], winner[b]);
                    }
                    put(q, best, winner);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // the next band's cells have landed
        __syncthreads();                // ... for every wave, and this band's reads are done
    };
    while (band < bands) {
        run(band, std::integral_constant<int, 0>{});
        band += gridDim.x;
        if (band >= bands) break;
        run(band, std::integral_constant<int, 1>{});
        band += gridDim.x;
    }
}

// Weight and bias gradient through ReLU -> 2x2 max pool (small_conv_pool_wgrad_kernel) over bands of
// 1 x 32 windows, for the fixed geometries, through the pool's winners.  Per band the LDS buffer
// holds the gradient and the pooled values [32 windows][64 columns], the winner bytes [32][64] and
// the input planes (streamed in by buffer_load ... lds, double-buffered).  Column n of a window takes
// its gradient at one pixel only -- its winner, when the pooled value is positive -- so the product
// over the window's four pixels is g * x at that pixel plus 0 * x at the other three, and the zeros
// change nothing while x is finite.  A lane per output column gathers its winner pixel's C*KH*KW
// input terms from the staged band (one LDS read each, at compile-time offsets from a per-lane
// base) and adds g * x to each term's sum, and g to the bias's: a quarter of the products, none of
// them padded.  A wave whose windows read a non-finite input value in a band then also adds the
// other three positions' 0 * x, so 0 * inf = NaN reaches the sums as in the dense product.  Wave w
// takes windows 8 w .. 8 w + 7 of each band; the sums run window by window, band by band
// (deterministic).
template <int C, int KH, int KW>
__global__ void __launch_bounds__(256, 3) small_conv_pool_wgrad_gather_kernel(SmallConvArgs a,
                                                                                const float *__restrict__ g,
                                                                                const float *__restrict__ pooled,
                                                                                const uint8_t *__restrict__ argmax,
                                                                                float *__restrict__ partial) {
    using F = Fixed<C, KH, KW, 1, 69, 335>;
    constexpr int W = F::BS;             // windows per band
    constexpr int GP = W * 64;           // floats of the band's gradient (and pooled values)
    constexpr int XO = 2 * GP + W * 16;  // the input planes, after the winner bytes
    constexpr int BUF = XO + C * F::PLANE;
    constexpr int T = F::K;              // input terms per pixel; term T is the bias
    static_assert(2 * BUF >= 4 * (T + 1) * 64, "the four waves' sums fit the buffers");
    // the wave's input region in a band: C planes x SH rows x 18 columns (8 windows and the halo)
    constexpr int RW = 2 * 8 + KW - 1;
    constexpr int REGION = C * F::SH * RW;
    constexpr int CHECKS = (REGION + 63) / 64;
    __shared__ __attribute__((aligned(16))) float lds[2 * BUF];
    const int tid = threadIdx.x, lane = tid & 63;
    const int32_t col0 = (int32_t)blockIdx.y * 64;

    StripStream<F> stream;
    stream.init(a, tid);
    const int wave = stream.wave;
    // Gradient and pooled loads e = wave, wave + 4 (16 bytes per lane): window 4 e + lane / 16,
    // columns col0 + 4 (lane % 16) ..; winner loads e = wave < 2: window 16 e + lane / 4, bytes
    // col0 + 16 (lane % 4) ..
    int32_t gwin[2];
    uint32_t grel[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        gwin[s] = 4 * (wave + 4 * s) + (lane >> 4);
        grel[s] = (uint32_t)((gwin[s] * a.n + col0 + 4 * (lane & 15)) * 4);
    }
    const int32_t awin = 16 * wave + (lane >> 2);
    const uint32_t arel = (uint32_t)(awin * a.n + col0 + 16 * (lane & 3));
    // the lane's cells of the wave's input region (the non-finite test), as offsets in the band
    int32_t check[CHECKS];
#pragma unroll
    for (int i = 0; i < CHECKS; ++i) {
        const int cell = lane + 64 * i < REGION ? lane + 64 * i : 0;
        const int plane = cell / (F::SH * RW), rest = cell % (F::SH * RW);
        check[i] = XO + plane * F::PLANE + (rest / RW) * F::SW + 16 * wave + rest % RW;
    }
    const uint32_t bands = (uint32_t)a.bands;

    auto load = [&](const Band &b, float *buf) {
        const int64_t first = (((int64_t)b.img * a.win_rows + b.wr0) * a.win_cols + b.wc0) * a.n;
        const int32_t room = a.win_cols - b.wc0;  // windows of the band inside the image
        const __amdgpu_buffer_rsrc_t rg = rsrc_of(uniform_ptr(g + first));
        const __amdgpu_buffer_rsrc_t rp = rsrc_of(uniform_ptr(pooled + first));
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint32_t off = gwin[s] < room ? grel[s] : kOutside;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void)(buf + 256 * (wave + 4 * s)), 16, off, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (lds_void)(buf + GP + 256 * (wave + 4 * s)), 16, off, 0, 0,
                                                     0);
        }
        if (wave < 2) {
            const __amdgpu_buffer_rsrc_t ra = rsrc_of(uniform_ptr(argmax + first));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void)(buf + 2 * GP + 256 * wave), 16,
                                                     awin < room ? arel : kOutside, 0, 0, 0);
        }
        stream.load(a, b, buf + XO);
    };

    float acc[T + 1];
#pragma unroll
    for (int t = 0; t <= T; ++t) acc[t] = 0.0f;

    uint32_t band = blockIdx.x;
    if (band < bands) load(decode_band(a, band), lds);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // one body for both buffers (the buffer a runtime offset): the sums stay in the same registers
    auto run = [&](uint32_t bnd, int P) {
        if (bnd + gridDim.x < bands) load(decode_band(a, bnd + gridDim.x), lds + (P ^ 1) * BUF);
        const float *buf = lds + P * BUF;
        bool bad = false;
#pragma unroll
        for (int i = 0; i < CHECKS; ++i)
            if (lane + 64 * i < REGION) bad |= !(__builtin_fabsf(buf[check[i]]) <= FLT_MAX);
        // the wave's window j: its gradient where its winner takes it (else 0) and the winner
        auto window = [&](int j, float &ge, uint32_t &key) {
            const int w = 8 * wave + j;
            const float gv = buf[w * 64 + lane];
            const float pv = buf[GP + w * 64 + lane];
            key = reinterpret_cast<const uint8_t *>(buf + 2 * GP)[w * 64 + lane];
            const bool take = pv > 0.0f && key < 4u;
            ge = take ? gv : 0.0f;
            key = take ? key : 0u;
        };
        // the winner's offset from the window's first pixel, (key / 2) * SW + key % 2, as byte key
        // of a packed table
        static_assert(F::SW + 1 < 256, "winner offsets fit a byte");
        constexpr uint32_t kWinnerOffsets = 0u | (1u << 8) | ((uint32_t)F::SW << 16) | ((uint32_t)(F::SW + 1) << 24);
        float ge_next;
        uint32_t key_next;
        window(0, ge_next, key_next);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float ge = ge_next;
            const uint32_t key = key_next;
            if (j + 1 < 8) window(j + 1, ge_next, key_next);  // the next window's operands ahead
            // one ds_read_b32 per term at a compile-time offset from the lane's base (read through
            // volatile so they are not paired into ds_read2, whose 8-bit offsets would take an
            // address add per pair)
            const uint32_t at = __builtin_amdgcn_ubfe(kWinnerOffsets, 8 * key, 8);
            const volatile lds_float *xp = (const volatile lds_float *)(buf + XO + 2 * (8 * wave + j) + at);
            float xv[T];
#pragma unroll
            for (int t = 0; t < T; ++t) xv[t] = xp[F::off(t)];
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = __builtin_fmaf(ge, xv[t], acc[t]);
            acc[T] = acc[T] + ge;
        }
        if (__builtin_amdgcn_ballot_w64(bad) != 0) {
            // a non-finite input in the wave's windows: the other three positions' 0 * x as well
#pragma unroll 1
            for (int j = 0; j < 8; ++j) {
                float ge;
                uint32_t key;
                window(j, ge, key);
#pragma unroll 1
                for (int p = 0; p < 4; ++p) {
                    // the winner's own term is in already (g * x, which is not 0 * x for infinite x)
                    if ((uint32_t)p == key) continue;
                    const float *xp = buf + XO + 2 * (8 * wave + j) + (p >> 1) * F::SW + (p & 1);
#pragma unroll
                    for (int t = 0; t < T; ++t) acc[t] = __builtin_fmaf(0.0f, xp[F::off(t)], acc[t]);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // the next band has landed
        __syncthreads();                // ... for every wave, and this band's reads are done
    };
    for (int P = 0; band < bands; band += gridDim.x, P ^= 1) run(band, P);

    // The four waves' sums meet in LDS ([wave][term][64 columns]) and are added in wave order.
    float *const red = lds;
#pragma unroll
    for (int t = 0; t <= T; ++t) red[(wave * (T + 1) + t) * 64 + lane] = acc[t];
    __syncthreads();
    float *dst = partial + (int64_t)blockIdx.x * 32 * a.n;
    constexpr int SUMS = (T + 1) * 64;
    for (int32_t e = tid; e < SUMS; e += 256) {
        const int32_t t = e >> 6, col = col0 + (e & 63);
        const float sum = ((red[e] + red[SUMS + e]) + red[2 * SUMS + e]) + red[3 * SUMS + e];
        dst[(int64_t)t * a.n + col] = sum;
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

unsigned persistent_blocks(axis_device device, int64_t bands, int64_t columns, int per_cu = 4) {
    const int64_t slots = (int64_t)device->multiprocessors * per_cu / (columns > 0 ? columns : 1);
    int64_t per = (bands + (slots > 0 ? slots : 1) - 1) / (slots > 0 ? slots : 1);
    if (per < 1) per = 1;
    return (unsigned)((bands + per - 1) / per);
}

// The fixed-geometry instances: a 3x3 kernel over 1 or 3 channels, bands of `rows` x 32 windows,
// whole 64-column groups, and every input cell's byte offset (and the band corners') within 31 bits.
bool fixed_applies(const SmallConvArgs &a, int32_t rows) {
    if (a.kh != 3 || a.kw != 3 || (a.c_in != 1 && a.c_in != 3)) return false;
    if (a.band_s != 32 || a.band_r != rows || a.n % 64 != 0) return false;
    if (a.ld_h < 0 || a.ld_w < 0 || a.ld_c < 0) return false;
    const int64_t reach = ((int64_t)a.height + 8) * a.ld_h + ((int64_t)a.width + 72) * a.ld_w + (int64_t)a.c_in * a.ld_c;
    return reach * 4 < ((int64_t)1 << 31);
}

template <int C>
int launch_pool_forward_fixed(axis_device device, const SmallConvArgs &a, dim3 grid) {
    small_conv_pool_forward_fixed_kernel<C, 3, 3><<<grid, 256, 0, device->stream>>>(a);
    return axis::launch_status("small_conv_pool_forward_fixed_kernel");
}

template <bool POOL>
int launch_forward(axis_device device, const SmallConvArgs &a) {
    const int kp = (a.k + 2) / 2;  // the k terms and the bias term
    const unsigned columns = (unsigned)((a.n + 63) / 64);
    dim3 grid(persistent_blocks(device, a.bands, columns), columns);
    if (POOL && a.wide && fixed_applies(a, 2))
        return a.c_in == 3 ? launch_pool_forward_fixed<3>(device, a, grid) : launch_pool_forward_fixed<1>(device, a, grid);
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
    const bool fixed = a.vec && aligned16(argmax) && fixed_applies(a, 1);
    const unsigned blocks = persistent_blocks(device, a.bands, columns, fixed ? 3 : 4);
    Scratch partial;
    if (int st = partial.get(device, sizeof(float) * (size_t)blocks * 32 * (size_t)a.n)) return st;
    const size_t lds = strip_bytes(a, 1) + gradient_bytes(a);
    {
        TimedLaunch timed(device, "gemm", 2.0 * (double)s.batch * s.out_h * s.out_w * s.out_channels * a.k);
        const dim3 grid(blocks, columns);
        if (fixed && a.c_in == 3) {
            small_conv_pool_wgrad_gather_kernel<3, 3, 3><<<grid, 256, 0, device->stream>>>(a, gradient, pooled, argmax,
                                                                                             partial.as<float>());
        } else if (fixed) {
            small_conv_pool_wgrad_gather_kernel<1, 3, 3><<<grid, 256, 0, device->stream>>>(a, gradient, pooled, argmax,
                                                                                             partial.as<float>());
        } else {
            small_conv_pool_wgrad_kernel<<<grid, 256, lds, device->stream>>>(a, gradient, pooled, argmax,
                                                                              partial.as<float>());
        }
        if (int st = launch_status("small_conv_pool_wgrad_kernel")) return st;
    }
    // d_weight[t][n] (t < k) and d_bias[n] (t = k) = the sum over blocks of partial[block][t][n]
    const int64_t outputs = (int64_t)(a.k + (d_bias ? 1 : 0)) * a.n;
    return column_block_sum(device, partial, blocks, outputs, 32 * (int64_t)a.n, (int64_t)a.k * a.n, d_weight,
                            d_bias);
}

}  // namespace axis
