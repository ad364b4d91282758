// fp32 GEMM family on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32) for the reference's
// matmul / matmul_left_backward / matmul_right_backward (runtime/backend.rs:934-1021,
// kernels :2190-2290).
//
// One kernel template computes C[i][j] = sum_r X(i,r) Y(r,j) for a batch of row-major C,
// with each operand either contiguous along the reduction (r) or along its output dimension:
//   matmul      : X = a [m,k] (r-contiguous),        Y = b [k,n] (j-contiguous)
//   left_bwd    : X = gradient [m,n] (r-contiguous), Y = rhs [k,n] read as rhs^T (r-contiguous)
//   right_bwd   : X = lhs [m,k] read as lhs^T (i-contiguous), Y = gradient [m,n] (j-contiguous)
// Tiles are staged through LDS as [r][i] / [r][j] so every MFMA operand read is a unit-stride
// LDS access across the wave.  The next K tile is prefetched into registers while the current
// one feeds the MFMAs.  When the output has too few tiles to fill 256 CUs, the reduction is
// split into slices whose partial tiles are summed afterwards in slice order (deterministic,
// no atomics).
#include <algorithm>

#include "common.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

struct GemmParams {
    const float *x;
    const float *y;
    float *c;
    int64_t m, n, k;           // C is [m, n]; reduction length k
    int64_t x_si, x_sr;        // X(i, r) = x[i * x_si + r * x_sr]
    int64_t y_sr, y_sj;        // Y(r, j) = y[r * y_sr + j * y_sj]
    int64_t x_batch, y_batch;  // batch strides (elements)
    int64_t c_batch;           // batch stride of the output (or of one slice of partials)
    int64_t c_split;           // stride between reduction slices in the output (partials)
    int64_t k_chunk;           // reduction length per slice (multiple of the tile depth)
    int32_t splits;
    int32_t tiles_m, tiles_n;
};

// Stage one BK x BT tile of an operand into registers.  OUTER is the operand's output-dimension
// extent (m for X, n for Y).  RCONTIG: the operand is contiguous along r.
template <int BT, int BK, int NT, bool RCONTIG, int VEC>
struct TileLoader {
    static constexpr int kElems = BT * BK / NT;  // floats per thread
    static constexpr int kVecs = kElems / VEC;
    static constexpr int LD = RCONTIG ? BT + 2 : BT + 4;  // LDS row pitch ([r][t] layout)

    float reg[kElems];

    // s_t: stride along the output dimension; s_r: stride along r.
    __device__ __forceinline__ void load(const float *__restrict__ base, int64_t s_t, int64_t s_r,
                                         int64_t t0, int64_t r0, int64_t t_end, int64_t r_end,
                                         int tid) {
#pragma unroll
        for (int e = 0; e < kVecs; ++e) {
            int idx = tid + e * NT;
            int tt, rr;
            if (RCONTIG) {
                constexpr int per = BK / VEC;
                rr = (idx % per) * VEC;
                tt = idx / per;
            } else {
                constexpr int per = BT / VEC;
                tt = (idx % per) * VEC;
                rr = idx / per;
            }
            int64_t gt = t0 + tt, gr = r0 + rr;
            bool valid = gt < t_end && gr < r_end;
            if (VEC == 4) {
                floatx4 v = {0.f, 0.f, 0.f, 0.f};
                if (valid) v = *reinterpret_cast<const floatx4 *>(base + gt * s_t + gr * s_r);
                reg[e * 4 + 0] = v[0];
                reg[e * 4 + 1] = v[1];
                reg[e * 4 + 2] = v[2];
                reg[e * 4 + 3] = v[3];
            } else {
                reg[e] = valid ? base[gt * s_t + gr * s_r] : 0.f;
            }
        }
    }

    __device__ __forceinline__ void store(float *__restrict__ lds, int tid) const {
#pragma unroll
        for (int e = 0; e < kVecs; ++e) {
            int idx = tid + e * NT;
            if (RCONTIG) {
                constexpr int per = BK / VEC;
                int rr = (idx % per) * VEC;
                int tt = idx / per;
#pragma unroll
                for (int c = 0; c < VEC; ++c) lds[(rr + c) * LD + tt] = reg[e * VEC + c];
            } else {
                constexpr int per = BT / VEC;
                int tt = (idx % per) * VEC;
                int rr = idx / per;
                if (VEC == 4) {
                    floatx4 v = {reg[e * 4 + 0], reg[e * 4 + 1], reg[e * 4 + 2], reg[e * 4 + 3]};
                    *reinterpret_cast<floatx4 *>(lds + rr * LD + tt) = v;
                } else {
                    lds[rr * LD + tt] = reg[e];
                }
            }
        }
    }
};

template <int BM, int BN, int BK, int WM, int WN, bool XR, bool YR, int VX, int VY>
__global__ void __launch_bounds__(WM *WN * 64)
    gemm_kernel(GemmParams p) {
    constexpr int NT = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    using LX = TileLoader<BM, BK, NT, XR, VX>;
    using LY = TileLoader<BN, BK, NT, YR, VY>;
    __shared__ float xs[BK * LX::LD];
    __shared__ float ys[BK * LY::LD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;

    const int tile = blockIdx.x;
    const int64_t i0 = (int64_t)(tile % p.tiles_m) * BM;
    const int64_t j0 = (int64_t)(tile / p.tiles_m) * BN;
    const int split = blockIdx.y % p.splits;
    const int64_t batch = blockIdx.y / p.splits;
    const int64_t r_begin = (int64_t)split * p.k_chunk;
    const int64_t r_end = r_begin + p.k_chunk < p.k ? r_begin + p.k_chunk : p.k;

    const float *x = p.x + batch * p.x_batch;
    const float *y = p.y + batch * p.y_batch;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

    LX lx;
    LY ly;
    if (r_begin < r_end) {
        lx.load(x, p.x_si, p.x_sr, i0, r_begin, p.m, r_end, tid);
        ly.load(y, p.y_sj, p.y_sr, j0, r_begin, p.n, r_end, tid);
        lx.store(xs, tid);
        ly.store(ys, tid);
    }
    __syncthreads();

    const int half = lane >> 5;  // which k of the pair this lane feeds
    const int l32 = lane & 31;
    for (int64_t r0 = r_begin; r0 < r_end; r0 += BK) {
        const bool more = r0 + BK < r_end;
        if (more) {
            lx.load(x, p.x_si, p.x_sr, i0, r0 + BK, p.m, r_end, tid);
            ly.load(y, p.y_sj, p.y_sr, j0, r0 + BK, p.n, r_end, tid);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float av[FM], bv[FN];
#pragma unroll
            for (int a = 0; a < FM; ++a) av[a] = xs[(kk + half) * LX::LD + wm * TM + a * 32 + l32];
#pragma unroll
            for (int b = 0; b < FN; ++b) bv[b] = ys[(kk + half) * LY::LD + wn * TN + b * 32 + l32];
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int b = 0; b < FN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
        if (more) {
            lx.store(xs, tid);
            ly.store(ys, tid);
            __syncthreads();
        }
    }

    // Accumulator layout of the 32x32 block: lane -> column l32; register v -> row
    // 8*(v/4) + 4*(lane/32) + (v%4).
    float *c = p.c + batch * p.c_batch + (int64_t)split * p.c_split;
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) {
            const int64_t col = j0 + wn * TN + b * 32 + l32;
            if (col >= p.n) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t row = i0 + wm * TM + a * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
                if (row < p.m) c[row * p.n + col] = acc[a][b][v];
            }
        }
}

// Sum of reduction slices: lane group g (of 4) adds slices g, g+4, g+8, ... in order, then the
// four group sums are added in group order -- a fixed association for a given slice count, so
// the result is deterministic and independent of scheduling.
__global__ void __launch_bounds__(256) split_sum_kernel(const float *__restrict__ partial,
                                                        float *__restrict__ out, int64_t len,
                                                        int32_t splits, int64_t split_stride) {
    __shared__ float acc[4][64];
    const int lane = threadIdx.x & 63, group = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (i < len)
        for (int32_t k = group; k < splits; k += 4) s += partial[k * split_stride + i];
    acc[group][lane] = s;
    __syncthreads();
    if (group == 0 && i < len) out[i] = ((acc[0][lane] + acc[1][lane]) + acc[2][lane]) + acc[3][lane];
}

template <int BM, int BN, int BK, int WM, int WN, bool XR, bool YR, int VX, int VY>
void launch_config(const GemmParams &p, dim3 grid, hipStream_t stream) {
    gemm_kernel<BM, BN, BK, WM, WN, XR, YR, VX, VY><<<grid, WM * WN * 64, 0, stream>>>(p);
}

template <int BM, int BN, int BK, int WM, int WN, bool XR, bool YR>
void launch_vec(const GemmParams &p, dim3 grid, hipStream_t stream, bool vx, bool vy) {
    if (vx && vy)
        launch_config<BM, BN, BK, WM, WN, XR, YR, 4, 4>(p, grid, stream);
    else if (vx)
        launch_config<BM, BN, BK, WM, WN, XR, YR, 4, 1>(p, grid, stream);
    else if (vy)
        launch_config<BM, BN, BK, WM, WN, XR, YR, 1, 4>(p, grid, stream);
    else
        launch_config<BM, BN, BK, WM, WN, XR, YR, 1, 1>(p, grid, stream);
}

// Vector loads need the contiguous extent, the other stride and the base to be 4-aligned.
bool vec_ok(const float *base, int64_t contiguous_extent, int64_t other_stride) {
    return axis::aligned16(base) && contiguous_extent % 4 == 0 && other_stride % 4 == 0;
}

template <bool XR, bool YR>
int run_gemm(axis_device device, GemmParams p, int64_t batch, float *out) {
    const int64_t cus = device->multiprocessors;
    // Large tiles whenever both output extents fill them; a reduction split restores the block
    // count when the output alone has too few tiles.  Large tiles run 32 deep per LDS stage.
    const bool big = p.m >= 128 && p.n >= 128;
    const int BK = big ? 32 : 16;
    const int bm = big ? 128 : 64, bn = big ? 128 : 64;
    p.tiles_m = static_cast<int32_t>((p.m + bm - 1) / bm);
    p.tiles_n = static_cast<int32_t>((p.n + bn - 1) / bn);
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n * batch;
    // Split the reduction when the tiles alone cannot fill the chip.
    int64_t splits = 1;
    if (tiles < 2 * cus && p.k >= 8 * BK) {
        splits = std::min<int64_t>((4 * cus + tiles - 1) / tiles, 2 * cus);
        splits = std::min<int64_t>(splits, p.k / (BK * 4));
        splits = std::max<int64_t>(splits, 1);
    }
    int64_t chunk = (p.k + splits - 1) / splits;
    chunk = (chunk + BK - 1) / BK * BK;
    if (chunk < BK) chunk = BK;
    splits = (p.k + chunk - 1) / chunk;
    if (splits < 1) splits = 1;
    p.k_chunk = chunk;
    p.splits = static_cast<int32_t>(splits);

    const bool vx = XR ? vec_ok(p.x, p.k, p.x_si) && p.x_batch % 4 == 0
                       : vec_ok(p.x, p.m, p.x_sr) && p.x_batch % 4 == 0;
    const bool vy = YR ? vec_ok(p.y, p.k, p.y_sj) && p.y_batch % 4 == 0
                       : vec_ok(p.y, p.n, p.y_sr) && p.y_batch % 4 == 0;

    axis::Scratch partial;
    const int64_t out_len = batch * p.m * p.n;
    if (splits > 1) {
        int status = partial.get(device, sizeof(float) * (size_t)(out_len * splits));
        if (status) return status;
        p.c = partial.as<float>();
        p.c_split = out_len;
        p.c_batch = p.m * p.n;
    } else {
        p.c = out;
        p.c_split = 0;
        p.c_batch = p.m * p.n;
    }
    if (batch * splits > 65535)
        return axis::fail(AXIS_ERROR_INVALID, "matmul batch too large for one launch");
    axis::TimedLaunch timed(device, "gemm", 2.0 * (double)batch * (double)p.m * (double)p.n * (double)p.k);
    dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n), static_cast<unsigned>(batch * splits));
    if (big)
        launch_vec<128, 128, 32, 2, 2, XR, YR>(p, grid, device->stream, vx, vy);
    else
        launch_vec<64, 64, 16, 2, 2, XR, YR>(p, grid, device->stream, vx, vy);
    int status = axis::launch_status("gemm_kernel");
    if (status) return status;
    if (splits > 1) {
        split_sum_kernel<<<axis::blocks_for(out_len, 64, INT32_MAX), 256, 0, device->stream>>>(
            partial.as<float>(), out, out_len, static_cast<int32_t>(splits), out_len);
        status = axis::launch_status("split_sum_kernel");
    }
    return status;
}

int check_dims(const void *a, const void *b, const void *out, int64_t batch, int64_t m, int64_t k,
               int64_t n) {
    AXIS_REQUIRE(a && b && out, "null matmul operand");
    AXIS_REQUIRE(batch >= 1 && m >= 1 && k >= 1 && n >= 1, "matmul extents must be positive");
    AXIS_REQUIRE(batch * m * k < (int64_t(1) << 40) && batch * m * n < (int64_t(1) << 40) &&
                     batch * k * n < (int64_t(1) << 40),
                 "matmul operand too large");
    AXIS_REQUIRE(m < (int64_t(1) << 31) / 2 && n < (int64_t(1) << 31) / 2,
                 "matmul output extent too large for one launch");
    return AXIS_OK;
}

}  // namespace

extern "C" {

int axis_matmul(axis_device device, const float *a, const float *b, float *out, int64_t batch,
                int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    if (int s = check_dims(a, b, out, batch, m, k, n)) return s;
    GemmParams p{};
    p.x = a;
    p.y = b;
    p.m = m;
    p.n = n;
    p.k = k;
    p.x_si = k;
    p.x_sr = 1;
    p.y_sr = n;
    p.y_sj = 1;
    p.x_batch = m * k;
    p.y_batch = k * n;
    return run_gemm<true, false>(device, p, batch, out);
}

int axis_matmul_left_backward(axis_device device, const float *gradient, const float *rhs,
                              float *out, int64_t batch, int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    if (int s = check_dims(gradient, rhs, out, batch, m, k, n)) return s;
    // out [m, k] = gradient [m, n] . rhs[k, n]^T : i = m, j = k, r = n.
    GemmParams p{};
    p.x = gradient;
    p.y = rhs;
    p.m = m;
    p.n = k;
    p.k = n;
    p.x_si = n;
    p.x_sr = 1;
    p.y_sr = 1;
    p.y_sj = n;
    p.x_batch = m * n;
    p.y_batch = k * n;
    return run_gemm<true, true>(device, p, batch, out);
}

int axis_matmul_right_backward(axis_device device, const float *lhs, const float *gradient,
                               float *out, int64_t batch, int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    if (int s = check_dims(lhs, gradient, out, batch, m, k, n)) return s;
    // out [k, n] = lhs[m, k]^T . gradient [m, n] : i = k, j = n, r = m.
    GemmParams p{};
    p.x = lhs;
    p.y = gradient;
    p.m = k;
    p.n = n;
    p.k = m;
    p.x_si = 1;
    p.x_sr = k;
    p.y_sr = n;
    p.y_sj = 1;
    p.x_batch = m * k;
    p.y_batch = m * n;
    return run_gemm<false, false>(device, p, batch, out);
}

}  // extern "C"
