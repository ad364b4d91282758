// bf16 matrix-core product of the dense matmul family on a bf16 device (interface and the
// reference kernels it stands for: gemm_bf16.hpp).
//
// Staging: each operand becomes bf16 rows [b][t][kp], reduction index contiguous, so every
// MFMA operand (eight consecutive reduction elements of one row) is one 16-byte LDS read and
// every global read of the product kernel a 16-byte row chunk.  Operands already contiguous
// along the reduction are rounded in place order; those contiguous along t go through a 64 x 64
// LDS transpose so both the fp32 reads and the bf16 writes stay coalesced.
//
// Product: WM x WN waves per BM x BN tile (2 x 2 for 128 x 128 and 64 x 64, two blocks per CU;
// 2 x 4 waves of 128 x 64 for 256 x 256, one block per CU), 64-deep LDS stages of both operands in
// two LDS buffers; the next stage streams straight into the idle buffer (buffer_load ... lds)
// while the current one feeds v_mfma_f32_16x16x32_bf16, then one wait and one barrier per stage.
// The 256 x 256 tile halves the operand bytes per product of two 128 x 128 blocks (the stage
// loads of a CU: 64 KB per 2048 MFMA cycles instead of 64 KB per 1024).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "bf16.hpp"
#include "gemm_bf16.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t bf16_bits(float x) { return __builtin_bit_cast(uint32_t, bf16_round(x)) >> 16; }

// One thread per 8-element chunk of a staged row; reads along r (coalesced when s_r == 1).
// VEC: s_r == 1 with 16-byte aligned rows, so a chunk inside k is two 16-byte reads.
template <bool VEC>
__global__ void stage_rows_kernel(axis::Bf16Source s, int64_t rows, int64_t k, int64_t kp, int64_t total,
                                  uint16_t *dst) {
    const int64_t chunks = kp / 8;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t c8 = idx % chunks;
        const int64_t row = idx / chunks;  // b * rows + t
        const int64_t b = row / rows, t = row - b * rows;
        const float *src = s.base + b * s.s_b + t * s.s_t;
        uint32_t h[8];
        if (VEC && c8 * 8 + 8 <= k) {
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(src + c8 * 8);
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(src + c8 * 8 + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                h[j] = bf16_bits(lo[j]);
                h[j + 4] = bf16_bits(hi[j]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t r = c8 * 8 + j;
                h[j] = r < k ? bf16_bits(src[r * s.s_r]) : 0u;
            }
        }
        const u32x4 v = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
        *reinterpret_cast<u32x4 *>(dst + row * kp + c8 * 8) = v;
    }
}

// Operands contiguous along t (s_t == 1): block (tt, rt, b) moves the 64 x 64 tile at
// t0 = 64 tt, r0 = 64 rt through LDS; reads run along t, writes along r.  VEC (16-byte aligned
// base and batch / reduction strides): a lane reads four consecutive t of one r as one 16-byte
// load (4 loads per lane and tile instead of 16).
template <bool VEC>
__global__ void __launch_bounds__(256) stage_transpose_kernel(axis::Bf16Source s, int64_t batch, int64_t rows,
                                                              int64_t k, int64_t kp, uint16_t *dst) {
    constexpr int PITCH = 66;  // bf16 per LDS row: 2-byte stores of 64 consecutive rows hit distinct banks
    __shared__ uint16_t tile[64 * PITCH];
    const int tid = threadIdx.x;
    const int64_t t0 = (int64_t)blockIdx.x * 64;
    const int tl = tid & 63;
    const int64_t t = t0 + tl;
    // Reduction tiles and batches past the grid's y / z extents are walked by the same block.
    for (int64_t b = blockIdx.z; b < batch; b += gridDim.z) {
        const float *src = s.base + b * s.s_b;
        for (int64_t r0 = (int64_t)blockIdx.y * 64; r0 < kp; r0 += (int64_t)gridDim.y * 64) {
            if constexpr (VEC) {
                const int tq = tid & 15;  // t quad of the tile
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int rl = e * 16 + (tid >> 4);
                    const int64_t r = r0 + rl;
                    const int64_t tb = t0 + 4 * tq;
                    floatx4 v = {0.f, 0.f, 0.f, 0.f};
                    if (r < k) {
                        if (tb + 4 <= rows) {
                            v = *reinterpret_cast<const floatx4 *>(src + tb + r * s.s_r);
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                if (tb + j < rows) v[j] = src[tb + j + r * s.s_r];
                        }
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        tile[(4 * tq + j) * PITCH + rl] = (uint16_t)(r < k && tb + j < rows ? bf16_bits(v[j]) : 0u);
                }
            } else {
#pragma unroll 4
                for (int e = 0; e < 16; ++e) {
                    const int rl = e * 4 + (tid >> 6);
                    const int64_t r = r0 + rl;
                    tile[tl * PITCH + rl] = (uint16_t)(t < rows && r < k ? bf16_bits(src[t * s.s_t + r * s.s_r]) : 0u);
                }
            }
            __syncthreads();
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int idx = tid + e * 256;
                const int row = idx >> 3, ch = idx & 7;
                if (t0 + row >= rows) continue;
                const uint32_t *q = reinterpret_cast<const uint32_t *>(tile + row * PITCH + ch * 8);
                const u32x4 v = {q[0], q[1], q[2], q[3]};
                *reinterpret_cast<u32x4 *>(dst + (b * rows + t0 + row) * kp + r0 + ch * 8) = v;
            }
            __syncthreads();  // the tile is rewritten by the next reduction tile
        }
    }
}

// Buffer loads: an offset at or past the resource's record count reads as zero (rows past the
// end of the operand).
constexpr uint32_t kOutside = 0x80000000u;

__device__ __forceinline__ const uint16_t *uniform_ptr(const uint16_t *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint16_t *>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t *base) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
}

// LDS layout of one operand's stage of depth BK: row t (BK reduction elements, unpadded) at
// t * BK, its 16-byte chunk c at chunk position c ^ Layout<BK>::swizzle(t).  With these swizzles
// an MFMA operand read (16 consecutive rows, one chunk) meets no bank conflict
// (SQ_LDS_BANK_CONFLICT reads 0, against 2.7 cycles per LDS instruction for 64-deep rows at a
// 144-byte padded pitch).  A swizzle depends on t % 16 only, so the rows 16 i apart
// that one lane reads share it.
template <int BK>
struct Layout {
    static constexpr int chunks = BK / 8;
    static __device__ __forceinline__ constexpr int swizzle(int t) { return BK == 64 ? t & 7 : (t >> 1) & 3; }
    static __device__ __forceinline__ constexpr int at(int t, int c) { return t * BK + ((c ^ swizzle(t)) << 3); }
};

struct KernelArgs {
    axis::Bf16Gemm g;
    int32_t tiles_m, tiles_n;
    uint32_t xcd_span;  // blocks / 8: the first 8 * xcd_span blocks are remapped, the rest keep their order
};

// + bias[col], then beta * d + alpha * v, each product and the sum rounded separately.
__device__ __forceinline__ float finish(const float *bias, const float *d, float alpha, float beta, float v,
                                        int64_t idx, int64_t col) {
#pragma clang fp contract(off)
    if (bias) v = v + bias[col];
    if (d) {
        const float t1 = beta * d[idx];
        const float t2 = alpha * v;
        v = t1 + t2;
    }
    return v;
}

// Rows [t0, t0 + BT) of a staged operand, one 64-deep stage, loaded straight into LDS: one
// buffer_load ... lds moves 16 bytes per lane to the wave's M0 base + 16 * lane (checked on the
// device), with no registers or LDS store instructions in between.  Instruction q of a stage fills
// rows 8q..8q+7 (1 KB); lane i writes row 8q + i/8 at chunk position i % 8, so it loads that row's
// chunk (i % 8) ^ ((i / 8) & 7), the swizzled layout above.  Rows past the operand's end read
// out of range; they only reach output rows or columns that are never stored.
template <int BT, int NW>
struct DirectLoader {
    static_assert(axis::kBf16Depth == 64, "eight 16-byte chunks per staged row");
    static constexpr int CH = BT * 64 / 8 / (64 * NW);  // instructions per wave and stage (NW waves)
    static_assert(CH * 64 * NW * 8 == BT * 64, "the block's waves split the stage's rows evenly");
    uint32_t off[CH];
    const uint16_t *base;
    int wave;
    __device__ __forceinline__ void init(const uint16_t *b, int64_t t0, int64_t rows, int64_t kp, int tid) {
        base = uniform_ptr(b + t0 * kp);
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int i = tid & 63;
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int q = e * NW + wave;
            const int row = 8 * q + (i >> 3);
            const int c = (i & 7) ^ ((i >> 3) & 7);
            off[e] = t0 + row < rows ? (uint32_t)((row * kp + c * 8) * 2) : kOutside;
        }
    }
    __device__ __forceinline__ void load(int64_t r0, uint16_t *stage) const {
        const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(uniform_ptr(base + r0));
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int q = e * NW + wave;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc, (__attribute__((address_space(3))) void *)(stage + q * 512), 16, off[e], 0, 0, 0);
        }
    }
};

// Logical tile -> (row panel, column panel): groups of 8 row panels, column-major inside a group,
// so consecutive tiles (one XCD's resident blocks) cover a compact patch and share panels in L2.
__device__ __forceinline__ void grouped_tile(uint32_t tile, uint32_t tiles_m, uint32_t tiles_n, uint32_t &ti,
                                             uint32_t &tj) {
    const uint32_t per_group = 8u * tiles_n;
    const uint32_t group = tile / per_group;
    const uint32_t first = group * 8u;
    const uint32_t height = tiles_m - first < 8u ? tiles_m - first : 8u;
    const uint32_t in = tile - group * per_group;
    ti = first + in % height;
    tj = in / height;
}

template <int BM, int BN, int BK, int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64, WM * WN == 8 ? 1 : 2) bf16_gemm_kernel(KernelArgs a) {
    static_assert(axis::kBf16Depth % BK == 0 && BK % 32 == 0, "stages tile the staged depth");
    using Lay = Layout<BK>;
    constexpr int LDK = BK;  // bf16 per LDS row
    constexpr int NW = WM * WN, TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
    constexpr int kBuf = (BM + BN) * LDK;  // one stage of both operands
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kBuf];
    const axis::Bf16Gemm &g = a.g;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int quad = lane >> 4, l16 = lane & 15;

    // XCD-aware order: block L takes logical tile (L % 8) * (blocks / 8) + L / 8, so each XCD's
    // L2 serves a contiguous range of tiles (the last blocks % 8 blocks keep their own order).
    const uint32_t tiles = (uint32_t)a.tiles_m * (uint32_t)a.tiles_n;
    const uint32_t L = blockIdx.x;
    const uint32_t logical = L < 8u * a.xcd_span ? (L % 8u) * a.xcd_span + L / 8u : L;
    const uint32_t tile = logical % tiles;
    const uint32_t slice = logical / tiles;
    uint32_t ti, tj;
    grouped_tile(tile, (uint32_t)a.tiles_m, (uint32_t)a.tiles_n, ti, tj);
    const int64_t i0 = (int64_t)ti * BM;
    const int64_t j0 = (int64_t)tj * BN;
    const int split = (int)(slice % (uint32_t)g.splits);
    const int64_t batch = slice / (uint32_t)g.splits;
    const int64_t r_begin = (int64_t)split * g.k_chunk;
    const int64_t r_end = r_begin + g.k_chunk < g.kp ? r_begin + g.k_chunk : g.kp;
    const int stages = (int)((r_end - r_begin) / BK);  // the host splits in whole stages

    floatx4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    using LX = DirectLoader<BM, NW>;
    using LY = DirectLoader<BN, NW>;
    LX lx;
    LY ly;
    lx.init(g.x + batch * g.x_batch, i0, g.m, g.kp, tid);
    ly.init(g.y + batch * g.y_batch, j0, g.n, g.kp, tid);
    if (stages > 0) {
        lx.load(r_begin, lds);
        ly.load(r_begin, lds + BM * LDK);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // v_mfma_f32_16x16x32_bf16: lane l supplies row l % 16 of A and column l % 16 of B at
    // reduction elements 8 * (l / 16) .. + 7; result register v is row 4 * (l / 16) + v,
    // column l % 16.  Block i of a wave covers its rows 16 i .. 16 i + 15, block j its columns.
    // operand offsets of the lane's chunk for each 32-deep part h of a stage (chunk 4 h + quad)
    constexpr int KS = BK / 32;
    int xa[KS], yb[KS];
#pragma unroll
    for (int h = 0; h < KS; ++h) {
        xa[h] = Lay::at(wm * TM + l16, 4 * h + quad);
        yb[h] = BM * LDK + Lay::at(wn * TN + l16, 4 * h + quad);
    }
    auto compute = [&](const uint16_t *buf) {
        bf16x8 av[2][FM], bv[2][FN];
        auto read_operands = [&](int kk, bf16x8 *avk, bf16x8 *bvk) {
            const int h = kk / 32;
#pragma unroll
            for (int i = 0; i < FM; ++i) avk[i] = *reinterpret_cast<const bf16x8 *>(buf + xa[h] + 16 * i * LDK);
#pragma unroll
            for (int j = 0; j < FN; ++j) bvk[j] = *reinterpret_cast<const bf16x8 *>(buf + yb[h] + 16 * j * LDK);
        };
        read_operands(0, av[0], bv[0]);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            const int cur = (kk / 32) & 1;
            if (kk + 32 < BK) read_operands(kk + 32, av[cur ^ 1], bv[cur ^ 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[cur][i], bv[cur][j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Stage s: stage s + 1 streams into the other buffer (whose stage s - 1 every wave finished
    // before the last barrier) while stage s is computed; then its loads are waited for and one
    // barrier makes it visible to every wave.
    auto step = [&](int s, auto parity) {
        constexpr int P = decltype(parity)::value;
        const int64_t r0 = r_begin + (int64_t)s * BK;
        if (s + 1 < stages) {
            lx.load(r0 + BK, lds + (P ^ 1) * kBuf);
            ly.load(r0 + BK, lds + (P ^ 1) * kBuf + BM * LDK);
        }
        compute(lds + P * kBuf);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    for (int s = 0; s < stages; s += 2) {
        step(s, std::integral_constant<int, 0>{});
        if (s + 1 < stages) step(s + 1, std::integral_constant<int, 1>{});
    }

    // acc[i][j][v]: tile row wm*TM + 16 i + 4 quad + v, column wn*TN + 16 j + l16.  Bias and
    // axpby apply to whole sums only; a split reduction's slices are finished by its sum.
    float *c = g.c + batch * g.c_batch + (int64_t)split * g.c_split;
    const bool whole = g.splits == 1;
    const float *bias = whole ? g.bias : nullptr;
    const float *d = whole ? g.d : nullptr;
    const int64_t out_base = batch * g.m * g.n;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t col = j0 + wn * TN + 16 * j + l16;
        if (col >= g.n) continue;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t row = i0 + wm * TM + 16 * i + 4 * quad + v;
                if (row < g.m)
                    c[row * g.n + col] =
                        finish(bias, d, g.alpha, g.beta, acc[i][j][v], out_base + row * g.n + col, col);
            }
    }
}

}  // namespace

namespace axis {

int stage_bf16(axis_device device, const Bf16Source &src, int64_t batch, int64_t rows, int64_t k, int64_t kp,
               uint16_t *dst) {
    if (kp % kBf16Depth != 0 || kp < k) return fail(AXIS_ERROR_INVALID, "bf16 staging depth must cover k in whole stages");
    if (src.s_t == 1 && src.s_r != 1) {
        if (rows > (int64_t)64 * INT32_MAX) return fail(AXIS_ERROR_INVALID, "bf16 staging grid too large");
        dim3 grid((unsigned)((rows + 63) / 64), (unsigned)std::min<int64_t>(kp / 64, 65535),
                  (unsigned)std::min<int64_t>(batch, 65535));
        if (aligned16(src.base) && src.s_r % 4 == 0 && src.s_b % 4 == 0)
            stage_transpose_kernel<true><<<grid, 256, 0, device->stream>>>(src, batch, rows, k, kp, dst);
        else
            stage_transpose_kernel<false><<<grid, 256, 0, device->stream>>>(src, batch, rows, k, kp, dst);
        return launch_status("stage_transpose_kernel");
    }
    const int64_t total = batch * rows * (kp / 8);
    const bool vec = src.s_r == 1 && aligned16(src.base) && src.s_t % 4 == 0 && src.s_b % 4 == 0;
    if (vec)
        stage_rows_kernel<true><<<blocks_for(total, 256, 1 << 16), 256, 0, device->stream>>>(src, rows, k, kp, total, dst);
    else
        stage_rows_kernel<false><<<blocks_for(total, 256, 1 << 16), 256, 0, device->stream>>>(src, rows, k, kp, total, dst);
    return launch_status("stage_rows_kernel");
}

Bf16Tile bf16_gemm_tile(int64_t m, int64_t n, int64_t batch, int64_t kp, int64_t cus) {
    // 256 x 256 tiles when they alone fill the chip (one per CU) and cover the output with at most
    // 1/8 of their rows and columns past its edges (a batch of small products keeps the smaller
    // tiles): 4096^3 data and weight gradients 870 / 852 -> 919 / 907 TFLOP/s, staging included.
    // (Their 32-bit row offsets reach 257 * kp * 2 bytes: longer reductions keep 128 x 128.)
    const int64_t pm = (m + 255) / 256 * 256, pn = (n + 255) / 256 * 256;
    if ((pm / 256) * (pn / 256) * batch >= cus && 8 * m * n >= 7 * pm * pn &&
        (int64_t)257 * kp * 2 < (int64_t(1) << 31))
        return Bf16Tile{256, 256};
    // (A 256 x 128 tile of 32-deep stages, 128 x 64 per wave, measured no faster.)  A reduction
    // long enough to split keeps the 128 x 128 tile and fills the chip with slices instead: the
    // skinny 784 x 1024 x 8192 weight gradient runs 15% faster that way than on 64 x 64 tiles.
    const int64_t large = ((m + 127) / 128) * ((n + 127) / 128) * batch;
    return large * 2 >= cus || kp >= 8 * kBf16Depth ? Bf16Tile{128, 128} : Bf16Tile{64, 64};
}

bool bf16_gemm_fits(int64_t m, int64_t n, int64_t batch, int64_t kp, int64_t cus) {
    const Bf16Tile tile = bf16_gemm_tile(m, n, batch, kp, cus);
    const int64_t tiles = ((m + tile.rows - 1) / tile.rows) * ((n + tile.cols - 1) / tile.cols) * batch;
    return (int64_t)(std::max(tile.rows, tile.cols) + 1) * kp * 2 < (int64_t(1) << 31) &&
           std::max<int64_t>(tiles, cus * 2) < INT32_MAX;
}

int bf16_gemm(axis_device device, const Bf16Gemm &g, int64_t batch, Bf16Tile tile) {
    KernelArgs a{};
    a.g = g;
    a.tiles_m = (int32_t)((g.m + tile.rows - 1) / tile.rows);
    a.tiles_n = (int32_t)((g.n + tile.cols - 1) / tile.cols);
    const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n * batch * g.splits;
    if (blocks >= INT32_MAX) return fail(AXIS_ERROR_INVALID, "matmul too large for one launch");
    // 32-bit byte offsets inside one tile's rows: (tile rows + 1) * kp * 2 bytes
    if ((int64_t)(std::max(tile.rows, tile.cols) + 1) * g.kp * 2 >= (int64_t(1) << 31))
        return fail(AXIS_ERROR_INVALID, "bf16 matmul reduction too long");
    a.xcd_span = (uint32_t)(blocks / 8);
    dim3 grid((unsigned)blocks);
    if (tile.rows == 256)
        bf16_gemm_kernel<256, 256, 64, 2, 4><<<grid, 512, 0, device->stream>>>(a);
    else if (tile.rows == 128)
        bf16_gemm_kernel<128, 128, 64, 2, 2><<<grid, 256, 0, device->stream>>>(a);
    else
        bf16_gemm_kernel<64, 64, 64, 2, 2><<<grid, 256, 0, device->stream>>>(a);
    return launch_status("bf16_gemm_kernel");
}

}  // namespace axis
