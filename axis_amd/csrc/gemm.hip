// fp32 GEMM family on CDNA4 matrix cores (v_mfma_f32_16x16x4_f32) for the reference's
// matmul / matmul_left_backward / matmul_right_backward (runtime/backend.rs:934-1021,
// kernels :2190-2290), and implicit-GEMM convolution entries that compute the reference's
// unfold -> contract (forward), contract-backward -> unfold_backward (dgrad) and
// unfold -> contract-backward (wgrad) without materialising the patch matrix.
//
// One kernel template computes C[i][j] = sum_r X(i,r) Y(r,j) for a batch of row-major C.
// Dense operands are contiguous along the reduction (r) or along their output dimension:
//   matmul      : X = a [m,k] (r-contiguous),        Y = b [k,n] (j-contiguous)
//   left_bwd    : X = gradient [m,n] (r-contiguous), Y = rhs [k,n] read as rhs^T (r-contiguous)
//   right_bwd   : X = lhs [m,k] read as lhs^T (i-contiguous), Y = gradient [m,n] (j-contiguous)
// Convolution X operands gather from a channel-innermost tensor [batch, h, w, c]:
//   rows mode   : X(i = output pixel, r = (ky*kw + kx)*c + channel)   (forward, dgrad)
//   cols mode   : X(i = (ky*kw + kx)*c + channel, r = output pixel)   (wgrad)
// with zero outside the padded input.  Reordering the reduction as (ky, kx, channel) makes every
// gathered vector contiguous in memory when channels are innermost; the weights are permuted to
// match (a few KB).  Any other input layout (e.g. channel-major [batch, c, h, w]) is gathered
// element by element through its strides.
//
// The forward can end in a fused epilogue: bias, ReLU and a non-overlapping max pool over whole
// windows, with the pool's window-local winner emitted as a byte.  The tile is staged in LDS so
// every window is complete inside one block; the pre-activation never reaches HBM.
//
// Tiles are staged through LDS as [r][i] / [r][j] so every MFMA operand read is a unit-stride
// LDS access across the wave.  The next K tile is prefetched into registers while the current
// one feeds the MFMAs, and the last two k-quads of each stage are held in registers across the
// stage barriers.  MFMA and vector instructions do not overlap on this part (one wave of each on
// a SIMD takes the sum of their times), so the K loop keeps vector work to a few instructions
// per step.  When the output has too few tiles to fill 256 CUs, the reduction is split into
// slices whose partial tiles are summed afterwards in a fixed order (deterministic, no atomics).
#include <algorithm>
#include <cfloat>
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "common.hpp"
#include "bf16.hpp"
#include "conv_small.hpp"
#include "fastdiv.hpp"
#include "gemm_bf16.hpp"
#include "pool_rule.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Split partial sums of the allocation-free weight gradient (axis_matmul_right_backward_noalloc).
// One copy per GPU, alive until the process ends.  Host code never passes this name to a kernel:
// it is a host-side stand-in, and kernels take the device address hipGetSymbolAddress returns
// (axis_device_s::static_scratch).  The split rules of run_gemm keep a launch's partial slices
// within 64 MiB; one whose slices and range sums would not fit here is rejected before it runs.
constexpr int64_t kStaticScratchFloats = int64_t(16) << 20;  // 64 MiB
static __device__ __align__(256) float scratch[kStaticScratchFloats];

// Device memory a caller hands to run_gemm in place of allocations (split partials, then the
// range sums of more than 32 slices).
struct Workspace {
    float *ptr;
    int64_t floats;
};

// Geometry of a gathered convolution operand (tensor [batch, height, width, channels]).
struct ConvGeom {
    const float *src;
    int64_t ld_b;                     // element strides of batch, channel, row, column
    int32_t ld_c, ld_h, ld_w;
    int32_t height, width, channels;  // gathered tensor
    int32_t out_h, out_w;             // output pixel grid the reduction/rows enumerate
    int32_t kh, kw, sy, sx, py, px;
    FastDiv c_div, kw_div, ow_div, oh_div;
    bool tap_steps;                   // channels % 32 == 0: a 32-deep K step stays in one tap
    // With tap steps, the buffer rows loader walks the reduction in 32-channel blocks, every tap
    // of a block before the next block: r = (cb * taps + pos) * 32 + ci.  A tile then re-reads
    // the same 32 channels of its neighbourhood on consecutive steps, which stay in L2, instead
    // of the whole tensor slab between one tap and the next.
    bool block_major;
    FastDiv taps_div;                 // kh * kw
    // Rows mode, 2x2 pooling epilogue: tile row t holds position t % 4 (ky major) of the tile's
    // window t / 4, windows numbered row-major over the tile's window rows (pw per row).  A tile
    // starts on an even output row and holds whole window rows.
    bool window_major;
    FastDiv pw_div;
};

// Output pixel of tile row t for a tile starting at pixel t0.
__device__ __forceinline__ int64_t tile_pixel(const ConvGeom &g, int64_t t0, int t) {
    if (!g.window_major) return t0 + t;
    const uint32_t w = (uint32_t)t >> 2, pos = (uint32_t)t & 3u;
    const uint32_t wr = g.pw_div.div(w), wc = w - wr * g.pw_div.d;
    return t0 + (int64_t)(2 * wr + (pos >> 1)) * g.out_w + 2 * wc + (pos & 1u);
}

// Second operand read straight from a convolution weight in the reference's [(c, ky, kx), n]
// layout: the reduction index is r = pos * R + q (pos = ky * kw + kx, R rows per tap, R a
// multiple of the K step), and a K step starting at r0 = pos * R + q0 begins at element
// q0 * qa + pos * pb + pc, its rows s_r apart.
struct TapSteps {
    bool on;
    FastDiv r_div;   // R
    int64_t qa, pb, pc;
    // The rows loader's block-major order: step r0 = (cb * taps + pos) * 32 covers q0 = 32 cb.
    bool block_major;
    FastDiv taps_div;
};

struct GemmParams {
    const float *x;
    const float *y;
    float *c;
    const float *bias;         // added to every row of C (length n), or null
    const float *d;            // out = beta * d + alpha * (A.B) when non-null (d shaped like out)
    float alpha, beta;
    int64_t m, n, k;           // C is [m, n]; reduction length k
    int64_t x_si, x_sr;        // dense X(i, r) = x[i * x_si + r * x_sr]
    int64_t y_sr, y_sj;        // Y(r, j) = y[r * y_sr + j * y_sj]
    int64_t x_batch, y_batch;  // batch strides (elements)
    int64_t c_batch;           // batch stride of the output (or of one slice of partials)
    int64_t c_split;           // stride between reduction slices in the output (partials)
    int64_t k_chunk;           // reduction length per slice (multiple of the tile depth)
    int64_t k_work;            // algorithmic reduction length for timing (k without padding), or 0
    int32_t splits;
    int32_t tiles_m, tiles_n;
    uint32_t xcd_span;         // blocks / 8: the first 8 * xcd_span blocks are remapped, the rest keep their order
    ConvGeom conv;
    // Pooling epilogue: output rows are pixels of a [.., out_h, out_w] grid (out_w = pool_ow).
    float *pooled;
    uint8_t *argmax;
    int32_t pool_h, pool_w, pool_ow;
    FastDiv pool_cols;         // pooled columns per output row (pool_ow / pool_w)
    TapSteps ytaps;            // Y read as a tap-major convolution weight
    // Output rows ordered (pos, c) with perm_c channels and perm_taps taps are written as rows
    // c * perm_taps + pos (the reference's weight layout); 0 = rows as computed.
    int32_t perm_c, perm_taps;
    bool bf16;                 // operands rounded to bf16 as they are staged (Device::cuda_bf16)
};

template <int VEC>
__device__ __forceinline__ void load_into(float *reg, const float *src, bool valid) {
    if constexpr (VEC == 4) {
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (valid) v = *reinterpret_cast<const floatx4 *>(src);
        reg[0] = v[0];
        reg[1] = v[1];
        reg[2] = v[2];
        reg[3] = v[3];
    } else {
        reg[0] = valid ? src[0] : 0.f;
    }
}

// Buffer loads: an offset at or past the resource's record count (2^31 - 1 bytes) reads as zero,
// so padding taps and reduction tails need neither a branch nor zeroed registers.
constexpr uint32_t kOutside = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, int32_t bytes = 0x7fffffff) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, bytes, 0x00020000);
}
template <int VEC>
__device__ __forceinline__ void buffer_into(float *reg, __amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
    if constexpr (VEC == 4) {
        const floatx4 v = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_offset, 0, 0));
        reg[0] = v[0];
        reg[1] = v[1];
        reg[2] = v[2];
        reg[3] = v[3];
    } else {
        reg[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, byte_offset, 0, 0));
    }
}

// LDS staging shared by every loader: [r][t] layout, row pitch BT + 4 (16-byte aligned rows),
// and column t of row r stored at t ^ swizzle(r) with swizzle(r) = 8 * ((r / 4) % 8).  The XOR
// moves whole aligned groups of 8 columns, so the MFMA operand reads (4 or 2 consecutive columns
// of one row per lane) stay single 16- or 8-byte reads, and one k-quad (4 rows) shares one
// swizzle.  It spreads the transposing stores of r-contiguous operands (a lane writes rows
// 4j..4j+3 of one column) over distinct banks.
// Tiles 32 wide (the folded products) permute inside their 32 columns: swizzle(r) = 8 * ((r / 4) % 4).
template <int BT>
__device__ __forceinline__ constexpr int stage_swizzle(int r) {
    return 8 * ((r >> 2) & (BT >= 64 ? 7 : 3));
}

template <int BT, int BK, int NT, bool RCONTIG, int VEC>
struct Staging {
    static_assert(BT % 64 == 0 || BT == 32, "the swizzle permutes columns inside aligned groups of 64 (or 32)");
    static constexpr int kElems = BT * BK / NT;  // floats per thread
    static constexpr int kVecs = kElems / VEC;
    // Row pitch: t-contiguous operands BT + 4 (their 16-byte stores along t spread over the banks
    // by the padding); r-contiguous ones BT + 64, a multiple of 64 words, so the four rows a lane
    // writes sit 3 x 256 bytes apart and two ds_write2st64 reach them from one address register
    // (the XOR swizzle alone keeps those stores and the operand reads free of bank conflicts).
    // 32-wide tiles (the folded products' four stages share one CU's LDS): BT + 4 for both.
    static constexpr int LD = RCONTIG && BT >= 64 ? BT + 64 : BT + 4;
    static constexpr int kPer = RCONTIG ? BK / VEC : BT / VEC;  // vectors per contiguous line
    float reg[kElems];

    // bf16: round every staged operand to bf16 first (products of bf16 values are exact in fp32).
    __device__ __forceinline__ void store(float *__restrict__ lds, int tid, int bf16 = 0) {
        if (bf16) {
#pragma unroll
            for (int e = 0; e < kElems; ++e) reg[e] = bf16_round(reg[e]);
        }
#pragma unroll
        for (int e = 0; e < kVecs; ++e) {
            const int idx = tid + e * NT;
            if (RCONTIG) {
                const int rr = (idx % kPer) * VEC;
                const int tt = idx / kPer;
#pragma unroll
                for (int c = 0; c < VEC; ++c) lds[(rr + c) * LD + (tt ^ stage_swizzle<BT>(rr + c))] = reg[e * VEC + c];
            } else {
                const int tt = (idx % kPer) * VEC;
                const int rr = idx / kPer;
                if (VEC == 4) {
                    floatx4 v = {reg[e * 4 + 0], reg[e * 4 + 1], reg[e * 4 + 2], reg[e * 4 + 3]};
                    *reinterpret_cast<floatx4 *>(lds + rr * LD + (tt ^ stage_swizzle<BT>(rr))) = v;
                } else {
                    lds[rr * LD + (tt ^ stage_swizzle<BT>(rr))] = reg[e];
                }
            }
        }
    }
};

// A wave-uniform pointer moved to scalar registers, so that buffer resources built from it need no
// per-lane loop (the compiler cannot always prove such values uniform).
__device__ __forceinline__ const float *uniform_ptr(const float *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const float *>(((uint64_t)hi << 32) | lo);
}

// Dense operand: element (t, r) at base[t * s_t + r * s_r], read through buffer loads.  One buffer
// resource per K step, based at the tile's element (t0, step) (wave-uniform: a 64-bit scalar add and
// the descriptor words), and one 32-bit element offset per lane and vector inside the tile, fixed at
// init.  The host keeps those offsets below 2^29 elements (127 * s_t + 31 * s_r, strides
// nonnegative).
template <int BT, int BK, int NT, bool RCONTIG, int VEC>
struct DenseLoader : Staging<BT, BK, NT, RCONTIG, VEC> {
    using S = Staging<BT, BK, NT, RCONTIG, VEC>;
    const float *tile_base;        // element (t0, 0) (wave-uniform)
    uint32_t voff[S::kVecs];       // this lane's byte offset from (t0, r0) per vector; kOutside past the end
    int32_t r_wave[S::kVecs];      // r of each vector's first lane inside the tile (wave-uniform)
    int32_t r_lane;                // this lane's r from its vector's first lane
    int64_t s_r;
    TapSteps taps{};               // tap-major steps (convolution weights), if on

    static __device__ __forceinline__ void split(int idx, int &tt, int &r) {
        if (RCONTIG) {
            r = (idx % S::kPer) * VEC;
            tt = idx / S::kPer;
        } else {
            tt = (idx % S::kPer) * VEC;
            r = idx / S::kPer;
        }
    }
    __device__ __forceinline__ void init(const float *b, int64_t st, int64_t sr, int64_t t0,
                                         int64_t t_end, int tid) {
        s_r = sr;
        // 64 and NT are multiples of kPer, or kPer of 64: a lane adds split(lane) to its vector's
        // first lane with no carry between the two fields.
        static_assert(64 % S::kPer == 0 || S::kPer % 64 == 0, "lane split must not carry");
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        int t_l, r_l;
        split(tid & 63, t_l, r_l);
        r_lane = r_l;
        tile_base = uniform_ptr(b + t0 * st);
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            int t_w, r_w;
            split(wave * 64 + e * NT, t_w, r_w);
            r_wave[e] = r_w;
            voff[e] = t0 + t_w + t_l < t_end ? (uint32_t)((t_w + t_l) * st + (r_w + r_l) * sr) * 4u : kOutside;
        }
    }
    // room: k of this step inside the reduction (1..BK); WHOLE: every step of the launch is whole
    template <bool WHOLE = false>
    __device__ __forceinline__ void load(const ConvGeom &, int64_t r0, int32_t room, int) {
        int64_t step = r0 * s_r;
        if (taps.on) {
            uint32_t pos;
            int64_t q0;
            if (taps.block_major) {
                const uint32_t st = (uint32_t)r0 >> 5;
                const uint32_t cb = taps.taps_div.div(st);
                pos = st - cb * taps.taps_div.d;
                q0 = (int64_t)cb * 32;
            } else {
                pos = taps.r_div.div((uint32_t)r0);
                q0 = r0 - (int64_t)pos * taps.r_div.d;
            }
            step = q0 * taps.qa + (int64_t)pos * taps.pb + taps.pc;
        }
        if constexpr (RCONTIG) {
            const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(uniform_ptr(tile_base + step));
            // Branch-free: split into whole-step and partial-step paths, the loads' wait counts
            // merge conservatively and the next loads wait on this step's.  room - r_wave is
            // scalar work, and every vector shares the one compare.
#pragma unroll
            for (int e = 0; e < S::kVecs; ++e)
                buffer_into<VEC>(this->reg + e * VEC, rsrc, WHOLE || r_lane < room - r_wave[e] ? voff[e] : kOutside);
        } else {
            // t-contiguous rows (s_t = 1 and rows no longer than their pitch, which the host
            // checks): a row past the step's depth starts at or after byte room * s_r * 4 of the
            // step, so the resource's record count masks it with no vector instruction.
            const int32_t bytes = WHOLE || room >= BK ? 0x7fffffff : (int32_t)(room * s_r * 4);
            const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(uniform_ptr(tile_base + step), bytes);
#pragma unroll
            for (int e = 0; e < S::kVecs; ++e) buffer_into<VEC>(this->reg + e * VEC, rsrc, voff[e]);
        }
    }
};

// Convolution operand, rows mode: t = output pixel, r = (ky*kw + kx)*channels + channel.
// Per row: the offset of its window origin and the origin's coordinates (for the padding test);
// per K step: one decode of the thread's r into a 32-bit offset shared by every row.
template <int BT, int BK, int NT, int VEC>
struct ConvRowsLoader : Staging<BT, BK, NT, true, VEC> {
    using S = Staging<BT, BK, NT, true, VEC>;
    uint32_t origin[S::kVecs];   // b*ld_b + iy0*ld_h + ix0*ld_w (mod 2^32; exact when valid)
    int32_t iy0[S::kVecs], ix0[S::kVecs];
    int rr;

    __device__ __forceinline__ void init(const ConvGeom &geom, int64_t t0, int64_t t_end, int tid) {
        rr = (tid % S::kPer) * VEC;  // NT is a multiple of kPer, so rr is the same for every e
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            const int64_t gt = tile_pixel(geom, t0, (tid + e * NT) / S::kPer);
            // Rows past the end get an origin far outside the image, so every tap is padding;
            // computed branch-free so the per-row arrays stay in registers.
            const bool live = gt < t_end;
            const uint32_t pix = live ? (uint32_t)gt : 0u;
            const uint32_t q = geom.ow_div.div(pix);
            const int32_t ox = (int32_t)(pix - q * (uint32_t)geom.out_w);
            const uint32_t b = geom.oh_div.div(q);
            const int32_t oy = (int32_t)(q - b * (uint32_t)geom.out_h);
            const int32_t y0 = oy * geom.sy - geom.py;
            ix0[e] = ox * geom.sx - geom.px;
            origin[e] = b * (uint32_t)geom.ld_b + (uint32_t)y0 * (uint32_t)geom.ld_h +
                        (uint32_t)ix0[e] * (uint32_t)geom.ld_w;
            iy0[e] = live ? y0 : -(1 << 30);
        }
    }
    __device__ __forceinline__ void load(const ConvGeom &geom, int64_t r0, int32_t room, int) {
        const bool r_ok = rr < room;
        const uint32_t g = r_ok ? (uint32_t)(r0 + rr) : 0u;
        const uint32_t pos = geom.c_div.div(g);
        const int32_t c = (int32_t)(g - pos * (uint32_t)geom.channels);
        const int32_t ky = (int32_t)geom.kw_div.div(pos);
        const int32_t kx = (int32_t)pos - ky * geom.kw;
        const uint32_t delta = (uint32_t)(ky * geom.ld_h + kx * geom.ld_w + c * geom.ld_c);
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            const bool valid = r_ok && (uint32_t)(iy0[e] + ky) < (uint32_t)geom.height &&
                               (uint32_t)(ix0[e] + kx) < (uint32_t)geom.width;
            load_into<VEC>(this->reg + e * VEC, geom.src + (valid ? origin[e] + delta : 0u), valid);
        }
    }
};

// Rows mode through buffer loads, for gathered tensors whose offsets fit 31-bit byte offsets and
// kernels of at most 32 taps.  Each row keeps its window origin's offset and a mask of the taps
// that fall outside the image (bit ky*kw + kx), so a K step tests one bit per vector.  When the
// channel count is a multiple of BK (geom.tap_steps), a K step covers BK channels of one tap and
// the step's tap decode is wave-uniform.
template <int BT, int BK, int NT, int VEC>
struct ConvRowsBufferLoader : Staging<BT, BK, NT, true, VEC> {
    using S = Staging<BT, BK, NT, true, VEC>;
    uint32_t origin4[S::kVecs];  // 4 * (b*ld_b + iy0*ld_h + ix0*ld_w) (mod 2^32; exact when valid)
    uint32_t outside[S::kVecs];  // taps of the row's window outside the image (all, for rows past the end)
    int rr;
    uint32_t lane_c4;            // 4 * rr * ld_c: the thread's channel offset inside a tap step, bytes

    __device__ __forceinline__ void init(const ConvGeom &geom, int64_t t0, int64_t t_end, int tid) {
        rr = (tid % S::kPer) * VEC;
        lane_c4 = (uint32_t)(rr * geom.ld_c) * 4u;
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            const int64_t gt = tile_pixel(geom, t0, (tid + e * NT) / S::kPer);
            const bool live = gt < t_end;
            const uint32_t pix = live ? (uint32_t)gt : 0u;
            const uint32_t q = geom.ow_div.div(pix);
            const int32_t ox = (int32_t)(pix - q * (uint32_t)geom.out_w);
            const uint32_t b = geom.oh_div.div(q);
            const int32_t oy = (int32_t)(q - b * (uint32_t)geom.out_h);
            const int32_t y0 = oy * geom.sy - geom.py;
            const int32_t x0 = ox * geom.sx - geom.px;
            origin4[e] = (b * (uint32_t)geom.ld_b + (uint32_t)y0 * (uint32_t)geom.ld_h + (uint32_t)x0 * (uint32_t)geom.ld_w) * 4u;
            uint32_t cols = 0, taps = 0;
            for (int32_t kx = 0; kx < geom.kw; ++kx)
                cols |= (uint32_t)((uint32_t)(x0 + kx) < (uint32_t)geom.width) << kx;
            for (int32_t ky = 0; ky < geom.kh; ++ky)
                taps |= ((uint32_t)(y0 + ky) < (uint32_t)geom.height ? cols : 0u) << (ky * geom.kw);
            outside[e] = live ? ~taps : ~0u;
        }
    }
    __device__ __forceinline__ void load(const ConvGeom &geom, int64_t r0, int32_t room, int) {
        const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(geom.src);
        if (geom.tap_steps) {
            // The reduction is a multiple of BK here, so every k of the step is inside it; the
            // step's tap and first channel are wave-uniform (scalar arithmetic).  Per vector: the
            // offset, and the window's outside bit for this tap moved to bit 31, which puts a
            // masked lane's offset past the record count (three vector instructions).
            uint32_t pos;
            int32_t c0;
            if (geom.block_major) {
                const uint32_t st = (uint32_t)r0 >> 5;
                const uint32_t cb = geom.taps_div.div(st);
                pos = st - cb * geom.taps_div.d;
                c0 = (int32_t)cb * 32;
            } else {
                pos = geom.c_div.div((uint32_t)r0);
                c0 = (int32_t)((uint32_t)r0 - pos * (uint32_t)geom.channels);
            }
            const int32_t ky = (int32_t)geom.kw_div.div(pos);
            const int32_t kx = (int32_t)pos - ky * geom.kw;
            const uint32_t delta4 =
                __builtin_amdgcn_readfirstlane((uint32_t)(ky * geom.ld_h + kx * geom.ld_w + c0 * geom.ld_c) * 4u) +
                lane_c4;
            const uint32_t up = 31u - __builtin_amdgcn_readfirstlane(pos);
#pragma unroll
            for (int e = 0; e < S::kVecs; ++e)
                buffer_into<VEC>(this->reg + e * VEC, rsrc, (origin4[e] + delta4) | ((outside[e] << up) & kOutside));
        } else {
            const bool r_ok = rr < room;
            const uint32_t g = r_ok ? (uint32_t)(r0 + rr) : 0u;
            const uint32_t pos = geom.c_div.div(g);
            const int32_t c = (int32_t)(g - pos * (uint32_t)geom.channels);
            const int32_t ky = (int32_t)geom.kw_div.div(pos);
            const int32_t kx = (int32_t)pos - ky * geom.kw;
            const uint32_t delta4 = (uint32_t)(ky * geom.ld_h + kx * geom.ld_w + c * geom.ld_c) * 4u;
#pragma unroll
            for (int e = 0; e < S::kVecs; ++e) {
                const bool valid = r_ok && ((outside[e] >> pos) & 1u) == 0;
                buffer_into<VEC>(this->reg + e * VEC, rsrc, valid ? origin4[e] + delta4 : kOutside);
            }
        }
    }
};

// Convolution operand, cols mode: t = (ky*kw + kx)*channels + channel, r = output pixel.  The
// thread's t is fixed; each row keeps its pixel's coordinates and offset and walks forward BK
// pixels per K step.
template <int BT, int BK, int NT, int VEC>
struct ConvColsLoader : Staging<BT, BK, NT, false, VEC> {
    using S = Staging<BT, BK, NT, false, VEC>;
    static constexpr int kRowStep = NT / S::kPer;  // pixels between the thread's rows
    uint32_t tap;                // (ky-py)*ld_h + (kx-px)*ld_w + c*ld_c of the thread's t (mod 2^32)
    int32_t ky, kx;
    bool t_ok;
    int32_t ox[S::kVecs], oy[S::kVecs];
    uint32_t off[S::kVecs];      // b*ld_b + oy*sy*ld_h + ox*sx*ld_w (mod 2^32)
    int64_t next_r;              // r0 the state describes

    __device__ __forceinline__ void init(const ConvGeom &geom, int64_t t0, int64_t t_end, int tid) {
        const int64_t gt = t0 + (tid % S::kPer) * VEC;
        t_ok = gt < t_end;
        const uint32_t g = t_ok ? (uint32_t)gt : 0u;
        const uint32_t pos = geom.c_div.div(g);
        const int32_t c = (int32_t)(g - pos * (uint32_t)geom.channels);
        ky = (int32_t)geom.kw_div.div(pos);
        kx = (int32_t)pos - ky * geom.kw;
        tap = (uint32_t)(ky - geom.py) * (uint32_t)geom.ld_h + (uint32_t)(kx - geom.px) * (uint32_t)geom.ld_w +
              (uint32_t)c * (uint32_t)geom.ld_c;
        next_r = -1;
    }
    __device__ __forceinline__ void locate(const ConvGeom &geom, int64_t r0, int tid) {
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            const uint32_t pix = (uint32_t)(r0 + tid / S::kPer + e * kRowStep);
            const uint32_t q = geom.ow_div.div(pix);
            ox[e] = (int32_t)(pix - q * (uint32_t)geom.out_w);
            const uint32_t b = geom.oh_div.div(q);
            oy[e] = (int32_t)(q - b * (uint32_t)geom.out_h);
            off[e] = b * (uint32_t)geom.ld_b + (uint32_t)(oy[e] * geom.sy) * (uint32_t)geom.ld_h +
                     (uint32_t)(ox[e] * geom.sx) * (uint32_t)geom.ld_w;
        }
        next_r = r0;
    }
    __device__ __forceinline__ void advance(const ConvGeom &geom) {
        const uint32_t col_step = (uint32_t)(geom.sx * geom.ld_w), row_step = (uint32_t)(geom.sy * geom.ld_h);
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            ox[e] += BK;
            off[e] += BK * col_step;
            while (ox[e] >= geom.out_w) {
                ox[e] -= geom.out_w;
                off[e] += row_step - (uint32_t)geom.out_w * col_step;
                if (++oy[e] == geom.out_h) {
                    oy[e] = 0;
                    off[e] += (uint32_t)geom.ld_b - (uint32_t)geom.out_h * row_step;
                }
            }
        }
        next_r += BK;
    }
    __device__ __forceinline__ void load(const ConvGeom &geom, int64_t r0, int32_t room, int tid) {
        if (r0 != next_r) locate(geom, r0, tid);
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            const int32_t iy = oy[e] * geom.sy + ky - geom.py, ix = ox[e] * geom.sx + kx - geom.px;
            const bool valid = t_ok && tid / S::kPer + e * kRowStep < room && (uint32_t)iy < (uint32_t)geom.height &&
                               (uint32_t)ix < (uint32_t)geom.width;
            load_into<VEC>(this->reg + e * VEC, geom.src + (valid ? off[e] + tap : 0u), valid);
        }
        advance(geom);
    }
};

// Cols mode when every K step covers whole aligned pixel runs: BK divides the output width or is
// a multiple of it, and the image's pixel count is a multiple of BK.  Then a step starting at
// pixel p0 (a multiple of BK) never leaves one image and the in-step pixel s sits at
// (oy0 + s / out_w, ox0 + s % out_w) for every step, so each vector's window position relative
// to the step origin is fixed at init and a step decodes only its wave-uniform origin.
template <int BT, int BK, int NT, int VEC>
struct ConvColsStepLoader : Staging<BT, BK, NT, false, VEC> {
    using S = Staging<BT, BK, NT, false, VEC>;
    static constexpr int kRowStep = NT / S::kPer;  // pixels between the thread's rows
    static_assert(BK == 32, "steps of 32 pixels");
    uint32_t rel4[S::kVecs];  // bytes: (iy_rel + py)*ld_h + (ix_rel + px)*ld_w + c*ld_c (mod 2^32)
    // Bit (first | last << 1 | top << 2 | bottom << 3) set when the lane's element is padding (or
    // its row past the end) in a step whose pixels start the image's first / last 32-column
    // segment, first / last row group.  A step elsewhere has every element inside (the host
    // keeps px <= 32 sx and py <= (rows per step) sy), so these four flags decide.
    uint32_t bad[S::kVecs];

    __device__ __forceinline__ void init(const ConvGeom &geom, int64_t t0, int64_t t_end, int tid) {
        const int64_t gt = t0 + (tid % S::kPer) * VEC;
        const bool t_ok = gt < t_end;
        const uint32_t g = t_ok ? (uint32_t)gt : 0u;
        const uint32_t pos = geom.c_div.div(g);
        const int32_t c = (int32_t)(g - pos * (uint32_t)geom.channels);
        const int32_t ky = (int32_t)geom.kw_div.div(pos);
        const int32_t kx = (int32_t)pos - ky * geom.kw;
        const int32_t s0 = tid / S::kPer;
        const int32_t seg = geom.out_w < 32 ? geom.out_w : 32;       // columns a step spans
        const int32_t rows = geom.out_w < 32 ? 32 / geom.out_w : 1;  // rows a step spans
        const int32_t last_x = (geom.out_w - seg) * geom.sx, last_y = (geom.out_h - rows) * geom.sy;
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e) {
            const uint32_t s = (uint32_t)(s0 + e * kRowStep);
            const int32_t dy = (int32_t)geom.ow_div.div(s);
            const int32_t dx = (int32_t)s - dy * geom.out_w;
            const int32_t iy_rel = dy * geom.sy + ky - geom.py, ix_rel = dx * geom.sx + kx - geom.px;
            rel4[e] = ((uint32_t)(iy_rel + geom.py) * (uint32_t)geom.ld_h + (uint32_t)(ix_rel + geom.px) * (uint32_t)geom.ld_w +
                       (uint32_t)c * (uint32_t)geom.ld_c) * 4u;
            uint32_t b = 0;
            for (uint32_t f = 0; f < 16; ++f) {
                const bool first = f & 1u, last = f & 2u, top = f & 4u, bottom = f & 8u;
                const int32_t x = first ? ix_rel : last ? last_x + ix_rel : 0;
                const int32_t y = top ? iy_rel : bottom ? last_y + iy_rel : 0;
                const bool in = t_ok && (!(first || last) || (uint32_t)x < (uint32_t)geom.width) &&
                                (!(top || bottom) || (uint32_t)y < (uint32_t)geom.height);
                b |= (in ? 0u : 1u) << f;
            }
            bad[e] = b;
        }
    }
    // Every step is whole: the reduction (batch * image pixels) and the slices are multiples of 32.
    __device__ __forceinline__ void load(const ConvGeom &geom, int64_t r0, int32_t, int) {
        const uint32_t p0 = (uint32_t)r0;
        const uint32_t q = geom.ow_div.div(p0);
        const int32_t ox0 = (int32_t)(p0 - q * (uint32_t)geom.out_w);
        const uint32_t b = geom.oh_div.div(q);
        const int32_t oy0 = (int32_t)(q - b * (uint32_t)geom.out_h);
        const int32_t seg = geom.out_w < 32 ? geom.out_w : 32;
        const int32_t rows = geom.out_w < 32 ? 32 / geom.out_w : 1;
        // sign bits rather than comparisons: compared flags reach vector registers as lane masks
        const uint32_t flags = ((uint32_t)(ox0 - 1) >> 31) | ((uint32_t)(geom.out_w - ox0 - seg - 1) >> 31 << 1) |
                               ((uint32_t)(oy0 - 1) >> 31 << 2) | ((uint32_t)(geom.out_h - oy0 - rows - 1) >> 31 << 3);
        const int32_t oys = oy0 * geom.sy, oxs = ox0 * geom.sx;
        // Buffer base at the step origin moved back by the padding, so that every valid lane's
        // offset (at least -py rows and -px columns from the origin) is non-negative.
        const int64_t shift = (int64_t)geom.py * geom.ld_h + (int64_t)geom.px * geom.ld_w;
        const int64_t base = (int64_t)b * geom.ld_b + (int64_t)oys * geom.ld_h + (int64_t)oxs * geom.ld_w - shift;
        const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(geom.src + base);
        // the padding bit of this step's case moved to bit 31: past the record count (two vector
        // instructions per vector)
#pragma unroll
        for (int e = 0; e < S::kVecs; ++e)
            buffer_into<VEC>(this->reg + e * VEC, rsrc, (((bad[e] >> flags) & 1u) << 31) | rel4[e]);
    }
};

// Finishes one output value v (the whole reduction) at flat output index idx: + bias[col], then
using axis::finish_value;

// XMODE: 0 dense X, 1 convolution rows mode, 2 convolution cols mode, 3 cols mode over aligned
// pixel steps, 4 rows mode through buffer loads.
// EPI: 0 store C (+ bias), 1 bias + ReLU + max pool of whole windows (rows are output pixels).
// Blocks per CU the register budget is held to (two large, three tall or wide, four small tiles).
// tall4: the vectorised data gradient through the gathered convolution loader (128x64 tiles), which
// fits 128 VGPRs without spilling -- four blocks per CU, under which conv2's data gradient runs in
// 302 us against 343 at three (the other tall instances spill at that budget).
constexpr int gemm_blocks_per_cu(int bm, int bn, bool tall4 = false) {
    return bm == 128 && bn == 128 ? 2 : bm == 128 && bn == 64 && tall4 ? 4 : bm == 128 || bn == 128 ? 3 : 4;
}

// WS: waves of the block that split the reduction among them.  1: the WM x WN waves share the
// tile and its K steps.  WS > 1 (WM = WN = 1, EPI 0): wave w computes the whole tile over slice w
// of the launch's p.splits slices (none when w >= p.splits) through its own LDS stage, ordered by
// its own instruction stream (no barrier inside the K loop), and the block adds the WS partial
// tiles in the association of split_sum_part / split_sum_store: the same bits as split slices
// summed by split_sum_kernel, without their partial buffer and second launch.
template <int BM, int BN, int BK, int WM, int WN, bool XR, bool YR, int VX, int VY, int XMODE, int EPI, int WS>
__device__ __forceinline__ void gemm_body(const GemmParams &p) {
    static_assert(WS == 1 || (WS == 4 && WM == 1 && WN == 1 && EPI == 0 && XMODE == 0),
                  "reduction split among waves: one-wave dense tiles, four slices");
    constexpr int NT = WM * WN * 64;  // threads that stage one tile's operands
    static_assert(XMODE != 4 || BK == 32, "the buffer rows loader's tap steps are 32 deep");
    constexpr int TM = BM / WM, TN = BN / WN;
    // 16x16 MFMA blocks per wave side.  Block a of a wave holds the wave's tile rows FM*i + a
    // (i = 0..15) and block b its columns FN*j + b, so for one k a lane's FM (FN) operands are
    // consecutive staged columns: one 16- or 8-byte LDS read.
    constexpr int FM = TM / 16, FN = TN / 16;
    static_assert((FM == 2 || FM == 4) && (FN == 2 || FN == 4), "wave tiles 32 or 64 wide");
    static_assert(EPI == 0 || FM == 4, "the pooling epilogue takes 64-row wave tiles");
    using LX = std::conditional_t<
        XMODE == 0, DenseLoader<BM, BK, NT, XR, VX>,
        std::conditional_t<
            XMODE == 1, ConvRowsLoader<BM, BK, NT, VX>,
            std::conditional_t<XMODE == 2, ConvColsLoader<BM, BK, NT, VX>,
                               std::conditional_t<XMODE == 3, ConvColsStepLoader<BM, BK, NT, VX>,
                                                  ConvRowsBufferLoader<BM, BK, NT, VX>>>>>;
    using LY = DenseLoader<BN, BK, NT, YR, VY>;
    constexpr int kStage = BK * LX::LD + BK * LY::LD;
    constexpr int kPoolPitch = TN + 1;
    constexpr int kEpilogue = EPI == 1 ? BM * kPoolPitch : WS > 1 ? WS * BM * BN : 0;
    constexpr int kStages = WS * kStage;
    __shared__ __attribute__((aligned(16))) float lds[kStages > kEpilogue ? kStages : kEpilogue];
    // the wave's reduction slice inside the block (WS > 1), and its own stage
    const int kw = WS > 1 ? (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
    float *const xs = lds + kw * kStage;
    float *const ys = xs + BK * LX::LD;

    const int tid = WS > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;

    // Workgroups go to the 8 XCDs round-robin in launch order; block L takes logical tile
    // (L % 8) * (blocks / 8) + L / 8 so each XCD (its own L2) works through a contiguous range
    // of tiles: the tiles of one reduction slice, or neighbouring row panels, share its cache.
    // The last blocks % 8 blocks keep their own order.
    const uint32_t tiles = (uint32_t)p.tiles_m * (uint32_t)p.tiles_n;
    const uint32_t L = blockIdx.x;
    const uint32_t logical = L < 8u * p.xcd_span ? (L % 8u) * p.xcd_span + L / 8u : L;
    const uint32_t tile = logical % tiles;
    const uint32_t slice = logical / tiles;  // WS > 1: the batch index (the block holds every slice)
    const int64_t i0 = (int64_t)(tile % (uint32_t)p.tiles_m) * BM;
    const int64_t j0 = (int64_t)(tile / (uint32_t)p.tiles_m) * BN;
    const int split = WS > 1 ? kw : (int)(slice % (uint32_t)p.splits);
    const int64_t batch = WS > 1 ? (int64_t)slice : (int64_t)(slice / (uint32_t)p.splits);
    const int64_t r_begin = (int64_t)split * p.k_chunk;
    const int64_t r_end = r_begin + p.k_chunk < p.k ? r_begin + p.k_chunk : p.k;

    floatx4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[a][b][v] = 0.f;

    LX lx;
    LY ly;
    if constexpr (XMODE == 0)
        lx.init(p.x + batch * p.x_batch, p.x_si, p.x_sr, i0, p.m, tid);
    else
        lx.init(p.conv, i0, p.m, tid);
    ly.init(p.y + batch * p.y_batch, p.y_sj, p.y_sr, j0, p.n, tid);
    ly.taps = p.ytaps;
    // K steps of this slice, counted in 32 bits (scalar compares; 64-bit compares of scalars take
    // vector instructions), and the k of the last one
    const int32_t steps = r_begin < r_end ? (int32_t)((r_end - r_begin + BK - 1) / BK) : 0;
    const int32_t tail = (int32_t)(r_end - r_begin - (int64_t)(steps - 1) * BK);
    auto room_of = [&](int32_t step) { return step == steps - 1 ? tail : BK; };
    // cols mode over aligned steps: the reduction (batch * image pixels) is a multiple of BK
    constexpr bool kWholeSteps = XMODE == 3;
    // flags the loop tests, as ints from the scalar unit: kept as bools they cross the loop's
    // blocks as lane masks and cost two vector instructions per test
    const int bf16 = __builtin_amdgcn_readfirstlane(p.bf16 ? 1 : 0);
    if (steps > 0) {
        lx.load(p.conv, r_begin, room_of(0), tid);
        ly.template load<kWholeSteps>(p.conv, r_begin, room_of(0), tid);
        lx.store(xs, tid, bf16);
        ly.store(ys, tid, bf16);
    }
    // Orders a stage's LDS stores and reads: the block's barrier, or with one wave per stage
    // (WS > 1) the wave's own instruction order (its LDS operations run in issue order): a wait
    // for its LDS operations and a compiler-only fence.
    auto stage_sync = [&]() {
        if constexpr (WS > 1) {
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
        } else {
            __syncthreads();
        }
    };
    stage_sync();

    // v_mfma_f32_16x16x4_f32: lane l feeds k = l / 16 of the quad, A row i = l % 16, B column
    // j = l % 16; its result registers v hold rows 4 * (l / 16) + v of column l % 16.
    const int quad = lane >> 4;
    const int l16 = lane & 15;
    // MFMA operands of the k-quad starting at kk (its four rows share one swizzle).
    auto read_operands = [&](int kk, float *av, float *bv) {
        const float *xa = xs + (kk + quad) * LX::LD + ((wm * TM + FM * l16) ^ stage_swizzle<BM>(kk));
        const float *yb = ys + (kk + quad) * LY::LD + ((wn * TN + FN * l16) ^ stage_swizzle<BN>(kk));
        if constexpr (FM == 4) {
            const floatx4 v = *reinterpret_cast<const floatx4 *>(xa);
            av[0] = v[0], av[1] = v[1], av[2] = v[2], av[3] = v[3];
        } else {
            const float2 v = *reinterpret_cast<const float2 *>(xa);
            av[0] = v.x, av[1] = v.y;
        }
        if constexpr (FN == 4) {
            const floatx4 v = *reinterpret_cast<const floatx4 *>(yb);
            bv[0] = v[0], bv[1] = v[1], bv[2] = v[2], bv[3] = v[3];
        } else {
            const float2 v = *reinterpret_cast<const float2 *>(yb);
            bv[0] = v.x, bv[1] = v.y;
        }
    };
    auto mma_quad = [&](const float *av, const float *bv) {
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[b], acc[a][b], 0, 0, 0);
    };
    // Each stage's k-quads run from registers read one quad ahead, and the last two quads are read
    // before the stage barrier and held, so their MFMAs cover the stores of the next stage into
    // LDS and the first reads of it and no wave idles at either barrier (the register budget:
    // two 128x128, three 128x64 or four 64x64 blocks per CU).
    constexpr int kQuads = BK / 4;
    static_assert(kQuads >= 3, "the held-quad schedule needs three k-quads per stage");
    // Wave priority while a stage's k-quads issue their MFMAs and while the two held quads do, per
    // tile shape (measured on the CNN's convolution products and config 2's 4096^3 and skinny
    // products): the SIMD's arbiter then feeds the matrix pipe before the co-resident blocks'
    // loads, stores and address arithmetic.  128-row tiles: quads at 1, held quads at 0 (held at 1
    // cost 3-6%); 64x128 tiles (three blocks per CU): quads at 2, held at 1; 64x64 tiles (four per
    // CU): no change, which the skinny products lost 1-3% to.
    // With the reduction split among waves (one block per CU, one wave per SIMD) there is no
    // other wave to arbitrate against.
    constexpr int kQuadPrio = (WS > 1 || (BM == 64 && BN == 64)) ? 0 : (BM == 64 && BN == 128) ? 2 : 1;
    constexpr int kHeldPrio = (BM == 64 && BN == 128) ? 1 : 0;
    // The K loop in two forms for dense products: every step whole (the depth tests of
    // r-contiguous operands compiled out) or a partial last step; a launch takes one.
    // Convolution launches keep one form (their dense operand is bounded by the record count).
    auto k_loop = [&](auto whole) {
        constexpr bool kW = decltype(whole)::value;
        float av[2][FM], bv[2][FN];
        float hold_a[2][FM], hold_b[2][FN];
        if (steps > 0) read_operands(0, av[0], bv[0]);
        for (int32_t step = 0; step < steps; ++step) {
            const bool more = step + 1 < steps;
            if (more) {
                const int64_t r_next = r_begin + (int64_t)(step + 1) * BK;
                if constexpr (XMODE == 0)
                    lx.template load<kW>(p.conv, r_next, room_of(step + 1), tid);
                else
                    lx.load(p.conv, r_next, room_of(step + 1), tid);
                ly.template load<kW>(p.conv, r_next, room_of(step + 1), tid);
            }
            // The operands of the next k-quad are read before this quad's MFMAs issue, and the
            // scheduling barriers keep that order: each LDS read has a whole MFMA group to land
            // (left to itself the compiler sinks every read to just before its use).
#pragma unroll
            for (int q = 0; q < kQuads - 2; ++q) {
                const int cur = q & 1;
                if (q + 1 < kQuads - 2) {
                    read_operands(4 * (q + 1), av[cur ^ 1], bv[cur ^ 1]);
                } else {
                    read_operands(4 * (kQuads - 2), hold_a[0], hold_b[0]);
                    read_operands(4 * (kQuads - 1), hold_a[1], hold_b[1]);
                }
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (kQuadPrio > 0) __builtin_amdgcn_s_setprio(kQuadPrio);
                mma_quad(av[cur], bv[cur]);
                if constexpr (kQuadPrio > 0) __builtin_amdgcn_s_setprio(0);
                __builtin_amdgcn_sched_barrier(0);
            }
            // After the last step the stores, the barrier and the reads below handle stale
            // registers and LDS nothing reads: unconditional, they keep the loop free of flag tests.
            stage_sync();  // every wave is done reading this stage
            lx.store(xs, tid, bf16);
            ly.store(ys, tid, bf16);
            if constexpr (kHeldPrio > 0) __builtin_amdgcn_s_setprio(kHeldPrio);
            mma_quad(hold_a[0], hold_b[0]);
            if constexpr (kHeldPrio > 0) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            stage_sync();  // the next stage is in LDS
            read_operands(0, av[0], bv[0]);
            if constexpr (kHeldPrio > 0) __builtin_amdgcn_s_setprio(kHeldPrio);
            mma_quad(hold_a[1], hold_b[1]);
            if constexpr (kHeldPrio > 0) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if constexpr (kWholeSteps) {
        k_loop(std::true_type{});
    } else if constexpr (XMODE != 0) {
        k_loop(std::false_type{});
    } else {
        if (tail == BK)
            k_loop(std::true_type{});
        else
            k_loop(std::false_type{});
    }

    // acc[a][b][v] is tile row wm*TM + FM*(4*quad + v) + a, column wn*TN + FN*l16 + b: a lane's
    // FN columns are adjacent.  The bias (one value per column) is added only when the reduction
    // is not split; split sums add it once at the end.
    auto row_of = [&](int a, int v) { return wm * TM + FM * (4 * quad + v) + a; };
    const int col_l = wn * TN + FN * l16;  // tile column of the lane's first column
    if constexpr (WS > 1) {
        // The waves' partial tiles meet in LDS ([wave][row][column]), then each output is
        // 0 + slice w per wave (split_sum_part's group sums, one slice per group), added in wave
        // order and finished once (split_sum_store): the bits of the split launch and its sum.
        __syncthreads();  // every wave is done with its stage
        float *const red = lds + kw * BM * BN;
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float *row = red + row_of(a, v) * BN + col_l;
                if constexpr (FN == 4)
                    *reinterpret_cast<floatx4 *>(row) = floatx4{acc[a][0][v], acc[a][1][v], acc[a][2][v], acc[a][3][v]};
                else
                    *reinterpret_cast<float2 *>(row) = make_float2(acc[a][0][v], acc[a][1][v]);
            }
        __syncthreads();
        float *c = p.c + batch * p.c_batch;
        const int64_t out_base = batch * p.m * p.n;
        const bool vec = p.n % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & 15) == 0;
        for (int e = (int)threadIdx.x; e < BM * BN / 4; e += WS * 64) {
            const int r = e / (BN / 4), cl = (e % (BN / 4)) * 4;
            const int64_t row = i0 + r, col = j0 + cl;
            if (row >= p.m || col >= p.n) continue;
            float o[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float g[WS];
#pragma unroll
                for (int w = 0; w < WS; ++w) g[w] = 0.f + lds[w * BM * BN + r * BN + cl + u];
                const float total = ((g[0] + g[1]) + g[2]) + g[3];
                o[u] = finish_value(p.bias, p.d, p.alpha, p.beta, total, out_base + row * p.n + col + u, col + u);
            }
            const int64_t idx = row * p.n + col;
            if (vec) {
                *reinterpret_cast<floatx4 *>(c + idx) = floatx4{o[0], o[1], o[2], o[3]};
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (col + u < p.n) c[idx + u] = o[u];
            }
        }
    } else if constexpr (EPI == 0) {
        float *c = p.c + batch * p.c_batch + (int64_t)split * p.c_split;
        // bias / axpby apply to whole sums only; split sums finish them at the end
        const bool whole = p.splits == 1;
        const float *bias = whole ? p.bias : nullptr;
        const float *d = whole ? p.d : nullptr;
        const int64_t out_base = batch * p.m * p.n;
        const int64_t col = j0 + col_l;
        if (p.n % FN == 0 && (reinterpret_cast<uintptr_t>(c) & (4 * FN - 1)) == 0) {
            // one FN-wide vector store per row (col < n implies all FN columns are)
            if (col < p.n) {
#pragma unroll
                for (int a = 0; a < FM; ++a)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int64_t row = i0 + row_of(a, v);
                        if (row >= p.m) continue;
                        const int64_t idx = row * p.n + col;
                        if constexpr (FN == 4) {
                            floatx4 o;
#pragma unroll
                            for (int b = 0; b < 4; ++b)
                                o[b] = finish_value(bias, d, p.alpha, p.beta, acc[a][b][v], out_base + idx + b, col + b);
                            *reinterpret_cast<floatx4 *>(c + idx) = o;
                        } else {
                            float2 o;
                            o.x = finish_value(bias, d, p.alpha, p.beta, acc[a][0][v], out_base + idx, col);
                            o.y = finish_value(bias, d, p.alpha, p.beta, acc[a][1][v], out_base + idx + 1, col + 1);
                            *reinterpret_cast<float2 *>(c + idx) = o;
                        }
                    }
            }
        } else {
#pragma unroll
            for (int b = 0; b < FN; ++b) {
                if (col + b >= p.n) continue;
#pragma unroll
                for (int a = 0; a < FM; ++a)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int64_t row = i0 + row_of(a, v);
                        if (row < p.m)
                            c[row * p.n + col + b] = finish_value(bias, d, p.alpha, p.beta, acc[a][b][v],
                                                                  out_base + row * p.n + col + b, col + b);
                    }
            }
        }
    } else {
        // The block's BM rows are whole rows of pooling windows (the host guarantees
        // BM % (pool_h * pool_ow) == 0 and an exact tiling), so every window is complete here.
        const int kh = p.pool_h, kw = p.pool_w, ow = p.pool_ow;
        const int pw = ow / kw;
        const int windows = BM / (kh * kw);
        const int64_t pooled_row0 = i0 / ow / kh;
        if (p.conv.window_major) {
            // 2x2 windows, tile rows window-major: acc[a][b][v] is position a of the wave's window
            // 4 * quad + v, so each lane pools whole windows from its own registers (no LDS, no
            // barrier) and writes its FN adjacent columns as one vector of values and one of
            // winner bytes.
            float addv[FN];
            bool okv[FN];
#pragma unroll
            for (int b = 0; b < FN; ++b) {
                const int64_t col = j0 + col_l + b;
                okv[b] = col < p.n;
                addv[b] = (p.bias != nullptr && okv[b]) ? p.bias[col] : 0.0f;
            }
            const bool vec = p.n % FN == 0 && (reinterpret_cast<uintptr_t>(p.pooled) & (4 * FN - 1)) == 0 &&
                             (reinterpret_cast<uintptr_t>(p.argmax) & (FN - 1)) == 0;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int w = wm * (TM / 4) + 4 * quad + v;  // window inside the tile
                const int wr = (int)p.pool_cols.div((uint32_t)w), wc = w - wr * pw;
                if (i0 + (int64_t)wr * 2 * ow >= p.m) continue;
                float best[FN];
                int winner[FN];
#pragma unroll
                for (int b = 0; b < FN; ++b) {
                    float y[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) y[e] = acc[e][b][v] + addv[b];
                    relu_pool_window4(y, best[b], winner[b]);
                }
                const int64_t out = ((pooled_row0 + wr) * pw + wc) * p.n + j0 + col_l;
                if (vec && okv[0]) {
                    if constexpr (FN == 4) {
                        *reinterpret_cast<floatx4 *>(p.pooled + out) = floatx4{best[0], best[1], best[2], best[3]};
                        *reinterpret_cast<uint32_t *>(p.argmax + out) =
                            (uint32_t)winner[0] | ((uint32_t)winner[1] << 8) | ((uint32_t)winner[2] << 16) |
                            ((uint32_t)winner[3] << 24);
                    } else {
                        *reinterpret_cast<float2 *>(p.pooled + out) = make_float2(best[0], best[1]);
                        *reinterpret_cast<uint16_t *>(p.argmax + out) = (uint16_t)(winner[0] | (winner[1] << 8));
                    }
                } else {
#pragma unroll
                    for (int b = 0; b < FN; ++b) {
                        if (!okv[b]) continue;
                        p.pooled[out + b] = best[b];
                        p.argmax[out + b] = (uint8_t)winner[b];
                    }
                }
            }
            return;
        }
        // Other windows: one column half (the waves with wn == h) at a time goes through LDS as
        // relu(acc + bias); then all threads reduce windows: first strictly greater finite value
        // in window order (ky major, kx minor), winner 255 and NaN when no value qualifies.
#pragma unroll
        for (int h = 0; h < WN; ++h) {
            __syncthreads();
            if (wn == h) {
#pragma unroll
                for (int b = 0; b < FN; ++b) {
                    const int cl = FN * l16 + b;
                    const int64_t col = j0 + h * TN + cl;
                    const bool with_bias = p.bias != nullptr && col < p.n;
                    const float add = with_bias ? p.bias[col] : 0.0f;
#pragma unroll
                    for (int a = 0; a < FM; ++a)
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const float z = with_bias ? acc[a][b][v] + add : acc[a][b][v];
                            lds[row_of(a, v) * kPoolPitch + cl] = z > 0.0f ? z : 0.0f;
                        }
                }
            }
            __syncthreads();
            // Thread items: column cl (fixed per thread) of windows w, w + NT/TN, ...
            const int cl = tid % TN;
            const int64_t col = j0 + h * TN + cl;
            const bool col_ok = col < p.n;
            for (int w = tid / TN; w < windows; w += NT / TN) {
                const int wr = (int)p.pool_cols.div((uint32_t)w), px = w - wr * pw;
                if (!col_ok || i0 + (int64_t)wr * kh * ow >= p.m) continue;
                float best = -INFINITY;
                int winner = 255;
                const float *win = lds + ((wr * kh) * ow + px * kw) * kPoolPitch + cl;
                auto take = [&](float v, int at) {
                    if (v >= -FLT_MAX && v <= FLT_MAX && v > best) {
                        best = v;
                        winner = at;
                    }
                };
                for (int ky = 0; ky < kh; ++ky)
                    for (int kx = 0; kx < kw; ++kx) take(win[(ky * ow + kx) * kPoolPitch], ky * kw + kx);
                const int64_t out = ((pooled_row0 + wr) * pw + px) * p.n + col;
                p.pooled[out] = winner == 255 ? __builtin_nanf("") : best;
                p.argmax[out] = (uint8_t)winner;
            }
        }
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool XR, bool YR, int VX, int VY, int XMODE, int EPI>
__global__ void __launch_bounds__(WM *WN * 64,
                                  gemm_blocks_per_cu(BM, BN, XMODE == 4 && XR && YR && VX == 4 && VY == 4 && EPI == 0))
    gemm_kernel(GemmParams p) {
    gemm_body<BM, BN, BK, WM, WN, XR, YR, VX, VY, XMODE, EPI, 1>(p);
}

// Dense 32x32 tiles whose two to four reduction slices are the block's four waves (gemm_body,
// WS = 4), staged 64 deep: for short split reductions over few tiles, one launch instead of the
// slices' launch and their sum, a slice of up to 64 in one load round trip.
template <bool XR, bool YR, int VX, int VY>
__global__ void __launch_bounds__(256, 1) gemm_fold_kernel(GemmParams p) {
    gemm_body<32, 32, 64, 1, 1, XR, YR, VX, VY, 0, 0, 4>(p);
}

// Sum of reduction slices (split_sum_part / split_sum_store): lane group g (of 4) adds slices
// g, g+4, g+8, ... in order, then the four group sums are added in group order -- a fixed
// association for a given slice count, so the result is deterministic and independent of
// scheduling.  The bias, when present, is added to the total.
__global__ void __launch_bounds__(256) split_sum_kernel(const float *__restrict__ partial,
                                                        float *__restrict__ out, int64_t len,
                                                        int32_t splits, int64_t split_stride,
                                                        const float *__restrict__ bias, int64_t n,
                                                        const float *__restrict__ d, float alpha,
                                                        float beta, int32_t perm_c, int32_t perm_taps) {
    __shared__ float acc[4][64];
    const int lane = threadIdx.x & 63, group = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + lane;
    acc[group][lane] = axis::split_sum_part(partial, i, len, splits, split_stride, group);
    __syncthreads();
    if (group == 0 && i < len)
        axis::split_sum_store(out, i, acc[0][lane], acc[1][lane], acc[2][lane], acc[3][lane], bias, n, d, alpha,
                              beta, perm_c, perm_taps);
}

// split_sum_kernel for len % 4 == 0 over 16-byte aligned slices: 256 outputs per block, four per
// lane, the same association per output.
__global__ void __launch_bounds__(256) split_sum4_kernel(const float *__restrict__ partial,
                                                         float *__restrict__ out, int64_t len,
                                                         int32_t splits, int64_t split_stride,
                                                         const float *__restrict__ bias, int64_t n,
                                                         const float *__restrict__ d, float alpha,
                                                         float beta, int32_t perm_c, int32_t perm_taps) {
    __shared__ axis::finish_floatx4 acc[4][64];
    const int lane = threadIdx.x & 63, group = threadIdx.x >> 6;
    const int64_t i4 = ((int64_t)blockIdx.x * 64 + lane) * 4;
    acc[group][lane] = axis::split_sum_part4(partial, i4, len, splits, split_stride, group);
    __syncthreads();
    if (group == 0 && i4 < len) {
        axis::split_sum_store4(out, i4, acc[0][lane], acc[1][lane], acc[2][lane], acc[3][lane], bias, n, d, alpha,
                               beta, perm_c, perm_taps);
    }
}

// First level for many slices: mid[g][i] = sum of slices [g*span, (g+1)*span) in order.
__global__ void __launch_bounds__(256) split_range_kernel(const float *__restrict__ partial,
                                                          float *__restrict__ mid, int64_t len,
                                                          int32_t splits, int32_t span) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= len) return;
    const int32_t g = blockIdx.y;
    const int32_t k1 = (g + 1) * span < splits ? (g + 1) * span : splits;
    // slice order; eight loads in flight before their adds
    constexpr int kAhead = 8;
    float s = 0.f;
    for (int32_t k0 = g * span; k0 < k1; k0 += kAhead) {
        float v[kAhead];
#pragma unroll
        for (int u = 0; u < kAhead; ++u) v[u] = k0 + u < k1 ? partial[(int64_t)(k0 + u) * len + i] : 0.f;
#pragma unroll
        for (int u = 0; u < kAhead; ++u)
            if (k0 + u < k1) s += v[u];
    }
    mid[(int64_t)g * len + i] = s;
}

// Weight permutations between the reference's [(c, ky, kx), n] layout and the implicit-GEMM
// orders, with the channel axis padded to c_pad >= c_in (padding rows are zero).
//   mode 0: W'[(ky, kx, c), n] = W[(c, ky, kx), n]                 (forward; rows c >= c_in are 0)
//   mode 1: W''[(ky', kx', n), c] = W[(c, kh-1-ky', kw-1-kx'), n]   (dgrad, flipped; c_pad == c_in)
//   mode 2: W[(c, ky, kx), n] = W'[(ky, kx, c), n]                 (wgrad result back; c < c_in)
// block (modes 0 and 1): the reduction rows in the rows loader's block-major order instead,
// (cb, ky, kx, ci) with c = 32 cb + ci (mode 0), (nb, ky', kx', ni) with n = 32 nb + ni (mode 1).
__device__ __forceinline__ void block_row(int64_t r, int32_t taps, int32_t &pos, int32_t &c) {
    const int32_t ci = (int32_t)(r & 31);
    const int64_t st = r >> 5;
    const int32_t cb = (int32_t)(st / taps);
    pos = (int32_t)(st - (int64_t)cb * taps);
    c = cb * 32 + ci;
}

__global__ void __launch_bounds__(256) conv_weight_permute_kernel(const float *__restrict__ src,
                                                                  float *__restrict__ dst, int32_t c_in,
                                                                  int32_t c_pad, int32_t n_out, int32_t kh,
                                                                  int32_t kw, int32_t mode, int32_t block = 0) {
    const int64_t total = (int64_t)(mode == 0 ? c_pad : c_in) * kh * kw * n_out;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        if (mode == 0) {
            const int32_t n = (int32_t)(idx % n_out);
            const int64_t r = idx / n_out;
            int32_t c, pos;
            if (block) {
                block_row(r, kh * kw, pos, c);
            } else {
                c = (int32_t)(r % c_pad);
                pos = (int32_t)(r / c_pad);
            }
            dst[idx] = c < c_in ? src[((int64_t)c * kh * kw + pos) * n_out + n] : 0.0f;
        } else if (mode == 1) {
            const int32_t c = (int32_t)(idx % c_in);
            const int64_t r = idx / c_in;
            int32_t n, pos;
            if (block) {
                block_row(r, kh * kw, pos, n);
            } else {
                n = (int32_t)(r % n_out);
                pos = (int32_t)(r / n_out);
            }
            const int32_t ky = pos / kw, kx = pos % kw;
            const int32_t flipped = (kh - 1 - ky) * kw + (kw - 1 - kx);
            dst[idx] = src[((int64_t)c * kh * kw + flipped) * n_out + n];
        } else {
            const int32_t n = (int32_t)(idx % n_out);
            const int64_t r = idx / n_out;
            const int32_t pos = (int32_t)(r % (kh * kw));
            const int32_t c = (int32_t)(r / (kh * kw));
            dst[idx] = src[((int64_t)pos * c_pad + c) * n_out + n];
        }
    }
}

// Copies an input of any layout into channel-innermost [batch, height, width, c_pad] with the
// channels past c_in zero, so every gathered vector is 16 contiguous bytes.  Consecutive lanes
// take consecutive pixels, which keeps the reads of a channel-major source coalesced.
__global__ void __launch_bounds__(256) repack_channels_last_kernel(const float *__restrict__ src,
                                                                   int64_t ld_b, int64_t ld_c,
                                                                   int64_t ld_h, int64_t ld_w,
                                                                   float *__restrict__ dst, int64_t pixels,
                                                                   int32_t height, int32_t width,
                                                                   int32_t c_in, int32_t c_pad) {
    const int32_t groups = c_pad / 4;
    const int64_t total = pixels * groups;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        const int32_t g = (int32_t)(t / pixels);
        const int64_t pix = t - (int64_t)g * pixels;
        const int32_t x = (int32_t)(pix % width);
        const int64_t rest = pix / width;
        const int32_t y = (int32_t)(rest % height);
        const int64_t b = rest / height;
        const float *s0 = src + b * ld_b + (int64_t)y * ld_h + (int64_t)x * ld_w;
        floatx4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int32_t c = g * 4 + e;
            v[e] = c < c_in ? s0[(int64_t)c * ld_c] : 0.0f;
        }
        *reinterpret_cast<floatx4 *>(dst + pix * c_pad + g * 4) = v;
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool XR, bool YR, int VX, int VY, int XMODE, int EPI>
void launch_config(const GemmParams &p, dim3 grid, hipStream_t stream) {
    gemm_kernel<BM, BN, BK, WM, WN, XR, YR, VX, VY, XMODE, EPI><<<grid, WM * WN * 64, 0, stream>>>(p);
}

template <int BM, int BN, int BK, int WM, int WN, bool XR, bool YR, int XMODE, int EPI>
void launch_vec(const GemmParams &p, dim3 grid, hipStream_t stream, bool vx, bool vy) {
    if (vx && vy)
        launch_config<BM, BN, BK, WM, WN, XR, YR, 4, 4, XMODE, EPI>(p, grid, stream);
    else if (vx)
        launch_config<BM, BN, BK, WM, WN, XR, YR, 4, 1, XMODE, EPI>(p, grid, stream);
    else if (vy)
        launch_config<BM, BN, BK, WM, WN, XR, YR, 1, 4, XMODE, EPI>(p, grid, stream);
    else
        launch_config<BM, BN, BK, WM, WN, XR, YR, 1, 1, XMODE, EPI>(p, grid, stream);
}

template <bool XR, bool YR>
void launch_fold(const GemmParams &p, dim3 grid, hipStream_t stream, bool vx, bool vy) {
    if (vx && vy)
        gemm_fold_kernel<XR, YR, 4, 4><<<grid, 256, 0, stream>>>(p);
    else if (vx)
        gemm_fold_kernel<XR, YR, 4, 1><<<grid, 256, 0, stream>>>(p);
    else if (vy)
        gemm_fold_kernel<XR, YR, 1, 4><<<grid, 256, 0, stream>>>(p);
    else
        gemm_fold_kernel<XR, YR, 1, 1><<<grid, 256, 0, stream>>>(p);
}

// Vector loads need the contiguous extent, the other stride and the base to be 4-aligned.
bool vec_ok(const float *base, int64_t contiguous_extent, int64_t other_stride) {
    return axis::aligned16(base) && contiguous_extent % 4 == 0 && other_stride % 4 == 0;
}

// Tile shapes, all 32 deep per LDS stage: large 128x128 when both output extents fill it; 128x64
// when the columns are few (<= 64); 64x64 otherwise; 64x128 for the convolution weight gradients
// over aligned pixel steps: three blocks per CU, and twice the tiles of 128x128, so the split fills
// the chip with fewer slices of partial sums (conv2's 576 patch rows: 9 wide tiles, not 4.5 large
// ones; conv3's 1152: 278 us against 287, 21 slices against 28).
// Resident blocks per CU follow from the register budget of each shape.
enum class Shape { Large, Tall, Small, Wide };

struct Choice {
    Shape shape;
    int bm, bn, bk, per_cu;
};

Choice choose(int64_t m, int64_t n, int64_t k, int64_t batch, int64_t cus, bool pool_epilogue,
              bool wide_ok = false) {
    const Choice large{Shape::Large, 128, 128, 32, 2}, tall{Shape::Tall, 128, 64, 32, 3},
        small{Shape::Small, 64, 64, 32, 4}, wide{Shape::Wide, 64, 128, 32, 3};
    if (m < 128 && !pool_epilogue) return small;
    if (n < 128) return n <= 64 || pool_epilogue ? tall : small;
    if (wide_ok) return wide;
    const int64_t tiles = ((m + 127) / 128) * ((n + 127) / 128) * batch;
    // A short reduction over few large tiles (e.g. a classifier layer) would leave most CUs idle
    // and each block only a few K steps: four times as many small tiles finish sooner.
    if (!pool_epilogue && tiles * 2 < cus && k <= 2048) return small;
    return large;
}

// Dense products whose 128x128 tiles number fewer than two per CU (reductions of 4 K steps or
// more): every (tile shape, slice count) is priced as the time of the busiest CU --
// ceil(blocks / CUs) blocks of BM x BN x chunk products at a per-CU rate measured on these kernels
// (0.46 GFLOP/ms with two or more resident blocks; a CU left one resident block at a time runs 16%
// slower) scaled by the shape's efficiency, at least the load latency of each round's K steps --
// plus the slice sum (partials written and read once at ~5 TB/s and a launch).  The 8192 x 784 x 1024 products of a
// 784-wide layer: 128x128 tiles leave 64 CUs one block and 192 two (143 us); 64x64 tiles, unsplit
// for the data gradient and in six slices for the weight gradient, run in 130 us.
struct DenseSchedule {
    Choice choice;
    int64_t splits;
};

DenseSchedule dense_schedule(int64_t m, int64_t n, int64_t k, int64_t batch, int64_t cus) {
    const Choice shapes[3] = {{Shape::Large, 128, 128, 32, 2}, {Shape::Tall, 128, 64, 32, 3},
                              {Shape::Small, 64, 64, 32, 4}};
    const double eff[3] = {1.0, 0.96, 0.92};
    const int64_t out_len = batch * m * n;
    DenseSchedule best{shapes[0], 1};
    double best_us = 1e300;
    for (int c = 0; c < 3; ++c) {
        const Choice &sh = shapes[c];
        if (sh.shape == Shape::Tall && n > 64) continue;
        const int64_t tiles = ((m + sh.bm - 1) / sh.bm) * ((n + sh.bn - 1) / sh.bn) * batch;
        const int64_t most = std::max<int64_t>(1, k / (sh.bk * 2));
        for (int64_t want = 1; want <= std::min<int64_t>(most, 64); ++want) {
            int64_t chunk = (k + want - 1) / want;
            chunk = (chunk + sh.bk - 1) / sh.bk * sh.bk;
            const int64_t splits = (k + chunk - 1) / chunk;
            if (splits != want) continue;
            if (splits > 1 && out_len * splits > (int64_t(16) << 20)) break;
            const int64_t blocks = tiles * splits;
            const int64_t per_cu = (blocks + cus - 1) / cus;
            const double occ = std::min<int64_t>(per_cu, sh.per_cu) >= 2 ? 1.0 : 0.84;
            double us = (double)per_cu * 2.0 * sh.bm * sh.bn * (double)chunk / (0.46e6 * eff[c] * occ);
            // latency floor: a block's K steps each wait on their loads when the CU holds too few
            // blocks to cover them (~1 us per step, ~2 us to start), once per round of resident blocks
            const int64_t rounds = (per_cu + sh.per_cu - 1) / sh.per_cu;
            us = std::max(us, (double)rounds * (1.0 * (double)(chunk / sh.bk) + 2.0));
            if (splits > 1) us += (double)(splits + 1) * (double)out_len * 4.0 / 5.0e6 + 3.0;
            if (us < best_us) {
                best_us = us;
                best = {sh, splits};
            }
        }
    }
    return best;
}

// Deterministic sum of reduction slices (+ bias): up to 32 slices in one pass; beyond that, ranges
// of 32 consecutive slices first, then the range sums -- a fixed association for a given count.
// `owner` (the block holding `partial`), when given and the handle defers finishing sums, lets
// the last pass be recorded instead of launched: `out` is then a final gradient.
int sum_splits(axis_device device, const float *partial, float *out, int64_t len, int64_t splits,
               const float *bias, int64_t n, const float *d, float alpha, float beta, int32_t perm_c,
               int32_t perm_taps, float *mid_space = nullptr, axis::Scratch *owner = nullptr) {
    const unsigned blocks = axis::blocks_for(len, 64, INT32_MAX);
    const bool defer = owner && device->deferring && len <= (int64_t)INT32_MAX * 64 / 2;
    auto last_pass = [&](const float *slices, int64_t count, axis::Scratch &held) {
        // four outputs per lane when every slice and the output start 16-byte aligned
        const bool vec4 = len % 4 == 0 && axis::aligned16(slices) && axis::aligned16(out);
        if (defer) {
            axis::FinishTask t{};
            t.partial = slices;
            t.out_a = out;
            t.bias = bias;
            t.d = d;
            t.len = len;
            t.count = count;
            t.stride = len;
            t.n = n;
            t.alpha = alpha;
            t.beta = beta;
            t.perm_c = perm_c;
            t.perm_taps = perm_taps;
            t.kind = vec4 ? 2 : 0;
            t.blocks = (int32_t)(vec4 ? (len + 255) / 256 : (len + 63) / 64);
            return axis::defer_finish(device, t, held);
        }
        if (vec4) {
            split_sum4_kernel<<<axis::blocks_for(len, 256, INT32_MAX), 256, 0, device->stream>>>(
                slices, out, len, (int32_t)count, len, bias, n, d, alpha, beta, perm_c, perm_taps);
            return axis::launch_status("split_sum4_kernel");
        }
        split_sum_kernel<<<blocks, 256, 0, device->stream>>>(slices, out, len, (int32_t)count, len, bias, n, d,
                                                             alpha, beta, perm_c, perm_taps);
        return axis::launch_status("split_sum_kernel");
    };
    axis::Scratch none;
    if (splits <= 32) return last_pass(partial, splits, defer ? *owner : none);
    const int32_t span = 32;
    const int64_t ranges = (splits + span - 1) / span;
    axis::Scratch mid;
    float *sums = mid_space;
    if (!sums || defer) {
        if (int st = mid.get(device, sizeof(float) * (size_t)(ranges * len))) return st;
        sums = mid.as<float>();
    }
    dim3 grid(axis::blocks_for(len, 256, INT32_MAX), (unsigned)ranges);
    split_range_kernel<<<grid, 256, 0, device->stream>>>(partial, sums, len, (int32_t)splits, span);
    if (int st = axis::launch_status("split_range_kernel")) return st;
    return last_pass(sums, ranges, mid);
}

// Dense product on a bf16 device: both operands staged as bf16 rows, then bf16 matrix cores
// (gemm_bf16.hip).  The staging passes sit inside the timed launch.
int run_gemm_bf16(axis_device device, const GemmParams &p, int64_t batch, float *out) {
    constexpr int64_t D = axis::kBf16Depth;
    const int64_t kp = (p.k + D - 1) / D * D;
    const int64_t xb = p.x_batch ? batch : 1, yb = p.y_batch ? batch : 1;
    // A product of an operand with itself under the same layout (a Gram matrix, x . x^T) stages it once.
    const bool same = p.x == p.y && p.x_batch == p.y_batch && p.x_si == p.y_sj && p.x_sr == p.y_sr && p.m == p.n;
    axis::Scratch sx, sy, partial;
    if (int st = sx.get(device, sizeof(uint16_t) * (size_t)(xb * p.m * kp))) return st;
    if (!same)
        if (int st = sy.get(device, sizeof(uint16_t) * (size_t)(yb * p.n * kp))) return st;
    const double k_work = (double)(p.k_work > 0 ? p.k_work : p.k);
    axis::TimedLaunch timed(device, "gemm", 2.0 * (double)batch * (double)p.m * (double)p.n * k_work);
    if (int st = axis::stage_bf16(device, {p.x, p.x_batch, p.x_si, p.x_sr}, xb, p.m, p.k, kp, sx.as<uint16_t>()))
        return st;
    if (!same)
        if (int st = axis::stage_bf16(device, {p.y, p.y_batch, p.y_sj, p.y_sr}, yb, p.n, p.k, kp, sy.as<uint16_t>()))
            return st;
    const axis::Bf16Tile tile = axis::bf16_gemm_tile(p.m, p.n, batch, kp, device->multiprocessors);
    const int64_t tiles = ((p.m + tile.rows - 1) / tile.rows) * ((p.n + tile.cols - 1) / tile.cols) * batch;
    const int64_t slots = device->multiprocessors * (tile.rows == 256 ? 1 : 2);  // resident blocks
    const int64_t out_len = batch * p.m * p.n;
    // split as the fp32 path does: fill one round of resident blocks, reductions of 8 stages or more
    int64_t splits = 1;
    if (tiles < slots && kp >= 8 * D) {
        splits = std::min<int64_t>({slots / tiles, kp / (D * 4), (int64_t(16) << 20) / out_len});
        splits = std::max<int64_t>(splits, 1);
    }
    int64_t chunk = (kp + splits - 1) / splits;
    chunk = (chunk + D - 1) / D * D;
    splits = (kp + chunk - 1) / chunk;
    axis::Bf16Gemm g{};
    g.x = sx.as<uint16_t>();
    g.y = same ? sx.as<uint16_t>() : sy.as<uint16_t>();
    g.x_batch = p.x_batch ? p.m * kp : 0;
    g.y_batch = p.y_batch ? p.n * kp : 0;
    g.bias = p.bias;
    g.d = p.d;
    g.alpha = p.alpha;
    g.beta = p.beta;
    g.m = p.m;
    g.n = p.n;
    g.kp = kp;
    g.c_batch = p.m * p.n;
    g.k_chunk = chunk;
    g.splits = (int32_t)splits;
    if (splits > 1) {
        if (int st = partial.get(device, sizeof(float) * (size_t)(out_len * splits))) return st;
        g.c = partial.as<float>();
        g.c_split = out_len;
    } else {
        g.c = out;
        g.c_split = 0;
    }
    if (int st = axis::bf16_gemm(device, g, batch, tile)) return st;
    if (splits > 1)
        return sum_splits(device, partial.as<float>(), out, out_len, splits, p.bias, p.n, p.d, p.alpha, p.beta, 0, 0);
    return AXIS_OK;
}

// ws: when non-null, the partial sums live there (nothing is allocated, nothing is timed) and a
// launch whose partials would not fit is rejected before anything runs.
template <bool XR, bool YR, int XMODE, int EPI>
// final_out: `out` is the entry's own result, read by nothing in the entry after this product, so
// its split sum may be deferred (sum_splits).
int run_gemm(axis_device device, GemmParams p, int64_t batch, float *out, const Workspace *ws = nullptr,
             bool final_out = false) {
    if constexpr (XMODE == 0 && EPI == 0)
        if (device->bf16_matmul && !p.ytaps.on && !p.perm_c) {
            if (ws) return axis::fail(AXIS_ERROR_INVALID, "the allocation-free product is fp32 only");
            const int64_t kp = (p.k + axis::kBf16Depth - 1) / axis::kBf16Depth * axis::kBf16Depth;
            if (axis::bf16_gemm_fits(p.m, p.n, batch, kp, device->multiprocessors))
                return run_gemm_bf16(device, p, batch, out);
            // otherwise the fp32 matrix cores below, rounding the operands to bf16 as they are staged
        }
    p.bf16 = device->bf16_matmul;
    const int64_t cus = device->multiprocessors;
    Choice ch = choose(p.m, p.n, p.k, batch, cus, EPI == 1, XMODE == 3);
    int64_t scheduled_splits = 0;
    if constexpr (XMODE == 0 && EPI == 0) {
        const int64_t large_tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128) * batch;
        if (!p.perm_c && large_tiles < 2 * cus && p.k >= 4 * 32) {
            const DenseSchedule d = dense_schedule(p.m, p.n, p.k, batch, cus);
            ch = d.choice;
            scheduled_splits = d.splits;
        }
    }
    const int BK = ch.bk;
    p.tiles_m = static_cast<int32_t>((p.m + ch.bm - 1) / ch.bm);
    p.tiles_n = static_cast<int32_t>((p.n + ch.bn - 1) / ch.bn);
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n * batch;
    // Split the reduction when the tiles alone cannot fill the chip (dense products: as the
    // schedule above decided): aim at one full round of resident blocks so no round runs nearly
    // empty.  The pooling epilogue needs whole sums.  Other reductions under 16 K steps are not
    // split (the extra sum launch would cost more than it saves).  The partial slices stay within
    // 64 MiB.
    const int64_t slots = cus * ch.per_cu;
    const int64_t out_len = batch * p.m * p.n;
    int64_t splits = 1;
    if (scheduled_splits > 0) {
        splits = scheduled_splits;
    } else if (EPI == 0 && tiles < slots && p.k >= 16 * BK) {
        splits = std::min<int64_t>({slots / tiles, p.k / (BK * 4), (int64_t(16) << 20) / out_len});
        splits = std::max<int64_t>(splits, 1);
    }
    int64_t chunk = (p.k + splits - 1) / splits;
    chunk = (chunk + BK - 1) / BK * BK;
    if (chunk < BK) chunk = BK;
    splits = (p.k + chunk - 1) / chunk;
    if (splits < 1) splits = 1;
    p.k_chunk = chunk;
    p.splits = static_cast<int32_t>(splits);
    // Two to four slices of at most 128 over at most one 32x32 tile per CU: one block per tile whose
    // waves are the slices (gemm_fold_kernel), with no partial buffer and no sum launch; the same
    // bits as the slices and their sum.  Its 64-deep stages reach 31 * s_t + 63 * s_r elements.
    auto fold_reach = [](int64_t st, int64_t sr) { return 31 * st + 63 * sr < (int64_t(1) << 29); };
    const int64_t fold_tiles = ((p.m + 31) / 32) * ((p.n + 31) / 32) * batch;
    const bool fold = XMODE == 0 && EPI == 0 && scheduled_splits > 1 && ch.shape == Shape::Small && splits >= 2 &&
                      splits <= 4 && chunk <= 128 && fold_tiles <= cus && !p.perm_c && device->fold_splits &&
                      fold_reach(p.x_si, p.x_sr) && fold_reach(p.y_sj, p.y_sr);
    if (fold) {
        p.tiles_m = static_cast<int32_t>((p.m + 31) / 32);
        p.tiles_n = static_cast<int32_t>((p.n + 31) / 32);
    }

    // Dense operands read through 32-bit offsets inside a tile: at most 127 * s_t + 31 * s_r elements.
    auto reach = [](int64_t st, int64_t sr) { return st >= 0 && sr >= 0 && 127 * st + 31 * sr < (int64_t(1) << 29); };
    if (XMODE == 0 && !reach(p.x_si, p.x_sr))
        return axis::fail(AXIS_ERROR_INVALID, "matmul operand row pitch must stay below 4,227,000 elements");
    if (!reach(p.y_sj, p.y_sr))
        return axis::fail(AXIS_ERROR_INVALID, "matmul operand row pitch must stay below 4,227,000 elements");
    // t-contiguous dense operands bound a K step's rows by the resource's record count: unit
    // element stride and rows no longer than their pitch (every entry point lays them out so)
    if ((XMODE == 0 && !XR && (p.x_si != 1 || p.x_sr < p.m)) || (!YR && (p.y_sj != 1 || p.y_sr < p.n)))
        return axis::fail(AXIS_ERROR_INVALID, "t-contiguous product operand without unit stride and full-row pitch");
    bool vx;
    if constexpr (XMODE == 0)
        vx = XR ? vec_ok(p.x, p.k, p.x_si) && p.x_batch % 4 == 0
                : vec_ok(p.x, p.m, p.x_sr) && p.x_batch % 4 == 0;
    else
        vx = axis::aligned16(p.conv.src) && p.conv.channels % 4 == 0 && p.conv.ld_c == 1 &&
             p.conv.ld_w % 4 == 0 && p.conv.ld_h % 4 == 0 && p.conv.ld_b % 4 == 0;
    const bool vy = YR ? vec_ok(p.y, p.k, p.y_sj) && p.y_batch % 4 == 0
                       : vec_ok(p.y, p.n, p.y_sr) && p.y_batch % 4 == 0;

    axis::Scratch partial, ordered;
    // spare: the range sums of more than 32 slices, or an unsplit permuted product before its move
    float *partials = nullptr, *spare = nullptr;
    if (ws) {
        const int64_t ranges = splits > 32 ? (splits + 31) / 32 : 0;
        const int64_t need =
            (splits > 1 && !fold ? splits + ranges : 0) * out_len + (splits == 1 && p.perm_c ? out_len : 0);
        if (need > ws->floats)
            return axis::fail(AXIS_ERROR_INVALID, "product needs " + std::to_string(need * 4) +
                                                      " bytes of partial sums; the static scratch holds " +
                                                      std::to_string(ws->floats * 4));
        partials = ws->ptr;
        spare = ws->ptr + splits * out_len;
    }
    if (splits > 1 && !fold) {
        if (!partials) {
            int status = partial.get(device, sizeof(float) * (size_t)(out_len * splits));
            if (status) return status;
            partials = partial.as<float>();
        }
        p.c = partials;
        p.c_split = out_len;
        p.c_batch = p.m * p.n;
    } else {
        // an unsplit product with permuted rows is written in its own order, then moved
        if (p.perm_c) {
            if (partials) {
                spare = partials;
            } else {
                if (int status = ordered.get(device, sizeof(float) * (size_t)out_len)) return status;
                spare = ordered.as<float>();
            }
        }
        p.c = p.perm_c ? spare : out;
        p.c_split = 0;
        p.c_batch = p.m * p.n;
    }
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * batch * (fold ? 1 : splits);
    if (blocks >= INT32_MAX) return axis::fail(AXIS_ERROR_INVALID, "matmul too large for one launch");
    p.xcd_span = (uint32_t)(blocks / 8);
    const double k_work = (double)(p.k_work > 0 ? p.k_work : p.k);
    axis::TimedLaunch timed(ws ? nullptr : device, "gemm", 2.0 * (double)batch * (double)p.m * (double)p.n * k_work);
    dim3 grid(static_cast<unsigned>(blocks));
    if (fold) {
        if constexpr (XMODE == 0 && EPI == 0) launch_fold<XR, YR>(p, grid, device->stream, vx, vy);
    } else if constexpr (EPI == 1) {
        // the fused forward's 128x128 tiles in eight waves of 64x32 (307.8 -> 302.8 us per launch)
        if (ch.shape == Shape::Large)
            launch_vec<128, 128, 32, 2, 4, XR, YR, XMODE, EPI>(p, grid, device->stream, vx, vy);
        else
            launch_vec<128, 64, 32, 2, 2, XR, YR, XMODE, EPI>(p, grid, device->stream, vx, vy);
    } else {
        // 128x128 tiles of the gathered convolution loader, and dense ones with both operands
        // contiguous along the reduction, in eight waves of 64x32: two blocks and sixteen waves per
        // CU at 128 VGPRs (conv3's data gradient 293 -> 284 us, the 4096^3 data gradient 141 -> 144
        // TFLOP/s); other dense ones in four waves of 64x64 (the eight-wave instances need 132-154
        // VGPRs, one block per CU)
        if (ch.shape == Shape::Large) {
            if constexpr (XMODE == 4 || (XMODE == 0 && XR && YR))
                launch_vec<128, 128, 32, 2, 4, XR, YR, XMODE, EPI>(p, grid, device->stream, vx, vy);
            else
                launch_vec<128, 128, 32, 2, 2, XR, YR, XMODE, EPI>(p, grid, device->stream, vx, vy);
        }
        else if (ch.shape == Shape::Tall)
            launch_vec<128, 64, 32, 2, 2, XR, YR, XMODE, EPI>(p, grid, device->stream, vx, vy);
        else if (ch.shape == Shape::Small)
            launch_vec<64, 64, 32, 2, 2, XR, YR, XMODE, EPI>(p, grid, device->stream, vx, vy);
        else if constexpr (XMODE == 3)  // Wide: cols-mode weight gradients only
            launch_vec<64, 128, 32, 2, 2, XR, YR, XMODE, EPI>(p, grid, device->stream, vx, vy);
    }
    int status = axis::launch_status("gemm_kernel");
    if (status) return status;
    if (splits > 1 && !fold)
        status = sum_splits(device, partials, out, out_len, splits, p.bias, p.n, p.d, p.alpha, p.beta,
                            p.perm_c, p.perm_taps, spare, final_out && !ws ? &partial : nullptr);
    else if (p.perm_c) {
        // mode 2 of the weight permutation with the taps as one axis
        conv_weight_permute_kernel<<<axis::blocks_for(out_len, 256, 4096), 256, 0, device->stream>>>(
            spare, out, p.perm_c, p.perm_c, (int32_t)p.n, p.perm_taps, 1, 2);
        status = axis::launch_status("conv_weight_permute_kernel");
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

struct ConvShape {
    int64_t batch;
    int32_t height, width, channels, out_channels, kh, kw, sy, sx, py, px, out_h, out_w;
};

int conv_shape(int64_t batch, int32_t height, int32_t width, int32_t channels, int32_t out_channels,
               const int32_t *kernel, const int32_t *stride, const int32_t *padding, ConvShape *s) {
    AXIS_REQUIRE(kernel && stride && padding, "null convolution geometry");
    AXIS_REQUIRE(batch >= 1 && height >= 1 && width >= 1 && channels >= 1 && out_channels >= 1,
                 "convolution extents must be positive");
    AXIS_REQUIRE(kernel[0] >= 1 && kernel[1] >= 1 && stride[0] >= 1 && stride[1] >= 1 &&
                     padding[0] >= 0 && padding[1] >= 0,
                 "convolution kernel/stride must be positive and padding nonnegative");
    AXIS_REQUIRE(height + 2 * padding[0] >= kernel[0] && width + 2 * padding[1] >= kernel[1],
                 "convolution kernel exceeds the padded spatial extent");
    s->batch = batch;
    s->height = height;
    s->width = width;
    s->channels = channels;
    s->out_channels = out_channels;
    s->kh = kernel[0];
    s->kw = kernel[1];
    s->sy = stride[0];
    s->sx = stride[1];
    s->py = padding[0];
    s->px = padding[1];
    s->out_h = (height + 2 * padding[0] - kernel[0]) / stride[0] + 1;
    s->out_w = (width + 2 * padding[1] - kernel[1]) / stride[1] + 1;
    const int64_t in_len = batch * height * width * channels;
    const int64_t out_len = batch * (int64_t)s->out_h * s->out_w * out_channels;
    const int64_t patch = (int64_t)channels * kernel[0] * kernel[1];
    AXIS_REQUIRE(in_len < INT32_MAX && out_len < INT32_MAX && batch * s->out_h * s->out_w < INT32_MAX &&
                     patch * out_channels < INT32_MAX && batch * (int64_t)s->out_h * s->out_w * patch < (int64_t(1) << 40),
                 "convolution too large for 32-bit pixel indexing");
    return AXIS_OK;
}

axis::SmallConvShape small_shape(const ConvShape &s) {
    return axis::SmallConvShape{s.batch, s.height, s.width, s.channels, s.out_channels, s.kh, s.kw,
                                s.sy,    s.sx,     s.py,    s.px,       s.out_h,        s.out_w};
}

// Strides of a channel-innermost contiguous [batch, height, width, channels] tensor.
void channels_last(int32_t height, int32_t width, int32_t channels, int64_t ld[4]) {
    ld[0] = (int64_t)height * width * channels;
    ld[1] = 1;
    ld[2] = (int64_t)width * channels;
    ld[3] = channels;
}

// Validates caller strides {batch, channel, row, column} (null = channel-innermost contiguous).
int input_strides(const int64_t *given, int64_t batch, int32_t height, int32_t width,
                  int32_t channels, int64_t ld[4]) {
    if (!given) {
        channels_last(height, width, channels, ld);
        return AXIS_OK;
    }
    for (int i = 0; i < 4; ++i) ld[i] = given[i];
    AXIS_REQUIRE(ld[0] >= 0 && ld[1] >= 0 && ld[2] >= 0 && ld[3] >= 0, "input strides must be nonnegative");
    AXIS_REQUIRE(ld[1] < INT32_MAX && ld[2] < INT32_MAX && ld[3] < INT32_MAX, "input stride too large");
    const int64_t last = (batch - 1) * ld[0] + (int64_t)(channels - 1) * ld[1] +
                         (int64_t)(height - 1) * ld[2] + (int64_t)(width - 1) * ld[3];
    AXIS_REQUIRE(last < (int64_t(1) << 40), "input strides address too far");
    return AXIS_OK;
}

ConvGeom geom(const float *src, const int64_t ld[4], int32_t height, int32_t width, int32_t channels,
              int32_t out_h, int32_t out_w, int32_t kh, int32_t kw, int32_t sy, int32_t sx, int32_t py, int32_t px) {
    ConvGeom g{};
    g.src = src;
    g.ld_b = ld[0];
    g.ld_c = (int32_t)ld[1];
    g.ld_h = (int32_t)ld[2];
    g.ld_w = (int32_t)ld[3];
    g.height = height;
    g.width = width;
    g.channels = channels;
    g.out_h = out_h;
    g.out_w = out_w;
    g.kh = kh;
    g.kw = kw;
    g.sy = sy;
    g.sx = sx;
    g.py = py;
    g.px = px;
    g.c_div = FastDiv((uint32_t)channels);
    g.kw_div = FastDiv((uint32_t)kw);
    g.ow_div = FastDiv((uint32_t)out_w);
    g.oh_div = FastDiv((uint32_t)out_h);
    g.tap_steps = channels % 32 == 0;
    g.block_major = false;  // set by launches that take the buffer rows loader (use_block_major)
    g.taps_div = FastDiv((uint32_t)(kh * kw));
    return g;
}

// Rows mode reads through 31-bit byte offsets when every element of the gathered tensor is
// within reach of them and the kernel has at most 32 taps (the buffer loader); other
// convolutions keep 64-bit addresses.
bool buffer_reach(const ConvGeom &g, int64_t batch) {
    const int64_t last = (batch - 1) * g.ld_b + (int64_t)(g.height - 1) * g.ld_h + (int64_t)(g.width - 1) * g.ld_w +
                         (int64_t)(g.channels - 1) * g.ld_c;
    return (last + 4) * 4 < (int64_t(1) << 31) - 1 && g.kh * g.kw <= 32;
}

int permute_weight(axis_device device, const float *src, float *dst, const ConvShape &s, int mode,
                   int32_t c_pad, bool block = false) {
    const int64_t total = (int64_t)(mode == 0 ? c_pad : s.channels) * s.kh * s.kw * s.out_channels;
    conv_weight_permute_kernel<<<axis::blocks_for(total, 256, 4096), 256, 0, device->stream>>>(
        src, dst, s.channels, c_pad, s.out_channels, s.kh, s.kw, mode, block ? 1 : 0);
    return axis::launch_status("conv_weight_permute_kernel");
}

// Whether a rows-mode launch takes the buffer loader and, with tap steps, its block-major
// reduction order (the second operand must then be read in the same order).
bool use_block_major(ConvGeom &g, int64_t batch) {
    g.block_major = g.tap_steps && buffer_reach(g, batch);
    return g.block_major;
}

// The forward's second operand W'[(ky, kx, c), n]: read in place from the reference's
// [(c, ky, kx), n] weight when the channels need no padding and a K step stays in one tap
// (c % 32 == 0), otherwise permuted (and padded) into `permuted`.
int forward_weight(axis_device device, const float *weight, const ConvShape &s, int32_t c_pad,
                   axis::Scratch &permuted, GemmParams &p) {
    const int64_t taps = (int64_t)s.kh * s.kw;
    const bool block = p.conv.block_major;
    if (c_pad == s.channels && s.channels % 32 == 0) {
        p.y = weight;
        p.y_sj = 1;
        p.y_sr = taps * s.out_channels;
        p.ytaps = TapSteps{true, FastDiv((uint32_t)s.channels), taps * s.out_channels, s.out_channels, 0, block,
                           FastDiv((uint32_t)taps)};
        return AXIS_OK;
    }
    if (int st = permuted.get(device, sizeof(float) * (size_t)(c_pad * taps * s.out_channels))) return st;
    if (int st = permute_weight(device, weight, permuted.as<float>(), s, 0, c_pad, block)) return st;
    p.y = permuted.as<float>();
    p.y_sr = s.out_channels;
    p.y_sj = 1;
    return AXIS_OK;
}

// The gathered input of a forward or weight-gradient launch: the caller's tensor when it is
// channel-innermost with a multiple of 4 channels on a 16-byte boundary, otherwise a repacked
// channel-innermost copy with the channels padded to a multiple of 4.
struct GatherInput {
    axis::Scratch copy;
    const float *src = nullptr;
    int64_t ld[4];
    int32_t channels = 0;  // channel extent the GEMM reduces over (padded)

    int prepare(axis_device device, const float *input, const int64_t given[4], int64_t batch,
                int32_t height, int32_t width, int32_t c_in) {
        if (int st = input_strides(given, batch, height, width, c_in, ld)) return st;
        // Gathers address the tensor with 32-bit offsets.
        const int64_t last = (batch - 1) * ld[0] + (int64_t)(c_in - 1) * ld[1] +
                             (int64_t)(height - 1) * ld[2] + (int64_t)(width - 1) * ld[3];
        if (ld[1] == 1 && c_in % 4 == 0 && ld[2] % 4 == 0 && ld[3] % 4 == 0 && ld[0] % 4 == 0 &&
            axis::aligned16(input) && last < INT32_MAX && ld[0] < INT32_MAX) {
            src = input;
            channels = c_in;
            return AXIS_OK;
        }
        channels = (c_in + 3) / 4 * 4;
        const int64_t pixels = batch * height * width;
        AXIS_REQUIRE(pixels * channels < INT32_MAX, "convolution input too large for 32-bit gathers");
        if (int st = copy.get(device, sizeof(float) * (size_t)(pixels * channels))) return st;
        repack_channels_last_kernel<<<axis::blocks_for(pixels * (channels / 4), 256, 1 << 16), 256, 0,
                                      device->stream>>>(input, ld[0], ld[1], ld[2], ld[3], copy.as<float>(),
                                                        pixels, height, width, c_in, channels);
        if (int st = axis::launch_status("repack_channels_last_kernel")) return st;
        src = copy.as<float>();
        channels_last(height, width, channels, ld);
        return AXIS_OK;
    }
};

}  // namespace

namespace axis {

// The device address of this GPU's copy of `scratch`, looked up once per GPU with that GPU
// current (axis_device_create makes it current before calling this), and one event per GPU that
// serialises the array's users across handles (created once, like the array never released).
int bind_static_scratch(axis_device device) {
    static std::mutex guard;
    struct Bound {
        float *address;
        hipEvent_t done;
    };
    static std::unordered_map<int, Bound> bound;
    std::lock_guard<std::mutex> lock(guard);
    auto it = bound.find(device->ordinal);
    if (it == bound.end()) {
        void *address = nullptr;
        hipError_t e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        hipEvent_t done = nullptr;
        e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags(scratch)");
        it = bound.emplace(device->ordinal, Bound{static_cast<float *>(address), done}).first;
    }
    device->static_scratch = it->second.address;
    device->static_scratch_done = it->second.done;
    return AXIS_OK;
}

}  // namespace axis

extern "C" {

int axis_matmul(axis_device device, const float *a, const float *b, float *out, int64_t batch,
                int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * batch * m * k}, {b, 4 * batch * k * n}, {out, 4 * batch * m * n});
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
    return run_gemm<true, false, 0, 0>(device, p, batch, out);
}

int axis_matmul_bias(axis_device device, const float *a, const float *b, const float *bias, float *out,
                     int64_t batch, int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * batch * m * k}, {b, 4 * batch * k * n}, {bias, 4 * n}, {out, 4 * batch * m * n});
    if (int s = check_dims(a, b, out, batch, m, k, n)) return s;
    AXIS_REQUIRE(bias, "null matmul bias");
    AXIS_REQUIRE(bias + n <= out || bias >= out + batch * m * n, "matmul bias must not alias the output");
    GemmParams p{};
    p.x = a;
    p.y = b;
    p.bias = bias;
    p.m = m;
    p.n = n;
    p.k = k;
    p.x_si = k;
    p.x_sr = 1;
    p.y_sr = n;
    p.y_sj = 1;
    p.x_batch = m * k;
    p.y_batch = k * n;
    return run_gemm<true, false, 0, 0>(device, p, batch, out);
}

int axis_matmul_axpby(axis_device device, const float *a, const float *b, const float *d, float *out,
                      int64_t batch, int64_t m, int64_t k, int64_t n, float alpha, float beta) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * batch * m * k}, {b, 4 * batch * k * n}, {d, 4 * batch * m * n}, {out, 4 * batch * m * n});
    if (int s = check_dims(a, b, out, batch, m, k, n)) return s;
    AXIS_REQUIRE(d, "null axpby addend");
    AXIS_REQUIRE(d != out, "axpby addend must not alias the output");
    GemmParams p{};
    p.x = a;
    p.y = b;
    p.d = d;
    p.alpha = alpha;
    p.beta = beta;
    p.m = m;
    p.n = n;
    p.k = k;
    p.x_si = k;
    p.x_sr = 1;
    p.y_sr = n;
    p.y_sj = 1;
    p.x_batch = m * k;
    p.y_batch = k * n;
    return run_gemm<true, false, 0, 0>(device, p, batch, out);
}

int axis_matmul_left_backward(axis_device device, const float *gradient, const float *rhs,
                              float *out, int64_t batch, int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * batch * m * n}, {rhs, 4 * batch * k * n}, {out, 4 * batch * m * k});
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
    return run_gemm<true, true, 0, 0>(device, p, batch, out);
}

int axis_matmul_right_backward(axis_device device, const float *lhs, const float *gradient,
                               float *out, int64_t batch, int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {lhs, 4 * batch * m * k}, {gradient, 4 * batch * m * n}, {out, 4 * batch * k * n});
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
    return run_gemm<false, false, 0, 0>(device, p, batch, out, nullptr, true);
}

int axis_matmul_right_backward_noalloc(axis_device device, const float *lhs, const float *gradient,
                                       float *out, int64_t batch, int64_t m, int64_t k, int64_t n) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {lhs, 4 * batch * m * k}, {gradient, 4 * batch * m * n}, {out, 4 * batch * k * n});
    if (int s = check_dims(lhs, gradient, out, batch, m, k, n)) return s;
    AXIS_REQUIRE(!device->bf16_matmul, "the allocation-free product is fp32 only (a bf16 handle stages operands)");
    AXIS_REQUIRE(device->static_scratch, "static scratch is not bound on this device");
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
    const Workspace ws{device->static_scratch, kStaticScratchFloats};
    // Another handle on this GPU may still be running a call that uses the array: wait for its
    // last launch (a never-recorded event is complete), and mark this call's for the next user.
    // Under stream capture the graph's own order stands in (an event recorded outside the
    // capture is not a node the graph can wait on).
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    AXIS_HIP(hipStreamIsCapturing(device->stream, &capture));
    const bool order = capture == hipStreamCaptureStatusNone;
    if (order) AXIS_HIP(hipStreamWaitEvent(device->stream, device->static_scratch_done, 0));
    if (int st = run_gemm<false, false, 0, 0>(device, p, batch, out, &ws)) return st;
    if (order) AXIS_HIP(hipEventRecord(device->static_scratch_done, device->stream));
    return AXIS_OK;
}

int axis_conv2d_forward(axis_device device, const float *input, const int64_t input_strides_[4],
                        const float *weight, const float *bias, float *out, int64_t batch,
                        int32_t height, int32_t width, int32_t channels, int32_t out_channels,
                        const int32_t kernel[2], const int32_t stride[2], const int32_t padding[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {input, 1}, {weight, 1}, {bias, 4 * (int64_t)out_channels}, {out, 1});
    AXIS_REQUIRE(input && weight && out, "null convolution buffer");
    ConvShape s{};
    if (int st = conv_shape(batch, height, width, channels, out_channels, kernel, stride, padding, &s))
        return st;
    if (!device->bf16_matmul && axis::small_conv_applies(small_shape(s))) {
        int64_t ld[4];
        if (int st = input_strides(input_strides_, batch, height, width, channels, ld)) return st;
        return axis::small_conv_forward(device, small_shape(s), input, ld, weight, bias, out, nullptr, nullptr);
    }
    GatherInput in;
    if (int st = in.prepare(device, input, input_strides_, batch, height, width, channels)) return st;
    const int64_t patch = (int64_t)in.channels * s.kh * s.kw;
    axis::Scratch permuted;
    GemmParams p{};
    p.conv = geom(in.src, in.ld, height, width, in.channels, s.out_h, s.out_w, s.kh, s.kw, s.sy, s.sx, s.py, s.px);
    const bool buffered = buffer_reach(p.conv, batch);
    use_block_major(p.conv, batch);
    if (int st = forward_weight(device, weight, s, in.channels, permuted, p)) return st;
    p.bias = bias;
    p.m = batch * s.out_h * s.out_w;
    p.n = out_channels;
    p.k = patch;
    p.k_work = (int64_t)channels * s.kh * s.kw;
    return buffered ? run_gemm<true, false, 4, 0>(device, p, 1, out)
                    : run_gemm<true, false, 1, 0>(device, p, 1, out);
}

int axis_conv2d_relu_pool_forward(axis_device device, const float *input,
                                  const int64_t input_strides_[4], const float *weight,
                                  const float *bias, float *pooled, uint8_t *argmax, int64_t batch,
                                  int32_t height, int32_t width, int32_t channels,
                                  int32_t out_channels, const int32_t kernel[2],
                                  const int32_t stride[2], const int32_t padding[2],
                                  const int32_t pool[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {input, 1}, {weight, 1}, {bias, 4 * (int64_t)out_channels}, {pooled, 1}, {argmax, 1});
    AXIS_REQUIRE(input && weight && pooled && argmax && pool, "null convolution buffer");
    ConvShape s{};
    if (int st = conv_shape(batch, height, width, channels, out_channels, kernel, stride, padding, &s))
        return st;
    int64_t ld_check[4];
    if (int st = input_strides(input_strides_, batch, height, width, channels, ld_check)) return st;
    AXIS_REQUIRE(pool[0] >= 1 && pool[1] >= 1 && pool[0] * pool[1] < 255,
                 "pool window must be positive with fewer than 255 positions");
    AXIS_REQUIRE(s.out_h % pool[0] == 0 && s.out_w % pool[1] == 0,
                 "fused pooling needs windows that tile the convolution output exactly");
    if (pool[0] == 2 && pool[1] == 2 && !device->bf16_matmul && axis::small_conv_applies(small_shape(s)))
        return axis::small_conv_forward(device, small_shape(s), input, ld_check, weight, bias, nullptr, pooled,
                                        argmax);
    AXIS_REQUIRE(128 % (pool[0] * s.out_w) == 0,
                 "fused pooling needs pool height x output width to divide 128");
    GatherInput in;
    if (int st = in.prepare(device, input, input_strides_, batch, height, width, channels)) return st;
    const int64_t patch = (int64_t)in.channels * s.kh * s.kw;
    axis::Scratch permuted;
    GemmParams p{};
    p.conv = geom(in.src, in.ld, height, width, in.channels, s.out_h, s.out_w, s.kh, s.kw, s.sy, s.sx, s.py, s.px);
    const bool buffered = buffer_reach(p.conv, batch);
    use_block_major(p.conv, batch);
    if (int st = forward_weight(device, weight, s, in.channels, permuted, p)) return st;
    p.bias = bias;
    p.m = batch * s.out_h * s.out_w;
    p.n = out_channels;
    p.k = patch;
    p.k_work = (int64_t)channels * s.kh * s.kw;
    p.pooled = pooled;
    p.argmax = argmax;
    p.pool_h = pool[0];
    p.pool_w = pool[1];
    p.pool_ow = s.out_w;
    p.pool_cols = FastDiv((uint32_t)(s.out_w / pool[1]));
    // 2x2 windows: tile rows window-major, pooled in registers
    p.conv.window_major = pool[0] == 2 && pool[1] == 2;
    p.conv.pw_div = p.pool_cols;
    return buffered ? run_gemm<true, false, 4, 1>(device, p, 1, nullptr)
                    : run_gemm<true, false, 1, 1>(device, p, 1, nullptr);
}

int axis_conv2d_backward_data(axis_device device, const float *gradient, const float *weight,
                              float *d_input, int64_t batch, int32_t height, int32_t width,
                              int32_t channels, int32_t out_channels, const int32_t kernel[2],
                              const int32_t stride[2], const int32_t padding[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 1}, {weight, 1}, {d_input, 4 * batch * height * width * channels});
    AXIS_REQUIRE(gradient && weight && d_input, "null convolution buffer");
    ConvShape s{};
    if (int st = conv_shape(batch, height, width, channels, out_channels, kernel, stride, padding, &s))
        return st;
    AXIS_REQUIRE(s.sy == 1 && s.sx == 1, "implicit convolution dgrad supports stride 1 only");
    AXIS_REQUIRE(s.py <= s.kh - 1 && s.px <= s.kw - 1, "implicit convolution dgrad needs padding < kernel");
    const int64_t taps = (int64_t)s.kh * s.kw;
    // d_input[b, y, x, c] = sum over (ky', kx', n) of gradient[b, y + ky' - (kh-1-py),
    // x + kx' - (kw-1-px), n] * W[(c, kh-1-ky', kw-1-kx'), n]: a stride-1 convolution of the
    // output gradient with the flipped, transposed kernel -- the reference's col2im of
    // gradient . W^T, summed in a different (fp32) order.
    GemmParams p{};
    p.x = gradient;
    p.m = batch * (int64_t)height * width;
    p.n = channels;
    p.k = taps * out_channels;
    int64_t ld[4];
    channels_last(s.out_h, s.out_w, out_channels, ld);
    p.conv = geom(gradient, ld, s.out_h, s.out_w, out_channels, height, width, s.kh, s.kw, 1, 1,
                  s.kh - 1 - s.py, s.kw - 1 - s.px);
    const bool buffered = buffer_reach(p.conv, batch);
    const bool block = use_block_major(p.conv, batch);
    if (out_channels % 32 == 0 && axis::aligned16(weight)) {
        // The flipped, transposed kernel read in place: Y(r, c) with r = (ky', kx', n) is
        // W[c * taps * n_out + (taps - 1 - (ky' * kw + kx')) * n_out + n], so a K step (32
        // consecutive n of one tap, in either row order) is 128 contiguous bytes of each
        // column c, at tap offset (taps - 1) * n_out - pos * n_out.  Same values in the same
        // reduction order as the permuted copy below, so the same bits.
        p.y = weight;
        p.y_sr = 1;
        p.y_sj = taps * out_channels;
        p.ytaps = TapSteps{true, FastDiv((uint32_t)out_channels), 1, -(int64_t)out_channels,
                           (taps - 1) * out_channels, block, FastDiv((uint32_t)taps)};
        return buffered ? run_gemm<true, true, 4, 0>(device, p, 1, d_input)
                        : run_gemm<true, true, 1, 0>(device, p, 1, d_input);
    }
    axis::Scratch flipped;
    if (int st = flipped.get(device, sizeof(float) * (size_t)(taps * channels * out_channels))) return st;
    if (int st = permute_weight(device, weight, flipped.as<float>(), s, 1, channels, block)) return st;
    p.y = flipped.as<float>();
    p.y_sr = channels;
    p.y_sj = 1;
    return buffered ? run_gemm<true, false, 4, 0>(device, p, 1, d_input)
                    : run_gemm<true, false, 1, 0>(device, p, 1, d_input);
}

int axis_conv2d_backward_weight(axis_device device, const float *input,
                                const int64_t input_strides_[4], const float *gradient,
                                float *d_weight, int64_t batch, int32_t height, int32_t width,
                                int32_t channels, int32_t out_channels, const int32_t kernel[2],
                                const int32_t stride[2], const int32_t padding[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {input, 1}, {gradient, 1}, {d_weight, 1});
    AXIS_REQUIRE(input && gradient && d_weight, "null convolution buffer");
    ConvShape s{};
    if (int st = conv_shape(batch, height, width, channels, out_channels, kernel, stride, padding, &s))
        return st;
    GatherInput in;
    if (int st = in.prepare(device, input, input_strides_, batch, height, width, channels)) return st;
    const int64_t patch = (int64_t)in.channels * s.kh * s.kw;
    // Without channel padding the product's rows (ky, kx, c) go straight to the reference's
    // (c, ky, kx) order as the reduction slices are summed.
    const bool direct = in.channels == channels;
    axis::Scratch ordered;
    if (!direct)
        if (int st = ordered.get(device, sizeof(float) * (size_t)(patch * out_channels))) return st;
    GemmParams p{};
    if (direct) {
        p.perm_c = channels;
        p.perm_taps = s.kh * s.kw;
    }
    p.y = gradient;
    p.m = patch;
    p.n = out_channels;
    p.k = batch * (int64_t)s.out_h * s.out_w;
    // rows past the real channels are padding: time the algorithmic 2 * patch * n * pixels
    p.k_work = (int64_t)((double)p.k * (double)channels / (double)in.channels);
    p.y_sr = out_channels;
    p.y_sj = 1;
    p.conv = geom(in.src, in.ld, height, width, in.channels, s.out_h, s.out_w, s.kh, s.kw, s.sy, s.sx, s.py, s.px);
    // Every tile shape is 32 deep: when 32-pixel steps never straddle an image and cut its rows
    // the same way each time, the cheaper step loader applies.
    const int64_t image = (int64_t)s.out_h * s.out_w;
    // (the step loader also needs the padding inside the first column segment and row group)
    const int32_t rows_per_step = s.out_w < 32 ? 32 / s.out_w : 1;
    const bool aligned = (32 % s.out_w == 0 || s.out_w % 32 == 0) && image % 32 == 0 && s.px <= 32 * s.sx &&
                         s.py <= rows_per_step * s.sy;
    float *dst = direct ? d_weight : ordered.as<float>();
    const int st = aligned ? run_gemm<false, false, 3, 0>(device, p, 1, dst, nullptr, direct)
                           : run_gemm<false, false, 2, 0>(device, p, 1, dst, nullptr, direct);
    if (st || direct) return st;
    return permute_weight(device, ordered.as<float>(), d_weight, s, 2, in.channels);
}


int axis_conv2d_relu_pool_backward_weight(axis_device device, const float *input,
                                          const int64_t input_strides_[4], const float *gradient,
                                          const float *pooled, const uint8_t *argmax, float *d_weight,
                                          float *d_bias, int64_t batch, int32_t height, int32_t width,
                                          int32_t channels, int32_t out_channels, const int32_t kernel[2],
                                          const int32_t stride[2], const int32_t padding[2],
                                          const int32_t pool[2]) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {input, 1}, {gradient, 1}, {pooled, 1}, {argmax, 1}, {d_weight, 1}, {d_bias, 4 * (int64_t)out_channels});
    AXIS_REQUIRE(input && gradient && pooled && argmax && d_weight && pool, "null convolution buffer");
    ConvShape s{};
    if (int st = conv_shape(batch, height, width, channels, out_channels, kernel, stride, padding, &s))
        return st;
    int64_t ld[4];
    if (int st = input_strides(input_strides_, batch, height, width, channels, ld)) return st;
    AXIS_REQUIRE(pool[0] >= 1 && pool[1] >= 1 && pool[0] * pool[1] < 255 && s.out_h % pool[0] == 0 &&
                     s.out_w % pool[1] == 0,
                 "fused pooling needs windows that tile the convolution output exactly");
    if (pool[0] == 2 && pool[1] == 2 && !device->bf16_matmul && axis::small_conv_applies(small_shape(s)))
        return axis::small_conv_pool_backward_weight(device, small_shape(s), input, ld, gradient, pooled, argmax,
                                                     d_weight, d_bias);
    // Any other shape: the pre-activation gradient through axis_relu_pool_backward, then the
    // weight gradient of the convolution.
    axis::Scratch d_pre;
    if (int st = d_pre.get(device, sizeof(float) * (size_t)(batch * s.out_h * s.out_w * out_channels))) return st;
    if (int st = axis_relu_pool_backward(device, gradient, pooled, argmax, d_pre.as<float>(), d_bias, batch, s.out_h,
                                         s.out_w, out_channels, pool))
        return st;
    return axis_conv2d_backward_weight(device, input, input_strides_, d_pre.as<float>(), d_weight, batch, height,
                                       width, channels, out_channels, kernel, stride, padding);
}

}  // extern "C"
