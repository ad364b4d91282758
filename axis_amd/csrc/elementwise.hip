// Bandwidth-bound elementwise, layout and reduction entries (runtime/backend.rs kernels
// :2057-2188, :2588-2640, :2797-2801) and the fused bias/reduction entries of axis_hip.h.
//
// Streaming kernels move 16-byte vectors when every pointer is 16-byte aligned, with a scalar
// tail; reductions keep the reference's association (sequential chunks of 512, then chunk
// partials in order) so they are bit-identical to a sequential restatement.  Built with
// -ffp-contract=off: every expression rounds exactly as written.
#include <algorithm>
#include <cfloat>

#include "common.hpp"
#include "column_sum.hpp"
#include "fastdiv.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;

// ---------------------------------------------------------------- generic streaming map

template <class F>
__global__ void __launch_bounds__(kBlock) map_kernel(F f, int64_t len, bool vec) {
    const int64_t tid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    if (vec) {
        const int64_t nv = len / 4;
        for (int64_t v = tid; v < nv; v += stride) f.vec(v);
        for (int64_t i = nv * 4 + tid; i < len; i += stride) f.one(i);
    } else {
        for (int64_t i = tid; i < len; i += stride) f.one(i);
    }
}

template <class F>
int launch_map(axis_device device, const F &f, int64_t len, bool vec, const char *name) {
    if (len <= 0) return AXIS_OK;
    const int64_t work = vec ? (len + 3) / 4 : len;
    const unsigned blocks = axis::blocks_for(work, kBlock, (int64_t)device->multiprocessors * 16);
    map_kernel<<<blocks, kBlock, 0, device->stream>>>(f, len, vec);
    return axis::launch_status(name);
}

#define LOAD4(p, v) (reinterpret_cast<const floatx4 *>(p)[v])
#define STORE4(p, v, x) (reinterpret_cast<floatx4 *>(p)[v] = (x))

struct MaskGradient {
    const float *g, *w;
    float *out;
    __device__ void one(int64_t i) const { out[i] = w[i] > 0.0f ? g[i] : 0.0f; }
    __device__ void vec(int64_t v) const {
        floatx4 a = LOAD4(g, v), m = LOAD4(w, v), r;
        for (int c = 0; c < 4; ++c) r[c] = m[c] > 0.0f ? a[c] : 0.0f;
        STORE4(out, v, r);
    }
};

struct Relu {
    const float *a;
    float *out;
    __device__ void one(int64_t i) const { out[i] = a[i] > 0.0f ? a[i] : 0.0f; }
    __device__ void vec(int64_t v) const {
        floatx4 x = LOAD4(a, v), r;
        for (int c = 0; c < 4; ++c) r[c] = x[c] > 0.0f ? x[c] : 0.0f;
        STORE4(out, v, r);
    }
};

struct ReluBackward {
    const float *g, *a;
    float *out;
    __device__ void one(int64_t i) const { out[i] = a[i] > 0.0f ? g[i] : 0.0f; }
    __device__ void vec(int64_t v) const {
        floatx4 x = LOAD4(a, v), d = LOAD4(g, v), r;
        for (int c = 0; c < 4; ++c) r[c] = x[c] > 0.0f ? d[c] : 0.0f;
        STORE4(out, v, r);
    }
};

struct Scale {
    const float *a;
    float factor;
    float *out;
    __device__ void one(int64_t i) const { out[i] = a[i] * factor; }
    __device__ void vec(int64_t v) const { STORE4(out, v, LOAD4(a, v) * factor); }
};

template <int OP>
struct Binary {
    const float *a, *b;
    float *out;
    __device__ static float apply(float x, float y) {
        return OP == 0 ? x + y : OP == 1 ? x - y : OP == 2 ? x * y : x / y;
    }
    __device__ void one(int64_t i) const { out[i] = apply(a[i], b[i]); }
    __device__ void vec(int64_t v) const {
        floatx4 x = LOAD4(a, v), y = LOAD4(b, v), r;
        for (int c = 0; c < 4; ++c) r[c] = apply(x[c], y[c]);
        STORE4(out, v, r);
    }
};

struct InverseSqrt {
    const float *a;
    float eps;
    float *out;
    __device__ void one(int64_t i) const { out[i] = 1.0f / sqrtf(a[i] + eps); }
    __device__ void vec(int64_t v) const {
        floatx4 x = LOAD4(a, v), r;
        for (int c = 0; c < 4; ++c) r[c] = 1.0f / sqrtf(x[c] + eps);
        STORE4(out, v, r);
    }
};

struct MultiplyScalar {
    const float *a, *s;
    float *out;
    __device__ void one(int64_t i) const { out[i] = a[i] * s[0]; }
    __device__ void vec(int64_t v) const { STORE4(out, v, LOAD4(a, v) * s[0]); }
};

bool all_aligned(std::initializer_list<const void *> ptrs) {
    for (const void *p : ptrs)
        if (p && !axis::aligned16(p)) return false;
    return true;
}

// ---------------------------------------------------------------- select_axis

struct SelectArgs {
    int32_t rank;
    int32_t coordinate;
    FastDiv place[10];   // divisor giving the coordinate from the flat index
    FastDiv extent[10];
    int32_t far[10];     // stride on the other side
    int32_t selected[10];
    int32_t len;
};

__global__ void __launch_bounds__(kBlock) select_axis_kernel(const float *__restrict__ input,
                                                             float *__restrict__ out, SelectArgs a) {
    const uint32_t o = blockIdx.x * kBlock + threadIdx.x;
    if (o >= (uint32_t)a.len) return;
    int64_t index = 0;
    for (int d = 0; d < a.rank; ++d) {
        if (a.selected[d])
            index += (int64_t)a.coordinate * a.far[d];
        else
            index += (int64_t)a.extent[d].mod(a.place[d].div(o)) * a.far[d];
    }
    out[o] = input[index];
}

__global__ void __launch_bounds__(kBlock) select_axis_backward_kernel(const float *__restrict__ gradient,
                                                                      float *__restrict__ out,
                                                                      SelectArgs a) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= (uint32_t)a.len) return;
    int64_t index = 0;
    bool live = true;
    for (int d = 0; d < a.rank; ++d) {
        const int32_t c = (int32_t)a.extent[d].mod(a.place[d].div(i));
        if (a.selected[d])
            live = live && c == a.coordinate;
        else
            index += (int64_t)c * a.far[d];
    }
    out[i] = live ? gradient[index] : 0.0f;
}

// A permutation copy whose destination-innermost dim is strided in the source while another dim
// is source-contiguous goes through LDS 64 x 64 tiles: the tile is read along the source's
// contiguous dim (J) and written along the destination's (T), so both sides move whole cache
// lines.  Remaining dims are batch dims, one per grid row.
constexpr int kTile = 64;
constexpr int kMaxBatchDims = 8;

struct TransposeArgs {
    int64_t base;                 // source offset of the selected coordinate
    int64_t t_src;                // source stride of T (its destination stride is 1)
    int64_t j_dst;                // destination stride of J (its source stride is 1)
    int32_t t_extent, j_extent, tiles_t;
    int32_t batch_dims;
    int32_t b_extent[kMaxBatchDims];
    int64_t b_src[kMaxBatchDims], b_dst[kMaxBatchDims];
};

__global__ void __launch_bounds__(256) transpose_copy_kernel(const float *__restrict__ src,
                                                             float *__restrict__ dst, TransposeArgs a) {
    __shared__ float tile[kTile][kTile + 1];
    const int t0 = (int)(blockIdx.x % (uint32_t)a.tiles_t) * kTile;
    const int j0 = (int)(blockIdx.x / (uint32_t)a.tiles_t) * kTile;
    uint32_t b = blockIdx.y;
    int64_t s_off = a.base, d_off = 0;
    for (int d = a.batch_dims - 1; d >= 0; --d) {
        const uint32_t c = b % (uint32_t)a.b_extent[d];
        b /= (uint32_t)a.b_extent[d];
        s_off += (int64_t)c * a.b_src[d];
        d_off += (int64_t)c * a.b_dst[d];
    }
    const int lane = threadIdx.x & 63, row = threadIdx.x >> 6;
    const int j = j0 + lane;
#pragma unroll 4
    for (int tt = row; tt < kTile; tt += 4) {
        const int t = t0 + tt;
        if (j < a.j_extent && t < a.t_extent) tile[tt][lane] = src[s_off + j + (int64_t)t * a.t_src];
    }
    __syncthreads();
    const int t = t0 + lane;
#pragma unroll 4
    for (int jj = row; jj < kTile; jj += 4) {
        const int jo = j0 + jj;
        if (jo < a.j_extent && t < a.t_extent) dst[d_off + (int64_t)jo * a.j_dst + t] = tile[lane][jj];
    }
}

// Canonical form of a select_axis copy: dims of extent > 1 sorted by destination stride (outer
// first), runs contiguous on both sides merged, the selected coordinate folded into the source
// base.  Returns false when the copy is not a plain permutation/broadcast onto a dense
// destination (the backward of a selection, which zero-fills, is not).
struct CopyDims {
    int rank = 0;
    int64_t extent[10], src[10], dst[10];
    int64_t base = 0;
};

bool canonical_copy(const int32_t *metadata, int32_t rank, int32_t coordinate, bool forward, CopyDims *c) {
    c->rank = 0;
    c->base = 0;
    for (int d = 0; d < rank; ++d) {
        const int64_t extent = metadata[3 * d], in_stride = metadata[3 * d + 1], out_stride = metadata[3 * d + 2];
        if (out_stride < 0) {
            if (!forward) return false;
            c->base += (int64_t)coordinate * in_stride;
            continue;
        }
        if (extent == 1) continue;
        c->extent[c->rank] = extent;
        c->src[c->rank] = forward ? in_stride : out_stride;
        c->dst[c->rank] = forward ? out_stride : in_stride;
        ++c->rank;
    }
    for (int i = 1; i < c->rank; ++i)  // insertion sort, destination stride descending
        for (int k = i; k > 0 && c->dst[k] > c->dst[k - 1]; --k) {
            std::swap(c->extent[k], c->extent[k - 1]);
            std::swap(c->src[k], c->src[k - 1]);
            std::swap(c->dst[k], c->dst[k - 1]);
        }
    int merged = 0;
    for (int i = 0; i < c->rank; ++i) {
        if (merged > 0 && c->dst[merged - 1] == c->dst[i] * c->extent[i] &&
            c->src[merged - 1] == c->src[i] * c->extent[i]) {
            c->extent[merged - 1] *= c->extent[i];
            c->src[merged - 1] = c->src[i];
            c->dst[merged - 1] = c->dst[i];
            continue;
        }
        c->extent[merged] = c->extent[i];
        c->src[merged] = c->src[i];
        c->dst[merged] = c->dst[i];
        ++merged;
    }
    c->rank = merged;
    int64_t expect = 1;
    for (int i = c->rank - 1; i >= 0; --i) {
        if (c->dst[i] != expect) return false;
        expect *= c->extent[i];
    }
    return true;
}

// Launches the tiled transpose when the canonical copy has one; returns -1 when it does not.
int try_transpose(axis_device device, const float *src, float *dst, const int32_t *metadata, int32_t rank,
                  int32_t coordinate, bool forward) {
    CopyDims c;
    if (!canonical_copy(metadata, rank, coordinate, forward, &c) || c.rank < 2) return -1;
    const int last = c.rank - 1;
    if (c.src[last] == 1) return -1;  // rows already contiguous on both sides
    int j = -1;
    for (int i = 0; i < last; ++i)
        if (c.src[i] == 1) j = i;
    if (j < 0 || c.extent[last] < 16 || c.extent[j] < 16 || c.rank - 2 > kMaxBatchDims) return -1;
    TransposeArgs a{};
    a.base = c.base;
    a.t_src = c.src[last];
    a.j_dst = c.dst[j];
    a.t_extent = (int32_t)c.extent[last];
    a.j_extent = (int32_t)c.extent[j];
    a.tiles_t = (a.t_extent + kTile - 1) / kTile;
    const int64_t tiles_j = (a.j_extent + kTile - 1) / kTile;
    int64_t batch = 1;
    for (int i = 0; i < last; ++i) {
        if (i == j) continue;
        a.b_extent[a.batch_dims] = (int32_t)c.extent[i];
        a.b_src[a.batch_dims] = c.src[i];
        a.b_dst[a.batch_dims] = c.dst[i];
        ++a.batch_dims;
        batch *= c.extent[i];
    }
    if (batch > 65535 || a.tiles_t * tiles_j >= INT32_MAX) return -1;
    dim3 grid((unsigned)(a.tiles_t * tiles_j), (unsigned)batch);
    transpose_copy_kernel<<<grid, 256, 0, device->stream>>>(src, dst, a);
    return axis::launch_status("transpose_copy_kernel");
}

int select_args(const int32_t *metadata, int32_t rank, int32_t coordinate, int64_t len, bool forward,
                SelectArgs *a) {
    AXIS_REQUIRE(metadata, "null select metadata");
    AXIS_REQUIRE(rank >= 0 && rank <= 10, "select_axis rank must be 0..10");
    AXIS_REQUIRE(len >= 1 && len <= INT32_MAX - kBlock, "select_axis length out of range");
    a->rank = rank;
    a->coordinate = coordinate;
    a->len = (int32_t)len;
    for (int d = 0; d < rank; ++d) {
        const int32_t extent = metadata[3 * d], in_stride = metadata[3 * d + 1],
                      out_stride = metadata[3 * d + 2];
        AXIS_REQUIRE(extent >= 1, "select_axis extents must be positive");
        a->extent[d] = FastDiv((uint32_t)extent);
        a->selected[d] = out_stride < 0;
        if (forward) {
            // out index decodes through output_stride; the input is addressed by input_stride.
            a->place[d] = FastDiv((uint32_t)(out_stride < 0 ? 1 : out_stride));
            a->far[d] = in_stride;
        } else {
            a->place[d] = FastDiv((uint32_t)(in_stride < 1 ? 1 : in_stride));
            a->far[d] = out_stride;
        }
    }
    return AXIS_OK;
}

// ---------------------------------------------------------------- sum of squares

__device__ __forceinline__ float wave_sum(float v) {
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset);
    return v;
}

__global__ void __launch_bounds__(kBlock) sum_squares_kernel(const float *__restrict__ a, int64_t len,
                                                             float *__restrict__ partial) {
    __shared__ float waves[kBlock / 64];
    float s = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < len; i += (int64_t)gridDim.x * kBlock)
        s += a[i] * a[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < kBlock / 64; ++w) t += waves[w];
        partial[blockIdx.x] = t;
    }
}

__global__ void __launch_bounds__(kBlock) sum_kernel(const float *__restrict__ partial, int n,
                                                     float *__restrict__ out) {
    __shared__ float waves[kBlock / 64];
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kBlock) s += partial[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < kBlock / 64; ++w) t += waves[w];
        out[0] = t;
    }
}

// ---------------------------------------------------------------- bias entries

struct BiasAdd {
    const float *a, *bias;
    float *out, *relu_out;
    FastDiv width_div;
    int64_t width;
    __device__ void one(int64_t i) const {
        const float z = a[i] + bias[i % width];
        out[i] = z;
        if (relu_out) relu_out[i] = z > 0.0f ? z : 0.0f;
    }
    __device__ void vec(int64_t v) const {
        const floatx4 x = LOAD4(a, v);
        const int64_t c0 = (v * 4) % width;  // width % 4 == 0 on this path
        const floatx4 b = LOAD4(bias + c0, 0);
        const floatx4 z = x + b;
        STORE4(out, v, z);
        if (relu_out) {
            floatx4 r;
            for (int c = 0; c < 4; ++c) r[c] = z[c] > 0.0f ? z[c] : 0.0f;
            STORE4(relu_out, v, r);
        }
    }
};

// Stage one of the bias gradient: partial[q][c] = sum of rows [512q, 512q+512) of column c,
// sequentially; optionally masked by relu_input > 0 (and the masked gradient written out).
// Block (column group, chunk): the chunk's rows of 16 columns are staged in LDS first -- every
// load of the chunk in flight at once, coalesced in 64-byte row segments -- then one lane per
// column adds its 512 (or fewer) rows in row order.  A lane summing straight from memory waits on
// one round trip per batch of loads: 8.4 us for a [256, 1000] gradient against ~3 us staged.
constexpr int kChunkCols = 8;
template <bool MASK>
__global__ void __launch_bounds__(kBlock) column_chunk_kernel(const float *__restrict__ g,
                                                              const float *__restrict__ relu_input,
                                                              float *__restrict__ masked_out,
                                                              float *__restrict__ partial,
                                                              int64_t rows, int64_t width, int64_t chunks,
                                                              float *__restrict__ out) {
    static_assert(axis::kGroupedChunk * kChunkCols % kBlock == 0, "whole staging passes");
    constexpr int kPasses = axis::kGroupedChunk * kChunkCols / kBlock;
    constexpr int kRowsPerPass = kBlock / kChunkCols;
    __shared__ float staged[axis::kGroupedChunk][kChunkCols + 1];
    const int tid = threadIdx.x;
    const int cl = tid % kChunkCols;
    const int64_t c = (int64_t)blockIdx.x * kChunkCols + cl;
    for (int64_t q = blockIdx.y; q < chunks; q += gridDim.y) {
        const int64_t r0 = q * axis::kGroupedChunk;
        const int n_rows = (int)(r0 + axis::kGroupedChunk < rows ? axis::kGroupedChunk : rows - r0);
        float v[kPasses];
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
            const int r = u * kRowsPerPass + tid / kChunkCols;
            v[u] = 0.0f;
            if (r < n_rows && c < width) {
                const int64_t idx = (r0 + r) * width + c;
                v[u] = g[idx];
                if (MASK) {
                    v[u] = relu_input[idx] > 0.0f ? v[u] : 0.0f;
                    masked_out[idx] = v[u];
                }
            }
        }
        __syncthreads();  // the previous chunk's sums have read the stage
#pragma unroll
        for (int u = 0; u < kPasses; ++u) staged[u * kRowsPerPass + tid / kChunkCols][cl] = v[u];
        __syncthreads();
        if (tid < kChunkCols && c < width) {
            float sum = 0.0f;
            for (int r = 0; r < n_rows; ++r) sum = sum + staged[r][tid];
            // A single chunk is also the whole sum: the combine's 0 + p0 (scale 1) written here.
            if (out)
                out[c] = 0.0f + sum;
            else
                partial[q * width + c] = sum;
        }
    }
}

// The same chunk sums for wide operands: 64 columns per block, so every row read (and masked
// write) is one 256-byte segment per wave.  A chunk's 512 rows pass through LDS 128 at a time;
// wave 0's lane per column keeps adding in row order across the passes, so each sum has the
// association of column_chunk_kernel.
constexpr int kWideCols = 64, kWideRows = 128;
template <bool MASK>
__global__ void __launch_bounds__(kBlock) column_chunk_wide_kernel(const float *__restrict__ g,
                                                                   const float *__restrict__ relu_input,
                                                                   float *__restrict__ masked_out,
                                                                   float *__restrict__ partial, int64_t rows,
                                                                   int64_t width, int64_t chunks,
                                                                   float *__restrict__ out) {
    static_assert(kBlock == 256 && kWideRows % 4 == 0, "four waves stage whole row groups");
    constexpr int kPerLane = kWideRows / 4;
    __shared__ float staged[kWideRows][kWideCols + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * kWideCols + lane;
    for (int64_t q = blockIdx.y; q < chunks; q += gridDim.y) {
        const int64_t r0 = q * axis::kGroupedChunk;
        const int n_rows = (int)(r0 + axis::kGroupedChunk < rows ? axis::kGroupedChunk : rows - r0);
        float sum = 0.0f;
        for (int base = 0; base < n_rows; base += kWideRows) {
            float v[kPerLane];
#pragma unroll
            for (int u = 0; u < kPerLane; ++u) {
                const int r = base + 4 * u + wave;
                v[u] = 0.0f;
                if (r < n_rows && c < width) {
                    const int64_t idx = (r0 + r) * width + c;
                    v[u] = g[idx];
                    if (MASK) {
                        v[u] = relu_input[idx] > 0.0f ? v[u] : 0.0f;
                        masked_out[idx] = v[u];
                    }
                }
            }
            __syncthreads();  // the previous pass's sums have read the stage
#pragma unroll
            for (int u = 0; u < kPerLane; ++u) staged[4 * u + wave][lane] = v[u];
            __syncthreads();
            if (wave == 0 && c < width) {
                const int lim = n_rows - base < kWideRows ? n_rows - base : kWideRows;
                for (int r = 0; r < lim; ++r) sum = sum + staged[r][lane];
            }
        }
        if (wave == 0 && c < width) {
            if (out)
                out[c] = 0.0f + sum;
            else
                partial[q * width + c] = sum;
        }
    }
}

// out[o][i] = factor * sum_r a[o][r][i] in the reference's chunked order.
__global__ void __launch_bounds__(kBlock) reduce_middle_kernel(const float *__restrict__ a,
                                                               float *__restrict__ out, int64_t outer,
                                                               int64_t reduce, int64_t inner,
                                                               float factor) {
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= outer * inner) return;
    const int64_t o = t / inner, i = t % inner;
    const float *base = a + o * reduce * inner + i;
    // Sequential sums in the plan's order; the loads of 32 terms are issued before their adds so
    // each thread keeps 32 reads in flight instead of one.
    constexpr int kBatch = 32;
    float total = 0.0f;
    for (int64_t r0 = 0; r0 < reduce; r0 += axis::kGroupedChunk) {
        const int64_t r1 = r0 + axis::kGroupedChunk < reduce ? r0 + axis::kGroupedChunk : reduce;
        float partial = 0.0f;
        int64_t r = r0;
        for (; r + kBatch <= r1; r += kBatch) {
            float v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) v[u] = base[(r + u) * inner];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) partial = partial + v[u];
        }
        for (; r < r1; ++r) partial = partial + base[r * inner];
        total = total + partial;
    }
    out[t] = total * factor;
}

// ---------------------------------------------------------------- reductions over any axis set

// Sum over any set of dims of a densely laid-out tensor, without an index plan.  The reduced
// dims are walked in decreasing input stride (row-major over them), i.e. every group's
// contributions in increasing memory position -- the order Plan::reverse lists them
// (runtime/backend.rs:1577-1583) -- summed in chunks of 512, then the chunk partials in order,
// then scaled (backend.rs:2964-3016).  The output is row-major over the kept dims in shape order.
constexpr int kMaxReduceDims = 10;

struct ReduceAxesArgs {
    int32_t kept_rank, red_rank;
    FastDiv kept_place[kMaxReduceDims], kept_extent[kMaxReduceDims];
    int64_t kept_src[kMaxReduceDims];
    FastDiv red_place[kMaxReduceDims], red_extent[kMaxReduceDims];
    int64_t red_src[kMaxReduceDims];
    int64_t outputs, count, chunks;
    float factor;
};

// Thread (q, o): the sum of chunk q of output o's contributions.  With one chunk the value is
// final (0 + partial == partial, then the scale); otherwise it goes to partial[q][o].
__global__ void __launch_bounds__(kBlock) reduce_axes_chunk_kernel(const float *__restrict__ a,
                                                                   float *__restrict__ dst, ReduceAxesArgs r) {
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= r.outputs * r.chunks) return;
    const uint32_t o = (uint32_t)(t % r.outputs);
    const int64_t q = t / r.outputs;
    int64_t base = 0;
    for (int d = 0; d < r.kept_rank; ++d) base += (int64_t)r.kept_extent[d].mod(r.kept_place[d].div(o)) * r.kept_src[d];
    const int64_t j0 = q * axis::kGroupedChunk;
    const int64_t j1 = j0 + axis::kGroupedChunk < r.count ? j0 + axis::kGroupedChunk : r.count;
    float sum = 0.0f;
    if (r.red_rank == 1) {
        const float *p = a + base;
        for (int64_t j = j0; j < j1; ++j) sum = sum + p[j * r.red_src[0]];
    } else {
        for (int64_t j = j0; j < j1; ++j) {
            int64_t off = base;
            for (int d = 0; d < r.red_rank; ++d)
                off += (int64_t)r.red_extent[d].mod(r.red_place[d].div((uint32_t)j)) * r.red_src[d];
            sum = sum + a[off];
        }
    }
    if (r.chunks == 1)
        dst[o] = sum * r.factor;
    else
        dst[q * r.outputs + o] = sum;
}

__global__ void __launch_bounds__(kBlock) reduce_axes_combine_kernel(const float *__restrict__ partial,
                                                                     float *__restrict__ out, int64_t outputs,
                                                                     int64_t chunks, float factor) {
    const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (o >= outputs) return;
    float total = 0.0f;
    for (int64_t q = 0; q < chunks; ++q) total = total + partial[q * outputs + o];
    out[o] = total * factor;
}

// Backward: every input element (in memory order) gets factor * gradient[its kept coordinates].
struct BroadcastAxesArgs {
    int32_t rank;
    FastDiv place[kMaxReduceDims], extent[kMaxReduceDims];  // dims in decreasing input stride
    int64_t out_stride[kMaxReduceDims];                     // 0 for reduced dims
    int64_t len;
    float factor;
};

__global__ void __launch_bounds__(kBlock) broadcast_axes_kernel(const float *__restrict__ g, float *__restrict__ out,
                                                                BroadcastAxesArgs b) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= b.len) return;
    int64_t off = 0;
    for (int d = 0; d < b.rank; ++d)
        off += (int64_t)b.extent[d].mod(b.place[d].div((uint32_t)i)) * b.out_stride[d];
    out[i] = g[off] * b.factor;
}

// Validates a dense layout (strides a permutation of row-major ones over the extents) and
// returns the dims ordered by decreasing stride.
int dense_order(int32_t rank, const int64_t *extents, const int64_t *strides, int *order, int64_t *len) {
    AXIS_REQUIRE(rank >= 1 && rank <= kMaxReduceDims, "reduce_axes rank must be 1..10");
    AXIS_REQUIRE(extents && strides, "null reduce_axes geometry");
    *len = 1;
    for (int d = 0; d < rank; ++d) {
        AXIS_REQUIRE(extents[d] >= 1 && strides[d] >= 0, "reduce_axes extents must be positive");
        *len *= extents[d];
        AXIS_REQUIRE(*len <= INT32_MAX - kBlock, "reduce_axes tensor too large");
        order[d] = d;
    }
    for (int i = 1; i < rank; ++i)  // stable: unit dims keep their order
        for (int k = i; k > 0 && strides[order[k]] > strides[order[k - 1]]; --k) std::swap(order[k], order[k - 1]);
    int64_t expect = 1;
    for (int i = rank - 1; i >= 0; --i) {
        const int d = order[i];
        AXIS_REQUIRE(extents[d] == 1 || strides[d] == expect, "reduce_axes needs a dense layout");
        expect *= extents[d];
    }
    return AXIS_OK;
}

// ---------------------------------------------------------------- extreme over one axis

// Tensor::min over one axis (tensor.rs:2880-2946: grouped_minimum over a forward plan that lists
// each output's members in increasing coordinate along the axis, then the winner mask over the
// gather plan, backend.rs:1365-1440, kernels :3019-3116) without the plans.  A thread per output:
// the first strictly better FINITE value in axis order wins; NaN and an all-zero mask when none is
// finite.  Outputs are row-major over the kept dims in dim order.
struct ExtremeAxisArgs {
    int32_t kept_rank;
    FastDiv kept_place[kMaxReduceDims], kept_extent[kMaxReduceDims];
    int64_t kept_src[kMaxReduceDims];
    int64_t axis_extent, axis_stride, outputs;
};

__device__ __forceinline__ int64_t extreme_base(const ExtremeAxisArgs &x, int64_t o) {
    int64_t off = 0;
    for (int d = 0; d < x.kept_rank; ++d)
        off += (int64_t)x.kept_extent[d].mod(x.kept_place[d].div((uint32_t)o)) * x.kept_src[d];
    return off;
}

template <bool MAXIMUM>
__global__ void __launch_bounds__(kBlock) extreme_axis_kernel(const float *__restrict__ a, float *__restrict__ out,
                                                              float *__restrict__ mask, ExtremeAxisArgs x) {
    const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (o >= x.outputs) return;
    const int64_t base = extreme_base(x, o);
    float best = MAXIMUM ? -INFINITY : INFINITY;
    int64_t winner = -1;
    for (int64_t c = 0; c < x.axis_extent; ++c) {
        const float v = a[base + c * x.axis_stride];
        const bool finite = v >= -FLT_MAX && v <= FLT_MAX;
        if (finite && (MAXIMUM ? v > best : v < best)) {
            best = v;
            winner = c;
        }
    }
    out[o] = winner >= 0 ? best : __builtin_nanf("");
    for (int64_t c = 0; c < x.axis_extent; ++c) mask[base + c * x.axis_stride] = c == winner ? 1.0f : 0.0f;
}

// Its backward (Rule::Minimum, tensor.rs:5679-5683): the gather plan's grouped sum gives every
// member (0 + g) * 1 of its output, and mask_gradient keeps it at the winner.
__global__ void __launch_bounds__(kBlock) extreme_axis_backward_kernel(const float *__restrict__ g,
                                                                       const float *__restrict__ mask,
                                                                       float *__restrict__ out, ExtremeAxisArgs x) {
    const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (o >= x.outputs) return;
    const int64_t base = extreme_base(x, o);
    const float expanded = (0.0f + g[o]) * 1.0f;
    for (int64_t c = 0; c < x.axis_extent; ++c) {
        const int64_t at = base + c * x.axis_stride;
        out[at] = mask[at] > 0.0f ? expanded : 0.0f;
    }
}

int extreme_axis_args(int32_t rank, const int64_t *extents, const int64_t *strides, int32_t axis,
                      ExtremeAxisArgs &x) {
    int order[kMaxReduceDims];
    int64_t len = 0;
    if (int st = dense_order(rank, extents, strides, order, &len)) return st;
    AXIS_REQUIRE(axis >= 0 && axis < rank, "extreme_axis axis out of range");
    x = ExtremeAxisArgs{};
    x.axis_extent = extents[axis];
    x.axis_stride = strides[axis];
    x.outputs = len / extents[axis];
    int64_t place = 1;
    int kr = 0;
    int kept[kMaxReduceDims];
    for (int d = 0; d < rank; ++d)
        if (d != axis) kept[kr++] = d;
    x.kept_rank = kr;
    for (int i = kr - 1; i >= 0; --i) {
        const int d = kept[i];
        x.kept_place[i] = FastDiv((uint32_t)place);
        x.kept_extent[i] = FastDiv((uint32_t)extents[d]);
        x.kept_src[i] = strides[d];
        place *= extents[d];
    }
    return AXIS_OK;
}

struct BroadcastMiddle {
    const float *g;
    float *out;
    int64_t reduce, inner;
    float factor;
    __device__ void one(int64_t idx) const {
        const int64_t i = idx % inner;
        const int64_t o = idx / (reduce * inner);
        out[idx] = g[o * inner + i] * factor;
    }
    __device__ void vec(int64_t v) const {
        const int64_t idx = v * 4;  // inner % 4 == 0 on this path
        const int64_t i = idx % inner;
        const int64_t o = idx / (reduce * inner);
        STORE4(out, v, LOAD4(g + o * inner + i, 0) * factor);
    }
};

}  // namespace

extern "C" {

int axis_mask_gradient(axis_device device, const float *gradient, const float *winners, float *out,
                       int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * len}, {winners, 4 * len}, {out, 4 * len});
    AXIS_REQUIRE(len >= 0 && (len == 0 || (gradient && winners && out)), "bad mask_gradient args");
    return launch_map(device, MaskGradient{gradient, winners, out}, len,
                      all_aligned({gradient, winners, out}), "mask_gradient");
}

int axis_relu(axis_device device, const float *a, float *out, int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * len}, {out, 4 * len});
    AXIS_REQUIRE(len >= 0 && (len == 0 || (a && out)), "bad relu args");
    return launch_map(device, Relu{a, out}, len, all_aligned({a, out}), "relu");
}

int axis_relu_backward(axis_device device, const float *gradient, const float *a, float *out,
                       int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * len}, {a, 4 * len}, {out, 4 * len});
    AXIS_REQUIRE(len >= 0 && (len == 0 || (gradient && a && out)), "bad relu_backward args");
    return launch_map(device, ReluBackward{gradient, a, out}, len, all_aligned({gradient, a, out}),
                      "relu_backward");
}

int axis_scale(axis_device device, const float *a, float factor, float *out, int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * len}, {out, 4 * len});
    AXIS_REQUIRE(len >= 0 && (len == 0 || (a && out)), "bad scale args");
    return launch_map(device, Scale{a, factor, out}, len, all_aligned({a, out}), "scale");
}

int axis_binary(axis_device device, const float *a, const float *b, int32_t op, float *out,
                int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * len}, {b, 4 * len}, {out, 4 * len});
    AXIS_REQUIRE(op >= 0 && op <= 3, "binary op must be 0 (add), 1 (sub), 2 (mul) or 3 (div)");
    AXIS_REQUIRE(len >= 0 && (len == 0 || (a && b && out)), "bad binary args");
    const bool v = all_aligned({a, b, out});
    switch (op) {
    case 0: return launch_map(device, Binary<0>{a, b, out}, len, v, "binary_add");
    case 1: return launch_map(device, Binary<1>{a, b, out}, len, v, "binary_sub");
    case 2: return launch_map(device, Binary<2>{a, b, out}, len, v, "binary_mul");
    default: return launch_map(device, Binary<3>{a, b, out}, len, v, "binary_div");
    }
}

int axis_select_axis(axis_device device, const float *input, float *out, const int32_t *metadata,
                     int32_t rank, int32_t coordinate, int64_t output_len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {input, 1}, {out, 4 * output_len});
    AXIS_REQUIRE(input && out, "null select_axis buffer");
    SelectArgs a{};
    if (int s = select_args(metadata, rank, coordinate, output_len, true, &a)) return s;
    const int tiled = try_transpose(device, input, out, metadata, rank, coordinate, true);
    if (tiled >= 0) return tiled;
    select_axis_kernel<<<axis::blocks_for(output_len, kBlock, INT32_MAX), kBlock, 0, device->stream>>>(
        input, out, a);
    return axis::launch_status("select_axis_kernel");
}

int axis_select_axis_backward(axis_device device, const float *gradient, float *out,
                              const int32_t *metadata, int32_t rank, int32_t coordinate,
                              int64_t input_len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 1}, {out, 4 * input_len});
    AXIS_REQUIRE(gradient && out, "null select_axis_backward buffer");
    SelectArgs a{};
    if (int s = select_args(metadata, rank, coordinate, input_len, false, &a)) return s;
    const int tiled = try_transpose(device, gradient, out, metadata, rank, coordinate, false);
    if (tiled >= 0) return tiled;
    select_axis_backward_kernel<<<axis::blocks_for(input_len, kBlock, INT32_MAX), kBlock, 0,
                                  device->stream>>>(gradient, out, a);
    return axis::launch_status("select_axis_backward_kernel");
}

int axis_inverse_sqrt(axis_device device, const float *a, float epsilon, float *out, int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * len}, {out, 4 * len});
    AXIS_REQUIRE(len >= 0 && (len == 0 || (a && out)), "bad inverse_sqrt args");
    return launch_map(device, InverseSqrt{a, epsilon, out}, len, all_aligned({a, out}),
                      "inverse_sqrt");
}

int axis_multiply_scalar(axis_device device, const float *a, const float *scalar, float *out,
                         int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * len}, {scalar, 4}, {out, 4 * len});
    AXIS_REQUIRE(scalar, "device scalar multiplier must contain exactly one value");
    AXIS_REQUIRE(len >= 0 && (len == 0 || (a && out)), "bad multiply_scalar args");
    return launch_map(device, MultiplyScalar{a, scalar, out}, len, all_aligned({a, out}),
                      "multiply_scalar");
}

int axis_sum_squares(axis_device device, const float *a, int64_t len, float *out) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * len}, {out, 4});
    AXIS_REQUIRE(len >= 1, "sum of squares requires a nonempty buffer");
    AXIS_REQUIRE(a && out, "null sum_squares buffer");
    const int blocks = (int)axis::blocks_for(len, kBlock * 8, 1024);
    axis::Scratch partial;
    if (int s = partial.get(device, sizeof(float) * blocks)) return s;
    sum_squares_kernel<<<blocks, kBlock, 0, device->stream>>>(a, len, partial.as<float>());
    if (int s = axis::launch_status("sum_squares_kernel")) return s;
    sum_kernel<<<1, kBlock, 0, device->stream>>>(partial.as<float>(), blocks, out);
    return axis::launch_status("sum_kernel");
}

int axis_bias_add(axis_device device, const float *a, const float *bias, float *out,
                  float *relu_out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * rows * width}, {bias, 4 * width}, {out, 4 * rows * width}, {relu_out, 4 * rows * width});
    AXIS_REQUIRE(a && bias && out, "null bias_add buffer");
    AXIS_REQUIRE(rows >= 1 && width >= 1, "bias_add extents must be positive");
    const bool v = width % 4 == 0 && all_aligned({a, bias, out, relu_out});
    return launch_map(device, BiasAdd{a, bias, out, relu_out, FastDiv(1), width}, rows * width, v,
                      "bias_add");
}

int axis_bias_gradient(axis_device device, const float *gradient, const float *relu_input,
                       float *masked_out, float *out, int64_t rows, int64_t width) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * rows * width}, {relu_input, 4 * rows * width}, {masked_out, 4 * rows * width}, {out, 4 * width});
    AXIS_REQUIRE(gradient && out, "null bias_gradient buffer");
    AXIS_REQUIRE(!relu_input || masked_out, "a masked bias gradient needs masked_out");
    AXIS_REQUIRE(rows >= 1 && width >= 1, "bias_gradient extents must be positive");
    const int64_t chunks = (rows + axis::kGroupedChunk - 1) / axis::kGroupedChunk;
    const int64_t pairs = chunks * width;
    AXIS_REQUIRE(width / kChunkCols < INT32_MAX, "bias_gradient too large");
    axis::Scratch partial;
    if (chunks > 1)
        if (int s = partial.get(device, sizeof(float) * (size_t)pairs)) return s;
    float *direct = chunks == 1 ? out : nullptr;
    if (width >= 2048) {  // enough 64-column blocks to fill the chip
        const dim3 grid((unsigned)((width + kWideCols - 1) / kWideCols), (unsigned)std::min<int64_t>(chunks, 65535));
        if (relu_input)
            column_chunk_wide_kernel<true><<<grid, kBlock, 0, device->stream>>>(
                gradient, relu_input, masked_out, partial.as<float>(), rows, width, chunks, direct);
        else
            column_chunk_wide_kernel<false><<<grid, kBlock, 0, device->stream>>>(
                gradient, nullptr, nullptr, partial.as<float>(), rows, width, chunks, direct);
        if (int s = axis::launch_status("column_chunk_wide_kernel")) return s;
    } else {
        const dim3 grid((unsigned)((width + kChunkCols - 1) / kChunkCols), (unsigned)std::min<int64_t>(chunks, 65535));
        if (relu_input)
            column_chunk_kernel<true><<<grid, kBlock, 0, device->stream>>>(
                gradient, relu_input, masked_out, partial.as<float>(), rows, width, chunks, direct);
        else
            column_chunk_kernel<false><<<grid, kBlock, 0, device->stream>>>(
                gradient, nullptr, nullptr, partial.as<float>(), rows, width, chunks, direct);
        if (int s = axis::launch_status("column_chunk_kernel")) return s;
    }
    if (chunks == 1) return AXIS_OK;
    axis::column_combine_kernel<<<(unsigned)width, 256, 0, device->stream>>>(partial.as<float>(), chunks,
                                                                           width, 1.0f, out);
    return axis::launch_status("column_combine_kernel");
}

int axis_reduce_middle(axis_device device, const float *a, float *out, int64_t outer,
                       int64_t reduce, int64_t inner, float factor) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * outer * reduce * inner}, {out, 4 * outer * inner});
    AXIS_REQUIRE(a && out, "null reduce_middle buffer");
    AXIS_REQUIRE(outer >= 1 && reduce >= 1 && inner >= 1, "reduce_middle extents must be positive");
    reduce_middle_kernel<<<axis::blocks_for(outer * inner, kBlock, INT32_MAX), kBlock, 0,
                           device->stream>>>(a, out, outer, reduce, inner, factor);
    return axis::launch_status("reduce_middle_kernel");
}

int axis_reduce_axes(axis_device device, const float *a, float *out, int32_t rank, const int64_t *extents,
                     const int64_t *strides, const int32_t *reduced, float factor) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 1}, {out, 1});
    AXIS_REQUIRE(a && out && reduced, "null reduce_axes buffer");
    int order[kMaxReduceDims];
    int64_t len = 0;
    if (int st = dense_order(rank, extents, strides, order, &len)) return st;
    ReduceAxesArgs r{};
    r.factor = factor;
    // kept dims in shape order; neighbours contiguous in the input merge (the output is
    // row-major over them, so it is contiguous there too)
    int64_t ke[kMaxReduceDims], ks[kMaxReduceDims];
    int kr = 0;
    for (int d = 0; d < rank; ++d) {
        if (reduced[d] || extents[d] == 1) continue;
        if (kr > 0 && ks[kr - 1] == strides[d] * extents[d]) {
            ke[kr - 1] *= extents[d];
            ks[kr - 1] = strides[d];
            continue;
        }
        ke[kr] = extents[d];
        ks[kr] = strides[d];
        ++kr;
    }
    // reduced dims in decreasing stride, contiguous runs merged
    int64_t re[kMaxReduceDims], rs[kMaxReduceDims];
    int rr = 0;
    for (int i = 0; i < rank; ++i) {
        const int d = order[i];
        if (!reduced[d] || extents[d] == 1) continue;
        if (rr > 0 && rs[rr - 1] == strides[d] * extents[d]) {
            re[rr - 1] *= extents[d];
            rs[rr - 1] = strides[d];
            continue;
        }
        re[rr] = extents[d];
        rs[rr] = strides[d];
        ++rr;
    }
    r.outputs = 1;
    for (int d = kr - 1; d >= 0; --d) {
        r.kept_place[d] = FastDiv((uint32_t)r.outputs);
        r.kept_extent[d] = FastDiv((uint32_t)ke[d]);
        r.kept_src[d] = ks[d];
        r.outputs *= ke[d];
    }
    r.count = 1;
    for (int d = rr - 1; d >= 0; --d) {
        r.red_place[d] = FastDiv((uint32_t)r.count);
        r.red_extent[d] = FastDiv((uint32_t)re[d]);
        r.red_src[d] = rs[d];
        r.count *= re[d];
    }
    r.kept_rank = kr;
    r.red_rank = rr;
    if (rr == 0) {  // nothing reduced (unit extents only): a scaled copy in output order
        r.red_rank = 1;
        r.red_place[0] = FastDiv(1u);
        r.red_extent[0] = FastDiv(1u);
        r.red_src[0] = 0;
    }
    r.chunks = (r.count + axis::kGroupedChunk - 1) / axis::kGroupedChunk;
    const int64_t threads = r.outputs * r.chunks;
    axis::Scratch partial;
    float *dst = out;
    if (r.chunks > 1) {
        if (int st = partial.get(device, sizeof(float) * (size_t)threads)) return st;
        dst = partial.as<float>();
    }
    reduce_axes_chunk_kernel<<<axis::blocks_for(threads, kBlock, INT32_MAX), kBlock, 0, device->stream>>>(a, dst, r);
    if (int st = axis::launch_status("reduce_axes_chunk_kernel")) return st;
    if (r.chunks == 1) return AXIS_OK;
    reduce_axes_combine_kernel<<<axis::blocks_for(r.outputs, kBlock, INT32_MAX), kBlock, 0, device->stream>>>(
        dst, out, r.outputs, r.chunks, factor);
    return axis::launch_status("reduce_axes_combine_kernel");
}

int axis_reduce_axes_backward(axis_device device, const float *gradient, float *out, int32_t rank,
                              const int64_t *extents, const int64_t *strides, const int32_t *reduced,
                              float factor) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 1}, {out, 1});
    AXIS_REQUIRE(gradient && out && reduced, "null reduce_axes_backward buffer");
    int order[kMaxReduceDims];
    int64_t len = 0;
    if (int st = dense_order(rank, extents, strides, order, &len)) return st;
    // output strides of the kept dims (row-major over them in shape order)
    int64_t out_stride[kMaxReduceDims];
    int64_t s = 1;
    for (int d = rank - 1; d >= 0; --d) {
        out_stride[d] = reduced[d] ? 0 : s;
        if (!reduced[d]) s *= extents[d];
    }
    BroadcastAxesArgs b{};
    b.len = len;
    b.factor = factor;
    int64_t place = 1;
    for (int i = rank - 1; i >= 0; --i) {
        const int d = order[i];
        b.place[i] = FastDiv((uint32_t)place);
        b.extent[i] = FastDiv((uint32_t)extents[d]);
        b.out_stride[i] = out_stride[d];
        place *= extents[d];
    }
    b.rank = rank;
    broadcast_axes_kernel<<<axis::blocks_for(len, kBlock, INT32_MAX), kBlock, 0, device->stream>>>(gradient, out, b);
    return axis::launch_status("broadcast_axes_kernel");
}

int axis_extreme_axis(axis_device device, const float *a, int32_t rank, const int64_t *extents,
                      const int64_t *strides, int32_t axis, int32_t maximum, float *out, float *winner_mask) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 1}, {out, 1}, {winner_mask, 1});
    AXIS_REQUIRE(a && out && winner_mask, "null extreme_axis buffer");
    ExtremeAxisArgs x;
    if (int st = extreme_axis_args(rank, extents, strides, axis, x)) return st;
    const unsigned blocks = axis::blocks_for(x.outputs, kBlock, INT32_MAX);
    if (maximum)
        extreme_axis_kernel<true><<<blocks, kBlock, 0, device->stream>>>(a, out, winner_mask, x);
    else
        extreme_axis_kernel<false><<<blocks, kBlock, 0, device->stream>>>(a, out, winner_mask, x);
    return axis::launch_status("extreme_axis_kernel");
}

int axis_extreme_axis_backward(axis_device device, const float *gradient, const float *winner_mask, int32_t rank,
                               const int64_t *extents, const int64_t *strides, int32_t axis, float *out) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 1}, {winner_mask, 1}, {out, 1});
    AXIS_REQUIRE(gradient && winner_mask && out, "null extreme_axis_backward buffer");
    ExtremeAxisArgs x;
    if (int st = extreme_axis_args(rank, extents, strides, axis, x)) return st;
    extreme_axis_backward_kernel<<<axis::blocks_for(x.outputs, kBlock, INT32_MAX), kBlock, 0, device->stream>>>(
        gradient, winner_mask, out, x);
    return axis::launch_status("extreme_axis_backward_kernel");
}

int axis_broadcast_middle(axis_device device, const float *gradient, float *out, int64_t outer,
                          int64_t reduce, int64_t inner, float factor) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * outer * inner}, {out, 4 * outer * reduce * inner});
    AXIS_REQUIRE(gradient && out, "null broadcast_middle buffer");
    AXIS_REQUIRE(outer >= 1 && reduce >= 1 && inner >= 1, "broadcast_middle extents must be positive");
    const bool v = inner % 4 == 0 && all_aligned({gradient, out});
    return launch_map(device, BroadcastMiddle{gradient, out, reduce, inner, factor},
                      outer * reduce * inner, v, "broadcast_middle");
}

}  // extern "C"
