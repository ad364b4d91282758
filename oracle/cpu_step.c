/*
 * CPU performance baseline for the 3-block CNN training step -- the figure
 * bench.py reports as `cpu_baseline`.  NOT the checker (axis_oracle.c is) and never part of the
 * product: only bench.py's cpu_baseline leg and tests/ load it.  Its results are checked against
 * the oracle to fp32 tolerance in tests/test_cpu_baseline.py.
 *
 * The same step as the reference's lowering (model/convolution.rs:211-235, :1334-1370,
 * model/nn.rs:268-282, algebra/tensor.rs:1485-1557, the reverse sweep of tensor.rs:5591-5718 and
 * Adam, runtime/backend.rs:2545-2586), restated for speed on the host cores:
 *   - blocked fp32 SGEMM (A and B packed into MR x KC / KC x NR panels, an MR x NR register tile
 *     of fused multiply-adds, OpenMP over 128 x 256 output tiles; reductions much longer than the
 *     output is large are split over threads and the partial products summed), used in the three
 *     forms the step needs: NN (forward), NT (data gradients) and TN (weight gradients);
 *   - im2col / col2im over channel-innermost activations, taps in (ky, kx, c) order (the weight
 *     is permuted from the reference's (c, ky, kx) patch order once per step, and its gradient
 *     back);
 *   - bias + ReLU + 2x2 max pool in one pass with a byte winner (first strictly greater value),
 *     the pool backward scatter, global mean pool, softmax cross-entropy, Adam.
 * Accumulation is fp32 in blocked order, so results differ from the oracle's fp64-accumulated
 * products by rounding only.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define KC 256
#define MC 128
#define NC 256
#define MR_MAX 8
#define NR_MAX 32

/* ------------------------------------------------------------------ micro-kernels */

/* c[MR][NR] (+)= sum_p a[p][MR] b[p][NR] over packed panels; ldc is c's row pitch. */
typedef void (*kernel_fn)(int64_t kc, const float *a, const float *b, float *c, int64_t ldc, int accumulate);

typedef float v16 __attribute__((vector_size(64)));
typedef float v16u __attribute__((vector_size(64), aligned(4)));
typedef float v8 __attribute__((vector_size(32)));
typedef float v8u __attribute__((vector_size(32), aligned(4)));

/* AVX-512: 8 rows x 32 columns, 16 zmm accumulators. */
__attribute__((target("avx512f,fma"))) static void kernel_8x32(int64_t kc, const float *restrict a,
                                                                 const float *restrict b, float *restrict c,
                                                                 int64_t ldc, int accumulate) {
    v16 acc[8][2];
    for (int r = 0; r < 8; ++r) acc[r][0] = acc[r][1] = (v16){0};
    for (int64_t p = 0; p < kc; ++p) {
        const v16 b0 = *(const v16 *)(b + p * 32), b1 = *(const v16 *)(b + p * 32 + 16);
#pragma GCC unroll 8
        for (int r = 0; r < 8; ++r) {
            const float av = a[p * 8 + r];
            acc[r][0] += av * b0;
            acc[r][1] += av * b1;
        }
    }
    for (int r = 0; r < 8; ++r) {
        v16u *row = (v16u *)(c + r * ldc);
        if (accumulate) {
            row[0] += acc[r][0];
            row[1] += acc[r][1];
        } else {
            row[0] = acc[r][0];
            row[1] = acc[r][1];
        }
    }
}

/* AVX2: 6 rows x 16 columns, 12 ymm accumulators. */
__attribute__((target("avx2,fma"))) static void kernel_6x16(int64_t kc, const float *restrict a,
                                                              const float *restrict b, float *restrict c,
                                                              int64_t ldc, int accumulate) {
    v8 acc[6][2];
    for (int r = 0; r < 6; ++r) acc[r][0] = acc[r][1] = (v8){0};
    for (int64_t p = 0; p < kc; ++p) {
        const v8 b0 = *(const v8 *)(b + p * 16), b1 = *(const v8 *)(b + p * 16 + 8);
#pragma GCC unroll 6
        for (int r = 0; r < 6; ++r) {
            const float av = a[p * 6 + r];
            acc[r][0] += av * b0;
            acc[r][1] += av * b1;
        }
    }
    for (int r = 0; r < 6; ++r) {
        v8u *row = (v8u *)(c + r * ldc);
        if (accumulate) {
            row[0] += acc[r][0];
            row[1] += acc[r][1];
        } else {
            row[0] = acc[r][0];
            row[1] = acc[r][1];
        }
    }
}

static int g_mr, g_nr;
static kernel_fn g_kernel;

/* The widest kernel the host runs; AXCPU_KERNEL=avx2 forces the AVX2 one (tests cover both). */
static void pick_kernel(void) {
    if (g_kernel) return;
    __builtin_cpu_init();
    const char *force = getenv("AXCPU_KERNEL");
    if (__builtin_cpu_supports("avx512f") && !(force && strcmp(force, "avx2") == 0)) {
        g_mr = 8, g_nr = 32, g_kernel = kernel_8x32;
    } else {
        g_mr = 6, g_nr = 16, g_kernel = kernel_6x16;
    }
}

int axcpu_kernel_width(void) {
    pick_kernel();
    return g_nr;
}

/* ------------------------------------------------------------------ SGEMM */

/* Element (i, j) of a matrix view at p[i * rs + j * cs]. */
typedef struct {
    const float *p;
    int64_t rs, cs;
} view;

static int threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* A rows [i0, i0 + mc) x reduction [p0, p0 + kc) into MR-row panels (rows past m are zero). */
static void pack_a(view A, int64_t m, int64_t i0, int64_t mc, int64_t p0, int64_t kc, float *dst) {
    const int mr = g_mr;
    for (int64_t ir = 0; ir < mc; ir += mr) {
        float *panel = dst + ir * kc;
        for (int r = 0; r < mr; ++r) {
            const int64_t i = i0 + ir + r;
            if (ir + r < mc && i < m) {
                const float *src = A.p + i * A.rs + p0 * A.cs;
                for (int64_t p = 0; p < kc; ++p) panel[p * mr + r] = src[p * A.cs];
            } else {
                for (int64_t p = 0; p < kc; ++p) panel[p * mr + r] = 0.f;
            }
        }
    }
}

/* B reduction [p0, p0 + kc) x columns [j0, j0 + nc) into NR-column panels (zero past n). */
static void pack_b(view B, int64_t n, int64_t p0, int64_t kc, int64_t j0, int64_t nc, float *dst) {
    const int nr = g_nr;
    for (int64_t jr = 0; jr < nc; jr += nr) {
        float *panel = dst + jr * kc;
        const int64_t width = (j0 + jr + nr <= n) ? nr : (n - j0 - jr > 0 ? n - j0 - jr : 0);
        if (B.cs == 1) {
            for (int64_t p = 0; p < kc; ++p) {
                const float *src = B.p + (p0 + p) * B.rs + j0 + jr;
                float *d = panel + p * nr;
                int64_t j = 0;
                for (; j < width; ++j) d[j] = src[j];
                for (; j < nr; ++j) d[j] = 0.f;
            }
        } else {
            for (int j = 0; j < nr; ++j) {
                if (j < width) {
                    const float *src = B.p + p0 * B.rs + (j0 + jr + j) * B.cs;
                    for (int64_t p = 0; p < kc; ++p) panel[p * nr + j] = src[p * B.rs];
                } else {
                    for (int64_t p = 0; p < kc; ++p) panel[p * nr + j] = 0.f;
                }
            }
        }
    }
}

/* One MC x NC tile of C (rows i0.., columns j0..) over the reduction [k0, k1). */
static void gemm_tile(int64_t m, int64_t n, int64_t k0, int64_t k1, view A, view B, float *C, int64_t ldc,
                      int accumulate, int64_t i0, int64_t j0, float *ap, float *bp) {
    const int mr = g_mr, nr = g_nr;
    const int64_t mc = (m - i0 < MC) ? m - i0 : MC, nc = (n - j0 < NC) ? n - j0 : NC;
    float edge[MR_MAX * NR_MAX];
    for (int64_t p0 = k0; p0 < k1; p0 += KC) {
        const int64_t kc = (k1 - p0 < KC) ? k1 - p0 : KC;
        const int acc = accumulate || p0 > k0;
        pack_a(A, m, i0, mc, p0, kc, ap);
        pack_b(B, n, p0, kc, j0, nc, bp);
        for (int64_t jr = 0; jr < nc; jr += nr) {
            for (int64_t ir = 0; ir < mc; ir += mr) {
                float *c = C + (i0 + ir) * ldc + j0 + jr;
                const int64_t rows = (mc - ir < mr) ? mc - ir : mr, cols = (nc - jr < nr) ? nc - jr : nr;
                if (rows == mr && cols == nr) {
                    g_kernel(kc, ap + ir * kc, bp + jr * kc, c, ldc, acc);
                } else {
                    g_kernel(kc, ap + ir * kc, bp + jr * kc, edge, nr, 0);
                    for (int64_t r = 0; r < rows; ++r)
                        for (int64_t j = 0; j < cols; ++j)
                            c[r * ldc + j] = acc ? c[r * ldc + j] + edge[r * nr + j] : edge[r * nr + j];
                }
            }
        }
    }
}

static float *aligned_floats(int64_t count) {
    size_t bytes = ((size_t)count * sizeof(float) + 63) & ~(size_t)63;
    return (float *)aligned_alloc(64, bytes ? bytes : 64);
}

/* C[m][n] (row pitch ldc) = (C +) sum_p A(i, p) B(p, j), p < k. */
static void gemm(int64_t m, int64_t n, int64_t k, view A, view B, float *C, int64_t ldc, int accumulate) {
    pick_kernel();
    const int64_t tm = (m + MC - 1) / MC, tn = (n + NC - 1) / NC;
    const int nt = threads();
    if (tm * tn < 2 * nt && k >= 4 * KC * (int64_t)nt && !accumulate) {
        /* A short, wide output over a long reduction (weight gradients): each thread takes a slice
         * of the reduction into its own copy of C, then the copies are added. */
        float *part = aligned_floats((int64_t)nt * m * n);
        const int64_t per = ((k + nt - 1) / nt + KC - 1) / KC * KC;
#pragma omp parallel num_threads(nt)
        {
            int t = 0;
#ifdef _OPENMP
            t = omp_get_thread_num();
#endif
            float *ap = aligned_floats((MC + MR_MAX) * KC), *bp = aligned_floats(KC * (NC + NR_MAX));
            float *mine = part + (int64_t)t * m * n;
            const int64_t k0 = t * per, k1 = (k0 + per < k) ? k0 + per : k;
            if (k0 < k1) {
                for (int64_t i0 = 0; i0 < m; i0 += MC)
                    for (int64_t j0 = 0; j0 < n; j0 += NC)
                        gemm_tile(m, n, k0, k1, A, B, mine, n, 0, i0, j0, ap, bp);
            } else {
                memset(mine, 0, sizeof(float) * (size_t)(m * n));
            }
            free(ap);
            free(bp);
        }
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < m; ++i)
            for (int64_t j = 0; j < n; ++j) {
                float s = 0.f;
                for (int t = 0; t < nt; ++t) s += part[(int64_t)t * m * n + i * n + j];
                C[i * ldc + j] = s;
            }
        free(part);
        return;
    }
#pragma omp parallel num_threads(nt)
    {
        float *ap = aligned_floats((MC + MR_MAX) * KC), *bp = aligned_floats(KC * (NC + NR_MAX));
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int64_t ti = 0; ti < tm; ++ti)
            for (int64_t tj = 0; tj < tn; ++tj)
                gemm_tile(m, n, 0, k, A, B, C, ldc, accumulate, ti * MC, tj * NC, ap, bp);
        free(ap);
        free(bp);
    }
}

/* The three forms, row-major operands.  NN: c[m][n] = a[m][k] b[k][n].  NT: c[m][k] =
 * g[m][n] b[k][n]^T.  TN: c[k][n] = a[m][k]^T g[m][n]. */
void axcpu_sgemm_nn(int64_t m, int64_t k, int64_t n, const float *a, const float *b, float *c) {
    gemm(m, n, k, (view){a, k, 1}, (view){b, n, 1}, c, n, 0);
}
void axcpu_sgemm_nt(int64_t m, int64_t k, int64_t n, const float *g, const float *b, float *c) {
    gemm(m, k, n, (view){g, n, 1}, (view){b, 1, n}, c, k, 0);
}
void axcpu_sgemm_tn(int64_t m, int64_t k, int64_t n, const float *a, const float *g, float *c) {
    gemm(k, n, m, (view){a, 1, k}, (view){g, n, 1}, c, n, 0);
}

/* ------------------------------------------------------------------ convolution pieces */

/* x [b][h][w][c] -> patches [b*h*w][9*c], taps (ky, kx) outer, channels inner, zero padding 1. */
static void im2col3(const float *x, int64_t b, int h, int w, int c, float *patches) {
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t n = 0; n < b; ++n)
        for (int y = 0; y < h; ++y)
            for (int xx = 0; xx < w; ++xx) {
                float *row = patches + ((n * h + y) * w + xx) * 9 * c;
                for (int ky = 0; ky < 3; ++ky)
                    for (int kx = 0; kx < 3; ++kx) {
                        float *dst = row + (ky * 3 + kx) * c;
                        const int sy = y + ky - 1, sx = xx + kx - 1;
                        if (sy < 0 || sy >= h || sx < 0 || sx >= w) {
                            memset(dst, 0, sizeof(float) * (size_t)c);
                        } else {
                            memcpy(dst, x + ((n * h + sy) * w + sx) * c, sizeof(float) * (size_t)c);
                        }
                    }
            }
}

/* The adjoint: dx[b][y][x][c] = sum over the taps that read it of dpatches. */
static void col2im3(const float *dpatches, int64_t b, int h, int w, int c, float *dx) {
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t n = 0; n < b; ++n)
        for (int y = 0; y < h; ++y)
            for (int xx = 0; xx < w; ++xx) {
                float *dst = dx + ((n * h + y) * w + xx) * c;
                memset(dst, 0, sizeof(float) * (size_t)c);
                for (int ky = 0; ky < 3; ++ky)
                    for (int kx = 0; kx < 3; ++kx) {
                        const int oy = y - ky + 1, ox = xx - kx + 1;
                        if (oy < 0 || oy >= h || ox < 0 || ox >= w) continue;
                        const float *src = dpatches + ((n * h + oy) * w + ox) * 9 * c + (ky * 3 + kx) * c;
                        for (int ch = 0; ch < c; ++ch) dst[ch] += src[ch];
                    }
            }
}

/* x [b][c][h][w] -> [b][h][w][c]. */
static void nchw_to_nhwc(const float *x, int64_t b, int c, int size, float *out) {
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t n = 0; n < b; ++n)
        for (int yy = 0; yy < size; ++yy)
            for (int xx = 0; xx < size; ++xx)
                for (int ch = 0; ch < c; ++ch)
                    out[((n * size + yy) * size + xx) * c + ch] = x[((n * c + ch) * size + yy) * size + xx];
}

/* Reference weight [(c, ky, kx)][out] <-> tap-major [(ky, kx, c)][out]. */
static void weight_to_taps(const float *w, int cin, int cout, float *taps) {
    for (int ch = 0; ch < cin; ++ch)
        for (int t = 0; t < 9; ++t)
            memcpy(taps + ((int64_t)t * cin + ch) * cout, w + ((int64_t)ch * 9 + t) * cout, sizeof(float) * (size_t)cout);
}
static void taps_to_weight(const float *taps, int cin, int cout, float *w) {
    for (int ch = 0; ch < cin; ++ch)
        for (int t = 0; t < 9; ++t)
            memcpy(w + ((int64_t)ch * 9 + t) * cout, taps + ((int64_t)t * cin + ch) * cout, sizeof(float) * (size_t)cout);
}

/* z [b][h][w][c] + bias, ReLU, 2x2 max pool (first strictly greater value wins) -> pooled
 * [b][h/2][w/2][c] and the winner byte ky*2 + kx. */
static void bias_relu_pool(const float *z, const float *bias, int64_t b, int h, int w, int c, float *pooled,
                           uint8_t *winner) {
    const int oh = h / 2, ow = w / 2;
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t n = 0; n < b; ++n)
        for (int oy = 0; oy < oh; ++oy)
            for (int ox = 0; ox < ow; ++ox)
                for (int ch = 0; ch < c; ++ch) {
                    float best = 0.f;
                    int arg = 0;
                    for (int p = 0; p < 4; ++p) {
                        const int y = 2 * oy + p / 2, xx = 2 * ox + p % 2;
                        float v = z[((n * h + y) * w + xx) * c + ch] + bias[ch];
                        v = v > 0.f ? v : 0.f;
                        if (p == 0 || v > best) {
                            best = v;
                            arg = p;
                        }
                    }
                    const int64_t o = ((n * oh + oy) * ow + ox) * c + ch;
                    pooled[o] = best;
                    winner[o] = (uint8_t)arg;
                }
}

/* dz [b][h][w][c]: the pooled gradient at each window's winner when the pooled value is positive
 * (ReLU passes it), zero elsewhere; dbias = column sums of dz. */
static void pool_relu_backward(const float *g, const float *pooled, const uint8_t *winner, int64_t b, int h, int w,
                               int c, float *dz, float *dbias) {
    const int oh = h / 2, ow = w / 2;
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t n = 0; n < b; ++n)
        for (int oy = 0; oy < oh; ++oy)
            for (int ox = 0; ox < ow; ++ox)
                for (int ch = 0; ch < c; ++ch) {
                    const int64_t o = ((n * oh + oy) * ow + ox) * c + ch;
                    const float v = pooled[o] > 0.f ? g[o] : 0.f;
                    for (int p = 0; p < 4; ++p) {
                        const int y = 2 * oy + p / 2, xx = 2 * ox + p % 2;
                        dz[((n * h + y) * w + xx) * c + ch] = p == winner[o] ? v : 0.f;
                    }
                }
    const int nt = threads();
    float *part = (float *)calloc((size_t)nt * (size_t)c, sizeof(float));
    const int64_t rows = b * oh * ow;
#pragma omp parallel num_threads(nt)
    {
        int t = 0;
#ifdef _OPENMP
        t = omp_get_thread_num();
#endif
        float *mine = part + (int64_t)t * c;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r)
            for (int ch = 0; ch < c; ++ch)
                if (pooled[r * c + ch] > 0.f) mine[ch] += g[r * c + ch];
    }
    for (int ch = 0; ch < c; ++ch) {
        float s = 0.f;
        for (int t = 0; t < nt; ++t) s += part[(int64_t)t * c + ch];
        dbias[ch] = s;
    }
    free(part);
}

static void adam(float *p, const float *g, float *m, float *v, int64_t len, float lr, float c1, float c2) {
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) {
        const float mi = b1 * m[i] + (1.f - b1) * g[i];
        const float vi = b2 * v[i] + (1.f - b2) * g[i] * g[i];
        m[i] = mi;
        v[i] = vi;
        p[i] = p[i] - lr * ((mi / c1) / (sqrtf(vi / c2) + eps));
    }
}

/* ------------------------------------------------------------------ the step */

/* Buffers kept across steps (grown on demand), so a timed step does not page in gigabytes of
 * fresh allocations; phase timers of the last step (axcpu_phase_seconds). */
enum { kSlots = 32 };
static void *g_slot[kSlots];
static size_t g_slot_bytes[kSlots];

static void *slot(int id, size_t bytes) {
    bytes = (bytes + 63) & ~(size_t)63;
    if (g_slot_bytes[id] < bytes) {
        free(g_slot[id]);
        g_slot[id] = aligned_alloc(64, bytes ? bytes : 64);
        g_slot_bytes[id] = bytes;
    }
    return g_slot[id];
}
#define FSLOT(id, count) ((float *)slot((id), sizeof(float) * (size_t)(count)))

enum { P_INPUT, P_IM2COL, P_GEMM_FWD, P_POOL, P_HEAD, P_POOL_BWD, P_GEMM_WGRAD, P_GEMM_DGRAD, P_COL2IM, P_ADAM,
       P_COUNT };
static double g_phase[P_COUNT];

static double now(void) {
#ifdef _OPENMP
    return omp_get_wtime();
#else
    return 0.0;
#endif
}
#define PHASE(id, stmt)                  \
    do {                                 \
        const double phase_t0 = now();   \
        stmt;                            \
        g_phase[id] += now() - phase_t0; \
    } while (0)

/* Seconds per phase of the last step: input repack, im2col, forward GEMMs, bias+ReLU+pool, head
 * (mean pool, classifier, cross-entropy and its backward), pool backward, weight-gradient GEMMs,
 * data-gradient GEMMs, col2im, Adam. */
int axcpu_phase_seconds(double *out, int count) {
    for (int i = 0; i < count && i < P_COUNT; ++i) out[i] = g_phase[i];
    return P_COUNT;
}

/* One forward + backward + Adam step of the 3-block CNN.  x is [batch][ch0][size][size] (NCHW),
 * y one-hot [batch][classes]; params / m / v / grads hold, in order, conv0.weight, conv0.bias,
 * conv1.weight, conv1.bias, conv2.weight, conv2.bias, linear.weight, linear.bias in the
 * reference's layouts (conv weight [ch_in * 9][ch_out] in (c, ky, kx) patch order, linear
 * [ch3][classes]).  params, m, v are updated in place (Adam step t, lr); grads may be null.
 * Returns the mean cross-entropy of the forward. */
float axcpu_cnn_step(int batch, int size, int classes, const int *ch, const float *x, const float *y,
                     float *const *params, float *const *m, float *const *v, float *const *grads, int t, float lr) {
    pick_kernel();
    for (int i = 0; i < P_COUNT; ++i) g_phase[i] = 0.0;
    const int64_t B = batch;
    int hw[4] = {size, size / 2, size / 4, size / 8};
    float *act[4]; /* block inputs, channel-innermost: act[0] = x as [b][h][w][3] */
    float *patches[3], *pooled[3], *wt[3];
    uint8_t *win[3];
    float *g_own[8];
    const int64_t lens[8] = {(int64_t)ch[0] * 9 * ch[1], ch[1], (int64_t)ch[1] * 9 * ch[2], ch[2],
                             (int64_t)ch[2] * 9 * ch[3], ch[3], (int64_t)ch[3] * classes, classes};
    for (int i = 0; i < 8; ++i) g_own[i] = grads && grads[i] ? grads[i] : FSLOT(20 + i, lens[i]);

    act[0] = FSLOT(0, B * size * size * ch[0]);
    PHASE(P_INPUT, nchw_to_nhwc(x, B, ch[0], size, act[0]));
    /* ---- forward */
    for (int j = 0; j < 3; ++j) {
        const int h = hw[j], cin = ch[j], cout = ch[j + 1];
        const int64_t rows = B * h * h, k = 9 * (int64_t)cin, pooled_len = B * (h / 2) * (h / 2) * cout;
        patches[j] = FSLOT(1 + j, rows * k);
        PHASE(P_IM2COL, im2col3(act[j], B, h, h, cin, patches[j]));
        wt[j] = FSLOT(4 + j, k * cout);
        weight_to_taps(params[2 * j], cin, cout, wt[j]);
        float *z = FSLOT(7, rows * cout);
        PHASE(P_GEMM_FWD, axcpu_sgemm_nn(rows, k, cout, patches[j], wt[j], z));
        pooled[j] = FSLOT(8 + j, pooled_len);
        win[j] = (uint8_t *)slot(11 + j, (size_t)pooled_len);
        PHASE(P_POOL, bias_relu_pool(z, params[2 * j + 1], B, h, h, cout, pooled[j], win[j]));
        act[j + 1] = pooled[j];
    }
    const double head_t0 = now();
    const int c3 = ch[3], s3 = hw[3];
    const int64_t cells = (int64_t)s3 * s3;
    float *gap = FSLOT(14, B * c3);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < B; ++n)
        for (int c = 0; c < c3; ++c) {
            float s = 0.f;
            for (int64_t q = 0; q < cells; ++q) s += pooled[2][(n * cells + q) * c3 + c];
            gap[n * c3 + c] = s * (1.0f / (float)cells);
        }
    float *logits = FSLOT(15, B * classes);
    axcpu_sgemm_nn(B, c3, classes, gap, params[6], logits);
    double loss = 0.0;
    float *dlogits = FSLOT(16, B * classes);
#pragma omp parallel for schedule(static) reduction(+ : loss)
    for (int64_t n = 0; n < B; ++n) {
        float *row = logits + n * classes;
        float mx = -INFINITY;
        for (int c = 0; c < classes; ++c) {
            row[c] += params[7][c];
            mx = row[c] > mx ? row[c] : mx;
        }
        float s = 0.f;
        for (int c = 0; c < classes; ++c) s += expf(row[c] - mx);
        const float lse = mx + logf(s);
        float l = 0.f;
        for (int c = 0; c < classes; ++c) {
            const float yv = y[n * classes + c];
            l -= yv * (row[c] - lse);
            dlogits[n * classes + c] = (expf(row[c] - lse) - yv) * (1.0f / (float)B);
        }
        loss += l;
    }
    /* ---- backward */
    float *dgap = FSLOT(17, B * c3);
    axcpu_sgemm_tn(B, c3, classes, gap, dlogits, g_own[6]);
    for (int c = 0; c < classes; ++c) {
        float s = 0.f;
        for (int64_t n = 0; n < B; ++n) s += dlogits[n * classes + c];
        g_own[7][c] = s;
    }
    axcpu_sgemm_nt(B, c3, classes, dlogits, params[6], dgap);
    /* the pooled gradient of the block being walked back; two buffers alternate */
    float *g = FSLOT(18, B * cells * c3);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < B; ++n)
        for (int64_t q = 0; q < cells; ++q)
            for (int c = 0; c < c3; ++c) g[(n * cells + q) * c3 + c] = dgap[n * c3 + c] * (1.0f / (float)cells);
    g_phase[P_HEAD] += now() - head_t0;
    for (int j = 2; j >= 0; --j) {
        const int h = hw[j], cin = ch[j], cout = ch[j + 1];
        const int64_t rows = B * h * h, k = 9 * (int64_t)cin;
        float *dz = FSLOT(28, rows * cout);
        PHASE(P_POOL_BWD, pool_relu_backward(g, pooled[j], win[j], B, h, h, cout, dz, g_own[2 * j + 1]));
        float *dwt = FSLOT(29, k * cout);
        PHASE(P_GEMM_WGRAD, axcpu_sgemm_tn(rows, k, cout, patches[j], dz, dwt));
        taps_to_weight(dwt, cin, cout, g_own[2 * j]);
        if (j > 0) {
            float *dp = FSLOT(30, rows * k);
            PHASE(P_GEMM_DGRAD, axcpu_sgemm_nt(rows, k, cout, dz, wt[j], dp));
            g = FSLOT(j % 2 ? 19 : 18, rows * cin);
            PHASE(P_COL2IM, col2im3(dp, B, h, h, cin, g));
        }
    }
    /* ---- Adam */
    const float c1 = 1.0f - powf(0.9f, (float)t), c2 = 1.0f - powf(0.999f, (float)t);
    const double adam_t0 = now();
    for (int i = 0; i < 8; ++i) adam(params[i], g_own[i], m[i], v[i], lens[i], lr, c1, c2);
    g_phase[P_ADAM] += now() - adam_t0;
    return (float)(loss / (double)B);
}

int axcpu_threads(void) { return threads(); }
