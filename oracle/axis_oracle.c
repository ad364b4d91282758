/*
 * CPU restatement of furkanhaney/axis's training hot path -- TEST INFRASTRUCTURE ONLY.
 * See axis_oracle.h for the contract; every function cites the reference code it follows
 * (paths relative to the reference's src/library/src/).
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off -fPIC -shared (oracle/Makefile).
 * Parallel loops split the OUTPUT index space only; each output is produced by the same
 * sequential expression whatever the thread count, so results do not depend on it.
 */
#include "axis_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int axo_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void axo_set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

/* ---------------------------------------------------------------- RNG */

/* algebra/tensor.rs:29-40: xorshift64 (13, 7, 17) seeded max(seed, 1); sample = (r >> 40) / 2^24. */
void axo_xorshift_unit_stream(uint64_t seed, int64_t count, float *out) {
    uint64_t rng = seed > 1 ? seed : 1;
    for (int64_t i = 0; i < count; ++i) {
        rng ^= rng << 13;
        rng ^= rng >> 7;
        rng ^= rng << 17;
        out[i] = (float)(rng >> 40) / (float)(1u << 24);
    }
}

/* algebra/tensor.rs:45-50: low + raw * (high - low), fp32. */
void axo_uniform_host_values(uint64_t seed, int64_t count, float low, float high, float *out) {
    axo_xorshift_unit_stream(seed, count, out);
    const float span = high - low;
    for (int64_t i = 0; i < count; ++i) out[i] = low + out[i] * span;
}

/* algebra/tensor.rs:60-71: Box-Muller on consecutive raw pairs with ln(1 - u1); an odd count
 * drops the final sine value.  fp32 libm calls, as Rust's f32::{ln, sqrt, cos, sin}. */
void axo_normal_host_values(uint64_t seed, int64_t count, float mean, float std, float *out) {
    int64_t pairs = (count + 1) / 2;
    float *raw = (float *)malloc(sizeof(float) * (size_t)(pairs * 2));
    axo_xorshift_unit_stream(seed, pairs * 2, raw);
    const float two_pi = 2.0f * 3.14159265358979323846f;
    int64_t written = 0;
    for (int64_t p = 0; p < pairs; ++p) {
        float radius = sqrtf(-2.0f * logf(1.0f - raw[2 * p]));
        float angle = two_pi * raw[2 * p + 1];
        out[written++] = mean + std * (radius * cosf(angle));
        if (written < count) out[written++] = mean + std * (radius * sinf(angle));
    }
    free(raw);
}

/* f32::powi as lowered by LLVM to compiler-rt's __powisf2 (repeated squaring in fp32);
 * the reference uses it for Adam's bias corrections (model/optim.rs:103-105). */
float axo_powi(float base, int32_t exponent) {
    int recip = exponent < 0;
    float r = 1.0f;
    for (;;) {
        if (exponent & 1) r *= base;
        exponent /= 2;
        if (exponent == 0) break;
        base *= base;
    }
    return recip ? 1.0f / r : r;
}

/* ---------------------------------------------------------------- contractions */

/* runtime/backend.rs:2209-2312 (matmul_bf16 and its backward kernels): convert_tile of each fp32
 * operand tile to bf16 before the mma -- round to nearest, ties to even, on the bit pattern; NaN
 * stays a (quiet) NaN.  The result is returned widened back to fp32. */
void axo_bf16_round(const float *a, int64_t len, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) {
        uint32_t bits;
        memcpy(&bits, &a[i], 4);
        if ((bits & 0x7fffffffu) > 0x7f800000u)
            bits = (bits | 0x00400000u) & 0xffff0000u;
        else
            bits = (bits + 0x7fffu + ((bits >> 16) & 1u)) & 0xffff0000u;
        memcpy(&out[i], &bits, 4);
    }
}

/* runtime/backend.rs:2190-2207: out[b] = a[b] . b[b], a [batch,m,k], b [batch,k,n].
 * fp64 accumulation (cuTile's mma order is not observable). */
void axo_matmul(const float *a, const float *b, int64_t batch, int64_t m, int64_t k, int64_t n,
                float *out) {
#pragma omp parallel
    {
        double *row = (double *)malloc(sizeof(double) * (size_t)n);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < batch * m; ++r) {
            int64_t bi = r / m;
            const float *ar = a + r * k;
            const float *bb = b + bi * k * n;
            for (int64_t j = 0; j < n; ++j) row[j] = 0.0;
            for (int64_t kk = 0; kk < k; ++kk) {
                double av = ar[kk];
                const float *br = bb + kk * n;
                for (int64_t j = 0; j < n; ++j) row[j] += av * (double)br[j];
            }
            for (int64_t j = 0; j < n; ++j) out[r * n + j] = (float)row[j];
        }
        free(row);
    }
}

/* runtime/backend.rs:2228-2247 (dgrad): out[b] = gradient[b] . rhs[b]^T,
 * gradient [batch,m,n], rhs [batch,k,n] -> out [batch,m,k]. */
void axo_matmul_left_backward(const float *gradient, const float *rhs, int64_t batch, int64_t m,
                              int64_t k, int64_t n, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < batch * m; ++r) {
        int64_t bi = r / m;
        const float *gr = gradient + r * n;
        const float *rb = rhs + bi * k * n;
        for (int64_t kk = 0; kk < k; ++kk) {
            const float *rr = rb + kk * n;
            double acc = 0.0;
            for (int64_t j = 0; j < n; ++j) acc += (double)gr[j] * (double)rr[j];
            out[r * k + kk] = (float)acc;
        }
    }
}

/* runtime/backend.rs:2271-2290 (wgrad): out[b] = lhs[b]^T . gradient[b],
 * lhs [batch,m,k], gradient [batch,m,n] -> out [batch,k,n]. */
void axo_matmul_right_backward(const float *lhs, const float *gradient, int64_t batch, int64_t m,
                               int64_t k, int64_t n, float *out) {
#pragma omp parallel
    {
        double *row = (double *)malloc(sizeof(double) * (size_t)n);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < batch * k; ++r) {
            int64_t bi = r / k, kk = r % k;
            const float *lb = lhs + bi * m * k;
            const float *gb = gradient + bi * m * n;
            for (int64_t j = 0; j < n; ++j) row[j] = 0.0;
            for (int64_t i = 0; i < m; ++i) {
                double lv = lb[i * k + kk];
                if (lv == 0.0) continue;
                const float *gr = gb + i * n;
                for (int64_t j = 0; j < n; ++j) row[j] += lv * (double)gr[j];
            }
            for (int64_t j = 0; j < n; ++j) out[r * n + j] = (float)row[j];
        }
        free(row);
    }
}

/* ---------------------------------------------------------------- im2col / col2im */

/* runtime/backend.rs:1604-1689 (unfold2d): one output element at a time; the rank-generic
 * metadata decode gives the non-spatial input offset and (oy, ox, group, patch); patch is
 * (channel_in_group, ky, kx) with kx fastest; positions outside the input read `fill`. */
void axo_unfold2d(const float *input, const axo_unfold_spec *s, float *out) {
    const int32_t kh = s->kernel[0], kw = s->kernel[1];
    const int32_t sy = s->stride[0], sx = s->stride[1];
    const int32_t py = s->padding[0], px = s->padding[1];
    const int32_t h = s->input_spatial[0], w = s->input_spatial[1];
    const int64_t cs = s->input_special_strides[0], hs = s->input_special_strides[1],
                  ws = s->input_special_strides[2];
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < s->output_len; ++o) {
        int64_t input_index = 0;
        int32_t oy = 0, ox = 0, group = 0, patch = 0;
        for (int32_t d = 0; d < s->output_rank; ++d) {
            const int32_t *md = s->forward_metadata + 4 * d;
            int32_t coordinate = (int32_t)((o / md[1]) % md[0]);
            switch (md[3]) {
            case 0: input_index += (int64_t)coordinate * md[2]; break;
            case 1: oy = coordinate; break;
            case 2: ox = coordinate; break;
            case 3: group = coordinate; break;
            default: patch = coordinate; break;
            }
        }
        int32_t kx = patch % kw, rest = patch / kw;
        int32_t ky = rest % kh, channel_in_group = rest / kh;
        int32_t channel = group * s->channels_per_group + channel_in_group;
        int32_t iy = oy * sy + ky - py, ix = ox * sx + kx - px;
        int valid = iy >= 0 && iy < h && ix >= 0 && ix < w;
        out[o] = valid ? input[input_index + channel * cs + iy * hs + ix * ws] : s->fill;
    }
}

/* runtime/backend.rs:1795-1889 (unfold2d_backward): gather-form col2im, one input element at a
 * time, summing the patch gradients that read it in ky-major, kx-minor order from +0.0. */
void axo_unfold2d_backward(const float *gradient, const axo_unfold_spec *s, float *out) {
    const int32_t kh = s->kernel[0], kw = s->kernel[1];
    const int32_t sy = s->stride[0], sx = s->stride[1];
    const int32_t py = s->padding[0], px = s->padding[1];
    const int32_t oh = s->output_spatial[0], ow = s->output_spatial[1];
    const int64_t ohs = s->output_special_strides[0], ows = s->output_special_strides[1],
                  ogs = s->output_special_strides[3], ops = s->output_special_strides[4];
    const int32_t cpg = s->channels_per_group;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < s->input_len; ++i) {
        int64_t output_base = 0;
        int32_t channel = 0, iy = 0, ix = 0;
        for (int32_t d = 0; d < s->input_rank; ++d) {
            const int32_t *md = s->backward_metadata + 4 * d;
            int32_t coordinate = (int32_t)((i / md[1]) % md[0]);
            switch (md[3]) {
            case 0: output_base += (int64_t)coordinate * md[2]; break;
            case 1: channel = coordinate; break;
            case 2: iy = coordinate; break;
            default: ix = coordinate; break;
            }
        }
        int32_t group = channel / cpg, channel_in_group = channel % cpg;
        float sum = 0.0f;
        for (int32_t ky = 0; ky < kh; ++ky) {
            int32_t padded_y = iy + (py - ky);
            int32_t oy = padded_y / sy;
            int valid_y = padded_y >= 0 && padded_y % sy == 0 && oy < oh;
            for (int32_t kx = 0; kx < kw; ++kx) {
                int32_t padded_x = ix + (px - kx);
                int32_t ox = padded_x / sx;
                int valid = valid_y && padded_x >= 0 && padded_x % sx == 0 && ox < ow;
                if (!valid) continue; /* the reference adds a masked 0.0: a no-op on the sum */
                int32_t patch = (channel_in_group * kh + ky) * kw + kx;
                int64_t index = output_base + oy * ohs + ox * ows + group * ogs + patch * ops;
                sum = sum + gradient[index];
            }
        }
        out[i] = sum;
    }
}

/* ---------------------------------------------------------------- CSR plans */

#define AXO_GROUPED_CHUNK 512 /* runtime/backend.rs:27 */

/* runtime/backend.rs:1089-1125 with chunked_offsets (:37-50) and grouped_partial/combine
 * (:2964-3016): each group's range splits into chunks of <= 512 contributions, each chunk is
 * summed sequentially from +0.0, the chunk partials are summed in chunk order from +0.0, and the
 * total is multiplied by `scale` once. */
void axo_grouped(const float *a, const float *b, const int32_t *offsets, const int32_t *left,
                 const int32_t *right, int64_t groups, float scale, float *out) {
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t g = 0; g < groups; ++g) {
        int32_t start = offsets[g], end = offsets[g + 1];
        float total = 0.0f;
        for (int32_t cursor = start; cursor < end;) {
            int32_t chunk_end = cursor + AXO_GROUPED_CHUNK < end ? cursor + AXO_GROUPED_CHUNK : end;
            float partial = 0.0f;
            for (int32_t i = cursor; i < chunk_end; ++i) {
                float value = a[left[i]];
                if (b) {
                    float product = value * b[right[i]];
                    partial = partial + product;
                } else {
                    partial = partial + value;
                }
            }
            total = total + partial;
            cursor = chunk_end;
        }
        out[g] = total * scale;
    }
}

/* runtime/backend.rs:3019-3056 (grouped_minimum): first strictly smaller FINITE candidate in
 * plan order wins; a group with no finite candidate yields NaN and winner -1. */
void axo_grouped_minimum(const float *a, const int32_t *offsets, const int32_t *left,
                         int64_t groups, float *out, int32_t *winners) {
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < groups; ++g) {
        int32_t winner = -1;
        float minimum = INFINITY;
        for (int32_t i = offsets[g]; i < offsets[g + 1]; ++i) {
            int32_t candidate = left[i];
            float value = a[candidate];
            int finite = value >= -FLT_MAX && value <= FLT_MAX;
            if (finite && value < minimum) {
                minimum = value;
                winner = candidate;
            }
        }
        winners[g] = winner;
        out[g] = minimum <= FLT_MAX ? minimum : NAN;
    }
}

/* runtime/backend.rs:3059-3099 (grouped_maximum): mirror of grouped_minimum. */
void axo_grouped_maximum(const float *a, const int32_t *offsets, const int32_t *left,
                         int64_t groups, float *out, int32_t *winners) {
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < groups; ++g) {
        int32_t winner = -1;
        float maximum = -INFINITY;
        for (int32_t i = offsets[g]; i < offsets[g + 1]; ++i) {
            int32_t candidate = left[i];
            float value = a[candidate];
            int finite = value >= -FLT_MAX && value <= FLT_MAX;
            if (finite && value > maximum) {
                maximum = value;
                winner = candidate;
            }
        }
        winners[g] = winner;
        out[g] = maximum >= -FLT_MAX ? maximum : NAN;
    }
}

/* runtime/backend.rs:3102-3116: mask[p] = 1 where p is its group's winner, else 0. */
void axo_reduction_winner_mask(const int32_t *winners, const int32_t *group_of_input, int64_t len,
                               float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < len; ++p) out[p] = winners[group_of_input[p]] == p ? 1.0f : 0.0f;
}

/* ---------------------------------------------------------------- elementwise */

/* runtime/backend.rs:2606-2617 */
void axo_mask_gradient(const float *gradient, const float *winners, int64_t len, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) out[i] = winners[i] > 0.0f ? gradient[i] : 0.0f;
}

/* runtime/backend.rs:2624-2628: max(x, 0) */
void axo_relu(const float *a, int64_t len, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) out[i] = a[i] > 0.0f ? a[i] : 0.0f;
}

/* runtime/backend.rs:2629-2640: x > 0 ? g : 0 (input-based mask, zero at x == 0) */
void axo_relu_backward(const float *gradient, const float *a, int64_t len, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) out[i] = a[i] > 0.0f ? gradient[i] : 0.0f;
}

/* runtime/backend.rs:2619-2622 */
void axo_scale(const float *a, int64_t len, float factor, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) out[i] = a[i] * factor;
}

/* runtime/backend.rs:2588-2604: op 0 add, 1 sub, 2 mul, 3 div */
void axo_binary(const float *a, const float *b, int64_t len, int32_t op, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) {
        float x = a[i], y = b[i];
        out[i] = op == 0 ? x + y : op == 1 ? x - y : op == 2 ? x * y : x / y;
    }
}

/* runtime/backend.rs:2057-2101: per output element, (extent, input_stride, output_stride)
 * per dimension; output_stride < 0 marks the selected dimension. */
void axo_select_axis(const float *input, const int32_t *metadata, int32_t rank, int32_t coordinate,
                     int64_t output_len, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < output_len; ++o) {
        int64_t index = 0;
        for (int32_t d = 0; d < rank; ++d) {
            const int32_t *md = metadata + 3 * d;
            if (md[2] < 0)
                index += (int64_t)coordinate * md[1];
            else
                index += ((o / md[2]) % md[0]) * (int64_t)md[1];
        }
        out[o] = input[index];
    }
}

/* runtime/backend.rs:2104-2148: inverse copy; elements off the selected coordinate get 0. */
void axo_select_axis_backward(const float *gradient, const int32_t *metadata, int32_t rank,
                              int32_t coordinate, int64_t input_len, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < input_len; ++i) {
        int64_t index = 0;
        int live = 1;
        for (int32_t d = 0; d < rank; ++d) {
            const int32_t *md = metadata + 3 * d;
            int64_t c = (i / md[1]) % md[0];
            if (md[2] < 0)
                live = live && c == coordinate;
            else
                index += c * (int64_t)md[2];
        }
        out[i] = live ? gradient[index] : 0.0f;
    }
}

/* ---------------------------------------------------------------- softmax / cross-entropy */

/* runtime/backend.rs:2509-2527: p = exp(x - max) / sum.  The reference's reduce_sum tree order is
 * a cuTile internal; the oracle sums in fp64. */
void axo_softmax(const float *a, int64_t rows, int64_t width, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float *x = a + r * width;
        float maximum = -INFINITY;
        for (int64_t j = 0; j < width; ++j) maximum = x[j] > maximum ? x[j] : maximum;
        double sum = 0.0;
        for (int64_t j = 0; j < width; ++j) sum += (double)expf(x[j] - maximum);
        float total = (float)sum;
        for (int64_t j = 0; j < width; ++j) out[r * width + j] = expf(x[j] - maximum) / total;
    }
}

/* runtime/backend.rs:2529-2543: p * (g - sum(g * p)) */
void axo_softmax_backward(const float *gradient, const float *probability, int64_t rows,
                          int64_t width, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        double dot = 0.0;
        for (int64_t j = 0; j < width; ++j)
            dot += (double)gradient[r * width + j] * (double)probability[r * width + j];
        float d = (float)dot;
        for (int64_t j = 0; j < width; ++j) {
            int64_t p = r * width + j;
            out[p] = probability[p] * (gradient[p] - d);
        }
    }
}

/* runtime/backend.rs:2424-2448: three sequential fp32 loops per row -- running max,
 * sum of exp(z - max), loss = sum_j y_j * ((max + ln sum) - z_j). */
void axo_categorical_cross_entropy(const float *logits, const float *targets, int64_t rows,
                                   int64_t width, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float *z = logits + r * width;
        const float *y = targets + r * width;
        float maximum = z[0];
        for (int64_t j = 1; j < width; ++j) maximum = z[j] > maximum ? z[j] : maximum;
        float exponential_sum = 0.0f;
        for (int64_t j = 0; j < width; ++j) exponential_sum = exponential_sum + expf(z[j] - maximum);
        float log_normalizer = maximum + logf(exponential_sum);
        float loss = 0.0f;
        for (int64_t j = 0; j < width; ++j) {
            float term = y[j] * (log_normalizer - z[j]);
            loss = loss + term;
        }
        out[r] = loss;
    }
}

/* runtime/backend.rs:2450-2463: out[pos] = g[row] * (p[pos] - y[pos]) */
void axo_categorical_cross_entropy_backward(const float *gradient, const float *probability,
                                            const float *targets, int64_t rows, int64_t width,
                                            float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < rows * width; ++p)
        out[p] = gradient[p / width] * (probability[p] - targets[p]);
}

/* ---------------------------------------------------------------- Adam */

/* runtime/backend.rs:2545-2586 (adam_moment x2, adam_update), in that expression order:
 *   m' = b1*m + (1-b1)*g ;  v' = b2*v + (1-b2)*(g*g)
 *   p' = p - lr * ((m'/c1) / (sqrt(v'/c2) + eps) + wd*p)                                  */
void axo_adam(const float *value, const float *gradient, const float *first, const float *second,
              int64_t len, float learning_rate, const float *learning_rates, float beta1,
              float beta2, float correction1, float correction2, float epsilon,
              float weight_decay, float *out_value, float *out_first, float *out_second) {
    const float one_minus_b1 = 1.0f - beta1, one_minus_b2 = 1.0f - beta2;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) {
        float g = gradient[i];
        float m = beta1 * first[i] + one_minus_b1 * g;
        float gg = g * g;
        float v = beta2 * second[i] + one_minus_b2 * gg;
        float lr = learning_rates ? learning_rates[i] : learning_rate;
        float mh = m / correction1;
        float vh = v / correction2;
        float p = value[i];
        float denom = sqrtf(vh) + epsilon;
        float step = mh / denom + weight_decay * p;
        out_value[i] = p - lr * step;
        out_first[i] = m;
        out_second[i] = v;
    }
}

/* ---------------------------------------------------------------- Muon helpers */

/* runtime/backend.rs:411-440 with kernels :2150-2180: sum of squares (fp64 accumulate here). */
void axo_sum_squares(const float *a, int64_t len, float *out) {
    double total = 0.0;
#pragma omp parallel for reduction(+ : total) schedule(static)
    for (int64_t i = 0; i < len; ++i) total += (double)a[i] * (double)a[i];
    out[0] = (float)total;
}

/* runtime/backend.rs:2797-2801: 1 / sqrt(x + eps) */
void axo_inverse_sqrt(const float *a, int64_t len, float epsilon, float *out) {
    for (int64_t i = 0; i < len; ++i) out[i] = 1.0f / sqrtf(a[i] + epsilon);
}

/* runtime/backend.rs:2181-2188 */
void axo_multiply_scalar(const float *a, int64_t len, const float *scalar, float *out) {
    const float s = scalar[0];
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) out[i] = a[i] * s;
}
