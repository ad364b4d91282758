/*
 * CPU restatement of furkanhaney/axis's training hot path (the parity oracle).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (axis_amd/, include/) links,
 * loads or calls this code: it is the checker that tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg compare the HIP path against.
 *
 * Every function names the reference file:line whose arithmetic it restates
 * (paths relative to the reference root, src/library/src/...).  Where the
 * reference fixes an evaluation order (sequential sums in CSR chunks, col2im in
 * ky-major/kx-minor order, scalar loops in cross-entropy, the Adam update
 * expression) the oracle follows it in fp32 with contraction disabled
 * (built with -ffp-contract=off), so the GPU path can be checked bit-exactly
 * where it follows the same order.  Where the reference's order is a cuTile
 * internal (the mma accumulation order of matmul, the reduce_sum tree of
 * softmax and sum_squares) the oracle accumulates in fp64 and parity is
 * tolerance-level by construction.
 */
#ifndef AXIS_ORACLE_H
#define AXIS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Geometry of one 2-D unfold (im2col) / unfold_backward (col2im), field for field
 * the reference's UnfoldSpec (runtime/backend.rs:1481-1501). */
typedef struct {
    int32_t spatial_rank;
    int64_t input_len;
    int64_t output_len;
    int32_t input_rank;
    int32_t output_rank;
    int32_t forward_metadata[32];  /* 4 per output dim: extent, output_stride, input_stride, role */
    int32_t backward_metadata[32]; /* 4 per input dim: extent, input_stride, output_stride, role */
    int32_t channels_per_group;
    float fill;
    int32_t kernel[3];
    int32_t stride[3];
    int32_t padding[3];
    int32_t input_spatial[3];
    int32_t output_spatial[3];
    int32_t input_special_strides[4];
    int32_t output_special_strides[5];
} axo_unfold_spec;

/* RNG: algebra/tensor.rs:29-71 */
void axo_xorshift_unit_stream(uint64_t seed, int64_t count, float *out);
void axo_uniform_host_values(uint64_t seed, int64_t count, float low, float high, float *out);
void axo_normal_host_values(uint64_t seed, int64_t count, float mean, float std, float *out);
float axo_powi(float base, int32_t exponent);

/* Contractions: runtime/backend.rs:934-1021 (kernels :2190-2290) */
void axo_bf16_round(const float *a, int64_t len, float *out);
void axo_matmul(const float *a, const float *b, int64_t batch, int64_t m, int64_t k, int64_t n, float *out);
void axo_matmul_left_backward(const float *gradient, const float *rhs, int64_t batch, int64_t m,
                              int64_t k, int64_t n, float *out);
void axo_matmul_right_backward(const float *lhs, const float *gradient, int64_t batch, int64_t m,
                               int64_t k, int64_t n, float *out);

/* im2col / col2im: runtime/backend.rs:1604-1689, :1795-1889 */
void axo_unfold2d(const float *input, const axo_unfold_spec *spec, float *out);
void axo_unfold2d_backward(const float *gradient, const axo_unfold_spec *spec, float *out);

/* CSR plans: runtime/backend.rs:1089-1125, :37-50, kernels :2964-3116 */
void axo_grouped(const float *a, const float *b, const int32_t *offsets, const int32_t *left,
                 const int32_t *right, int64_t groups, float scale, float *out);
void axo_grouped_minimum(const float *a, const int32_t *offsets, const int32_t *left,
                         int64_t groups, float *out, int32_t *winners);
void axo_grouped_maximum(const float *a, const int32_t *offsets, const int32_t *left,
                         int64_t groups, float *out, int32_t *winners);
void axo_reduction_winner_mask(const int32_t *winners, const int32_t *group_of_input, int64_t len,
                               float *out);

/* Elementwise: runtime/backend.rs kernels :2588-2640 */
void axo_mask_gradient(const float *gradient, const float *winners, int64_t len, float *out);
void axo_relu(const float *a, int64_t len, float *out);
void axo_relu_backward(const float *gradient, const float *a, int64_t len, float *out);
void axo_scale(const float *a, int64_t len, float factor, float *out);
void axo_binary(const float *a, const float *b, int64_t len, int32_t op, float *out);

/* Layout copier: runtime/backend.rs:2057-2148 */
void axo_select_axis(const float *input, const int32_t *metadata, int32_t rank, int32_t coordinate,
                     int64_t output_len, float *out);
void axo_select_axis_backward(const float *gradient, const int32_t *metadata, int32_t rank,
                              int32_t coordinate, int64_t input_len, float *out);

/* Softmax and categorical cross-entropy: runtime/backend.rs:2424-2543 */
void axo_softmax(const float *a, int64_t rows, int64_t width, float *out);
void axo_softmax_backward(const float *gradient, const float *probability, int64_t rows,
                          int64_t width, float *out);
void axo_categorical_cross_entropy(const float *logits, const float *targets, int64_t rows,
                                   int64_t width, float *out);
void axo_categorical_cross_entropy_backward(const float *gradient, const float *probability,
                                            const float *targets, int64_t rows, int64_t width,
                                            float *out);

/* Adam / AdamW: runtime/backend.rs:1023-1075, kernels :2545-2586 */
void axo_adam(const float *value, const float *gradient, const float *first, const float *second,
              int64_t len, float learning_rate, const float *learning_rates, float beta1,
              float beta2, float correction1, float correction2, float epsilon,
              float weight_decay, float *out_value, float *out_first, float *out_second);

/* Muon helpers: runtime/backend.rs:411-440 (sum_squares), :2797-2801, :2181-2188 */
void axo_sum_squares(const float *a, int64_t len, float *out);
void axo_inverse_sqrt(const float *a, int64_t len, float epsilon, float *out);
void axo_multiply_scalar(const float *a, int64_t len, const float *scalar, float *out);

int axo_threads(void);
void axo_set_threads(int threads);

#ifdef __cplusplus
}
#endif

#endif
