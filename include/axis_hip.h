/*
 * axis_hip.h -- C ABI of the MI355X (gfx950) backend for furkanhaney/axis's training hot path.
 *
 * One entry point per hot-path method of the reference's `Device`
 * (src/library/src/runtime/backend.rs; signature mirror in runtime/backend_docs.rs), plus a few
 * fused entries a tensor layer may pick when shapes match.  Citations are relative to the
 * reference's src/library/src/.
 *
 * Conventions
 *  - A device handle owns one GPU, one HIP stream and one stream-ordered caching allocator
 *    (replacing the reference's pending/retired buffer lists, backend.rs:297-351).
 *  - Every compute entry is asynchronous on the handle's stream and writes caller-owned device
 *    buffers; inputs are never modified unless an output pointer aliases them (entries that
 *    allow aliasing say so).  The reference's ops return a fresh buffer instead
 *    (backend.rs:1039-1074); a caller reproduces that by allocating the output first.
 *  - All floating-point data is fp32; plan indices and winners are int32.
 *  - Status: 0 on success.  On failure nothing is launched, and axis_last_error() returns a
 *    thread-local message (the reference's Result<_, Box<dyn Error>>, lib.rs:130).  Shape and
 *    limit errors are raised before any launch, as Plan::check_size does (backend.rs:1588).
 */
#ifndef AXIS_HIP_H
#define AXIS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AXIS_OK 0
#define AXIS_ERROR_INVALID 1 /* bad argument or shape: nothing was launched */
#define AXIS_ERROR_HIP 2     /* the HIP runtime reported an error */
#define AXIS_ERROR_MEMORY 3  /* device allocation failed */

typedef struct axis_device_s *axis_device;
typedef struct axis_plan_s *axis_plan;

/* ------------------------------------------------------------------ runtime (backend.rs:203-392) */

/* Thread-local text of the most recent failure in this thread. */
const char *axis_last_error(void);
/* Library version string (also names the offload target). */
const char *axis_version(void);

/* Device::cuda (backend.rs:268): bind GPU `ordinal`, create its stream and allocator. */
int axis_device_create(int ordinal, axis_device *out);
/* Device::cuda_bf16 (backend.rs:274-283): the same device with bf16 matrix products -- every
 * matmul, matmul_left/right_backward and convolution product of this handle rounds its operands to
 * bf16 (nearest, ties to even) and accumulates in fp32 (the operand conversion of matmul_bf16,
 * :2209-2312); parameters, activations outside the products, optimizer state and reductions stay
 * fp32.  axis_device_bf16_matmul reports the mode. */
int axis_device_create_bf16(int ordinal, axis_device *out);
int axis_device_bf16_matmul(axis_device device, int *enabled);
int axis_device_destroy(axis_device device);
/* Device::synchronize (backend.rs:352): wait for every launch on the stream. */
int axis_device_synchronize(axis_device device);
/* The hipStream_t all launches of this handle use. */
int axis_device_stream(axis_device device, void **stream);
/* Device memory from the caching allocator (the allocation behind zeros/track, backend.rs:297-301,
 * :385).  Blocks are 256-byte aligned.  axis_free returns a block for reuse by LATER launches on
 * the same stream, so a buffer may be released as soon as its last use has been enqueued. */
int axis_alloc(axis_device device, size_t bytes, void **out);
int axis_free(axis_device device, void *ptr);
/* Bytes currently handed out, and bytes cached for reuse. */
int axis_memory_stats(axis_device device, size_t *in_use, size_t *cached);
/* Release every cached (free) block back to the driver. */
int axis_empty_cache(axis_device device);
/* Device::upload (backend.rs:365): host -> device; returns once the host buffer may be reused. */
int axis_upload(axis_device device, void *dst, const void *src, size_t bytes);
/* Device::read (backend.rs:372-384): device -> host after all earlier launches; blocking. */
int axis_read(axis_device device, void *dst, const void *src, size_t bytes);
/* Device-to-device copy on the stream (stack_contiguous/contiguous_slice, backend.rs:1311-1362). */
int axis_copy(axis_device device, void *dst, const void *src, size_t bytes);
/* Device::zeros_buffer (backend.rs:385-392) generalised to any fill value. */
int axis_fill(axis_device device, float *out, float value, int64_t len);

/* Launch timing, off by default.  While enabled, every launch of a kernel family is bracketed
 * by HIP events on the handle's stream.  axis_timing_read synchronizes and returns, for the
 * family, the launches since the last reset, their summed duration and their summed algorithmic
 * work: "gemm" (matmul, left and right backward; 2*batch*m*k*n flops each) and "adam"
 * (axis_adam_multi; 28 bytes per parameter, 32 with per-element rates). */
int axis_timing_enable(axis_device device, int enabled);
int axis_timing_reset(axis_device device);
int axis_timing_read(axis_device device, const char *family, int64_t *launches, double *milliseconds,
                     double *work);

/* Deferred finishing sums, off by default (no counterpart in the reference: a launch schedule of
 * this library, used by the autograd tape's backward pass).  While enabled, the entries that
 * produce weight and bias gradients -- axis_matmul_right_backward, axis_conv2d_backward_weight,
 * axis_conv2d_relu_pool_backward_weight, and the d_bias of axis_relu_pool_backward(_mean) --
 * enqueue their products and scatters but record the last sum over their partial results instead
 * of launching it; those outputs hold their values only once the recorded sums have run.
 * axis_finish_flush runs every recorded sum in one launch, with the same results bit for bit;
 * axis_finish_before_read flushes when a recorded sum writes into [ptr, ptr + bytes);
 * axis_finish_defer(device, 0) flushes and stops deferring.  Every entry that touches such an
 * output flushes first by itself: axis_read, axis_copy, axis_upload, axis_fill, axis_free and
 * axis_device_synchronize, and every compute entry, for each buffer it reads or writes (a buffer
 * read through strides is checked at its first byte).  A batch that holds more than 256 MiB of
 * partial results is launched early. */
int axis_finish_defer(axis_device device, int enabled);
int axis_finish_flush(axis_device device);
int axis_finish_before_read(axis_device device, const void *ptr, size_t bytes);
/* Sums recorded and not yet run. */
int axis_finish_pending(axis_device device, int64_t *tasks);

/* ------------------------------------------------------------------ contractions */

/* Device::matmul (backend.rs:934-957): out[b] = a[b] . b[b]; a [batch,m,k], b [batch,k,n],
 * out [batch,m,n], all row-major.  fp32 on MFMA. */
int axis_matmul(axis_device device, const float *a, const float *b, float *out, int64_t batch,
                int64_t m, int64_t k, int64_t n);
/* Linear::forward with a bias (model/nn.rs:268-280): Device::matmul (backend.rs:934-957), then the
 * bias add of the projected output (tensor.rs:779-818 broadcasting `bias` [n] along the rows):
 * out[b][i][j] = (a[b] . b[b])[i][j] + bias[j], the product rounded once and the add once, as the
 * two operations round them.  bias must not alias out. */
int axis_matmul_bias(axis_device device, const float *a, const float *b, const float *bias, float *out,
                     int64_t batch, int64_t m, int64_t k, int64_t n);
/* out[b] = beta * d[b] + alpha * (a[b] . b[b]) for row-major [m,k] x [k,n] (d and out [m,n], d not
 * aliasing out): the Newton-Schulz steps of Muon::zeroth_power (optim.rs:728-752),
 * `gram.scale(b).add(gram2.scale(c))` and `x.scale(a).add(b.x)`, with the product's scale, the
 * addend's scale and the sum each rounded once, as the separate operations round them. */
int axis_matmul_axpby(axis_device device, const float *a, const float *b, const float *d, float *out,
                      int64_t batch, int64_t m, int64_t k, int64_t n, float alpha, float beta);
/* Device::matmul_left_backward (backend.rs:958-989), dgrad: out[b] = gradient[b] . rhs[b]^T;
 * gradient [batch,m,n], rhs [batch,k,n], out [batch,m,k]. */
int axis_matmul_left_backward(axis_device device, const float *gradient, const float *rhs,
                              float *out, int64_t batch, int64_t m, int64_t k, int64_t n);
/* Device::matmul_right_backward (backend.rs:990-1021), wgrad: out[b] = lhs[b]^T . gradient[b];
 * lhs [batch,m,k], gradient [batch,m,n], out [batch,k,n].  Deterministic split over m. */
int axis_matmul_right_backward(axis_device device, const float *lhs, const float *gradient,
                               float *out, int64_t batch, int64_t m, int64_t k, int64_t n);
/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same product as
 * axis_matmul_right_backward, bit for bit, with its split partial sums in a file-scope 64 MiB
 * device array (one per GPU, held until the process ends) instead of the caching allocator; it
 * calls no allocator.  Nothing in the array needs to start at zero.  A product whose partial
 * sums exceed 64 MiB is rejected before any launch (on MI355X's 256 CUs the split rule never
 * needs more than about 53 MB); bf16 handles are rejected.  Calls on one GPU share the array and
 * one event per GPU: each call's launches wait for the previous call's (from any handle on that
 * GPU) and it records its own, so calls from different handles run one after the other instead of
 * racing.  Calls from different host threads at the same moment must be serialised by the caller
 * (the wait and record pair is not atomic across threads). */
int axis_matmul_right_backward_noalloc(axis_device device, const float *lhs, const float *gradient,
                                       float *out, int64_t batch, int64_t m, int64_t k, int64_t n);

/* ------------------------------------------------------------------ unfold / fold (im2col) */

/* Field-for-field the reference's UnfoldSpec (backend.rs:1481-1501), built by the tensor layer
 * (tensor.rs:3751-3946).  Only spatial_rank == 2 is supported here. */
typedef struct {
    int32_t spatial_rank;
    int64_t input_len;
    int64_t output_len;
    int32_t input_rank;
    int32_t output_rank;
    int32_t forward_metadata[32];  /* per output dim: extent, output_stride, input_stride, role */
    int32_t backward_metadata[32]; /* per input dim: extent, input_stride, output_stride, role */
    int32_t channels_per_group;
    float fill;
    int32_t kernel[3];
    int32_t stride[3];
    int32_t padding[3];
    int32_t input_spatial[3];
    int32_t output_spatial[3];
    int32_t input_special_strides[4];
    int32_t output_special_strides[5];
} axis_unfold_spec;

/* Device::unfold (backend.rs:1127-1189), kernel unfold2d (:1604-1689): im2col gather with
 * `fill` outside the input.  out has spec->output_len elements. */
int axis_unfold(axis_device device, const float *input, float *out, const axis_unfold_spec *spec);
/* Device::unfold_backward (backend.rs:1191-1253), kernel unfold2d_backward (:1795-1889):
 * gather-form col2im, no atomics, each input sums its patch gradients in ky-major/kx-minor
 * order.  out has spec->input_len elements. */
int axis_unfold_backward(axis_device device, const float *gradient, float *out,
                         const axis_unfold_spec *spec);

/* ------------------------------------------------------------------ CSR plans (backend.rs:1542-1597) */

/* Plan::groups/gather/reverse uploaded once (the reference's device_plan cache,
 * backend.rs:1449-1475, plus the chunk tables of chunked_offsets, :37-50, which the reference
 * re-uploads per call).  Arrays are host pointers; `right` may be NULL when the plan is not a
 * product plan.  count = offsets[groups].  Rejects 0 or more than 16,777,216 contributions
 * unless `uncapped` is nonzero (the reference's experimental bound, backend.rs:1588-1596). */
int axis_plan_create(axis_device device, const int32_t *offsets, const int32_t *left,
                     const int32_t *right, int64_t groups, int uncapped, axis_plan *out);
int axis_plan_destroy(axis_device device, axis_plan plan);
/* Device::grouped (backend.rs:1089-1125): out[g] = scale * sum over the group's contributions of
 * a[left[i]] (times b[right[i]] when b != NULL), summed in chunks of 512 and then over chunks in
 * order, exactly as grouped_partial/grouped_combine (:2964-3016).  out has `groups` elements. */
int axis_grouped(axis_device device, const float *a, const float *b, axis_plan plan, float scale,
                 float *out);
/* Device::grouped_minimum / grouped_maximum (backend.rs:1365-1440, kernels :3019-3116): first
 * strictly better FINITE candidate in plan order; NaN and winner -1 for a group with none.
 * `winner_mask` (input_len floats) is the one-hot reduction_winner_mask in input order, built from
 * the reverse (gather) plan.  `winners` may be NULL. */
int axis_grouped_minimum(axis_device device, const float *a, int64_t input_len, axis_plan forward,
                         axis_plan reverse, float *out, int32_t *winners, float *winner_mask);
int axis_grouped_maximum(axis_device device, const float *a, int64_t input_len, axis_plan forward,
                         axis_plan reverse, float *out, int32_t *winners, float *winner_mask);

/* ------------------------------------------------------------------ elementwise */

/* Device::mask_gradient (backend.rs:482-491): out = winners > 0 ? gradient : 0. */
int axis_mask_gradient(axis_device device, const float *gradient, const float *winners, float *out,
                       int64_t len);
/* Device::relu / relu_backward (backend.rs:514-524): max(x,0); x > 0 ? g : 0. */
int axis_relu(axis_device device, const float *a, float *out, int64_t len);
int axis_relu_backward(axis_device device, const float *gradient, const float *a, float *out,
                       int64_t len);
/* Device::scale (backend.rs:492-497). out may alias a. */
int axis_scale(axis_device device, const float *a, float factor, float *out, int64_t len);
/* Device::binary (backend.rs:441-447): op 0 add, 1 sub, 2 mul, 3 div.  out may alias a or b. */
int axis_binary(axis_device device, const float *a, const float *b, int32_t op, float *out,
                int64_t len);
/* Device::select_axis / select_axis_backward (backend.rs:1271-1309, kernels :2057-2148):
 * rank-generic strided copier; metadata (host, 3 ints per dim: extent, input_stride,
 * output_stride, output_stride < 0 marking the selected dim), rank <= 10. */
int axis_select_axis(axis_device device, const float *input, float *out, const int32_t *metadata,
                     int32_t rank, int32_t coordinate, int64_t output_len);
int axis_select_axis_backward(axis_device device, const float *gradient, float *out,
                              const int32_t *metadata, int32_t rank, int32_t coordinate,
                              int64_t input_len);

/* ------------------------------------------------------------------ softmax / cross-entropy */

/* Device::softmax / softmax_backward (backend.rs:893-932): rows of `width` contiguous values. */
int axis_softmax(axis_device device, const float *a, float *out, int64_t rows, int64_t width);
int axis_softmax_backward(axis_device device, const float *gradient, const float *probability,
                          float *out, int64_t rows, int64_t width);
/* Device::categorical_cross_entropy (backend.rs:829-845, kernel :2424-2448): per row, the
 * running max, sum of exp(z - max) and sum_j y_j ((max + ln sum) - z_j), each in column order. */
int axis_categorical_cross_entropy(axis_device device, const float *logits, const float *targets,
                                   float *out, int64_t rows, int64_t width);
/* Device::categorical_cross_entropy_backward (backend.rs:846-863, kernel :2450-2463):
 * out[pos] = gradient[row] * (probability[pos] - targets[pos]). */
int axis_categorical_cross_entropy_backward(axis_device device, const float *gradient,
                                            const float *probability, const float *targets,
                                            float *out, int64_t rows, int64_t width);
/* The same backward for a loss that is the mean of the rows' losses (`.mean([rows])`,
 * tensor.rs:2837-2845, a grouped sum times 1/rows): its backward broadcasts the scalar gradient
 * times factor (1/rows) to every row (axis_broadcast_middle), which this entry folds in:
 * out[pos] = (gradient[0] * factor) * (probability[pos] - targets[pos]), the values of the two
 * launches it replaces.  d_bias (or NULL) also receives the column sums of out in
 * axis_bias_gradient's order (the bias gradient of the layer that produced the logits). */
int axis_categorical_cross_entropy_backward_mean(axis_device device, const float *gradient, float factor,
                                                 const float *probability, const float *targets, float *out,
                                                 float *d_bias, int64_t rows, int64_t width);

/* ------------------------------------------------------------------ optimizer */

/* Device::adam (backend.rs:1023-1075): m' = b1 m + (1-b1) g; v' = b2 v + (1-b2) g^2;
 * p' = p - lr ((m'/c1) / (sqrt(v'/c2) + eps) + wd p), one fused pass (28 bytes per element).
 * learning_rates (per element) may be NULL.  Outputs may alias value/first/second (in place). */
int axis_adam(axis_device device, const float *value, const float *gradient, const float *first,
              const float *second, const float *learning_rates, int64_t len, float learning_rate,
              float beta1, float beta2, float correction1, float correction2, float epsilon,
              float weight_decay, float *out_value, float *out_first, float *out_second);

/* One tensor of a multi-tensor Adam launch (updated in place). */
typedef struct {
    float *value;
    const float *gradient;
    float *first;
    float *second;
    const float *learning_rates; /* may be NULL */
    int64_t len;
} axis_adam_tensor;
/* Adam over many tensors in one launch (Adam::prepare's per-parameter loop, optim.rs:102-142,
 * fused); same arithmetic as axis_adam, in place.  `tensors` is a host array. */
int axis_adam_multi(axis_device device, const axis_adam_tensor *tensors, int32_t count,
                    float learning_rate, float beta1, float beta2, float correction1,
                    float correction2, float epsilon, float weight_decay);

/* Muon::prepare's elementwise steps (model/optim.rs:644-657 and :666-669) in one pass each, every
 * operation rounded as the reference's separate scale / add / sub tensor ops round it:
 *   axis_muon_momentum: next = previous * momentum + gradient * (1 - momentum) (previous NULL on the
 *     first step: gradient * (1 - momentum)); with nesterov != 0 also
 *     direction = gradient * (1 - momentum) + next * momentum.
 *   axis_muon_apply: out = value * decay - orthogonal * rate, with decay = 1 - lr * weight_decay and
 *     rate = lr * scaling computed by the caller in fp32 as the reference does.
 * All buffers hold `len` elements in the same layout, 16-byte aligned; outputs must not alias
 * inputs. */
int axis_muon_momentum(axis_device device, const float *gradient, const float *previous, float *next,
                       float *direction, float momentum, int nesterov, int64_t len);
int axis_muon_apply(axis_device device, const float *value, const float *orthogonal, float *out, float decay,
                    float rate, int64_t len);

/* Device::sum_squares (backend.rs:411-440): out[0] = sum of a^2 (out is a device scalar). */
int axis_sum_squares(axis_device device, const float *a, int64_t len, float *out);
/* Device::inverse_sqrt (backend.rs:630-635, kernel :2797-2801): 1 / sqrt(x + eps). */
int axis_inverse_sqrt(axis_device device, const float *a, float epsilon, float *out, int64_t len);
/* Device::multiply_scalar (backend.rs:466-481): out = a * scalar[0], scalar on the device. */
int axis_multiply_scalar(axis_device device, const float *a, const float *scalar, float *out,
                         int64_t len);

/* ------------------------------------------------------------------ fused entries
 * Each equals a composition of the entries above on the layouts named; none has a single
 * Device counterpart in the reference. */

/* align(bias) + binary(add) (tensor.rs:706-778, 819-821) for a row-major [rows, width] operand
 * and a [width] bias: out[r][c] = a[r][c] + bias[c].  With relu_out != NULL also writes
 * max(out, 0) there (Tensor::relu, tensor.rs:2136-2147).  out may alias a. */
int axis_bias_add(axis_device device, const float *a, const float *bias, float *out,
                  float *relu_out, int64_t rows, int64_t width);
/* The bias's Group rule over the align reverse plan of [rows, width] <- [width]
 * (tensor.rs:679-698 + Device::grouped): out[c] = sum_r gradient[r][c] in chunks of 512 rows,
 * chunk partials in order -- the reference's exact summation order.  With relu_input != NULL the
 * gradient is first masked by relu_input > 0 (Device::relu_backward) and the masked gradient is
 * also written to masked_out. */
int axis_bias_gradient(axis_device device, const float *gradient, const float *relu_input,
                       float *masked_out, float *out, int64_t rows, int64_t width);
/* Max pooling of a [outer, height, width, channels] (channel-innermost) tensor, window
 * kernel/stride/padding per spatial axis: the forward of -min(-unfold(x, -inf)) over the window
 * (convolution.rs:1357-1370) plus the window-local winner index (ky*kw + kx, 255 = none) as one
 * byte per output.  out [outer, oh, ow, channels]. */
int axis_max_pool2d(axis_device device, const float *input, float *out, uint8_t *argmax,
                    int64_t outer, int32_t height, int32_t width, int64_t channels,
                    const int32_t kernel[2], const int32_t stride[2], const int32_t padding[2]);
/* Its backward: Rule::Minimum (mask at the winner) followed by the window col2im, summing, per
 * input element, the gradients of the windows it won in ky-major/kx-minor order. */
int axis_max_pool2d_backward(axis_device device, const float *gradient, const uint8_t *argmax,
                             float *out, int64_t outer, int32_t height, int32_t width,
                             int64_t channels, const int32_t kernel[2], const int32_t stride[2],
                             const int32_t padding[2]);
/* mean/sum over the middle axis of a row-major [outer, reduce, inner] tensor
 * (reduce_grouped, tensor.rs:2808-2845): out[o][i] = factor * sum_r a[o][r][i], summed in the
 * reference's order (chunks of 512, then chunks). */
int axis_reduce_middle(axis_device device, const float *a, float *out, int64_t outer,
                       int64_t reduce, int64_t inner, float factor);
/* Tensor::reduce_grouped for any set of axes (tensor.rs:2755-2854: reduction_plans, then
 * Device::grouped, backend.rs:1089-1125) without an index plan, so without its 16,777,216 cap.
 * The tensor has rank dims with the given extents and element strides (a dense layout: the
 * strides are a permutation of row-major ones); reduced[d] != 0 marks the summed dims.  out is
 * row-major over the kept dims in dim order: out = factor * sum, each group's contributions in
 * increasing memory position, chunks of 512 then the chunk partials in order -- bit-identical to
 * grouped() over the reference's reverse plan.  rank <= 10, at most INT32_MAX elements. */
int axis_reduce_axes(axis_device device, const float *a, float *out, int32_t rank, const int64_t *extents,
                     const int64_t *strides, const int32_t *reduced, float factor);
/* Its backward (the gather plan's grouped, tensor.rs:2805-2854): out, laid out like the input,
 * gets factor * gradient[kept coordinates] at every element. */
int axis_reduce_axes_backward(axis_device device, const float *gradient, float *out, int32_t rank,
                              const int64_t *extents, const int64_t *strides, const int32_t *reduced,
                              float factor);
/* Tensor::min / max over one axis (tensor.rs:2880-2946: Device::grouped_minimum over the forward
 * plan, then the winner mask over the gather plan, backend.rs:1365-1440, kernels :3019-3116)
 * without the plans, so without their 16,777,216 cap.  The tensor is dense (rank <= 10 dims with
 * the given extents and element strides); out is row-major over the other dims in dim order and
 * holds the first strictly smaller (maximum != 0: greater) FINITE value along `axis`, NaN when
 * none is finite; winner_mask (laid out like the input) is 1 at each output's winner, else 0 --
 * bit-identical to axis_grouped_minimum/maximum over the reference's plans. */
int axis_extreme_axis(axis_device device, const float *a, int32_t rank, const int64_t *extents,
                      const int64_t *strides, int32_t axis, int32_t maximum, float *out, float *winner_mask);
/* Its backward (Rule::Minimum, tensor.rs:5679-5683: grouped over the gather plan, then
 * mask_gradient): out, laid out like the input, is 0 + gradient[output] at each winner, else 0. */
int axis_extreme_axis_backward(axis_device device, const float *gradient, const float *winner_mask, int32_t rank,
                               const int64_t *extents, const int64_t *strides, int32_t axis, float *out);
/* Its Group-rule backward: out[o][r][i] = factor * gradient[o][i]. */
int axis_broadcast_middle(axis_device device, const float *gradient, float *out, int64_t outer,
                          int64_t reduce, int64_t inner, float factor);
/* Implicit-GEMM convolution, one group: the reference's Conv2d lowering (convolution.rs:211-235:
 * unfold -> contract -> merge -> + bias) without materialising the patch matrix.  input is read
 * through input_strides {batch, channel, row, column} (elements; NULL = channel-innermost
 * contiguous [batch, height, width, channels]); weight in the reference's layout
 * [(channel, ky, kx), out_channels]; bias [out_channels] or NULL;
 * out [batch, out_h, out_w, out_channels] (the reference's unfold output order).  The patch
 * reduction runs in (ky, kx, channel) order on fp32 MFMA -- in (channel, ky, kx) order for short
 * layers (stride 1, channels * kh * kw <= 31) -- so results agree with the explicit path to fp32
 * tolerance. */
int axis_conv2d_forward(axis_device device, const float *input, const int64_t input_strides[4],
                        const float *weight, const float *bias, float *out, int64_t batch,
                        int32_t height, int32_t width, int32_t channels, int32_t out_channels,
                        const int32_t kernel[2], const int32_t stride[2], const int32_t padding[2]);
/* The same convolution followed by ReLU and a non-overlapping max pool (window = stride = pool,
 * no padding) in the GEMM epilogue: Conv2d -> ReLU -> MaxPool2d (convolution.rs:211-235,
 * tensor.rs:2136-2147, convolution.rs:1357-1370) with the pre-activation never written.
 * pooled and argmax are [batch, out_h/pool[0], out_w/pool[1], out_channels]; argmax holds the
 * window-local winner ky*pool[1]+kx (255 with a NaN output when no finite value exists), as
 * axis_max_pool2d.  Requires out_h % pool[0] == 0, out_w % pool[1] == 0 and, unless the
 * layer is short (stride 1, channels * kh * kw <= 31, 2x2 pool), 128 % (pool[0] * out_w) == 0.
 * Short layers reduce in the reference's patch order (channel, ky, kx), as axis_conv2d_forward
 * does for them, so the two entries agree bit for bit there. */
int axis_conv2d_relu_pool_forward(axis_device device, const float *input,
                                  const int64_t input_strides[4], const float *weight,
                                  const float *bias, float *pooled, uint8_t *argmax, int64_t batch,
                                  int32_t height, int32_t width, int32_t channels,
                                  int32_t out_channels, const int32_t kernel[2],
                                  const int32_t stride[2], const int32_t padding[2],
                                  const int32_t pool[2]);
/* Its input gradient (Rule::MatmulLeft then Rule::Unfold, tensor.rs:5650-5680): d_input
 * [batch, height, width, channels] (channel-innermost) from gradient
 * [batch, out_h, out_w, out_channels], computed as a stride-1 convolution with the flipped kernel
 * (no col2im pass).  Stride 1 and padding < kernel only. */
int axis_conv2d_backward_data(axis_device device, const float *gradient, const float *weight,
                              float *d_input, int64_t batch, int32_t height, int32_t width,
                              int32_t channels, int32_t out_channels, const int32_t kernel[2],
                              const int32_t stride[2], const int32_t padding[2]);
/* Its weight gradient (Rule::MatmulRight over the patches): d_weight in the reference's layout
 * [(channel, ky, kx), out_channels], deterministic split over output pixels; input strides as in
 * axis_conv2d_forward. */
int axis_conv2d_backward_weight(axis_device device, const float *input,
                                const int64_t input_strides[4], const float *gradient,
                                float *d_weight, int64_t batch, int32_t height, int32_t width,
                                int32_t channels, int32_t out_channels, const int32_t kernel[2],
                                const int32_t stride[2], const int32_t padding[2]);
/* Weight and bias gradients of Conv2d -> ReLU -> MaxPool2d (the composition
 * axis_conv2d_relu_pool_forward computes) straight from the pool's outputs: the reference's
 * Rule::Minimum gather + mask and Rule::Relu (tensor.rs:5679-5683, :2136-2147) into the
 * convolution's Rule::MatmulRight (tensor.rs:5650-5680) and the bias's column sum
 * (tensor.rs:706-778).  Equals axis_relu_pool_backward followed by axis_conv2d_backward_weight
 * (to fp32 tolerance; deterministic run to run); when stride is 1, channels * kh * kw <= 31 and
 * the pool is 2x2, the pre-activation gradient is never written to device memory.  gradient,
 * pooled and argmax are [batch, out_h/pool[0], out_w/pool[1], out_channels]; d_weight
 * [(channel, ky, kx), out_channels]; d_bias [out_channels] or NULL; input strides as in
 * axis_conv2d_forward. */
int axis_conv2d_relu_pool_backward_weight(axis_device device, const float *input,
                                          const int64_t input_strides[4], const float *gradient,
                                          const float *pooled, const uint8_t *argmax, float *d_weight,
                                          float *d_bias, int64_t batch, int32_t height, int32_t width,
                                          int32_t channels, int32_t out_channels, const int32_t kernel[2],
                                          const int32_t stride[2], const int32_t padding[2],
                                          const int32_t pool[2]);
/* Backward of ReLU -> non-overlapping max pool given the pool's outputs (Rule::Minimum gather +
 * mask, col2im, tensor.rs:5679-5683; Rule::Relu, tensor.rs:2136-2147): d_pre
 * [outer, height, width, channels] holds 0.0f + gradient at each window's winner when the pooled
 * value is > 0, and 0 elsewhere -- exactly axis_max_pool2d_backward then axis_relu_backward.
 * d_bias (or NULL) receives the column sums of d_pre in a fixed association (identical on every
 * run; equal to axis_bias_gradient's chunked order to fp32 tolerance, bit for bit when 256 is not
 * a multiple of the channel-vector count).  height % pool[0] == 0 and width % pool[1] == 0. */
int axis_relu_pool_backward(axis_device device, const float *gradient, const float *pooled,
                            const uint8_t *argmax, float *d_pre, float *d_bias, int64_t outer,
                            int32_t height, int32_t width, int32_t channels, const int32_t pool[2]);
/* The same backward when the pooled tensor's only reader is a mean over its pooled height and width
 * (tensor.rs:2837-2845): gradient is that mean's output gradient [outer, channels], and every
 * pooled position's gradient is gradient[o][c] * factor (factor = 1 / pooled positions) -- the
 * values the mean's backward (axis_broadcast_middle) would store, without storing them. */
int axis_relu_pool_backward_mean(axis_device device, const float *gradient, float factor, const float *pooled,
                                 const uint8_t *argmax, float *d_pre, float *d_bias, int64_t outer,
                                 int32_t height, int32_t width, int32_t channels, const int32_t pool[2]);
/* Softmax + categorical cross-entropy of [rows, width] logits in one pass (tensor.rs:1540-1543):
 * writes probability [rows, width] and per-row loss [rows]; each equals the separate entries. */
int axis_softmax_cross_entropy(axis_device device, const float *logits, const float *targets,
                               float *probability, float *loss, int64_t rows, int64_t width);

#ifdef __cplusplus
}
#endif

#endif
