//! Raw declarations of libaxis_hip, the C ABI in `include/axis_hip.h` (MI355X / gfx950 backend of
//! axis's training hot path).  One `extern "C"` item per header prototype, same order of
//! arguments and the same C types (`tests/test_abi.py` compares the two argument by argument).
//! A `hip` backend of the reference's `Device` (src/library/src/runtime/backend.rs:116) wraps
//! these calls; see `backend.rs:116-129` and `runtime/backend_docs.rs:13-80` for the method set.
#![allow(non_camel_case_types)]
use std::os::raw::{c_char, c_int, c_void};

#[repr(C)] pub struct axis_device_s { _p: [u8; 0] }
pub type axis_device = *mut axis_device_s;
#[repr(C)] pub struct axis_plan_s { _p: [u8; 0] }
pub type axis_plan = *mut axis_plan_s;

#[repr(C)]
pub struct axis_unfold_spec {            // == backend.rs:1481-1501 UnfoldSpec, flattened
    pub spatial_rank: i32, pub input_len: i64, pub output_len: i64,
    pub input_rank: i32, pub output_rank: i32,
    pub forward_metadata: [i32; 32], pub backward_metadata: [i32; 32],
    pub channels_per_group: i32, pub fill: f32,
    pub kernel: [i32; 3], pub stride: [i32; 3], pub padding: [i32; 3],
    pub input_spatial: [i32; 3], pub output_spatial: [i32; 3],
    pub input_special_strides: [i32; 4], pub output_special_strides: [i32; 5],
}

#[repr(C)]
pub struct axis_adam_tensor {
    pub value: *mut f32, pub gradient: *const f32, pub first: *mut f32, pub second: *mut f32,
    pub learning_rates: *const f32, pub len: i64,
}

#[link(name = "axis_hip")]
extern "C" {
    pub fn axis_last_error() -> *const c_char;
    pub fn axis_version() -> *const c_char;
    pub fn axis_device_create(ordinal: c_int, out: *mut axis_device) -> c_int;
    pub fn axis_device_create_bf16(ordinal: c_int, out: *mut axis_device) -> c_int;
    pub fn axis_device_bf16_matmul(d: axis_device, enabled: *mut c_int) -> c_int;
    pub fn axis_device_destroy(d: axis_device) -> c_int;
    pub fn axis_device_synchronize(d: axis_device) -> c_int;
    pub fn axis_device_stream(d: axis_device, stream: *mut *mut c_void) -> c_int;
    pub fn axis_alloc(d: axis_device, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn axis_free(d: axis_device, p: *mut c_void) -> c_int;
    pub fn axis_memory_stats(d: axis_device, in_use: *mut usize, cached: *mut usize) -> c_int;
    pub fn axis_empty_cache(d: axis_device) -> c_int;
    pub fn axis_copy(d: axis_device, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn axis_upload(d: axis_device, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn axis_read(d: axis_device, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn axis_fill(d: axis_device, out: *mut f32, value: f32, len: i64) -> c_int;
    pub fn axis_matmul(d: axis_device, a: *const f32, b: *const f32, out: *mut f32,
                       batch: i64, m: i64, k: i64, n: i64) -> c_int;
    pub fn axis_matmul_bias(d: axis_device, a: *const f32, b: *const f32, bias: *const f32,
                            out: *mut f32, batch: i64, m: i64, k: i64, n: i64) -> c_int;
    pub fn axis_matmul_axpby(d: axis_device, a: *const f32, b: *const f32, addend: *const f32,
                             out: *mut f32, batch: i64, m: i64, k: i64, n: i64,
                             alpha: f32, beta: f32) -> c_int;
    pub fn axis_matmul_left_backward(d: axis_device, g: *const f32, rhs: *const f32, out: *mut f32,
                                     batch: i64, m: i64, k: i64, n: i64) -> c_int;
    pub fn axis_matmul_right_backward(d: axis_device, lhs: *const f32, g: *const f32, out: *mut f32,
                                      batch: i64, m: i64, k: i64, n: i64) -> c_int;
    // No reference counterpart: the same product for callers that cannot allocate (graph capture).
    pub fn axis_matmul_right_backward_noalloc(d: axis_device, lhs: *const f32, g: *const f32,
                                              out: *mut f32, batch: i64, m: i64, k: i64,
                                              n: i64) -> c_int;
    pub fn axis_unfold(d: axis_device, input: *const f32, out: *mut f32,
                       spec: *const axis_unfold_spec) -> c_int;
    pub fn axis_unfold_backward(d: axis_device, g: *const f32, out: *mut f32,
                                spec: *const axis_unfold_spec) -> c_int;
    pub fn axis_reduce_axes(d: axis_device, a: *const f32, out: *mut f32, rank: i32,
                            extents: *const i64, strides: *const i64, reduced: *const i32,
                            factor: f32) -> c_int;
    pub fn axis_reduce_axes_backward(d: axis_device, g: *const f32, out: *mut f32, rank: i32,
                                     extents: *const i64, strides: *const i64, reduced: *const i32,
                                     factor: f32) -> c_int;
    pub fn axis_extreme_axis(d: axis_device, a: *const f32, rank: i32, extents: *const i64,
                             strides: *const i64, axis: i32, maximum: i32, out: *mut f32,
                             winner_mask: *mut f32) -> c_int;
    pub fn axis_extreme_axis_backward(d: axis_device, g: *const f32, winner_mask: *const f32, rank: i32,
                                      extents: *const i64, strides: *const i64, axis: i32,
                                      out: *mut f32) -> c_int;
    pub fn axis_plan_create(d: axis_device, offsets: *const i32, left: *const i32, right: *const i32,
                            groups: i64, uncapped: c_int, out: *mut axis_plan) -> c_int;
    pub fn axis_plan_destroy(d: axis_device, p: axis_plan) -> c_int;
    pub fn axis_grouped(d: axis_device, a: *const f32, b: *const f32, plan: axis_plan, scale: f32,
                        out: *mut f32) -> c_int;
    pub fn axis_grouped_minimum(d: axis_device, a: *const f32, input_len: i64, forward: axis_plan,
                                reverse: axis_plan, out: *mut f32, winners: *mut i32,
                                winner_mask: *mut f32) -> c_int;
    pub fn axis_grouped_maximum(d: axis_device, a: *const f32, input_len: i64, forward: axis_plan,
                                reverse: axis_plan, out: *mut f32, winners: *mut i32,
                                winner_mask: *mut f32) -> c_int;
    pub fn axis_mask_gradient(d: axis_device, g: *const f32, w: *const f32, out: *mut f32, len: i64) -> c_int;
    pub fn axis_relu(d: axis_device, a: *const f32, out: *mut f32, len: i64) -> c_int;
    pub fn axis_relu_backward(d: axis_device, g: *const f32, a: *const f32, out: *mut f32, len: i64) -> c_int;
    pub fn axis_scale(d: axis_device, a: *const f32, f: f32, out: *mut f32, len: i64) -> c_int;
    pub fn axis_binary(d: axis_device, a: *const f32, b: *const f32, op: i32, out: *mut f32, len: i64) -> c_int;
    pub fn axis_softmax(d: axis_device, a: *const f32, out: *mut f32, rows: i64, width: i64) -> c_int;
    pub fn axis_softmax_backward(d: axis_device, g: *const f32, p: *const f32, out: *mut f32,
                                 rows: i64, width: i64) -> c_int;
    pub fn axis_select_axis(d: axis_device, input: *const f32, out: *mut f32, metadata: *const i32,
                            rank: i32, coordinate: i32, output_len: i64) -> c_int;
    pub fn axis_select_axis_backward(d: axis_device, g: *const f32, out: *mut f32, metadata: *const i32,
                                     rank: i32, coordinate: i32, input_len: i64) -> c_int;
    pub fn axis_categorical_cross_entropy(d: axis_device, z: *const f32, y: *const f32, out: *mut f32,
                                          rows: i64, width: i64) -> c_int;
    pub fn axis_categorical_cross_entropy_backward(d: axis_device, g: *const f32, p: *const f32,
                                                   y: *const f32, out: *mut f32,
                                                   rows: i64, width: i64) -> c_int;
    pub fn axis_categorical_cross_entropy_backward_mean(d: axis_device, g: *const f32, factor: f32,
                                                        p: *const f32, y: *const f32, out: *mut f32,
                                                        d_bias: *mut f32, rows: i64, width: i64) -> c_int;
    pub fn axis_adam(d: axis_device, value: *const f32, g: *const f32, m: *const f32, v: *const f32,
                     rates: *const f32, len: i64, lr: f32, b1: f32, b2: f32, c1: f32, c2: f32,
                     eps: f32, wd: f32, out_value: *mut f32, out_m: *mut f32, out_v: *mut f32) -> c_int;
    pub fn axis_adam_multi(d: axis_device, t: *const axis_adam_tensor, count: i32, lr: f32, b1: f32,
                           b2: f32, c1: f32, c2: f32, eps: f32, wd: f32) -> c_int;
    pub fn axis_muon_momentum(d: axis_device, g: *const f32, previous: *const f32, next: *mut f32,
                              direction: *mut f32, momentum: f32, nesterov: c_int, len: i64) -> c_int;
    pub fn axis_muon_apply(d: axis_device, value: *const f32, orthogonal: *const f32, out: *mut f32,
                           decay: f32, rate: f32, len: i64) -> c_int;
    pub fn axis_sum_squares(d: axis_device, a: *const f32, len: i64, out: *mut f32) -> c_int;
    pub fn axis_inverse_sqrt(d: axis_device, a: *const f32, eps: f32, out: *mut f32, len: i64) -> c_int;
    pub fn axis_multiply_scalar(d: axis_device, a: *const f32, s: *const f32, out: *mut f32, len: i64) -> c_int;
    // Dedicated entries the tensor layer picks when shapes match (SURVEY 8b "plus new dedicated
    // entries"); each is a composition of the methods above on a specific layout.
    pub fn axis_bias_add(d: axis_device, a: *const f32, bias: *const f32, out: *mut f32,
                         relu_out: *mut f32, rows: i64, width: i64) -> c_int;
    pub fn axis_bias_gradient(d: axis_device, g: *const f32, relu_input: *const f32,
                              masked_out: *mut f32, out: *mut f32, rows: i64, width: i64) -> c_int;
    pub fn axis_max_pool2d(d: axis_device, input: *const f32, out: *mut f32, argmax: *mut u8,
                           outer: i64, height: i32, width: i32, channels: i64,
                           kernel: *const i32, stride: *const i32, padding: *const i32) -> c_int;
    pub fn axis_max_pool2d_backward(d: axis_device, g: *const f32, argmax: *const u8, out: *mut f32,
                                    outer: i64, height: i32, width: i32, channels: i64,
                                    kernel: *const i32, stride: *const i32, padding: *const i32) -> c_int;
    pub fn axis_reduce_middle(d: axis_device, a: *const f32, out: *mut f32, outer: i64, reduce: i64,
                              inner: i64, factor: f32) -> c_int;
    pub fn axis_broadcast_middle(d: axis_device, g: *const f32, out: *mut f32, outer: i64,
                                 reduce: i64, inner: i64, factor: f32) -> c_int;
    pub fn axis_softmax_cross_entropy(d: axis_device, logits: *const f32, targets: *const f32,
                                      probability: *mut f32, loss: *mut f32, rows: i64, width: i64) -> c_int;
    // Implicit-GEMM convolution, one group; input_strides = {batch, channel, row, column} or null
    // for channel-innermost contiguous input.
    pub fn axis_conv2d_forward(d: axis_device, input: *const f32, input_strides: *const i64,
                               weight: *const f32, bias: *const f32, out: *mut f32, batch: i64,
                               height: i32, width: i32, channels: i32, out_channels: i32,
                               kernel: *const i32, stride: *const i32, padding: *const i32) -> c_int;
    pub fn axis_conv2d_relu_pool_forward(d: axis_device, input: *const f32, input_strides: *const i64,
                                         weight: *const f32, bias: *const f32, pooled: *mut f32,
                                         argmax: *mut u8, batch: i64, height: i32, width: i32,
                                         channels: i32, out_channels: i32, kernel: *const i32,
                                         stride: *const i32, padding: *const i32,
                                         pool: *const i32) -> c_int;
    pub fn axis_conv2d_backward_data(d: axis_device, g: *const f32, weight: *const f32,
                                     d_input: *mut f32, batch: i64, height: i32, width: i32,
                                     channels: i32, out_channels: i32, kernel: *const i32,
                                     stride: *const i32, padding: *const i32) -> c_int;
    pub fn axis_conv2d_backward_weight(d: axis_device, input: *const f32, input_strides: *const i64,
                                       g: *const f32, d_weight: *mut f32, batch: i64, height: i32,
                                       width: i32, channels: i32, out_channels: i32,
                                       kernel: *const i32, stride: *const i32,
                                       padding: *const i32) -> c_int;
    pub fn axis_conv2d_relu_pool_backward_weight(d: axis_device, input: *const f32, input_strides: *const i64,
                                                 g: *const f32, pooled: *const f32, argmax: *const u8,
                                                 d_weight: *mut f32, d_bias: *mut f32, batch: i64,
                                                 height: i32, width: i32, channels: i32, out_channels: i32,
                                                 kernel: *const i32, stride: *const i32, padding: *const i32,
                                                 pool: *const i32) -> c_int;
    pub fn axis_relu_pool_backward(d: axis_device, g: *const f32, pooled: *const f32,
                                   argmax: *const u8, d_pre: *mut f32, d_bias: *mut f32, outer: i64,
                                   height: i32, width: i32, channels: i32, pool: *const i32) -> c_int;
    pub fn axis_relu_pool_backward_mean(d: axis_device, g: *const f32, factor: f32, pooled: *const f32,
                                        argmax: *const u8, d_pre: *mut f32, d_bias: *mut f32, outer: i64,
                                        height: i32, width: i32, channels: i32, pool: *const i32) -> c_int;
    // Launch timers (bench): per family "gemm" / "adam", HIP events on the device's stream.
    pub fn axis_timing_enable(d: axis_device, on: c_int) -> c_int;
    pub fn axis_timing_reset(d: axis_device) -> c_int;
    pub fn axis_timing_read(d: axis_device, family: *const c_char, launches: *mut i64,
                            ms: *mut f64, work: *mut f64) -> c_int;
    // Deferred finishing sums (the tape's backward): weight/bias gradients' last sums in one launch.
    pub fn axis_finish_defer(d: axis_device, on: c_int) -> c_int;
    pub fn axis_finish_flush(d: axis_device) -> c_int;
    pub fn axis_finish_before_read(d: axis_device, ptr: *const c_void, bytes: usize) -> c_int;
    pub fn axis_finish_pending(d: axis_device, tasks: *mut i64) -> c_int;
}
