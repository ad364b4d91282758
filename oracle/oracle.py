"""CPU restatement of furkanhaney/axis's training hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
module, and only as the checker: the product (``axis_amd``) never imports, links or runs it.

Layers:
  * ctypes bindings to ``libaxis_oracle.so`` (oracle/axis_oracle.c), the per-kernel arithmetic;
  * host-side geometry the reference computes before a launch -- ``unfold_spec``
    (algebra/tensor.rs:3751-3946), CSR ``Plan`` builders (runtime/backend.rs:1542-1597),
    ``reduction_plans`` (tensor.rs:2755-2804), ``min`` plans (tensor.rs:2880-2946) and the
    ``align`` reverse plan (tensor.rs:679-698);
  * model-level steps (``mlp_step``, ``cnn_step``, ``muon_step``) that replay the exact
    Device-call sequence the reference's forward records and ``Tensor::backward``
    (tensor.rs:5551-5738) replays, followed by the optimizer update.

Axes are plain strings here; a shape is a list of ``(axis, extent)`` and a layout is the
per-logical-axis stride list, as ``axis::Layout`` (algebra/axis.rs:152-176).
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libaxis_oracle.so")
_lib = None

F32P = ctypes.POINTER(ctypes.c_float)
I32P = ctypes.POINTER(ctypes.c_int32)


class UnfoldSpec(ctypes.Structure):
    """Field-for-field the reference's UnfoldSpec (runtime/backend.rs:1481-1501)."""

    _fields_ = [
        ("spatial_rank", ctypes.c_int32),
        ("input_len", ctypes.c_int64),
        ("output_len", ctypes.c_int64),
        ("input_rank", ctypes.c_int32),
        ("output_rank", ctypes.c_int32),
        ("forward_metadata", ctypes.c_int32 * 32),
        ("backward_metadata", ctypes.c_int32 * 32),
        ("channels_per_group", ctypes.c_int32),
        ("fill", ctypes.c_float),
        ("kernel", ctypes.c_int32 * 3),
        ("stride", ctypes.c_int32 * 3),
        ("padding", ctypes.c_int32 * 3),
        ("input_spatial", ctypes.c_int32 * 3),
        ("output_spatial", ctypes.c_int32 * 3),
        ("input_special_strides", ctypes.c_int32 * 4),
        ("output_special_strides", ctypes.c_int32 * 5),
    ]


def build() -> None:
    """Compile oracle/axis_oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _f(a):
    return a.ctypes.data_as(F32P)


def _i(a):
    return a.ctypes.data_as(I32P)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def threads() -> int:
    return int(lib().axo_threads())


def set_threads(n: int) -> None:
    lib().axo_set_threads(ctypes.c_int(n))


# ------------------------------------------------------------------ RNG (tensor.rs:29-71)

def xorshift_unit_stream(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().axo_xorshift_unit_stream(ctypes.c_uint64(seed), ctypes.c_int64(count), _f(out))
    return out


def uniform(seed: int, count: int, low: float = 0.0, high: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().axo_uniform_host_values(ctypes.c_uint64(seed), ctypes.c_int64(count),
                                  ctypes.c_float(low), ctypes.c_float(high), _f(out))
    return out


def normal(seed: int, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().axo_normal_host_values(ctypes.c_uint64(seed), ctypes.c_int64(count),
                                 ctypes.c_float(mean), ctypes.c_float(std), _f(out))
    return out


def powi(base: float, exponent: int) -> float:
    f = lib().axo_powi
    f.restype = ctypes.c_float
    return float(f(ctypes.c_float(base), ctypes.c_int32(exponent)))


def he_std(fan_in: int) -> float:
    """He-normal standard deviation sqrt(2 / fan_in), evaluated in fp32."""
    return float(np.sqrt(np.float32(2.0) / np.float32(fan_in), dtype=np.float32))


def one_hot_labels(seed: int, rows: int, classes: int) -> tuple[np.ndarray, np.ndarray]:
    """Labels l_i = min(floor(u_i * classes), classes - 1) from the xorshift stream, one-hot."""
    u = xorshift_unit_stream(seed, rows)
    labels = np.minimum(np.floor(u.astype(np.float64) * classes).astype(np.int64), classes - 1)
    y = np.zeros((rows, classes), np.float32)
    y[np.arange(rows), labels] = 1.0
    return labels, y


# ------------------------------------------------------------------ contractions

def bf16_round(a):
    """fp32 -> bf16 (nearest, ties to even) -> fp32: the operand conversion of the reference's bf16
    matrix products (backend.rs:2209-2312)."""
    a = _f32(a)
    out = np.empty_like(a)
    lib().axo_bf16_round(_f(a), ctypes.c_int64(a.size), _f(out))
    return out


def matmul(a, b, batch, m, k, n):
    a, b = _f32(a), _f32(b)
    out = np.empty(batch * m * n, np.float32)
    lib().axo_matmul(_f(a), _f(b), ctypes.c_int64(batch), ctypes.c_int64(m), ctypes.c_int64(k),
                     ctypes.c_int64(n), _f(out))
    return out


def matmul_left_backward(gradient, rhs, batch, m, k, n):
    g, r = _f32(gradient), _f32(rhs)
    out = np.empty(batch * m * k, np.float32)
    lib().axo_matmul_left_backward(_f(g), _f(r), ctypes.c_int64(batch), ctypes.c_int64(m),
                                   ctypes.c_int64(k), ctypes.c_int64(n), _f(out))
    return out


def matmul_right_backward(lhs, gradient, batch, m, k, n):
    l, g = _f32(lhs), _f32(gradient)
    out = np.empty(batch * k * n, np.float32)
    lib().axo_matmul_right_backward(_f(l), _f(g), ctypes.c_int64(batch), ctypes.c_int64(m),
                                    ctypes.c_int64(k), ctypes.c_int64(n), _f(out))
    return out


# ------------------------------------------------------------------ shapes and layouts

def contiguous(dims):
    """Layout::contiguous (axis.rs:152-171): strides of the logical order, last axis fastest."""
    strides = [0] * len(dims)
    s = 1
    for i in range(len(dims) - 1, -1, -1):
        strides[i] = s
        s *= dims[i][1]
    return strides


def layout_for(dims, order):
    """Layout::new (axis.rs:156-168): strides when stored in `order` (outermost first)."""
    names = [a for a, _ in dims]
    strides = [0] * len(dims)
    s = 1
    for axis in reversed(order):
        i = names.index(axis)
        strides[i] = s
        s *= dims[i][1]
    return strides


def shape_len(dims):
    n = 1
    for _, e in dims:
        n *= e
    return n


def coords(dims, flat):
    out = [0] * len(dims)
    for i in range(len(dims) - 1, -1, -1):
        out[i] = flat % dims[i][1]
        flat //= dims[i][1]
    return out


def to_logical(values, dims, strides):
    """Tensor::to_vec (tensor.rs:423-452): values in logical order from physical storage."""
    n = shape_len(dims)
    idx = np.zeros(n, np.int64)
    grid = np.indices([e for _, e in dims]).reshape(len(dims), -1) if dims else np.zeros((0, 1), np.int64)
    for d, s in enumerate(strides):
        idx += grid[d] * s
    return np.asarray(values)[idx]


# ------------------------------------------------------------------ unfold (tensor.rs:3654-3946)

@dataclass
class Unfold:
    shape: list
    strides: list
    spec: UnfoldSpec | None  # None: the reference's UnfoldPlans::Zero (no window touches input)


def unfold_spec(image_dims, image_strides, channels, spatial, group, patch, kernel, stride,
                padding, fill):
    """Restates unfold_shape + unfold_spec (tensor.rs:3654-3946) for two spatial axes.

    `group` is ``(axis, extent)`` or None; `patch` is ``(axis, extent)``.  Returns the patch
    tensor's logical shape, its physical strides (order: group, other axes, patch) and the
    packed spec."""
    names = [a for a, _ in image_dims]
    ext = dict(image_dims)
    n = 2
    channel_extent = ext[channels]
    input_spatial = [ext[spatial[i]] for i in range(n)]
    groups = group[1] if group else 1
    if channel_extent % groups:
        raise ValueError("channels must be divisible by groups")
    output_spatial = []
    for i in range(n):
        padded = input_spatial[i] + 2 * padding[i]
        if kernel[i] > padded:
            raise ValueError("kernel exceeds the padded spatial extent")
        output_spatial.append((padded - kernel[i]) // stride[i] + 1)
    cpg = channel_extent // groups
    expected_patch = cpg * kernel[0] * kernel[1]
    if patch[1] != expected_patch:
        raise ValueError("patch extent must equal channels per group * kernel volume")
    dims = []
    for a, e in image_dims:
        if a == channels:
            if group is None:
                dims.append((patch[0], expected_patch))
        elif a in spatial:
            dims.append((a, output_spatial[spatial.index(a)]))
        else:
            dims.append((a, e))
    if group is not None:
        dims += [group, (patch[0], expected_patch)]
    order = ([group[0]] if group else []) + [
        a for a, _ in dims if (group is None or a != group[0]) and a != patch[0]] + [patch[0]]
    out_strides = layout_for(dims, order)
    has_input = all(
        any(any(0 <= o * stride[d] + off - padding[d] < input_spatial[d]
                for off in range(kernel[d])) for o in range(output_spatial[d]))
        for d in range(n))
    if not has_input:
        return Unfold(dims, out_strides, None)
    s = UnfoldSpec()
    s.spatial_rank = 2
    s.input_len = shape_len(image_dims)
    s.output_len = shape_len(dims)
    s.input_rank = len(image_dims)
    s.output_rank = len(dims)
    for index, (a, e) in enumerate(dims):
        if a in spatial:
            istride, role = 0, spatial.index(a) + 1
        elif group is not None and a == group[0]:
            istride, role = 0, n + 1
        elif a == patch[0]:
            istride, role = 0, n + 2
        else:
            istride, role = image_strides[names.index(a)], 0
        s.forward_metadata[4 * index:4 * index + 4] = [e, out_strides[index], istride, role]
    out_names = [a for a, _ in dims]
    for index, (a, e) in enumerate(image_dims):
        if a == channels:
            ostride, role = 0, 1
        elif a in spatial:
            ostride, role = 0, spatial.index(a) + 2
        else:
            ostride, role = out_strides[out_names.index(a)], 0
        s.backward_metadata[4 * index:4 * index + 4] = [e, image_strides[index], ostride, role]
    s.channels_per_group = cpg
    s.fill = fill
    s.kernel[:] = [kernel[0], kernel[1], 1]
    s.stride[:] = [stride[0], stride[1], 1]
    s.padding[:] = [padding[0], padding[1], 0]
    s.input_spatial[:] = [input_spatial[0], input_spatial[1], 1]
    s.output_spatial[:] = [output_spatial[0], output_spatial[1], 1]
    s.input_special_strides[:] = [image_strides[names.index(channels)],
                                  image_strides[names.index(spatial[0])],
                                  image_strides[names.index(spatial[1])], 0]
    s.output_special_strides[:] = [out_strides[out_names.index(spatial[0])],
                                   out_strides[out_names.index(spatial[1])], 0,
                                   out_strides[out_names.index(group[0])] if group else 0,
                                   out_strides[out_names.index(patch[0])]]
    return Unfold(dims, out_strides, s)


def unfold2d(x, u: Unfold):
    out = np.empty(shape_len(u.shape), np.float32)
    if u.spec is None:
        out[:] = 0.0
        return out
    x = _f32(x)
    lib().axo_unfold2d(_f(x), ctypes.byref(u.spec), _f(out))
    return out


def unfold2d_backward(g, u: Unfold, input_len):
    out = np.empty(input_len, np.float32)
    if u.spec is None:
        out[:] = 0.0
        return out
    g = _f32(g)
    lib().axo_unfold2d_backward(_f(g), ctypes.byref(u.spec), _f(out))
    return out


# ------------------------------------------------------------------ CSR plans (backend.rs:1542-1597)

PLAN_CAP = 16_777_216


@dataclass
class Plan:
    offsets: np.ndarray
    left: np.ndarray
    right: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))


def plan_groups(groups, product=False, cap=True):
    count = sum(len(g) for g in groups)
    if cap and (count == 0 or count > PLAN_CAP):
        raise ValueError("index plan must have 1..=16777216 contributions")
    offsets = [0]
    left, right = [], []
    for g in groups:
        for a, b in g:
            left.append(a)
            if product:
                right.append(b)
        offsets.append(len(left))
    return Plan(_i32(offsets), _i32(left), _i32(right))


def plan_gather(mapping, cap=True):
    mapping = np.asarray(mapping, np.int64)
    if cap and (len(mapping) == 0 or len(mapping) > PLAN_CAP):
        raise ValueError("index plan must have 1..=16777216 contributions")
    return Plan(_i32(np.arange(len(mapping) + 1)), _i32(mapping))


def plan_reverse(mapping, length, cap=True):
    """Plan::reverse (backend.rs:1577-1583): group g lists, in increasing position order, every
    position whose mapping is g."""
    mapping = np.asarray(mapping, np.int64)
    if cap and (len(mapping) == 0 or len(mapping) > PLAN_CAP):
        raise ValueError("index plan must have 1..=16777216 contributions")
    order = np.argsort(mapping, kind="stable")
    counts = np.bincount(mapping, minlength=length)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    return Plan(_i32(offsets), _i32(order))


def reduction_plans(dims, strides, axes, mean: bool, cap=True):
    """tensor.rs:2755-2804: (output dims, forward plan, reverse plan, factor)."""
    out_dims = [(a, e) for a, e in dims if a not in axes]
    out_strides = contiguous(out_dims)
    n = shape_len(dims)
    grid = np.indices([e for _, e in dims]).reshape(len(dims), -1)
    physical = np.zeros(n, np.int64)
    for d, s in enumerate(strides):
        physical += grid[d] * s
    retained = np.zeros(n, np.int64)
    k = 0
    for d, (a, _) in enumerate(dims):
        if a not in axes:
            retained += grid[d] * out_strides[k]
            k += 1
    mapping = np.zeros(n, np.int64)
    mapping[physical] = retained
    olen = shape_len(out_dims)
    factor = np.float32(olen) / np.float32(n) if mean else np.float32(1.0)
    return out_dims, plan_reverse(mapping, olen, cap), plan_gather(mapping, cap), float(factor)


def min_plans(dims, strides, axis, cap=True):
    """tensor.rs:2880-2929: forward groups in output order, members in coordinate order."""
    red = [a for a, _ in dims].index(axis)
    extent = dims[red][1]
    out_dims = [(a, e) for a, e in dims if a != axis]
    olen = shape_len(out_dims)
    # a rank-0 result (the only axis reduced) is one group
    grid = (np.indices([e for _, e in out_dims]).reshape(len(out_dims), -1) if out_dims
            else np.zeros((0, 1), np.int64))
    base = np.zeros(olen, np.int64)
    k = 0
    for d in range(len(dims)):
        if d == red:
            continue
        base += grid[k] * strides[d]
        k += 1
    members = base[:, None] + np.arange(extent)[None, :] * strides[red]  # [olen, extent]
    mapping = np.zeros(shape_len(dims), np.int64)
    mapping[members.reshape(-1)] = np.repeat(np.arange(olen), extent)
    if cap and (members.size == 0 or members.size > PLAN_CAP):
        raise ValueError("index plan must have 1..=16777216 contributions")
    forward = Plan(_i32(np.arange(olen + 1) * extent), _i32(members.reshape(-1)))
    return out_dims, forward, plan_gather(mapping, cap)


def align_reverse_plan(small_dims, small_strides, target_dims, cap=True):
    """tensor.rs:679-698: for every target position, the small tensor's physical offset it reads;
    the reverse plan groups those target positions per small offset."""
    tnames = [a for a, _ in target_dims]
    positions = [tnames.index(a) for a, _ in small_dims]
    n = shape_len(target_dims)
    grid = np.indices([e for _, e in target_dims]).reshape(len(target_dims), -1)
    mapping = np.zeros(n, np.int64)
    for own, p in enumerate(positions):
        mapping += grid[p] * small_strides[own]
    return plan_reverse(mapping, shape_len(small_dims), cap)


def grouped(a, b, plan: Plan, scale):
    a = _f32(a)
    groups = len(plan.offsets) - 1
    out = np.empty(groups, np.float32)
    bb = _f32(b) if b is not None else None
    lib().axo_grouped(_f(a), _f(bb) if bb is not None else None, _i(plan.offsets), _i(plan.left),
                      _i(plan.right) if len(plan.right) else None, ctypes.c_int64(groups),
                      ctypes.c_float(scale), _f(out))
    return out


def grouped_minimum(a, forward: Plan, reverse: Plan, maximum=False):
    a = _f32(a)
    groups = len(forward.offsets) - 1
    out = np.empty(groups, np.float32)
    winners = np.empty(groups, np.int32)
    fn = lib().axo_grouped_maximum if maximum else lib().axo_grouped_minimum
    fn(_f(a), _i(forward.offsets), _i(forward.left), ctypes.c_int64(groups), _f(out), _i(winners))
    mask = np.empty(len(a), np.float32)
    lib().axo_reduction_winner_mask(_i(winners), _i(reverse.left), ctypes.c_int64(len(a)), _f(mask))
    return out, mask, winners


# ------------------------------------------------------------------ elementwise

def _unary(name, a, *extra):
    a = _f32(a)
    out = np.empty_like(a)
    getattr(lib(), name)(_f(a), ctypes.c_int64(a.size), *extra, _f(out))
    return out


def relu(a):
    return _unary("axo_relu", a)


def scale(a, factor):
    return _unary("axo_scale", a, ctypes.c_float(factor))


def inverse_sqrt(a, eps):
    return _unary("axo_inverse_sqrt", a, ctypes.c_float(eps))


def relu_backward(g, a):
    g, a = _f32(g), _f32(a)
    out = np.empty_like(a)
    lib().axo_relu_backward(_f(g), _f(a), ctypes.c_int64(a.size), _f(out))
    return out


def mask_gradient(g, winners):
    g, w = _f32(g), _f32(winners)
    out = np.empty_like(g)
    lib().axo_mask_gradient(_f(g), _f(w), ctypes.c_int64(g.size), _f(out))
    return out


def binary(a, b, op):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().axo_binary(_f(a), _f(b), ctypes.c_int64(a.size), ctypes.c_int32(op), _f(out))
    return out


def select_axis(x, metadata, rank, coordinate, output_len):
    x, md = _f32(x), _i32(metadata)
    out = np.empty(output_len, np.float32)
    lib().axo_select_axis(_f(x), _i(md), ctypes.c_int32(rank), ctypes.c_int32(coordinate),
                          ctypes.c_int64(output_len), _f(out))
    return out


def select_axis_backward(g, metadata, rank, coordinate, input_len):
    g, md = _f32(g), _i32(metadata)
    out = np.empty(input_len, np.float32)
    lib().axo_select_axis_backward(_f(g), _i(md), ctypes.c_int32(rank), ctypes.c_int32(coordinate),
                                   ctypes.c_int64(input_len), _f(out))
    return out


def broadcast_metadata(small_dims, small_strides, target_dims):
    """The select_axis metadata Tensor::align builds for a broadcast (tensor.rs:731-750)."""
    names = [a for a, _ in small_dims]
    out_strides = contiguous(target_dims)
    md = []
    for index, (a, e) in enumerate(target_dims):
        istride = small_strides[names.index(a)] if a in names else 0
        md += [e, istride, out_strides[index]]
    return md


# ------------------------------------------------------------------ softmax / cross-entropy

def softmax(a, rows, width):
    a = _f32(a)
    out = np.empty_like(a)
    lib().axo_softmax(_f(a), ctypes.c_int64(rows), ctypes.c_int64(width), _f(out))
    return out


def softmax_backward(g, p, rows, width):
    g, p = _f32(g), _f32(p)
    out = np.empty_like(p)
    lib().axo_softmax_backward(_f(g), _f(p), ctypes.c_int64(rows), ctypes.c_int64(width), _f(out))
    return out


def categorical_cross_entropy(logits, targets, rows, width):
    z, y = _f32(logits), _f32(targets)
    out = np.empty(rows, np.float32)
    lib().axo_categorical_cross_entropy(_f(z), _f(y), ctypes.c_int64(rows), ctypes.c_int64(width),
                                        _f(out))
    return out


def categorical_cross_entropy_backward(g, p, y, rows, width):
    g, p, y = _f32(g), _f32(p), _f32(y)
    out = np.empty(rows * width, np.float32)
    lib().axo_categorical_cross_entropy_backward(_f(g), _f(p), _f(y), ctypes.c_int64(rows),
                                                 ctypes.c_int64(width), _f(out))
    return out


def check_targets(y, width):
    """tensor.rs:1520-1536: every target row finite, nonnegative and summing to 1 within 1e-5."""
    for row, dist in enumerate(np.asarray(y, np.float32).reshape(-1, width)):
        if not np.all(np.isfinite(dist)) or np.any(dist < 0):
            raise ValueError(f"categorical target row {row} must contain finite nonnegative probabilities")
        s = np.float32(0.0)
        for v in dist:
            s = np.float32(s + v)
        if abs(float(s) - 1.0) > 1e-5:
            raise ValueError(f"categorical target row {row} must sum to 1; observed {s}")


# ------------------------------------------------------------------ Adam (backend.rs:1023-1075)

def adam(value, grad, first, second, lr, b1, b2, c1, c2, eps, wd, learning_rates=None):
    p, g, m, v = _f32(value), _f32(grad), _f32(first), _f32(second)
    out_p, out_m, out_v = np.empty_like(p), np.empty_like(p), np.empty_like(p)
    lrs = _f(_f32(learning_rates)) if learning_rates is not None else None
    lib().axo_adam(_f(p), _f(g), _f(m), _f(v), ctypes.c_int64(p.size), ctypes.c_float(lr), lrs,
                   ctypes.c_float(b1), ctypes.c_float(b2), ctypes.c_float(c1), ctypes.c_float(c2),
                   ctypes.c_float(eps), ctypes.c_float(wd), _f(out_p), _f(out_m), _f(out_v))
    return out_p, out_m, out_v


class AdamOracle:
    """Adam::prepare/commit (model/optim.rs:102-157): bias corrections in fp32 powi, zero moments
    on a parameter's first step, one state pair per parameter."""

    def __init__(self, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0):
        self.lr, self.b1, self.b2, self.eps, self.wd = lr, b1, b2, eps, wd
        self.step_count = 0
        self.states = {}

    def step(self, params: dict, grads: dict):
        t = self.step_count + 1
        c1 = np.float32(1.0) - np.float32(powi(self.b1, t))
        c2 = np.float32(1.0) - np.float32(powi(self.b2, t))
        out = {}
        for name, p in params.items():
            m, v = self.states.get(name, (np.zeros_like(p), np.zeros_like(p)))
            np_, nm, nv = adam(p, grads[name], m, v, self.lr, self.b1, self.b2, float(c1),
                               float(c2), self.eps, self.wd)
            out[name] = np_
            self.states[name] = (nm, nv)
        self.step_count = t
        return out


# ------------------------------------------------------------------ Muon (model/optim.rs:610-752)

NS_A, NS_B, NS_C = np.float32(3.4445), np.float32(-4.7750), np.float32(2.0315)


def sum_squares(a):
    a = _f32(a)
    out = np.empty(1, np.float32)
    lib().axo_sum_squares(_f(a), ctypes.c_int64(a.size), _f(out))
    return out


def multiply_scalar(a, scalar):
    a, s = _f32(a), _f32(scalar)
    out = np.empty_like(a)
    lib().axo_multiply_scalar(_f(a), ctypes.c_int64(a.size), _f(s), _f(out))
    return out


def normalized_l2(x, epsilon):
    """tensor.rs:2100-2134: x * (1/sqrt(1/sqrt(s+m)*s + eps + m))^2 with s = sum of squares and
    m = f32::MIN_POSITIVE, each step a separate fp32 device op."""
    tiny = float(np.finfo(np.float32).tiny)
    s = sum_squares(x)
    inv_root = inverse_sqrt(s, tiny)
    norm = binary(s, inv_root, 2)
    denom = binary(norm, np.array([epsilon], np.float32), 0)
    inv_half = inverse_sqrt(denom, tiny)
    inv = binary(inv_half, inv_half, 2)
    return multiply_scalar(x, inv)


def zeroth_power(d, rows, cols, bf16=False):
    """optim.rs:728-752 on a row-major [rows, cols] matrix: X = d/||d||; five times
    A = X X^T (small side), B = b*A + c*A*A, X = a*X + B*X (transposed when cols < rows).
    bf16: every product takes bf16-rounded operands (Device::cuda_bf16, backend.rs:274-283); the
    scale-and-add terms stay fp32."""
    r = bf16_round if bf16 else (lambda v: v)
    x = normalized_l2(d, 1e-7).reshape(rows, cols)
    transposed = rows > cols
    if transposed:
        x = np.ascontiguousarray(x.T)
    s, l = x.shape
    for _ in range(5):
        gram = matmul(r(x), r(np.ascontiguousarray(x.T)), 1, s, l, s).reshape(s, s)
        gram2 = matmul(r(gram), r(gram), 1, s, s, s).reshape(s, s)
        b = binary(scale(gram, float(NS_B)), scale(gram2, float(NS_C)), 0).reshape(s, s)
        bx = matmul(r(b), r(x), 1, s, s, l).reshape(s, l)
        x = binary(scale(x, float(NS_A)), bx, 0).reshape(s, l)
    if transposed:
        x = np.ascontiguousarray(x.T)
    return x.reshape(-1)


class MuonOracle:
    """Muon::prepare/commit (optim.rs:610-678): EMA momentum, Nesterov direction, zeroth power,
    scaled decoupled update.  `fan` maps a parameter to (fan_in, fan_out)."""

    def __init__(self, lr, momentum=0.95, nesterov=True, wd=0.0, bf16=False):
        self.lr, self.mu, self.nesterov, self.wd, self.bf16 = lr, momentum, nesterov, wd, bf16
        self.states = {}
        self.step_count = 0

    def step(self, params: dict, grads: dict, shapes: dict, fans: dict):
        out = {}
        w = np.float32(1.0) - np.float32(self.mu)
        for name, p in params.items():
            g = _f32(grads[name])
            prev = self.states.get(name)
            gw = scale(g, float(w))
            m = gw if prev is None else binary(scale(prev, self.mu), gw, 0)
            d = binary(scale(g, float(w)), scale(m, self.mu), 0) if self.nesterov else m
            rows, cols = shapes[name]
            x = zeroth_power(d, rows, cols, self.bf16)
            fan_in, fan_out = fans[name]
            scaling = np.sqrt(max(np.float32(fan_out) / np.float32(fan_in), np.float32(1.0)),
                              dtype=np.float32)
            decayed = scale(p, float(np.float32(1.0) - np.float32(self.lr) * np.float32(self.wd)))
            out[name] = binary(decayed, scale(x, float(np.float32(self.lr) * scaling)), 1)
            self.states[name] = m
        self.step_count += 1
        return out


# ------------------------------------------------------------------ model-level steps

def linear_forward(x, w, b, rows, fan_in, fan_out):
    """nn.rs:268-282: rename + contract (one GEMM) + add(bias) (align broadcast, binary add)."""
    z = matmul(x, w, 1, rows, fan_in, fan_out)
    bias = select_axis(b, broadcast_metadata([("o", fan_out)], [1], [("r", rows), ("o", fan_out)]),
                       2, 0, rows * fan_out)
    return binary(z, bias, 0)


def bias_gradient(g, rows, width, cap=False):
    """The Group rule of the bias's align edge: reverse plan over [rows, width] (tensor.rs:679-698)."""
    plan = align_reverse_plan([("o", width)], [1], [("r", rows), ("o", width)], cap=cap)
    return grouped(g, None, plan, 1.0)


def mean_rows_backward(rows):
    """Backward of loss.mean(batch) from the seed 1.0: the Group rule's gather plan, factor
    out/in (tensor.rs:2808-2845, 5585)."""
    _, _, reverse, factor = reduction_plans([("batch", rows)], [1], ["batch"], mean=True, cap=False)
    return grouped(np.ones(1, np.float32), None, reverse, factor)


def ce_loss(logits, y, rows, width):
    """categorical_cross_entropy_with_logits + mean(batch) forward (tensor.rs:1485-1557)."""
    check_targets(y, width)
    p = softmax(logits, rows, width)
    per_row = categorical_cross_entropy(logits, y, rows, width)
    _, forward, _, factor = reduction_plans([("batch", rows)], [1], ["batch"], mean=True, cap=False)
    loss = grouped(per_row, None, forward, factor)[0]
    return p, per_row, float(loss)


def mlp_inputs(batch=128, sizes=(784, 256, 256, 10), x_seed=1, label_seed=2, weight_seed=10):
    x = uniform(x_seed, batch * sizes[0])
    _, y = one_hot_labels(label_seed, batch, sizes[-1])
    params = {}
    for j in range(len(sizes) - 1):
        fi, fo = sizes[j], sizes[j + 1]
        params[f"w{j}"] = normal(weight_seed + j, fi * fo, 0.0, he_std(fi))
        params[f"b{j}"] = np.zeros(fo, np.float32)
    return x, y.reshape(-1), params


def mlp_forward_backward(x, y, params, batch, sizes, bf16=False):
    """ReLU MLP forward, mean categorical cross-entropy, and the tape's reverse sweep.  bf16: the
    matrix products take bf16-rounded operands (Device::cuda_bf16, backend.rs:274-283)."""
    r = bf16_round if bf16 else (lambda v: v)
    acts, pre = [x], []
    h = x
    layers = len(sizes) - 1
    for j in range(layers):
        z = linear_forward(r(h), r(params[f"w{j}"]), params[f"b{j}"], batch, sizes[j], sizes[j + 1])
        pre.append(z)
        h = relu(z) if j < layers - 1 else z
        acts.append(h)
    p, per_row, loss = ce_loss(h, y, batch, sizes[-1])
    g_rows = mean_rows_backward(batch)
    g = categorical_cross_entropy_backward(g_rows, p, y, batch, sizes[-1])
    grads = {}
    for j in reversed(range(layers)):
        if j < layers - 1:
            g = relu_backward(g, pre[j])
        grads[f"b{j}"] = bias_gradient(g, batch, sizes[j + 1])
        grads[f"w{j}"] = matmul_right_backward(r(acts[j]), r(g), 1, batch, sizes[j], sizes[j + 1])
        if j > 0:
            g = matmul_left_backward(r(g), r(params[f"w{j}"]), 1, batch, sizes[j], sizes[j + 1])
    return loss, grads


def mlp_step(batch=128, sizes=(784, 256, 256, 10), lr=1e-3, bf16=False):
    """one forward + backward + Adam step; returns loss, grads, new params."""
    x, y, params = mlp_inputs(batch, sizes)
    loss, grads = mlp_forward_backward(x, y, params, batch, sizes, bf16)
    new = AdamOracle(lr).step(params, grads)
    return {"loss": loss, "grads": grads, "params": new, "initial": params, "x": x, "y": y}


# --- 3-block CNN ---

CNN_CHANNELS = (3, 64, 128, 256)


def cnn_inputs(batch=256, size=64, classes=1000, channels=CNN_CHANNELS, x_seed=1, label_seed=2,
               weight_seed=10):
    x = uniform(x_seed, batch * channels[0] * size * size)
    _, y = one_hot_labels(label_seed, batch, classes)
    params = {}
    for j in range(3):
        fan_in = channels[j] * 9
        params[f"conv{j}.weight"] = normal(weight_seed + j, fan_in * channels[j + 1], 0.0, he_std(fan_in))
        params[f"conv{j}.bias"] = np.zeros(channels[j + 1], np.float32)
    params["linear.weight"] = normal(weight_seed + 3, channels[3] * classes, 0.0, he_std(channels[3]))
    params["linear.bias"] = np.zeros(classes, np.float32)
    return x, y.reshape(-1), params


def _decision_masks(argmax, pooled, batch, hh, ww, cout):
    """The pool's winner mask in the unfolded window layout [channel, batch, oh, ow, pool] and a
    ReLU sign array in the activation layout [batch, h, w, channel] from one forward's decisions:
    `argmax` [batch, oh, ow, channel] window-local winners (ky*2 + kx) and `pooled` its pooled
    values (the winner's ReLU is positive exactly when the pooled value is)."""
    am = np.asarray(argmax, np.uint8).reshape(batch, hh // 2, ww // 2, cout)
    pos = np.asarray(pooled, np.float32).reshape(am.shape) > 0
    mask = (am.transpose(3, 0, 1, 2)[..., None] == np.arange(4, dtype=np.uint8)).astype(np.float32)
    sign = np.zeros((batch, hh // 2, 2, ww // 2, 2, cout), np.float32)
    for p in range(4):
        sign[:, :, p // 2, :, p % 2, :] = (am == p) & pos
    return mask.reshape(-1), sign.reshape(-1)


def cnn_forward_backward(x, y, params, batch=256, size=64, classes=1000, channels=CNN_CHANNELS,
                         decisions=None, return_decisions=False):
    """convolution.rs:211-235 (Conv2d) + ReLU + convolution.rs:1334-1370 (MaxPool2d as
    -min(-unfold(x, -inf))) per block, mean over [H, W], Linear, mean categorical
    cross-entropy; then the reverse sweep of tensor.rs:5591-5718 rule by rule.

    `decisions` (optional, one ``(argmax, pooled)`` pair per block, laid out [batch, oh, ow,
    channel]) replaces the backward's discrete choices -- each pool window's winner and the ReLU
    sign at it -- with those of another fp32 forward of the same step.  Two fp32 forwards that
    accumulate in different orders can break a near-tie (two window values, or a pre-activation
    and zero, within rounding) differently, which moves a whole gradient term; replaying one set
    of decisions leaves the arithmetic as the only difference.  `return_decisions` also returns
    this forward's own decisions in that form (argmax 255 where a window has no finite value),
    each pair extended by how clearly it was decided: the window's best ReLU output minus its
    runner-up, and its best pre-activation."""
    dims = [("batch", batch), ("channel", channels[0]), ("height", size), ("width", size)]
    strides = contiguous(dims)
    h = x
    saved, made = [], []
    for j in range(3):
        cin, cout = channels[j], channels[j + 1]
        conv = unfold_spec(dims, strides, "channel" if j == 0 else f"c{j}", ["height", "width"],
                           ("group", 1), ("patch", cin * 9), [3, 3], [1, 1], [1, 1], 0.0)
        patches = unfold2d(h, conv)
        hh = [e for a, e in dims if a == "height"][0]
        ww = [e for a, e in dims if a == "width"][0]
        m = batch * hh * ww
        z = matmul(patches, params[f"conv{j}.weight"], 1, m, cin * 9, cout)
        bias = select_axis(params[f"conv{j}.bias"],
                           broadcast_metadata([("o", cout)], [1], [("r", m), ("o", cout)]),
                           2, 0, m * cout)
        zb = binary(z, bias, 0)
        a = relu(zb)
        adims = [("batch", batch), ("height", hh), ("width", ww), (f"c{j + 1}", cout)]
        astrides = contiguous(adims)
        pool = unfold_spec(adims, astrides, f"c{j + 1}", ["height", "width"], (f"c{j + 1}", cout),
                           ("pool", 4), [2, 2], [2, 2], [0, 0], float("-inf"))
        q = unfold2d(a, pool)
        qn = scale(q, -1.0)
        out_dims, forward, reverse = min_plans(pool.shape, pool.strides, "pool", cap=False)
        mn, mask, _ = grouped_minimum(qn, forward, reverse)
        h = scale(mn, -1.0)
        relu_sign = zb
        if return_decisions:
            won = mask.reshape(cout, batch, hh // 2, ww // 2, 4)
            own = np.where(won.any(-1), won.argmax(-1), 255).astype(np.uint8).transpose(1, 2, 3, 0)
            # how clearly each window was decided: its best ReLU output minus the runner-up, and
            # its best pre-activation (the ReLU sign at the winner), both [batch, oh, ow, channel]
            windows = np.sort(q.reshape(cout, batch, hh // 2, ww // 2, 4), axis=-1)
            gap = (windows[..., 3] - windows[..., 2]).transpose(1, 2, 3, 0)
            zmax = zb.reshape(batch, hh // 2, 2, ww // 2, 2, cout).max(axis=(2, 4))
            made.append((np.ascontiguousarray(own), h.reshape(own.shape).copy(), np.ascontiguousarray(gap), zmax))
        if decisions is not None:
            mask, relu_sign = _decision_masks(decisions[j][0], decisions[j][1], batch, hh, ww, cout)
        saved.append(dict(conv=conv, patches=patches, zb=relu_sign, m=m, pool=pool, mask=mask,
                          reverse=reverse, in_len=shape_len(dims), a_len=len(a)))
        dims, strides = out_dims, contiguous(out_dims)
    # global average pool: mean over [height, width] of [batch, 8, 8, 256]
    c = channels[3]
    out_dims, gap_fwd, gap_rev, gap_factor = reduction_plans(dims, strides, ["height", "width"],
                                                             mean=True, cap=False)
    pooled = grouped(h, None, gap_fwd, gap_factor)
    logits = linear_forward(pooled, params["linear.weight"], params["linear.bias"], batch, c, classes)
    p, per_row, loss = ce_loss(logits, y, batch, classes)
    # ---- reverse sweep
    grads = {}
    g = categorical_cross_entropy_backward(mean_rows_backward(batch), p, y, batch, classes)
    grads["linear.bias"] = bias_gradient(g, batch, classes)
    grads["linear.weight"] = matmul_right_backward(pooled, g, 1, batch, c, classes)
    g = matmul_left_backward(g, params["linear.weight"], 1, batch, c, classes)
    g = grouped(g, None, gap_rev, gap_factor)
    for j in reversed(range(3)):
        s = saved[j]
        cin, cout = channels[j], channels[j + 1]
        g = scale(g, -1.0)                                   # Rule::Scale(-1) of -min
        expanded = grouped(g, None, s["reverse"], 1.0)       # Rule::Minimum: gather ...
        g = mask_gradient(expanded, s["mask"])               # ... then mask
        g = scale(g, -1.0)                                   # Rule::Scale(-1) of -patches
        g = unfold2d_backward(g, s["pool"], s["a_len"])      # Rule::Unfold (pool window col2im)
        g = relu_backward(g, s["zb"])                        # Rule::Relu
        grads[f"conv{j}.bias"] = bias_gradient(g, s["m"], cout)
        grads[f"conv{j}.weight"] = matmul_right_backward(s["patches"], g, 1, s["m"], cin * 9, cout)
        if j > 0:
            dp = matmul_left_backward(g, params[f"conv{j}.weight"], 1, s["m"], cin * 9, cout)
            g = unfold2d_backward(dp, s["conv"], s["in_len"])
    if return_decisions:
        return loss, grads, made
    return loss, grads


def cnn_step(batch=256, size=64, classes=1000, lr=1e-3, channels=CNN_CHANNELS):
    """one forward + backward + Adam step of the 3-block CNN."""
    x, y, params = cnn_inputs(batch, size, classes, channels)
    loss, grads = cnn_forward_backward(x, y, params, batch, size, classes, channels)
    new = AdamOracle(lr).step(params, grads)
    return {"loss": loss, "grads": grads, "params": new, "initial": params, "x": x, "y": y}
