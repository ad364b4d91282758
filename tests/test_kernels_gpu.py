"""Parity of every C-ABI entry (include/axis_hip.h) against the CPU oracle on the same inputs.

Index and byte work (im2col, winners, argmax) and every kernel that keeps the reference's
evaluation order (col2im, CSR sums, elementwise, Adam) must be bit-identical; GEMMs and the
softmax family are checked to the stated fp32 tolerance.
"""
import ctypes
import os

import numpy as np
import pytest

from axis_amd import hip
from axis_amd.hip import F32, I32, I64, VP
from tests.conftest import close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return hip.Device(0)


def up(dev, a, dtype=np.float32):
    return dev.upload(np.ascontiguousarray(a, dtype=dtype))


def rel_err(actual, expected):
    e = np.asarray(expected, np.float64)
    return float(np.abs(np.asarray(actual, np.float64) - e).max() / max(np.abs(e).max(), 1e-30))


# ---------------------------------------------------------------- contractions

GEMM_SHAPES = [(1, 1, 1, 1), (1, 7, 5, 9), (2, 33, 27, 64), (1, 130, 129, 131), (3, 64, 64, 64),
               (1, 256, 256, 1000), (1, 300, 576, 128), (1, 2048, 27, 64), (1, 40000, 27, 64),
               (1, 512, 1152, 256)]


@pytest.mark.parametrize("batch,m,k,n", GEMM_SHAPES)
def test_matmul_family(dev, oracle, batch, m, k, n):
    rng = np.random.default_rng(batch * 1000 + m + k + n)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    g = rng.standard_normal(batch * m * n).astype(np.float32)
    da, db, dg = up(dev, a), up(dev, b), up(dev, g)
    out = dev.empty(batch * m * n)
    dev.call("axis_matmul", da.vp, db.vp, out.vp, I64(batch), I64(m), I64(k), I64(n))
    assert rel_err(dev.read(out, batch * m * n), oracle.matmul(a, b, batch, m, k, n)) < 1e-5
    out = dev.empty(batch * m * k)
    dev.call("axis_matmul_left_backward", dg.vp, db.vp, out.vp, I64(batch), I64(m), I64(k), I64(n))
    assert rel_err(dev.read(out, batch * m * k), oracle.matmul_left_backward(g, b, batch, m, k, n)) < 1e-5
    out = dev.empty(batch * k * n)
    dev.call("axis_matmul_right_backward", da.vp, dg.vp, out.vp, I64(batch), I64(m), I64(k), I64(n))
    assert rel_err(dev.read(out, batch * k * n), oracle.matmul_right_backward(a, g, batch, m, k, n)) < 1e-5


@pytest.mark.parametrize("batch,m,k,n", [(1, 256, 256, 1000), (1, 256, 1000, 256), (2, 33, 27, 64),
                                         (1, 130, 129, 131), (1, 4096, 512, 64), (1, 7, 3000, 5)])
def test_matmul_bias_equals_product_then_bias_add(dev, dev_bf16, batch, m, k, n):
    # Linear's product + bias in one launch: bit-identical to axis_matmul then axis_bias_add, on
    # unsplit, split-K (classifier shapes) and batched products, fp32 and bf16 handles
    rng = np.random.default_rng(batch * 7 + m + k + n)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    for d in (dev, dev_bf16):
        da, db, dbias = up(d, a), up(d, b), up(d, bias)
        geo = (I64(batch), I64(m), I64(k), I64(n))
        fused, prod, sep = d.empty(batch * m * n), d.empty(batch * m * n), d.empty(batch * m * n)
        d.call("axis_matmul_bias", da.vp, db.vp, dbias.vp, fused.vp, *geo)
        d.call("axis_matmul", da.vp, db.vp, prod.vp, *geo)
        d.call("axis_bias_add", prod.vp, dbias.vp, sep.vp, None, I64(batch * m), I64(n))
        got = d.read(fused, batch * m * n)
        assert np.array_equal(got.view(np.uint32), d.read(sep, batch * m * n).view(np.uint32))
    with pytest.raises(hip.AxisError, match="alias"):
        d.call("axis_matmul_bias", da.vp, db.vp, fused.vp, fused.vp, *geo)


# Products whose two to four short slices run in one block's waves (gemm_fold_kernel): (batch, m,
# k, n) and the entries that fold at that shape on a 256-CU part
FOLD_CASES = [(1, 256, 256, 1000),   # the classifier: product and weight gradient, 4 slices of 64
              (1, 256, 1000, 256),   # left and right backward, 4 slices of 64
              (2, 200, 300, 90),     # batched, ragged tiles, odd width: product 4, right backward 3 slices of 96
              (1, 100, 200, 999),    # product in 3 slices, width not a multiple of 4
              (1, 300, 576, 128)]    # right backward in 4 slices of 96


@pytest.fixture(scope="module")
def unfolded():
    """fp32 and bf16 handles that keep every split product as slices plus a sum launch."""
    os.environ["AXIS_GEMM_UNFOLDED"] = "1"
    try:
        return hip.Device(0), hip.Device(0, bf16_matmul=True)
    finally:
        del os.environ["AXIS_GEMM_UNFOLDED"]


def _stats(d):
    in_use, cached = ctypes.c_size_t(), ctypes.c_size_t()
    d.call("axis_memory_stats", ctypes.byref(in_use), ctypes.byref(cached))
    return in_use.value, cached.value


@pytest.mark.parametrize("batch,m,k,n", FOLD_CASES)
def test_folded_split_products_match_split_launches(dev, dev_bf16, unfolded, oracle, batch, m, k, n):
    # bit for bit against the slices and their sum on handles that do not fold, on every product
    # entry (bias and axpby finished once, as the sum does), fp32 and bf16 handles; the oracle to
    # GEMM tolerance
    rng = np.random.default_rng(batch * 31 + m + k + n)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    g = rng.standard_normal(batch * m * n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    geo = (I64(batch), I64(m), I64(k), I64(n))
    entries = [("axis_matmul", (a, b), (), batch * m * n),
               ("axis_matmul_bias", (a, b, bias), (), batch * m * n),
               ("axis_matmul_axpby", (a, b, g), (F32(1.75), F32(-0.5)), batch * m * n),
               ("axis_matmul_left_backward", (g, b), (), batch * m * k),
               ("axis_matmul_right_backward", (a, g), (), batch * k * n)]
    for folded, split in ((dev, unfolded[0]), (dev_bf16, unfolded[1])):
        for name, operands, scalars, size in entries:
            print(f"fold case {name} batch={batch} m={m} k={k} n={n}", flush=True)
            got = []
            for d in (folded, split):
                ops = [up(d, x) for x in operands]
                out = d.empty(size)
                d.call(name, *[o.vp for o in ops], out.vp, *geo, *scalars)
                got.append(d.read(out, size))
            assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32)), name
            if folded is dev and name == "axis_matmul":
                assert rel_err(got[0], oracle.matmul(a, b, batch, m, k, n)) < 1e-5
            if folded is dev and name == "axis_matmul_left_backward":
                assert rel_err(got[0], oracle.matmul_left_backward(g, b, batch, m, k, n)) < 1e-5
            if folded is dev and name == "axis_matmul_right_backward":
                assert rel_err(got[0], oracle.matmul_right_backward(a, g, batch, m, k, n)) < 1e-5


def test_folded_classifier_product_allocates_no_partial_sums(unfolded):
    # the classifier's product (4 slices over 64 tiles) folds: no partial buffer is taken from the
    # allocator, where the unfolded handle takes one of 4 x 256 x 1000 floats
    m, k, n = 256, 256, 1000
    rng = np.random.default_rng(3)
    for d, folds in ((hip.Device(0), True), (unfolded[0], False)):
        a, b = up(d, rng.standard_normal(m * k)), up(d, rng.standard_normal(k * n))
        out = d.empty(m * n)
        d.call("axis_empty_cache")  # a cached block would serve the partials without a count change
        before = _stats(d)
        d.call("axis_matmul", a.vp, b.vp, out.vp, I64(1), I64(m), I64(k), I64(n))
        d.synchronize()
        after = _stats(d)
        if folds:
            assert after == before
        else:
            assert after[1] >= before[1] + 4 * m * n * 4


def test_matmul_rejects_bad_extents(dev):
    buf = dev.empty(4)
    with pytest.raises(hip.AxisError, match="positive"):
        dev.call("axis_matmul", buf.vp, buf.vp, buf.vp, I64(1), I64(0), I64(1), I64(1))


# ---------------------------------------------------------------- unfold / col2im

def _spec(oracle, u):
    s = hip.UnfoldSpec()
    ctypes.memmove(ctypes.byref(s), ctypes.byref(u.spec), ctypes.sizeof(s))
    return s


UNFOLD_CASES = [
    # dims, layout order, channels, group, kernel, stride, padding, fill
    ([("batch", 2), ("channel", 3), ("height", 9), ("width", 7)], None, 1, [3, 3], [1, 1], [1, 1], 0.0),
    ([("batch", 2), ("height", 8), ("width", 8), ("channel", 16)], None, 1, [3, 3], [1, 1], [1, 1], 0.0),
    ([("batch", 2), ("height", 9), ("width", 7), ("channel", 4)], None, 4, [2, 2], [2, 2], [0, 0], float("-inf")),
    ([("batch", 3), ("channel", 4), ("height", 6), ("width", 5)], ["width", "batch", "channel", "height"], 2,
     [3, 2], [2, 1], [2, 1], 0.0),
]


@pytest.mark.parametrize("case", range(len(UNFOLD_CASES)))
def test_unfold_and_col2im_bit_exact(dev, oracle, case):
    dims, order, groups, kernel, stride, padding, fill = UNFOLD_CASES[case]
    strides = oracle.layout_for(dims, order) if order else oracle.contiguous(dims)
    cin = dict(dims)["channel"]
    group = ("channel", cin) if groups == cin and fill != 0.0 else ("group", groups)
    u = oracle.unfold_spec(dims, strides, "channel", ["height", "width"], group,
                           ("patch", cin // groups * kernel[0] * kernel[1]), kernel, stride, padding, fill)
    rng = np.random.default_rng(case)
    x = rng.standard_normal(oracle.shape_len(dims)).astype(np.float32)
    spec = _spec(oracle, u)
    dx = up(dev, x)
    out = dev.empty(spec.output_len)
    dev.call("axis_unfold", dx.vp, out.vp, ctypes.byref(spec))
    assert np.array_equal(dev.read(out, spec.output_len), oracle.unfold2d(x, u))
    y = rng.standard_normal(spec.output_len).astype(np.float32)
    dy = up(dev, y)
    back = dev.empty(spec.input_len)
    dev.call("axis_unfold_backward", dy.vp, back.vp, ctypes.byref(spec))
    assert np.array_equal(dev.read(back, spec.input_len), oracle.unfold2d_backward(y, u, len(x)))


def test_unfold_conv2_shape_bit_exact(dev, oracle):
    # conv2 geometry of the 3-block CNN at batch 8 (NHWC input, 64 channels)
    dims = [("batch", 8), ("height", 32), ("width", 32), ("c", 64)]
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("group", 1),
                           ("patch", 576), [3, 3], [1, 1], [1, 1], 0.0)
    x = np.random.default_rng(9).standard_normal(oracle.shape_len(dims)).astype(np.float32)
    spec = _spec(oracle, u)
    dx, out = up(dev, x), dev.empty(spec.output_len)
    dev.call("axis_unfold", dx.vp, out.vp, ctypes.byref(spec))
    patches = dev.read(out, spec.output_len)
    assert np.array_equal(patches, oracle.unfold2d(x, u))
    back = dev.empty(spec.input_len)
    dev.call("axis_unfold_backward", out.vp, back.vp, ctypes.byref(spec))
    assert np.array_equal(dev.read(back, spec.input_len), oracle.unfold2d_backward(patches, u, len(x)))


# ---------------------------------------------------------------- CSR plans

def _plan(dev, plan, uncapped=False):
    handle = ctypes.c_void_p()
    right = plan.right.ctypes.data_as(VP) if len(plan.right) else None
    dev.call("axis_plan_create", plan.offsets.ctypes.data_as(VP), plan.left.ctypes.data_as(VP), right,
             I64(len(plan.offsets) - 1), ctypes.c_int(1 if uncapped else 0), ctypes.byref(handle))
    return handle


def test_grouped_sum_and_product_bit_exact(dev, oracle):
    rng = np.random.default_rng(4)
    a = rng.standard_normal(5000).astype(np.float32)
    b = rng.standard_normal(5000).astype(np.float32)
    groups = [[(int(rng.integers(5000)), int(rng.integers(5000))) for _ in range(n)]
              for n in (0, 1, 511, 512, 513, 1300, 7)]
    plan = oracle.plan_groups(groups, product=True)
    h = _plan(dev, plan)
    da, db = up(dev, a), up(dev, b)
    out = dev.empty(len(groups))
    dev.call("axis_grouped", da.vp, None, h, F32(0.5), out.vp)
    assert np.array_equal(dev.read(out, len(groups)), oracle.grouped(a, None, plan, 0.5))
    dev.call("axis_grouped", da.vp, db.vp, h, F32(1.0), out.vp)
    assert np.array_equal(dev.read(out, len(groups)), oracle.grouped(a, b, plan, 1.0))
    dev.call("axis_plan_destroy", h)


def test_plan_cap_is_enforced(dev, oracle):
    offsets = np.array([0, 16_777_217], np.int32)
    left = np.zeros(16_777_217, np.int32)
    handle = ctypes.c_void_p()
    with pytest.raises(hip.AxisError, match="16777216"):
        dev.call("axis_plan_create", offsets.ctypes.data_as(VP), left.ctypes.data_as(VP), None,
                 I64(1), ctypes.c_int(0), ctypes.byref(handle))


def test_grouped_minimum_pool_winners_bit_exact(dev, oracle):
    rng = np.random.default_rng(5)
    dims = [("batch", 2), ("height", 6), ("width", 6), ("c", 8)]
    x = rng.integers(-3, 3, oracle.shape_len(dims)).astype(np.float32)  # many ties
    x[::17] = np.inf
    x[::23] = np.nan
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("c", 8),
                           ("pool", 9), [3, 3], [2, 2], [1, 1], float("-inf"))
    q = oracle.scale(oracle.unfold2d(x, u), -1.0)
    out_dims, fwd, rev = oracle.min_plans(u.shape, u.strides, "pool")
    ref, ref_mask, ref_w = oracle.grouped_minimum(q, fwd, rev)
    hf, hr = _plan(dev, fwd), _plan(dev, rev)
    dq = up(dev, q)
    n_out = len(fwd.offsets) - 1
    out, winners, mask = dev.empty(n_out), dev.empty(n_out, np.int32), dev.empty(len(q))
    dev.call("axis_grouped_minimum", dq.vp, I64(len(q)), hf, hr, out.vp, winners.vp, mask.vp)
    got = dev.read(out, n_out)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])
    assert np.array_equal(dev.read(winners, n_out, np.int32), ref_w)
    assert np.array_equal(dev.read(mask, len(q)), ref_mask)


# ---------------------------------------------------------------- elementwise

@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_elementwise_bit_exact(dev, oracle, n):
    rng = np.random.default_rng(n)
    a = rng.standard_normal(n).astype(np.float32)
    a[: min(n, 3)] = [0.0, -0.0, 1.0][: min(n, 3)]
    b = rng.standard_normal(n).astype(np.float32) + 3.0
    da, db, out = up(dev, a), up(dev, b), dev.empty(n)
    dev.call("axis_relu", da.vp, out.vp, I64(n))
    assert np.array_equal(dev.read(out, n), oracle.relu(a))
    dev.call("axis_relu_backward", db.vp, da.vp, out.vp, I64(n))
    assert np.array_equal(dev.read(out, n), oracle.relu_backward(b, a))
    dev.call("axis_mask_gradient", db.vp, da.vp, out.vp, I64(n))
    assert np.array_equal(dev.read(out, n), oracle.mask_gradient(b, a))
    dev.call("axis_scale", da.vp, F32(-0.37), out.vp, I64(n))
    assert np.array_equal(dev.read(out, n), oracle.scale(a, -0.37))
    for op in range(4):
        dev.call("axis_binary", da.vp, db.vp, I32(op), out.vp, I64(n))
        assert np.array_equal(dev.read(out, n), oracle.binary(a, b, op)), op
    dev.call("axis_inverse_sqrt", db.vp, F32(1e-3), out.vp, I64(n))
    assert np.array_equal(dev.read(out, n), oracle.inverse_sqrt(b, 1e-3), equal_nan=True)
    s = up(dev, np.array([1.7], np.float32))
    dev.call("axis_multiply_scalar", da.vp, s.vp, out.vp, I64(n))
    assert np.array_equal(dev.read(out, n), oracle.multiply_scalar(a, [1.7]))
    one = dev.empty(1)
    dev.call("axis_sum_squares", da.vp, I64(n), one.vp)
    close("sum_squares", dev.read(one, 1), oracle.sum_squares(a), rtol=1e-5)


def test_select_axis_permutation_and_broadcast(dev, oracle):
    rng = np.random.default_rng(6)
    dims = [("a", 3), ("b", 4), ("c", 5)]
    x = rng.standard_normal(60).astype(np.float32)
    # permutation to [c, a, b] order: metadata per target dim (extent, input_stride, output_stride)
    md = np.array([5, 1, 12, 3, 20, 4, 4, 5, 1], np.int32)
    dx, out = up(dev, x), dev.empty(60)
    dev.call("axis_select_axis", dx.vp, out.vp, md.ctypes.data_as(VP), I32(3), I32(0), I64(60))
    got = dev.read(out, 60)
    assert np.array_equal(got, oracle.select_axis(x, md, 3, 0, 60))
    assert np.array_equal(got, x.reshape(3, 4, 5).transpose(2, 0, 1).reshape(-1))
    back = dev.empty(60)
    bmd = np.array([3, 20, 4, 4, 5, 1, 5, 1, 12], np.int32)
    dev.call("axis_select_axis_backward", out.vp, back.vp, bmd.ctypes.data_as(VP), I32(3), I32(0), I64(60))
    assert np.array_equal(dev.read(back, 60), oracle.select_axis_backward(got, bmd, 3, 0, 60))
    bias = rng.standard_normal(7).astype(np.float32)
    bmd2 = oracle.broadcast_metadata([("o", 7)], [1], [("r", 11), ("o", 7)])
    db, out2 = up(dev, bias), dev.empty(77)
    dev.call("axis_select_axis", db.vp, out2.vp, np.array(bmd2, np.int32).ctypes.data_as(VP), I32(2),
             I32(0), I64(77))
    assert np.array_equal(dev.read(out2, 77), np.tile(bias, 11))


def _permutation_metadata(shape, perm):
    """with_layout's metadata (tensor.rs:5278-5333): per source dim (extent, source stride,
    stride of that axis in the permuted row-major layout)."""
    src = [int(np.prod(shape[i + 1:])) for i in range(len(shape))]
    dst_shape = [shape[p] for p in perm]
    dst_of_axis = {perm[k]: int(np.prod(dst_shape[k + 1:])) for k in range(len(perm))}
    md = []
    for i, e in enumerate(shape):
        md += [e, src[i], dst_of_axis[i]]
    return np.array(md, np.int32)


# Copies whose destination-innermost dim is strided in the source take the LDS-tiled transpose
# (tails, batch dims, unit dims merged away); the rest keep the per-element copier.
TRANSPOSE_CASES = [
    ((70, 130), (1, 0)),
    ((64, 64), (1, 0)),
    ((17, 16), (1, 0)),
    ((5, 33, 100), (2, 0, 1)),
    ((5, 33, 100), (1, 2, 0)),
    ((5, 33, 100), (0, 2, 1)),
    ((5, 33, 100), (2, 1, 0)),
    ((3, 1, 40, 2, 65), (4, 1, 2, 3, 0)),
    ((6, 7, 20, 48), (0, 3, 1, 2)),
    ((8, 3, 5), (2, 1, 0)),
]


@pytest.mark.parametrize("shape,perm", TRANSPOSE_CASES)
def test_select_axis_tiled_permutations(dev, oracle, shape, perm):
    rng = np.random.default_rng(len(shape) * 100 + sum(shape))
    n = int(np.prod(shape))
    x = rng.standard_normal(n).astype(np.float32)
    md = _permutation_metadata(shape, perm)
    rank = len(shape)
    dx, out, back = up(dev, x), dev.empty(n), dev.empty(n)
    dev.call("axis_select_axis", dx.vp, out.vp, md.ctypes.data_as(VP), I32(rank), I32(0), I64(n))
    got = dev.read(out, n)
    assert np.array_equal(got, x.reshape(shape).transpose(perm).reshape(-1))
    if n <= 1 << 16:
        assert np.array_equal(got, oracle.select_axis(x, md, rank, 0, n))
    dev.call("axis_select_axis_backward", out.vp, back.vp, md.ctypes.data_as(VP), I32(rank), I32(0), I64(n))
    assert np.array_equal(dev.read(back, n), x)


def test_select_axis_tiled_with_selected_coordinate(dev, oracle):
    """Selecting one coordinate of a middle axis and transposing the rest in one copy."""
    rng = np.random.default_rng(11)
    a, b, c = 48, 5, 70
    x = rng.standard_normal(a * b * c).astype(np.float32)
    # output [c, a] = x[:, 3, :].T ; per output dim: (extent, input stride, output stride),
    # the selected axis marked by output stride -1
    md = np.array([c, 1, a, a, b * c, 1, b, c, -1], np.int32)
    dx, out = up(dev, x), dev.empty(a * c)
    dev.call("axis_select_axis", dx.vp, out.vp, md.ctypes.data_as(VP), I32(3), I32(3), I64(a * c))
    got = dev.read(out, a * c)
    assert np.array_equal(got, x.reshape(a, b, c)[:, 3, :].T.reshape(-1))
    assert np.array_equal(got, oracle.select_axis(x, md, 3, 3, a * c))


def test_select_axis_muon_sized_transpose(dev):
    """The [8192, 4096] -> [4096, 8192] layout copy of Muon's Newton-Schulz input."""
    rng = np.random.default_rng(12)
    shape = (8192, 4096)
    n = shape[0] * shape[1]
    x = rng.standard_normal(n).astype(np.float32)
    md = _permutation_metadata(shape, (1, 0))
    dx, out = up(dev, x), dev.empty(n)
    dev.call("axis_select_axis", dx.vp, out.vp, md.ctypes.data_as(VP), I32(2), I32(0), I64(n))
    assert np.array_equal(dev.read(out, n), x.reshape(shape).T.reshape(-1))


# ---------------------------------------------------------------- softmax / cross-entropy

@pytest.mark.parametrize("rows,width", [(2, 3), (256, 1000), (5, 2049)])
def test_softmax_cross_entropy(dev, oracle, rows, width):
    rng = np.random.default_rng(rows)
    z = (rng.standard_normal(rows * width) * 4).astype(np.float32)
    _, y = oracle.one_hot_labels(7, rows, width)
    y = y.reshape(-1)
    dz, dy = up(dev, z), up(dev, y)
    p, loss = dev.empty(rows * width), dev.empty(rows)
    dev.call("axis_softmax", dz.vp, p.vp, I64(rows), I64(width))
    pr = dev.read(p, rows * width)
    close("softmax", pr, oracle.softmax(z, rows, width), atol=1e-7, rtol=2e-6)
    dev.call("axis_categorical_cross_entropy", dz.vp, dy.vp, loss.vp, I64(rows), I64(width))
    close("CE", dev.read(loss, rows), oracle.categorical_cross_entropy(z, y, rows, width), rtol=2e-6)
    p2, l2 = dev.empty(rows * width), dev.empty(rows)
    dev.call("axis_softmax_cross_entropy", dz.vp, dy.vp, p2.vp, l2.vp, I64(rows), I64(width))
    assert np.array_equal(dev.read(p2, rows * width), pr)
    close("fused CE", dev.read(l2, rows), oracle.categorical_cross_entropy(z, y, rows, width), rtol=2e-6)
    g = rng.standard_normal(rows).astype(np.float32)
    dg, out = up(dev, g), dev.empty(rows * width)
    dev.call("axis_categorical_cross_entropy_backward", dg.vp, p.vp, dy.vp, out.vp, I64(rows), I64(width))
    assert np.array_equal(dev.read(out, rows * width),
                          oracle.categorical_cross_entropy_backward(g, pr, y, rows, width))
    gw = rng.standard_normal(rows * width).astype(np.float32)
    dgw = up(dev, gw)
    dev.call("axis_softmax_backward", dgw.vp, p.vp, out.vp, I64(rows), I64(width))
    close("softmax backward", dev.read(out, rows * width), oracle.softmax_backward(gw, pr, rows, width),
          atol=1e-6, rtol=1e-5)


# ---------------------------------------------------------------- Adam

@pytest.mark.parametrize("n", [1, 5, 4096, 65537])
def test_adam_bit_exact(dev, oracle, n):
    rng = np.random.default_rng(n + 1)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-4).astype(np.float32)
    v = np.abs(rng.standard_normal(n) * 1e-6).astype(np.float32)
    c1, c2 = 1 - oracle.powi(0.9, 4), 1 - oracle.powi(0.999, 4)
    ref = oracle.adam(p, g, m, v, 1e-3, 0.9, 0.999, c1, c2, 1e-8, 0.01)
    dp, dg, dm, dv = up(dev, p), up(dev, g), up(dev, m), up(dev, v)
    op, om, ov = dev.empty(n), dev.empty(n), dev.empty(n)
    dev.call("axis_adam", dp.vp, dg.vp, dm.vp, dv.vp, None, I64(n), F32(1e-3), F32(0.9), F32(0.999),
             F32(c1), F32(c2), F32(1e-8), F32(0.01), op.vp, om.vp, ov.vp)
    for got, exp in zip((op, om, ov), ref):
        assert np.array_equal(dev.read(got, n), exp)
    # in place, multi-tensor
    t = hip.AdamTensor(dp.ptr, dg.ptr, dm.ptr, dv.ptr, None, n)
    arr = (hip.AdamTensor * 2)(t, hip.AdamTensor(None, None, None, None, None, 0))
    dev.call("axis_adam_multi", arr, I32(2), F32(1e-3), F32(0.9), F32(0.999), F32(c1), F32(c2),
             F32(1e-8), F32(0.01))
    for got, exp in zip((dp, dm, dv), ref):
        assert np.array_equal(dev.read(got, n), exp)


def test_adam_multi_many_tensors(dev, oracle):
    rng = np.random.default_rng(11)
    sizes = [3, 64, 1000, 4097, 1, 123457] * 5  # 30 tensors: spans two launches
    tensors, host = [], []
    for s in sizes:
        arrs = [(rng.standard_normal(s) * 0.1).astype(np.float32) for _ in range(3)]
        arrs.append(np.abs(arrs[2]) * 0.01)
        bufs = [up(dev, a) for a in arrs]
        host.append(arrs)
        tensors.append(bufs)
    arr = (hip.AdamTensor * len(sizes))(*[hip.AdamTensor(b[0].ptr, b[1].ptr, b[2].ptr, b[3].ptr, None, s)
                                          for b, s in zip(tensors, sizes)])
    dev.call("axis_adam_multi", arr, I32(len(sizes)), F32(0.01), F32(0.9), F32(0.999), F32(0.1),
             F32(0.001), F32(1e-8), F32(0.0))
    for (p, g, m, v), bufs, s in zip(host, tensors, sizes):
        ref = oracle.adam(p, g, m, v, 0.01, 0.9, 0.999, 0.1, 0.001, 1e-8, 0.0)
        assert np.array_equal(dev.read(bufs[0], s), ref[0])
        assert np.array_equal(dev.read(bufs[2], s), ref[1])


# ---------------------------------------------------------------- fused entries

# the last three take the 64-column kernel (widths from 2048): ragged columns over three chunks,
# one chunk written directly, config 5's [4096, 8192] layer
@pytest.mark.parametrize("rows,width", [(1, 1), (600, 2), (1030, 64), (777, 130), (1300, 2100), (300, 4096),
                                        (4096, 8192)])
def test_bias_entries_bit_exact(dev, oracle, rows, width):
    rng = np.random.default_rng(rows)
    a = rng.standard_normal(rows * width).astype(np.float32)
    bias = rng.standard_normal(width).astype(np.float32)
    g = rng.standard_normal(rows * width).astype(np.float32)
    da, db, dg = up(dev, a), up(dev, bias), up(dev, g)
    out, act = dev.empty(rows * width), dev.empty(rows * width)
    dev.call("axis_bias_add", da.vp, db.vp, out.vp, act.vp, I64(rows), I64(width))
    z = oracle.binary(a, np.tile(bias, rows), 0)
    assert np.array_equal(dev.read(out, rows * width), z)
    assert np.array_equal(dev.read(act, rows * width), oracle.relu(z))
    gb = dev.empty(width)
    dev.call("axis_bias_gradient", dg.vp, None, None, gb.vp, I64(rows), I64(width))
    assert np.array_equal(dev.read(gb, width), oracle.bias_gradient(g, rows, width))
    masked = dev.empty(rows * width)
    dev.call("axis_bias_gradient", dg.vp, out.vp, masked.vp, gb.vp, I64(rows), I64(width))
    gm = oracle.relu_backward(g, z)
    assert np.array_equal(dev.read(masked, rows * width), gm)
    assert np.array_equal(dev.read(gb, width), oracle.bias_gradient(gm, rows, width))


@pytest.mark.parametrize("kernel,stride,padding", [([2, 2], [2, 2], [0, 0]), ([3, 3], [1, 1], [1, 1]),
                                                   ([3, 2], [2, 1], [1, 0])])
def test_max_pool_entries_match_generic_path(dev, oracle, kernel, stride, padding):
    rng = np.random.default_rng(sum(kernel) + sum(stride))
    b, h, w, c = 2, 7, 9, 6
    x = rng.integers(-2, 3, b * h * w * c).astype(np.float32)  # ties everywhere
    x[::31] = np.nan
    dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("c", c),
                           ("pool", kernel[0] * kernel[1]), kernel, stride, padding, float("-inf"))
    q = oracle.scale(oracle.unfold2d(x, u), -1.0)
    out_dims, fwd, rev = oracle.min_plans(u.shape, u.strides, "pool")
    mn, mask, _ = oracle.grouped_minimum(q, fwd, rev)
    ref = oracle.scale(mn, -1.0)
    n_out = len(ref)
    gout = rng.standard_normal(n_out).astype(np.float32)
    gg = oracle.mask_gradient(oracle.grouped(oracle.scale(gout, -1.0), None, rev, 1.0), mask)
    ref_dx = oracle.unfold2d_backward(oracle.scale(gg, -1.0), u, len(x))
    k, s, p = (I32 * 2)(*kernel), (I32 * 2)(*stride), (I32 * 2)(*padding)
    dx, out, arg = up(dev, x), dev.empty(n_out), dev.empty(n_out, np.uint8)
    dev.call("axis_max_pool2d", dx.vp, out.vp, arg.vp, I64(b), I32(h), I32(w), I64(c), k, s, p)
    got = dev.read(out, n_out)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    dg, back = up(dev, gout), dev.empty(len(x))
    dev.call("axis_max_pool2d_backward", dg.vp, arg.vp, back.vp, I64(b), I32(h), I32(w), I64(c), k, s, p)
    assert np.array_equal(dev.read(back, len(x)), ref_dx)


def test_reduce_and_broadcast_middle_bit_exact(dev, oracle):
    rng = np.random.default_rng(12)
    outer, red, inner = 3, 1100, 5
    a = rng.standard_normal(outer * red * inner).astype(np.float32)
    dims = [("o", outer), ("r", red), ("i", inner)]
    _, fwd, rev, factor = oracle.reduction_plans(dims, oracle.contiguous(dims), ["r"], mean=True)
    da, out = up(dev, a), dev.empty(outer * inner)
    dev.call("axis_reduce_middle", da.vp, out.vp, I64(outer), I64(red), I64(inner), F32(factor))
    got = dev.read(out, outer * inner)
    assert np.array_equal(got, oracle.grouped(a, None, fwd, factor))
    back = dev.empty(len(a))
    dev.call("axis_broadcast_middle", out.vp, back.vp, I64(outer), I64(red), I64(inner), F32(factor))
    assert np.array_equal(dev.read(back, len(a)), oracle.grouped(got, None, rev, factor))


# (dims, storage order outermost first, reduced axes, mean): non-consecutive axis sets, permuted
# layouts, unit dims, several chunks per group, a single output, nothing left to merge.
REDUCE_AXES_CASES = [
    ([("a", 3), ("b", 5), ("c", 7)], ["a", "b", "c"], ["a", "c"], False),
    ([("a", 3), ("b", 5), ("c", 7)], ["c", "a", "b"], ["b"], True),
    ([("n", 4), ("h", 9), ("w", 9), ("ch", 6)], ["n", "ch", "h", "w"], ["h", "w"], True),
    ([("n", 4), ("h", 9), ("w", 9), ("ch", 6)], ["n", "h", "w", "ch"], ["n", "w"], False),
    ([("p", 1), ("q", 600), ("u", 1), ("v", 5)], ["v", "q", "p", "u"], ["q", "u"], True),
    ([("x", 2), ("y", 1300), ("z", 3)], ["y", "z", "x"], ["x", "y", "z"], True),
    ([("x", 2), ("y", 13), ("z", 3)], ["x", "y", "z"], ["y"], False),
]


@pytest.mark.parametrize("dims,order,axes,mean", REDUCE_AXES_CASES)
def test_reduce_axes_bit_exact(dev, oracle, dims, order, axes, mean):
    rng = np.random.default_rng(len(dims) * 31 + sum(e for _, e in dims))
    n = int(np.prod([e for _, e in dims]))
    a = rng.standard_normal(n).astype(np.float32)  # physical storage
    strides = oracle.layout_for(dims, order)
    out_dims, fwd, rev, factor = oracle.reduction_plans(dims, strides, axes, mean)
    olen = int(np.prod([e for _, e in out_dims])) if out_dims else 1
    ext = np.array([e for _, e in dims], np.int64)
    st = np.array(strides, np.int64)
    red = np.array([1 if name in axes else 0 for name, _ in dims], np.int32)
    geo = (I32(len(dims)), ext.ctypes.data_as(VP), st.ctypes.data_as(VP), red.ctypes.data_as(VP), F32(factor))
    da, out = up(dev, a), dev.empty(olen)
    dev.call("axis_reduce_axes", da.vp, out.vp, *geo)
    got = dev.read(out, olen)
    assert np.array_equal(got, oracle.grouped(a, None, fwd, factor))
    back = dev.empty(n)
    dev.call("axis_reduce_axes_backward", out.vp, back.vp, *geo)
    assert np.array_equal(dev.read(back, n), oracle.grouped(got, None, rev, factor))


EXTREME_AXIS_CASES = [
    # dims, physical order, axis
    ([("g", 6), ("w", 4)], ["g", "w"], "w"),
    ([("a", 3), ("b", 5), ("c", 7)], ["c", "a", "b"], "b"),
    ([("n", 2), ("oh", 5), ("ow", 5), ("ch", 3), ("win", 9)], ["n", "ch", "oh", "ow", "win"], "win"),
    ([("n", 2), ("oh", 4), ("ow", 4), ("ch", 8), ("win", 4)], ["win", "n", "oh", "ow", "ch"], "win"),
    ([("x", 1), ("y", 700)], ["y", "x"], "y"),
]


@pytest.mark.parametrize("dims,order,axis", EXTREME_AXIS_CASES)
@pytest.mark.parametrize("maximum", [False, True])
def test_extreme_axis_matches_plan_reductions(dev, oracle, dims, order, axis, maximum):
    rng = np.random.default_rng(len(dims) * 7 + int(maximum))
    n = int(np.prod([e for _, e in dims]))
    a = np.round(rng.standard_normal(n) * 4).astype(np.float32) / 4  # physical storage, many ties
    a[::11] = np.inf
    a[::13] = -np.inf
    a[::17] = np.nan
    strides = oracle.layout_for(dims, order)
    out_dims, fwd, rev = oracle.min_plans(dims, strides, axis)
    olen = int(np.prod([e for _, e in out_dims]))
    ref, ref_mask, _ = oracle.grouped_minimum(a, fwd, rev, maximum)
    ext = np.array([e for _, e in dims], np.int64)
    st = np.array(strides, np.int64)
    ax = [name for name, _ in dims].index(axis)
    geo = (I32(len(dims)), ext.ctypes.data_as(VP), st.ctypes.data_as(VP), I32(ax))
    da, out, mask = up(dev, a), dev.empty(olen), dev.empty(n)
    dev.call("axis_extreme_axis", da.vp, *geo, I32(1 if maximum else 0), out.vp, mask.vp)
    got, got_mask = dev.read(out, olen), dev.read(mask, n)
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    assert np.array_equal(got_mask, ref_mask)
    # backward: the gather plan's grouped sum, then mask_gradient
    g = rng.standard_normal(olen).astype(np.float32)
    g[::5] = -0.0
    dg, back = up(dev, g), dev.empty(n)
    dev.call("axis_extreme_axis_backward", dg.vp, mask.vp, *geo, back.vp)
    expect = oracle.mask_gradient(oracle.grouped(g, None, rev, 1.0), ref_mask)
    assert np.array_equal(dev.read(back, n).view(np.uint32), expect.view(np.uint32))


def test_extreme_axis_past_the_plan_cap(dev, oracle):
    # a [batch, 32, 32, 64, window 9] unfolded pool input: 18.9M members, past the plan cap
    dims = [("n", 32), ("oh", 32), ("ow", 32), ("ch", 64), ("win", 9)]
    strides = oracle.contiguous(dims)
    n = int(np.prod([e for _, e in dims]))
    assert n > 16777216
    rng = np.random.default_rng(5)
    a = rng.standard_normal(n).astype(np.float32)
    ext = np.array([e for _, e in dims], np.int64)
    st = np.array(strides, np.int64)
    geo = (I32(len(dims)), ext.ctypes.data_as(VP), st.ctypes.data_as(VP), I32(4))
    da, out, mask = up(dev, a), dev.empty(n // 9), dev.empty(n)
    dev.call("axis_extreme_axis", da.vp, *geo, I32(0), out.vp, mask.vp)
    windows = a.reshape(-1, 9)
    assert np.array_equal(dev.read(out, n // 9), windows.min(axis=1))
    m = dev.read(mask, n).reshape(-1, 9)
    assert np.array_equal(np.argmax(m, axis=1), np.argmin(windows, axis=1)) and np.all(m.sum(axis=1) == 1)


def test_reduce_axes_past_the_plan_cap(dev, oracle):
    """A mean over two non-adjacent axes of 2^24 + 2^20 elements: past the reference's 16,777,216
    contribution cap, still in the reverse plan's order (plan built uncapped on the host)."""
    dims = [("b", 17), ("h", 64), ("w", 32), ("c", 512)]
    n = int(np.prod([e for _, e in dims]))
    assert n > 16777216
    rng = np.random.default_rng(5)
    a = rng.standard_normal(n).astype(np.float32)
    strides = oracle.contiguous(dims)
    out_dims, fwd, _, factor = oracle.reduction_plans(dims, strides, ["b", "w"], True, cap=False)
    olen = int(np.prod([e for _, e in out_dims]))
    ext = np.array([e for _, e in dims], np.int64)
    st = np.array(strides, np.int64)
    red = np.array([1, 0, 1, 0], np.int32)
    da, out = up(dev, a), dev.empty(olen)
    dev.call("axis_reduce_axes", da.vp, out.vp, I32(4), ext.ctypes.data_as(VP), st.ctypes.data_as(VP),
             red.ctypes.data_as(VP), F32(factor))
    assert np.array_equal(dev.read(out, olen), oracle.grouped(a, None, fwd, factor))


def test_reduce_axes_rejects_non_dense_layouts(dev):
    a, out = dev.empty(64), dev.empty(8)
    ext = np.array([8, 8], np.int64)
    st = np.array([16, 1], np.int64)  # row pitch 16 over 8 columns: not dense
    red = np.array([0, 1], np.int32)
    with pytest.raises(hip.AxisError, match="dense layout"):
        dev.call("axis_reduce_axes", a.vp, out.vp, I32(2), ext.ctypes.data_as(VP), st.ctypes.data_as(VP),
                 red.ctypes.data_as(VP), F32(1.0))


# ---------------------------------------------------------------- bf16 matrix products

@pytest.fixture(scope="module")
def dev_bf16():
    return hip.Device(0, bf16_matmul=True)


@pytest.mark.parametrize("m,k,n", [(96, 160, 130), (257, 512, 256), (64, 2048, 40)])
def test_bf16_matmul_family(dev, dev_bf16, oracle, m, k, n):
    # Device::cuda_bf16: each product rounds its operands to bf16 and accumulates in fp32
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal(m * k).astype(np.float32)
    b = rng.standard_normal(k * n).astype(np.float32)
    g = rng.standard_normal(m * n).astype(np.float32)
    ra, rb, rg = oracle.bf16_round(a), oracle.bf16_round(b), oracle.bf16_round(g)
    flag = ctypes.c_int()
    hip.check(hip.load().axis_device_bf16_matmul(dev_bf16.handle, ctypes.byref(flag)), "bf16 flag")
    assert flag.value == 1
    da, db, dg = up(dev_bf16, a), up(dev_bf16, b), up(dev_bf16, g)
    geo = (I64(1), I64(m), I64(k), I64(n))
    out = dev_bf16.empty(m * n)
    dev_bf16.call("axis_matmul", da.vp, db.vp, out.vp, *geo)
    got = dev_bf16.read(out, m * n)
    ref = oracle.matmul(ra, rb, 1, m, k, n)
    assert rel_err(got, ref) < 1e-5
    assert rel_err(got, oracle.matmul(a, b, 1, m, k, n)) > 1e-4  # the rounding is really there
    dx, dw = dev_bf16.empty(m * k), dev_bf16.empty(k * n)
    dev_bf16.call("axis_matmul_left_backward", dg.vp, db.vp, dx.vp, *geo)
    assert rel_err(dev_bf16.read(dx, m * k), oracle.matmul_left_backward(rg, rb, 1, m, k, n)) < 1e-5
    dev_bf16.call("axis_matmul_right_backward", da.vp, dg.vp, dw.vp, *geo)
    assert rel_err(dev_bf16.read(dw, k * n), oracle.matmul_right_backward(ra, rg, 1, m, k, n)) < 1e-5
    # an fp32 handle is unaffected
    out32 = dev.empty(m * n)
    d32a, d32b = up(dev, a), up(dev, b)
    dev.call("axis_matmul", d32a.vp, d32b.vp, out32.vp, *geo)
    assert rel_err(dev.read(out32, m * n), oracle.matmul(a, b, 1, m, k, n)) < 1e-5


@pytest.mark.parametrize("batch,m,k,n", [(3, 130, 70, 33), (2, 64, 1000, 200), (1, 1, 9, 1), (1, 4100, 96, 2050)])
def test_bf16_batched_products_and_axpby(dev_bf16, oracle, batch, m, k, n):
    # (1, 4100, 96, 2050): enough 128 x 128 output tiles to fill the chip, ragged on both sides
    # batched bf16 products (staged operands per batch, reduction tail padded) and the axpby
    # epilogue: beta * d + alpha * product, each operation rounded on its own
    rng = np.random.default_rng(batch * 1000 + m + k + n)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    g = rng.standard_normal(batch * m * n).astype(np.float32)
    ra, rb, rg = oracle.bf16_round(a), oracle.bf16_round(b), oracle.bf16_round(g)
    da, db, dg = up(dev_bf16, a), up(dev_bf16, b), up(dev_bf16, g)
    geo = (I64(batch), I64(m), I64(k), I64(n))
    out = dev_bf16.empty(batch * m * n)
    dev_bf16.call("axis_matmul", da.vp, db.vp, out.vp, *geo)
    prod = dev_bf16.read(out, batch * m * n)
    assert rel_err(prod, oracle.matmul(ra, rb, batch, m, k, n)) < 1e-5
    dx, dw = dev_bf16.empty(batch * m * k), dev_bf16.empty(batch * k * n)
    dev_bf16.call("axis_matmul_left_backward", dg.vp, db.vp, dx.vp, *geo)
    assert rel_err(dev_bf16.read(dx, batch * m * k), oracle.matmul_left_backward(rg, rb, batch, m, k, n)) < 1e-5
    dev_bf16.call("axis_matmul_right_backward", da.vp, dg.vp, dw.vp, *geo)
    assert rel_err(dev_bf16.read(dw, batch * k * n), oracle.matmul_right_backward(ra, rg, batch, m, k, n)) < 1e-5
    alpha, beta = 2.0315, -4.7750
    fused = dev_bf16.empty(batch * m * n)
    dev_bf16.call("axis_matmul_axpby", da.vp, db.vp, dg.vp, fused.vp, *geo, F32(alpha), F32(beta))
    # the epilogue applied to this handle's own product is bit-exact (d itself is not rounded)
    expect = (np.float32(beta) * g) + (np.float32(alpha) * prod)
    assert np.array_equal(dev_bf16.read(fused, batch * m * n).view(np.uint32), expect.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("s,l", [(64, 96), (48, 160)])
def test_bf16_newton_schulz_iterations(dev_bf16, oracle, s, l):
    """The Newton-Schulz iteration of Muon's fused path (optim.rs:728-752; gram through the NT
    product, both scale-and-adds in axpby epilogues) on a bf16 handle, one iteration at a time
    from the GPU's own state: each matches the oracle's bf16 iteration (operands of every product
    rounded, fp32 terms) to 2e-5 of its norm (measured: at most 3e-6), while one fp32 iteration from
    the same state lies about 1e-4 away -- four times the error at least."""
    rng = np.random.default_rng(s * l)
    x = oracle.normalized_l2(rng.standard_normal(s * l).astype(np.float32), 1e-7)
    R = oracle.bf16_round
    A, B, C = float(oracle.NS_A), float(oracle.NS_B), float(oracle.NS_C)

    def step(xh, r):
        xm = xh.reshape(s, l)
        gram = oracle.matmul(r(xm), r(np.ascontiguousarray(xm.T)), 1, s, l, s)
        b = oracle.binary(oracle.scale(gram, B), oracle.scale(oracle.matmul(r(gram), r(gram), 1, s, s, s), C), 0)
        return oracle.binary(oracle.scale(xh, A), oracle.matmul(r(b), r(xh), 1, s, s, l), 0)

    X = up(dev_bf16, x)
    for _ in range(5):
        xh = dev_bf16.read(X, s * l)
        gram, b, nx = dev_bf16.empty(s * s), dev_bf16.empty(s * s), dev_bf16.empty(s * l)
        dev_bf16.call("axis_matmul_left_backward", X.vp, X.vp, gram.vp, I64(1), I64(s), I64(s), I64(l))
        dev_bf16.call("axis_matmul_axpby", gram.vp, gram.vp, gram.vp, b.vp, I64(1), I64(s), I64(s), I64(s), F32(C), F32(B))
        dev_bf16.call("axis_matmul_axpby", b.vp, X.vp, X.vp, nx.vp, I64(1), I64(s), I64(s), I64(l), F32(1.0), F32(A))
        X = nx
        got = dev_bf16.read(X, s * l)
        want, want32 = step(xh, R), step(xh, lambda v: v)
        err = np.linalg.norm(got - want) / np.linalg.norm(want)
        gap = np.linalg.norm(want32 - want) / np.linalg.norm(want)
        assert err < 2e-5 and gap > 4 * max(err, 1e-5), (err, gap)


@pytest.mark.parametrize("m,k,n", [(4096, 4096, 4096), (8192, 784, 1024)])
def test_bf16_backward_at_config2_sizes(dev_bf16, oracle, m, k, n):
    """BASELINE config 2's shapes on a bf16 handle (the bench's workload): 16 sampled rows of dX and
    16 sampled columns of dW against float64 products of the bf16-rounded operands."""
    rng = np.random.default_rng(k)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = rng.standard_normal(k * n).astype(np.float32)
    dy = rng.standard_normal(m * n).astype(np.float32)
    X, W, DY = up(dev_bf16, x), up(dev_bf16, w), up(dev_bf16, dy)
    dx, dw = dev_bf16.empty(m * k), dev_bf16.empty(k * n)
    geo = (I64(1), I64(m), I64(k), I64(n))
    dev_bf16.call("axis_matmul_left_backward", DY.vp, W.vp, dx.vp, *geo)
    dev_bf16.call("axis_matmul_right_backward", X.vp, DY.vp, dw.vp, *geo)
    R = oracle.bf16_round
    rows = np.sort(rng.choice(m, 16, replace=False))
    cols = np.sort(rng.choice(n, 16, replace=False))
    rx, rw, rdy = R(x).reshape(m, k), R(w).reshape(k, n), R(dy).reshape(m, n)
    want_dx = rdy[rows].astype(np.float64) @ rw.astype(np.float64).T
    want_dw = rx.astype(np.float64).T @ rdy[:, cols].astype(np.float64)
    got_dx = dev_bf16.read(dx, m * k).reshape(m, k)[rows]
    got_dw = dev_bf16.read(dw, k * n).reshape(k, n)[:, cols]
    for got, want in ((got_dx, want_dx), (got_dw, want_dw)):
        # fp32 accumulation of exact bf16 products over n (dX) or m (dW) terms
        assert rel_err(got, want) < 1e-5


@pytest.mark.parametrize("batch,m,k,n", [(1, 4096, 192, 4096), (1, 4352, 320, 4100), (4, 2048, 96, 2048)])
def test_bf16_products_on_256_tiles(dev_bf16, oracle, batch, m, k, n):
    """Products whose 256 x 256 tiles alone fill a 256-CU part (one block of eight waves per CU):
    every output, ragged edges and batches included, against float64 products of the bf16-rounded
    operands (fp32 accumulation of exact bf16 products: rel 1e-5); the bias and axpby entries
    finish the same sums (each operation rounded on its own)."""
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    A, B, BIAS = up(dev_bf16, a), up(dev_bf16, b), up(dev_bf16, bias)
    out, out_b = dev_bf16.empty(batch * m * n), dev_bf16.empty(batch * m * n)
    geo = (I64(batch), I64(m), I64(k), I64(n))
    dev_bf16.call("axis_matmul", A.vp, B.vp, out.vp, *geo)
    dev_bf16.call("axis_matmul_bias", A.vp, B.vp, BIAS.vp, out_b.vp, *geo)
    R = oracle.bf16_round
    ra, rb = R(a).reshape(batch, m, k).astype(np.float64), R(b).reshape(batch, k, n).astype(np.float64)
    want = ra @ rb
    got = dev_bf16.read(out, batch * m * n).reshape(batch, m, n)
    assert rel_err(got, want) < 1e-5
    got_b = dev_bf16.read(out_b, batch * m * n).reshape(batch, m, n)
    assert np.array_equal(got_b.view(np.uint32), (got + bias).astype(np.float32).view(np.uint32))
    g = rng.standard_normal(batch * m * n).astype(np.float32)
    G, fused = up(dev_bf16, g), dev_bf16.empty(batch * m * n)
    alpha, beta = 0.8125, -1.4375
    dev_bf16.call("axis_matmul_axpby", A.vp, B.vp, G.vp, fused.vp, *geo, F32(alpha), F32(beta))
    expect = (np.float32(beta) * g) + (np.float32(alpha) * got.reshape(-1))
    assert np.array_equal(dev_bf16.read(fused, batch * m * n).view(np.uint32), expect.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("m", [4_194_368, 8_400_000])
def test_bf16_weight_gradient_over_long_reductions(dev_bf16, m):
    """matmul_right_backward on a bf16 handle reducing over more than 4,194,304 rows (its operands
    are staged through the LDS transpose, more than 65,535 reduction tiles) and over more than the
    bf16 kernel's 32-bit offsets reach (about 8.3M: the fp32 matrix cores take the same rounded
    operands).  Operands in {-1, 0, 1} are exact in bf16 and every partial sum is an integer below
    2^24, so the result is exact in any summation order."""
    k = n = 16
    rng = np.random.default_rng(m)
    x = rng.integers(-1, 2, m * k).astype(np.float32)
    g = rng.integers(-1, 2, m * n).astype(np.float32)
    X, G = up(dev_bf16, x), up(dev_bf16, g)
    out = dev_bf16.empty(k * n)
    dev_bf16.call("axis_matmul_right_backward", X.vp, G.vp, out.vp, I64(1), I64(m), I64(k), I64(n))
    want = x.reshape(m, k).astype(np.float64).T @ g.reshape(m, n).astype(np.float64)
    assert np.array_equal(dev_bf16.read(out, k * n), want.reshape(-1).astype(np.float32))


def test_bf16_products_carry_inf_and_nan(dev_bf16):
    # a NaN operand stays NaN after rounding, an infinity stays infinite: rows meeting them turn
    # NaN / inf exactly as the fp32 product of the rounded operands does
    m, k, n = 4, 80, 5
    a = np.ones(m * k, np.float32)
    a[1 * k + 3] = np.nan
    a[2 * k + 70] = np.inf
    b = np.full(k * n, 0.5, np.float32)
    da, db = up(dev_bf16, a), up(dev_bf16, b)
    out = dev_bf16.empty(m * n)
    dev_bf16.call("axis_matmul", da.vp, db.vp, out.vp, I64(1), I64(m), I64(k), I64(n))
    got = dev_bf16.read(out, m * n).reshape(m, n)
    assert np.all(np.isnan(got[1])) and np.all(np.isposinf(got[2]))
    assert np.array_equal(got[0], np.full(n, 40.0, np.float32)) and np.array_equal(got[3], got[0])


@pytest.mark.parametrize("layout,b,c,h,w,n", [("nchw", 2, 3, 16, 16, 64), ("nhwc", 2, 64, 8, 8, 128)])
def test_bf16_convolution_entries(dev_bf16, oracle, layout, b, c, h, w, n):
    # bf16 mode: the convolution's product (unfold -> matmul_bf16) takes rounded input and weight;
    # the bias is added in fp32 after it, as the separate add of the reference's lowering.
    k = 3
    rng = np.random.default_rng(c + n)
    x = rng.uniform(-1, 1, b * c * h * w).astype(np.float32)
    weight = (rng.standard_normal(c * k * k * n) * 0.2).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    if layout == "nchw":
        dims = [("batch", b), ("c", c), ("height", h), ("width", w)]
        strides = (I64 * 4)(c * h * w, h * w, w, 1)
    else:
        dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
        strides = None
    z, _ = _oracle_conv(oracle, oracle.bf16_round(x), oracle.bf16_round(weight), bias, dims, b, c, n, k, 1, 1, h, w)
    geo = [(I32 * 2)(k, k), (I32 * 2)(1, 1), (I32 * 2)(1, 1)]
    dx, dw, db = up(dev_bf16, x), up(dev_bf16, weight), up(dev_bf16, bias)
    out = dev_bf16.empty(b * h * w * n)
    dev_bf16.call("axis_conv2d_forward", dx.vp, strides, dw.vp, db.vp, out.vp, I64(b), I32(h), I32(w), I32(c),
                  I32(n), *geo)
    assert rel_err(dev_bf16.read(out, b * h * w * n), z) < 1e-5
    # fused ReLU + 2x2 pool: pooled values of the same bf16 products
    pooled_len = b * (h // 2) * (w // 2) * n
    pooled, arg = dev_bf16.empty(pooled_len), dev_bf16.empty(pooled_len, np.uint8)
    dev_bf16.call("axis_conv2d_relu_pool_forward", dx.vp, strides, dw.vp, db.vp, pooled.vp, arg.vp, I64(b), I32(h),
                  I32(w), I32(c), I32(n), *geo, (I32 * 2)(2, 2))
    ref, _ = _first_max(_windows(np.maximum(z, 0), b, h, w, n, 2, 2))
    scale = np.abs(z).max()
    assert np.abs(dev_bf16.read(pooled, pooled_len) - ref.reshape(-1)).max() <= 1e-5 * scale


# ---------------------------------------------------------------- implicit-GEMM convolution

# Outputs of 16x16, 8x8, 32x32 (stride 2, and padding 0), 64x64 and 128x128 pixels take the weight
# gradient's aligned-step loader (128 columns: steps inside the row as well as at its two ends; a 5x5
# kernel with padding 2 over 16-wide rows: two rows per step); the others its general one.  Two
# cases are data gradients of few channels over many pixels (aligned tap steps, then a ragged last
# tile with the general decode); 64 channels under 3x3 (576 patch rows) take 64x128 tiles.
@pytest.mark.parametrize("b,h,w,c,n,k,s,p", [(2, 9, 7, 8, 16, 3, 1, 1), (3, 16, 16, 64, 128, 3, 1, 1),
                                             (2, 11, 10, 5, 7, 3, 1, 0), (2, 9, 8, 12, 20, 3, 2, 1),
                                             (1, 8, 8, 128, 256, 3, 1, 1), (2, 6, 6, 4, 8, 2, 1, 1),
                                             (2, 64, 64, 8, 16, 3, 2, 1), (2, 34, 34, 4, 8, 3, 1, 0),
                                             (1, 64, 64, 3, 64, 3, 1, 1), (32, 64, 64, 32, 64, 3, 1, 1),
                                             (34, 63, 63, 24, 40, 3, 1, 1), (1, 128, 128, 4, 8, 3, 1, 1),
                                             (1, 128, 128, 8, 16, 3, 2, 1), (2, 16, 16, 8, 16, 5, 1, 2)])
def test_conv2d_entries_match_explicit_lowering(dev, oracle, b, h, w, c, n, k, s, p):
    rng = np.random.default_rng(b * 100 + c)
    x = rng.standard_normal(b * h * w * c).astype(np.float32)
    weight = rng.standard_normal(c * k * k * n).astype(np.float32) * 0.1
    bias = rng.standard_normal(n).astype(np.float32)
    dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("group", 1),
                           ("patch", c * k * k), [k, k], [s, s], [p, p], 0.0)
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    m = b * oh * ow
    patches = oracle.unfold2d(x, u)
    ref = oracle.binary(oracle.matmul(patches, weight, 1, m, c * k * k, n), np.tile(bias, m), 0)
    geo = [(I32 * 2)(k, k), (I32 * 2)(s, s), (I32 * 2)(p, p)]
    dx, dw, db, out = up(dev, x), up(dev, weight), up(dev, bias), dev.empty(m * n)
    dev.call("axis_conv2d_forward", dx.vp, None, dw.vp, db.vp, out.vp, I64(b), I32(h), I32(w), I32(c), I32(n), *geo)
    assert rel_err(dev.read(out, m * n), ref) < 1e-5
    g = rng.standard_normal(m * n).astype(np.float32)
    dg = up(dev, g)
    gw = dev.empty(c * k * k * n)
    dev.call("axis_conv2d_backward_weight", dx.vp, None, dg.vp, gw.vp, I64(b), I32(h), I32(w), I32(c), I32(n), *geo)
    assert rel_err(dev.read(gw, c * k * k * n), oracle.matmul_right_backward(patches, g, 1, m, c * k * k, n)) < 1e-5
    gx = dev.empty(b * h * w * c)
    if s == 1:
        dev.call("axis_conv2d_backward_data", dg.vp, dw.vp, gx.vp, I64(b), I32(h), I32(w), I32(c), I32(n), *geo)
        ref_dx = oracle.unfold2d_backward(oracle.matmul_left_backward(g, weight, 1, m, c * k * k, n), u, len(x))
        assert rel_err(dev.read(gx, len(x)), ref_dx) < 1e-5
    else:
        with pytest.raises(hip.AxisError, match="stride 1"):
            dev.call("axis_conv2d_backward_data", dg.vp, dw.vp, gx.vp, I64(b), I32(h), I32(w), I32(c), I32(n), *geo)


def _oracle_conv(oracle, x, weight, bias, dims, b, c, n, k, s, p, oh, ow):
    """unfold -> matmul -> + bias on the CPU oracle; returns (pre-activation [m, n], patches)."""
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("group", 1),
                           ("patch", c * k * k), [k, k], [s, s], [p, p], 0.0)
    m = b * oh * ow
    patches = oracle.unfold2d(x, u)
    z = oracle.matmul(patches, weight, 1, m, c * k * k, n)
    if bias is not None:
        z = oracle.binary(z, np.tile(bias, m), 0)
    return z, patches


def _first_max(windows):
    """The reference's pool winner: first strictly greater finite value in window order (255 and
    NaN when none); windows [..., positions]."""
    w = np.where(np.isfinite(windows), windows, -np.inf)
    best = w.max(axis=-1)
    arg = np.argmax(w == best[..., None], axis=-1).astype(np.uint8)
    none = ~np.isfinite(windows).any(axis=-1)
    arg[none] = 255
    return np.where(none, np.nan, best).astype(np.float32), arg


def _windows(y, b, oh, ow, n, ph, pw):
    t = y.reshape(b, oh // ph, ph, ow // pw, pw, n).transpose(0, 1, 3, 5, 2, 4)
    return t.reshape(b, oh // ph, ow // pw, n, ph * pw)


def test_conv2d_channel_major_input(dev, oracle):
    # conv1 of the CNN: [batch, channel, height, width] input gathered through its strides
    b, c, h, w, n, k = 2, 3, 17, 12, 64, 3
    rng = np.random.default_rng(31)
    x = rng.uniform(0, 1, b * c * h * w).astype(np.float32)
    weight = rng.standard_normal(c * k * k * n).astype(np.float32) * 0.2
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    dims = [("batch", b), ("c", c), ("height", h), ("width", w)]
    z, patches = _oracle_conv(oracle, x, weight, bias, dims, b, c, n, k, 1, 1, h, w)
    m = b * h * w
    strides = (I64 * 4)(c * h * w, h * w, w, 1)
    geo = [(I32 * 2)(k, k), (I32 * 2)(1, 1), (I32 * 2)(1, 1)]
    dx, dw, db, out = up(dev, x), up(dev, weight), up(dev, bias), dev.empty(m * n)
    dev.call("axis_conv2d_forward", dx.vp, strides, dw.vp, db.vp, out.vp, I64(b), I32(h), I32(w), I32(c),
             I32(n), *geo)
    assert rel_err(dev.read(out, m * n), z) < 1e-5
    g = rng.standard_normal(m * n).astype(np.float32)
    dg, gw = up(dev, g), dev.empty(c * k * k * n)
    dev.call("axis_conv2d_backward_weight", dx.vp, strides, dg.vp, gw.vp, I64(b), I32(h), I32(w), I32(c),
             I32(n), *geo)
    assert rel_err(dev.read(gw, c * k * k * n), oracle.matmul_right_backward(patches, g, 1, m, c * k * k, n)) < 1e-5


FUSED_CASES = [
    # layout, b, c, h, w, n, pool
    ("nchw", 2, 3, 16, 16, 64, (2, 2)),   # conv1 of the CNN
    ("nhwc", 3, 64, 8, 8, 128, (2, 2)),   # conv3-like, large tiles
    ("nhwc", 2, 5, 8, 8, 20, (2, 2)),     # scalar gathers, partial column tile
    ("nhwc", 2, 8, 8, 8, 72, (2, 4)),     # wide windows, two column tiles
    ("nhwc", 2, 64, 32, 32, 128, (2, 2)), # conv2-like: 32-wide output, windows pooled in registers
    ("nhwc", 2, 16, 16, 16, 256, (2, 2)), # 16-wide output in registers, two column tiles
    ("nchw", 2, 3, 64, 64, 64, (2, 2)),   # conv1 at full image size (short reduction)
    ("nchw", 1, 3, 14, 72, 96, (2, 2)),   # short reduction: 36 windows per row, partial column group
    ("nhwc", 2, 2, 6, 10, 32, (2, 2)),    # short reduction, bands of several window rows
]


@pytest.mark.parametrize("case", range(len(FUSED_CASES)))
def test_conv2d_relu_pool_forward(dev, oracle, case):
    layout, b, c, h, w, n, (ph, pw) = FUSED_CASES[case]
    k = 3
    rng = np.random.default_rng(40 + case)
    x = rng.standard_normal(b * c * h * w).astype(np.float32)
    weight = rng.standard_normal(c * k * k * n).astype(np.float32) * 0.2
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    bias[0] = np.inf    # every ReLU output infinite: no finite winner -> NaN, 255
    bias[1] = -np.inf   # every ReLU output 0: the first position wins with 0
    if layout == "nchw":
        dims = [("batch", b), ("c", c), ("height", h), ("width", w)]
        strides = (I64 * 4)(c * h * w, h * w, w, 1)
    else:
        dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
        strides = None
    z, _ = _oracle_conv(oracle, x, weight, bias, dims, b, c, n, k, 1, 1, h, w)
    y = np.where(z > 0, z, np.float32(0))
    ref, ref_arg = _first_max(_windows(y, b, h, w, n, ph, pw))
    ref, ref_arg = ref.reshape(-1), ref_arg.reshape(-1)
    pooled_len = len(ref)
    geo = [(I32 * 2)(k, k), (I32 * 2)(1, 1), (I32 * 2)(1, 1)]
    dx, dw, db = up(dev, x), up(dev, weight), up(dev, bias)
    pooled, arg = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
    dev.call("axis_conv2d_relu_pool_forward", dx.vp, strides, dw.vp, db.vp, pooled.vp, arg.vp, I64(b), I32(h),
             I32(w), I32(c), I32(n), *geo, (I32 * 2)(ph, pw))
    got, got_arg = dev.read(pooled, pooled_len), dev.read(arg, pooled_len, np.uint8)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == pooled_len // n
    scale = np.abs(np.where(np.isfinite(z), z, 0)).max()
    assert np.abs(got[~nan] - ref[~nan]).max() <= 1e-5 * scale
    assert np.array_equal(got_arg[nan], ref_arg[nan])
    # winners must agree wherever the window's best beats its runner-up by more than rounding
    wins = _windows(np.where(np.isfinite(y), y, -np.inf), b, h, w, n, ph, pw).reshape(pooled_len, -1)
    top2 = np.sort(wins, axis=-1)[:, -2:]
    top2 = np.where(np.isfinite(top2), top2, 0.0)  # all-infinite windows are NaN outputs, checked above
    all_negative = (_windows(z, b, h, w, n, ph, pw).reshape(pooled_len, -1) < -1e-4 * scale).all(axis=-1)
    clear = ((top2[:, 1] - top2[:, 0] > 1e-4 * scale) | all_negative) & ~nan
    assert np.all(got_arg[all_negative] == 0) and np.all(got[all_negative] == 0)
    assert clear.mean() > 0.5
    assert np.array_equal(got_arg[clear], ref_arg[clear])
    # bit-identical to the separate GPU entries when the plain forward runs unsplit (k < 256)
    if c * k * k < 256:
        zz = dev.empty(b * h * w * n)
        dev.call("axis_conv2d_forward", dx.vp, strides, dw.vp, db.vp, zz.vp, I64(b), I32(h), I32(w), I32(c),
                 I32(n), *geo)
        yy = dev.empty(b * h * w * n)
        dev.call("axis_relu", zz.vp, yy.vp, I64(b * h * w * n))
        p2, a2 = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
        dev.call("axis_max_pool2d", yy.vp, p2.vp, a2.vp, I64(b), I32(h), I32(w), I64(n), (I32 * 2)(ph, pw),
                 (I32 * 2)(ph, pw), (I32 * 2)(0, 0))
        p2v = dev.read(p2, pooled_len)
        assert np.array_equal(np.isnan(p2v), np.isnan(got))
        assert np.array_equal(p2v[~nan], got[~nan])
        assert np.array_equal(dev.read(a2, pooled_len, np.uint8), got_arg)


FIXED_GEOMETRY_CASES = [
    # layout, b, c, h, w, n: 3x3 under padding 1 over 1 or 3 channels, windows at least 25 columns
    # wide, whole 64-column groups -- the shapes the fixed-geometry kernels take
    ("nchw", 2, 3, 64, 64, 64),   # conv1 of the CNN
    ("nchw", 1, 3, 14, 72, 128),  # 36 windows per row (a partial second band), 7 window rows, two groups
    ("nhwc", 2, 1, 50, 52, 64),   # one channel, 26 windows per row (a partial band), 25 window rows
]


@pytest.mark.parametrize("values", ["normal", "ties", "special"])
@pytest.mark.parametrize("case", range(len(FIXED_GEOMETRY_CASES)))
def test_conv2d_relu_pool_forward_fixed_geometry(dev, oracle, case, values):
    """The fused forward on the fixed-geometry kernels is bit-identical to the separate GPU entries
    (plain convolution, ReLU, max pool; the pool rule is bit-exact against the oracle in
    test_relu_pool_backward_bit_exact and its neighbours) on both pooling paths: the bit-pattern
    comparison ("normal", "ties": exact integer pre-activations with tied maxima, zeros and
    all-negative windows) and the exact scan that tiles holding +inf or NaN take ("special")."""
    layout, b, c, h, w, n = FIXED_GEOMETRY_CASES[case]
    k = 3
    rng = np.random.default_rng(90 + case)
    size = b * c * h * w
    if values == "ties":
        x = rng.integers(-2, 3, size).astype(np.float32)
        weight = rng.integers(-1, 2, c * k * k * n).astype(np.float32)
        bias = rng.integers(-1, 2, n).astype(np.float32)
    else:
        x = rng.standard_normal(size).astype(np.float32)
        weight = rng.standard_normal(c * k * k * n).astype(np.float32) * 0.2
        bias = rng.standard_normal(n).astype(np.float32) * 0.1
    if values == "special":
        cells = rng.choice(size, 30, replace=False)
        x[cells[:10]], x[cells[10:20]], x[cells[20:]] = np.nan, np.inf, -np.inf
    if layout == "nchw":
        dims = [("batch", b), ("c", c), ("height", h), ("width", w)]
        strides = (I64 * 4)(c * h * w, h * w, w, 1)
    else:
        dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
        strides = None
    geo = [(I32 * 2)(k, k), (I32 * 2)(1, 1), (I32 * 2)(1, 1)]
    pooled_len = b * (h // 2) * (w // 2) * n
    dx, dw, db = up(dev, x), up(dev, weight), up(dev, bias)
    pooled, arg = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
    dev.call("axis_conv2d_relu_pool_forward", dx.vp, strides, dw.vp, db.vp, pooled.vp, arg.vp, I64(b), I32(h),
             I32(w), I32(c), I32(n), *geo, (I32 * 2)(2, 2))
    got, got_arg = dev.read(pooled, pooled_len), dev.read(arg, pooled_len, np.uint8)
    zz, yy = dev.empty(b * h * w * n), dev.empty(b * h * w * n)
    dev.call("axis_conv2d_forward", dx.vp, strides, dw.vp, db.vp, zz.vp, I64(b), I32(h), I32(w), I32(c), I32(n),
             *geo)
    dev.call("axis_relu", zz.vp, yy.vp, I64(b * h * w * n))
    p2, a2 = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
    dev.call("axis_max_pool2d", yy.vp, p2.vp, a2.vp, I64(b), I32(h), I32(w), I64(n), (I32 * 2)(2, 2),
             (I32 * 2)(2, 2), (I32 * 2)(0, 0))
    want, want_arg = dev.read(p2, pooled_len), dev.read(a2, pooled_len, np.uint8)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.array_equal(got_arg, want_arg)
    if values == "ties":
        z = dev.read(zz, b * h * w * n)
        wins = _windows(z, b, h, w, n, 2, 2).reshape(pooled_len, 4)
        tied = ((wins == wins.max(axis=1, keepdims=True)).sum(axis=1) > 1) & (wins.max(axis=1) > 0)
        assert tied.mean() > 0.05 and (wins.max(axis=1) <= 0).mean() > 0.05  # both cases are exercised
    if values == "special":
        assert 0 < nan.sum() and np.isinf(got).sum() == 0  # +inf outputs have no finite winner: NaN
        assert (~np.isfinite(dev.read(zz, b * h * w * n))).any()
    if values == "normal":
        z, _ = _oracle_conv(oracle, x, weight, bias, dims, b, c, n, k, 1, 1, h, w)
        ref, _ = _first_max(_windows(np.where(z > 0, z, np.float32(0)), b, h, w, n, 2, 2))
        assert np.abs(got - ref.reshape(-1)).max() <= 1e-5 * np.abs(z).max()


def test_conv2d_relu_pool_rejects_partial_windows(dev):
    buf = dev.empty(4096)
    arg = dev.empty(4096, np.uint8)
    geo = [(I32 * 2)(3, 3), (I32 * 2)(1, 1), (I32 * 2)(1, 1)]
    with pytest.raises(hip.AxisError, match="tile the convolution output"):
        dev.call("axis_conv2d_relu_pool_forward", buf.vp, None, buf.vp, None, buf.vp, arg.vp, I64(1), I32(7),
                 I32(8), I32(4), I32(8), *geo, (I32 * 2)(2, 2))
    with pytest.raises(hip.AxisError, match="divide 128"):
        dev.call("axis_conv2d_relu_pool_forward", buf.vp, None, buf.vp, None, buf.vp, arg.vp, I64(1), I32(8),
                 I32(96), I32(4), I32(8), *geo, (I32 * 2)(2, 2))


RELU_POOL_WGRAD_CASES = [
    # layout, b, c, h, w, n, padding, bias
    ("nchw", 2, 3, 16, 16, 64, 1, True),    # conv1 of the CNN (short reduction, fused)
    ("nchw", 1, 3, 64, 64, 64, 1, True),    # conv1 at full image size
    ("nhwc", 3, 2, 12, 20, 96, 1, True),    # two column groups, the second partial
    ("nchw", 2, 1, 10, 70, 32, 1, False),   # 35 windows per row: two bands across; no bias
    ("nchw", 2, 3, 18, 18, 64, 0, True),    # no padding
    ("nhwc", 2, 8, 8, 8, 16, 1, True),      # 72-term reduction: composed from the separate entries
    # the fixed-geometry kernel: 3x3 over 1 or 3 channels, windows >= 25 columns, 64-column groups
    ("nchw", 1, 3, 14, 72, 128, 1, True),   # 36 windows per row: a partial second band; two groups
    ("nhwc", 2, 1, 50, 52, 64, 1, False),   # one channel, 26 windows per row (a partial band)
    ("nchw", 2, 3, 66, 66, 64, 0, True),    # no padding
]


@pytest.mark.parametrize("case", range(len(RELU_POOL_WGRAD_CASES)))
def test_conv2d_relu_pool_backward_weight(dev, oracle, case):
    layout, b, c, h, w, n, p, with_bias = RELU_POOL_WGRAD_CASES[case]
    k = 3
    oh, ow = h + 2 * p - k + 1, w + 2 * p - k + 1
    rng = np.random.default_rng(70 + case)
    x = rng.uniform(-1, 1, b * c * h * w).astype(np.float32)
    weight = rng.standard_normal(c * k * k * n).astype(np.float32) * 0.3
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    if layout == "nchw":
        dims = [("batch", b), ("c", c), ("height", h), ("width", w)]
        strides = (I64 * 4)(c * h * w, h * w, w, 1)
    else:
        dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
        strides = None
    geo = [(I32 * 2)(k, k), (I32 * 2)(1, 1), (I32 * 2)(p, p)]
    win = (I32 * 2)(2, 2)
    pooled_len = b * (oh // 2) * (ow // 2) * n
    dx, dw, db = up(dev, x), up(dev, weight), up(dev, bias)
    pooled, arg = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
    dev.call("axis_conv2d_relu_pool_forward", dx.vp, strides, dw.vp, db.vp, pooled.vp, arg.vp, I64(b), I32(h),
             I32(w), I32(c), I32(n), *geo, win)
    pv, av = dev.read(pooled, pooled_len), dev.read(arg, pooled_len, np.uint8)
    g = rng.standard_normal(pooled_len).astype(np.float32)
    g[::13] = 0.0
    dg = up(dev, g)
    # the pre-activation gradient the pooled tensors imply: g at each positive window's winner
    d_pre = np.zeros((b, oh // 2, ow // 2, n, 4), np.float32)
    sel = (pv > 0).reshape(b, oh // 2, ow // 2, n)
    a4 = av.reshape(b, oh // 2, ow // 2, n)
    for pos in range(4):
        d_pre[..., pos] = np.where(sel & (a4 == pos), np.float32(0) + g.reshape(b, oh // 2, ow // 2, n), 0.0)
    d_pre = d_pre.reshape(b, oh // 2, ow // 2, n, 2, 2).transpose(0, 1, 4, 2, 5, 3).reshape(-1)
    _, patches = _oracle_conv(oracle, x, weight, None, dims, b, c, n, k, 1, p, oh, ow)
    m = b * oh * ow
    ref_w = oracle.matmul_right_backward(patches, d_pre, 1, m, c * k * k, n)
    ref_b = oracle.bias_gradient(d_pre, m, n)
    gw, gb = dev.empty(c * k * k * n), dev.empty(n)
    dev.call("axis_conv2d_relu_pool_backward_weight", dx.vp, strides, dg.vp, pooled.vp, arg.vp, gw.vp,
             gb.vp if with_bias else None, I64(b), I32(h), I32(w), I32(c), I32(n), *geo, win)
    got_w = dev.read(gw, c * k * k * n)
    assert rel_err(got_w, ref_w) < 1e-5
    if with_bias:
        got_b = dev.read(gb, n)
        mag = np.abs(d_pre.reshape(-1, n)).sum(axis=0).astype(np.float64)
        assert np.all(np.abs(got_b.astype(np.float64) - ref_b) <= 2e-6 * mag + 1e-30)
    # the same as the separate entries (pre-activation gradient, then weight gradient)
    pre, sep_b, sep_w = dev.empty(m * n), dev.empty(n), dev.empty(c * k * k * n)
    dev.call("axis_relu_pool_backward", dg.vp, pooled.vp, arg.vp, pre.vp, sep_b.vp, I64(b), I32(oh), I32(ow),
             I32(n), win)
    assert np.array_equal(dev.read(pre, m * n).view(np.uint32), d_pre.view(np.uint32))
    dev.call("axis_conv2d_backward_weight", dx.vp, strides, pre.vp, sep_w.vp, I64(b), I32(h), I32(w), I32(c),
             I32(n), *geo)
    assert rel_err(got_w, dev.read(sep_w, c * k * k * n)) < 1e-5
    # deterministic run to run
    gw2 = dev.empty(c * k * k * n)
    dev.call("axis_conv2d_relu_pool_backward_weight", dx.vp, strides, dg.vp, pooled.vp, arg.vp, gw2.vp, None,
             I64(b), I32(h), I32(w), I32(c), I32(n), *geo, win)
    assert np.array_equal(dev.read(gw2, c * k * k * n).view(np.uint32), got_w.view(np.uint32))


@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_conv2d_relu_pool_backward_weight_nonfinite_input(dev, layout):
    # conv1's weight gradient through the pool's winners adds g * x at each window's winner only; a
    # band with a non-finite input also adds the other positions' 0 * x, so NaN and inf reach the
    # sums as in the dense product over the pre-activation gradient (the separate entries).  At 64 x 64
    # with padding 1 every input pixel lies in some pooling window, so both see the same terms.
    b, c, h, w, n, k, p = 1, 3, 64, 64, 64, 3, 1
    rng = np.random.default_rng(91)
    x = rng.uniform(-1, 1, b * c * h * w).astype(np.float32)
    x[[5, 300, 4100]] = [np.inf, np.nan, -np.inf]  # channels 0 and 1; channel 2's terms stay finite
    weight = rng.standard_normal(c * k * k * n).astype(np.float32) * 0.3
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    if layout == "nchw":
        strides = (I64 * 4)(c * h * w, h * w, w, 1)
    else:
        x = x.reshape(b, c, h, w).transpose(0, 2, 3, 1).copy().reshape(-1)
        strides = None
    geo = [(I32 * 2)(k, k), (I32 * 2)(1, 1), (I32 * 2)(p, p)]
    win = (I32 * 2)(2, 2)
    pooled_len = b * (h // 2) * (w // 2) * n
    dx, dw, db = up(dev, x), up(dev, weight), up(dev, bias)
    pooled, arg = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
    dev.call("axis_conv2d_relu_pool_forward", dx.vp, strides, dw.vp, db.vp, pooled.vp, arg.vp, I64(b), I32(h),
             I32(w), I32(c), I32(n), *geo, win)
    dg = up(dev, rng.standard_normal(pooled_len).astype(np.float32))
    gw = dev.empty(c * k * k * n)
    dev.call("axis_conv2d_relu_pool_backward_weight", dx.vp, strides, dg.vp, pooled.vp, arg.vp, gw.vp, None,
             I64(b), I32(h), I32(w), I32(c), I32(n), *geo, win)
    m = b * h * w
    pre, sep_b, sep_w = dev.empty(m * n), dev.empty(n), dev.empty(c * k * k * n)
    dev.call("axis_relu_pool_backward", dg.vp, pooled.vp, arg.vp, pre.vp, sep_b.vp, I64(b), I32(h), I32(w),
             I32(n), win)
    dev.call("axis_conv2d_backward_weight", dx.vp, strides, pre.vp, sep_w.vp, I64(b), I32(h), I32(w), I32(c),
             I32(n), *geo)
    got, ref = dev.read(gw, c * k * k * n), dev.read(sep_w, c * k * k * n)
    assert np.isnan(ref).any()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref)) and np.array_equal(got[np.isinf(got)], ref[np.isinf(ref)])
    fin = np.isfinite(ref)
    assert rel_err(got[fin], ref[fin]) < 1e-5


@pytest.mark.parametrize("b,h,w,c,pool", [(5, 16, 18, 64, (2, 2)), (3, 10, 12, 6, (2, 3)), (2, 8, 8, 20, (4, 4)),
                                          (64, 32, 32, 128, (2, 2)), (4, 8, 8, 16, (2, 2))])
def test_relu_pool_backward_bit_exact(dev, oracle, b, h, w, c, pool):
    rng = np.random.default_rng(h * w + c)
    z = rng.integers(-3, 4, b * h * w * c).astype(np.float32) * 0.5  # ties and exact zeros
    z[::37] = np.nan
    y = oracle.relu(z)
    n_in = len(z)
    ph, pw = pool
    n_out = n_in // (ph * pw)
    win = (I32 * 2)(ph, pw)
    dy, pooled, arg = up(dev, y), dev.empty(n_out), dev.empty(n_out, np.uint8)
    dev.call("axis_max_pool2d", dy.vp, pooled.vp, arg.vp, I64(b), I32(h), I32(w), I64(c), win, win,
             (I32 * 2)(0, 0))
    g = rng.standard_normal(n_out).astype(np.float32)
    g[::11] = -0.0
    dg, back = up(dev, g), dev.empty(n_in)
    dev.call("axis_max_pool2d_backward", dg.vp, arg.vp, back.vp, I64(b), I32(h), I32(w), I64(c), win, win,
             (I32 * 2)(0, 0))
    expected = oracle.relu_backward(dev.read(back, n_in), z)
    expected_db = oracle.bias_gradient(expected, b * h * w, c)
    d_pre, d_bias = dev.empty(n_in), dev.empty(c)
    dev.call("axis_relu_pool_backward", dg.vp, pooled.vp, arg.vp, d_pre.vp, d_bias.vp, I64(b), I32(h), I32(w),
             I32(c), win)
    got = dev.read(d_pre, n_in)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
    got_db = dev.read(d_bias, c)
    exact = 256 % (c // 4 if c % 4 == 0 else c) != 0  # reference chunk order unless folded into the scatter
    if exact:
        assert np.array_equal(got_db.view(np.uint32), expected_db.view(np.uint32))
    else:
        # fixed per-block tree: fp32 tolerance against the chunked sum, scaled by the sum of |terms|
        mag = np.abs(expected.reshape(-1, c)).sum(axis=0).astype(np.float64)
        assert np.all(np.abs(got_db.astype(np.float64) - expected_db) <= 1e-6 * mag + 1e-30)
    # run-to-run determinism
    d_bias2 = dev.empty(c)
    dev.call("axis_relu_pool_backward", dg.vp, pooled.vp, arg.vp, d_pre.vp, d_bias2.vp, I64(b), I32(h), I32(w),
             I32(c), win)
    assert np.array_equal(dev.read(d_bias2, c).view(np.uint32), got_db.view(np.uint32))


@pytest.mark.parametrize("b,h,w,c,pool", [(256, 16, 16, 256, (2, 2)), (3, 10, 12, 6, (2, 3)), (2, 8, 8, 20, (4, 4))])
def test_relu_pool_backward_mean_equals_broadcast_then_backward(dev, b, h, w, c, pool):
    # the backward of mean([h, w]) over the pooled tensor folded into the ReLU/pool backward: the
    # same bits as axis_broadcast_middle then axis_relu_pool_backward (CNN conv3 shape first)
    rng = np.random.default_rng(b + h + w + c)
    z = (rng.integers(-3, 4, b * h * w * c).astype(np.float32) * 0.5)
    y = np.maximum(z, 0).astype(np.float32)
    ph, pw = pool
    n_in, n_out = len(z), len(z) // (ph * pw)
    positions = n_out // (b * c)
    win = (I32 * 2)(ph, pw)
    dy, pooled, arg = up(dev, y), dev.empty(n_out), dev.empty(n_out, np.uint8)
    dev.call("axis_max_pool2d", dy.vp, pooled.vp, arg.vp, I64(b), I32(h), I32(w), I64(c), win, win, (I32 * 2)(0, 0))
    g = rng.standard_normal(b * c).astype(np.float32)
    g[::7] = -0.0
    factor = np.float32(1.0) / np.float32(positions)
    dg, full = up(dev, g), dev.empty(n_out)
    dev.call("axis_broadcast_middle", dg.vp, full.vp, I64(b), I64(positions), I64(c), F32(factor))
    ref, ref_db = dev.empty(n_in), dev.empty(c)
    dev.call("axis_relu_pool_backward", full.vp, pooled.vp, arg.vp, ref.vp, ref_db.vp, I64(b), I32(h), I32(w),
             I32(c), win)
    got, got_db = dev.empty(n_in), dev.empty(c)
    dev.call("axis_relu_pool_backward_mean", dg.vp, F32(factor), pooled.vp, arg.vp, got.vp, got_db.vp, I64(b),
             I32(h), I32(w), I32(c), win)
    assert np.array_equal(dev.read(got, n_in).view(np.uint32), dev.read(ref, n_in).view(np.uint32))
    assert np.array_equal(dev.read(got_db, c).view(np.uint32), dev.read(ref_db, c).view(np.uint32))


@pytest.mark.parametrize("rows,width", [(256, 1000), (3, 7), (1300, 37)])
def test_cross_entropy_backward_mean_equals_broadcast_then_backward(dev, rows, width):
    rng = np.random.default_rng(rows + width)
    logits = rng.standard_normal(rows * width).astype(np.float32)
    targets = np.zeros(rows * width, np.float32)
    targets[np.arange(rows) * width + rng.integers(0, width, rows)] = 1.0
    dl, dt = up(dev, logits), up(dev, targets)
    prob, loss = dev.empty(rows * width), dev.empty(rows)
    dev.call("axis_softmax_cross_entropy", dl.vp, dt.vp, prob.vp, loss.vp, I64(rows), I64(width))
    seed = up(dev, np.array([0.75], np.float32))
    factor = np.float32(1.0) / np.float32(rows)
    rows_g, ref, got = dev.empty(rows), dev.empty(rows * width), dev.empty(rows * width)
    dev.call("axis_broadcast_middle", seed.vp, rows_g.vp, I64(1), I64(rows), I64(1), F32(factor))
    dev.call("axis_categorical_cross_entropy_backward", rows_g.vp, prob.vp, dt.vp, ref.vp, I64(rows), I64(width))
    dev.call("axis_categorical_cross_entropy_backward_mean", seed.vp, F32(factor), prob.vp, dt.vp, got.vp, None,
             I64(rows), I64(width))
    assert np.array_equal(dev.read(got, rows * width).view(np.uint32), dev.read(ref, rows * width).view(np.uint32))
    # with the logits' bias gradient: the same values, and the column sums of axis_bias_gradient
    got2, db, ref_db = dev.empty(rows * width), dev.empty(width), dev.empty(width)
    dev.call("axis_categorical_cross_entropy_backward_mean", seed.vp, F32(factor), prob.vp, dt.vp, got2.vp, db.vp,
             I64(rows), I64(width))
    dev.call("axis_bias_gradient", ref.vp, None, None, ref_db.vp, I64(rows), I64(width))
    assert np.array_equal(dev.read(got2, rows * width).view(np.uint32), dev.read(ref, rows * width).view(np.uint32))
    assert np.array_equal(dev.read(db, width).view(np.uint32), dev.read(ref_db, width).view(np.uint32))


@pytest.mark.parametrize("batch,m,k,n", [(1, 256, 256, 256), (1, 64, 4096, 96), (2, 130, 70, 33), (1, 512, 512, 1024)])
def test_matmul_axpby_equals_separate_operations(dev, oracle, batch, m, k, n):
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    d = rng.standard_normal(batch * m * n).astype(np.float32)
    alpha, beta = 2.0315, -4.7750
    da, db, dd = up(dev, a), up(dev, b), up(dev, d)
    fused = dev.empty(batch * m * n)
    dev.call("axis_matmul_axpby", da.vp, db.vp, dd.vp, fused.vp, I64(batch), I64(m), I64(k), I64(n), F32(alpha),
             F32(beta))
    got = dev.read(fused, batch * m * n)
    # the same arithmetic through the separate entries: bit-identical
    prod, t1, t2, summed = (dev.empty(batch * m * n) for _ in range(4))
    dev.call("axis_matmul", da.vp, db.vp, prod.vp, I64(batch), I64(m), I64(k), I64(n))
    dev.call("axis_scale", dd.vp, F32(beta), t1.vp, I64(batch * m * n))
    dev.call("axis_scale", prod.vp, F32(alpha), t2.vp, I64(batch * m * n))
    dev.call("axis_binary", t1.vp, t2.vp, I32(0), summed.vp, I64(batch * m * n))
    assert np.array_equal(got.view(np.uint32), dev.read(summed, batch * m * n).view(np.uint32))
    # and the oracle to GEMM tolerance
    ref = oracle.binary(oracle.scale(d, beta), oracle.scale(oracle.matmul(a, b, batch, m, k, n), alpha), 0)
    assert rel_err(got, ref) < 1e-5


def test_matmul_axpby_rejects_aliasing(dev):
    buf = dev.empty(16)
    with pytest.raises(hip.AxisError, match="alias"):
        dev.call("axis_matmul_axpby", buf.vp, buf.vp, buf.vp, buf.vp, I64(1), I64(4), I64(4), I64(4), F32(1.0),
                 F32(1.0))


# ---------------------------------------------------------------- deferred finishing sums

def _pending(dev):
    n = ctypes.c_int64()
    dev.call("axis_finish_pending", ctypes.byref(n))
    return n.value


def _gradient_entries(dev, rng):
    """Weight and bias gradient entries whose last sums a deferring handle records: each returns
    (list of (output buffer, length)) after enqueueing its call."""
    calls = []
    for (batch, m, k, n) in [(1, 8192, 64, 48),     # split-K, one level (<= 32 slices)
                             (1, 65536, 64, 64),    # more than 32 slices: range sums first
                             (2, 4096, 96, 40),     # batched split-K
                             (1, 64, 256, 256)]:    # unsplit: nothing to defer
        lhs = up(dev, rng.standard_normal(batch * m * k).astype(np.float32))
        g = up(dev, rng.standard_normal(batch * m * n).astype(np.float32))

        def right(out, lhs=lhs, g=g, geo=(batch, m, k, n)):
            dev.call("axis_matmul_right_backward", lhs.vp, g.vp, out.vp, *map(I64, geo))
        calls.append((right, [batch * k * n]))
    # convolution weight gradient (channels need no padding: the split sum writes the result)
    b, h, w, c, n = 4, 32, 32, 64, 128
    x = up(dev, rng.standard_normal(b * h * w * c).astype(np.float32))
    gc = up(dev, rng.standard_normal(b * h * w * n).astype(np.float32))
    geo = [(I32 * 2)(3, 3), (I32 * 2)(1, 1), (I32 * 2)(1, 1)]

    def conv_w(out):
        dev.call("axis_conv2d_backward_weight", x.vp, None, gc.vp, out.vp, I64(b), I32(h), I32(w), I32(c), I32(n),
                 *geo)
    calls.append((conv_w, [c * 9 * n]))
    # ReLU/pool backward with the bias folded into the scatter (per-block partials)
    z = rng.integers(-3, 4, b * h * w * n).astype(np.float32) * 0.5
    dz = up(dev, np.maximum(z, 0).astype(np.float32))
    win = (I32 * 2)(2, 2)
    pooled, arg = dev.empty(len(z) // 4), dev.empty(len(z) // 4, np.uint8)
    dev.call("axis_max_pool2d", dz.vp, pooled.vp, arg.vp, I64(b), I32(h), I32(w), I64(n), win, win, (I32 * 2)(0, 0))
    gp = up(dev, rng.standard_normal(len(z) // 4).astype(np.float32))
    d_pre = dev.empty(len(z))

    def pool_bias(out):
        dev.call("axis_relu_pool_backward", gp.vp, pooled.vp, arg.vp, d_pre.vp, out.vp, I64(b), I32(h), I32(w),
                 I32(n), win)
    calls.append((pool_bias, [n]))
    # conv1's fused weight and bias gradient straight from the pooled gradient (one partial sum
    # feeding two outputs)
    b1, h1, c1, n1 = 2, 64, 3, 64
    x1 = up(dev, rng.standard_normal(b1 * c1 * h1 * h1).astype(np.float32))
    s1 = (I64 * 4)(c1 * h1 * h1, h1 * h1, h1, 1)
    w1 = up(dev, rng.standard_normal(c1 * 9 * n1).astype(np.float32) * 0.2)
    bias1 = up(dev, rng.standard_normal(n1).astype(np.float32) * 0.1)
    pooled1, arg1 = dev.empty(b1 * 32 * 32 * n1), dev.empty(b1 * 32 * 32 * n1, np.uint8)
    dev.call("axis_conv2d_relu_pool_forward", x1.vp, s1, w1.vp, bias1.vp, pooled1.vp, arg1.vp, I64(b1), I32(h1),
             I32(h1), I32(c1), I32(n1), *geo, win)
    g1 = up(dev, rng.standard_normal(b1 * 32 * 32 * n1).astype(np.float32))

    def conv1_wb(out_w, out_b):
        dev.call("axis_conv2d_relu_pool_backward_weight", x1.vp, s1, g1.vp, pooled1.vp, arg1.vp, out_w.vp, out_b.vp,
                 I64(b1), I32(h1), I32(h1), I32(c1), I32(n1), *geo, win)
    calls.append((conv1_wb, [c1 * 9 * n1, n1]))
    return calls


def test_deferred_finishing_sums_are_bit_identical(dev):
    # every entry's outputs with the last sums deferred and run in one batched launch: the same bits
    # as the entry run alone; outputs hold their old contents until the flush
    rng = np.random.default_rng(2024)
    calls = _gradient_entries(dev, rng)
    ref = []
    for fn, lens in calls:
        outs = [dev.empty(n) for n in lens]
        fn(*outs)
        ref.append([dev.read(o, n) for o, n in zip(outs, lens)])
    assert _pending(dev) == 0
    sentinel = np.float32(-7.25)
    got = []
    dev.call("axis_finish_defer", I32(1))
    try:
        for fn, lens in calls:
            outs = [dev.empty(n) for n in lens]
            for o, n in zip(outs, lens):
                dev.call("axis_fill", o.vp, F32(sentinel), I64(n))
            fn(*outs)
            got.append(outs)
        # one task per split product (not the unsplit one), the convolution, the pool bias and conv1
        assert _pending(dev) == 3 + 1 + 1 + 1
        # a read of an unrelated buffer leaves them pending; one of a pending output runs them all
        other = dev.empty(16)
        dev.call("axis_finish_before_read", other.vp, ctypes.c_size_t(64))
        assert _pending(dev) == 6
        dev.call("axis_finish_before_read", got[1][0].vp, ctypes.c_size_t(4))
        assert _pending(dev) == 0
    finally:
        dev.call("axis_finish_defer", I32(0))
    for r, outs, (fn, lens) in zip(ref, got, calls):
        for expected, o, n in zip(r, outs, lens):
            assert np.array_equal(dev.read(o, n).view(np.uint32), expected.view(np.uint32))


def test_deferred_finishing_sums_flush_on_read_free_and_overflow(dev):
    # axis_read of a pending output runs the batch; more tasks than one launch carries flush early;
    # freeing a pending output runs its sum before the block is reused
    rng = np.random.default_rng(7)
    m, k, n = 8192, 32, 24
    lhs = up(dev, rng.standard_normal(m * k).astype(np.float32))
    g = up(dev, rng.standard_normal(m * n).astype(np.float32))
    geo = (I64(1), I64(m), I64(k), I64(n))
    ref = dev.empty(k * n)
    dev.call("axis_matmul_right_backward", lhs.vp, g.vp, ref.vp, *geo)
    expected = dev.read(ref, k * n)
    dev.call("axis_finish_defer", I32(1))
    try:
        outs = []
        for i in range(30):
            o = dev.empty(k * n)
            dev.call("axis_matmul_right_backward", lhs.vp, g.vp, o.vp, *geo)
            outs.append(o)
        assert 0 < _pending(dev) < 30
        got = dev.read(outs[-1], k * n)   # flushes
        assert _pending(dev) == 0
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
        for o in outs:
            assert np.array_equal(dev.read(o, k * n).view(np.uint32), expected.view(np.uint32))
        tmp = dev.empty(k * n)
        dev.call("axis_matmul_right_backward", lhs.vp, g.vp, tmp.vp, *geo)
        assert _pending(dev) == 1
        del tmp                            # axis_free of a pending output
        assert _pending(dev) == 0
        tmp = dev.empty(k * n)
        dev.call("axis_matmul_right_backward", lhs.vp, g.vp, tmp.vp, *geo)
        assert _pending(dev) == 1
        dev.call("axis_fill", tmp.vp, F32(3.0), I64(k * n))   # a later write into it wins
        assert _pending(dev) == 0
        assert np.all(dev.read(tmp, k * n) == 3.0)
    finally:
        dev.call("axis_finish_defer", I32(0))


def test_kernel_entries_run_a_pending_sum_before_touching_its_output(dev, oracle):
    # any compute entry given a buffer a pending finishing sum writes (as input or output) runs the
    # batch first: the reader sees the finished gradient, a later writer's values win; entries on
    # other buffers leave the batch pending
    rng = np.random.default_rng(11)
    m, k, n = 8192, 32, 24
    lhs = up(dev, rng.standard_normal(m * k).astype(np.float32))
    g = up(dev, rng.standard_normal(m * n).astype(np.float32))
    geo = (I64(1), I64(m), I64(k), I64(n))
    ref = dev.empty(k * n)
    dev.call("axis_matmul_right_backward", lhs.vp, g.vp, ref.vp, *geo)
    expected = dev.read(ref, k * n)
    other_in, other_out = up(dev, np.ones(64, np.float32)), dev.empty(64)
    dev.call("axis_finish_defer", I32(1))
    try:
        pend = dev.empty(k * n)
        dev.call("axis_matmul_right_backward", lhs.vp, g.vp, pend.vp, *geo)
        assert _pending(dev) == 1
        dev.call("axis_scale", other_in.vp, F32(2.0), other_out.vp, I64(64))      # unrelated
        assert _pending(dev) == 1
        scaled = dev.empty(k * n)
        dev.call("axis_scale", pend.vp, F32(2.0), scaled.vp, I64(k * n))          # reads it
        assert _pending(dev) == 0
        assert np.array_equal(dev.read(scaled, k * n), np.float32(2.0) * expected)
        # an Adam update whose gradient is pending
        p0 = up(dev, np.zeros(k * n, np.float32))
        m0, v0 = up(dev, np.zeros(k * n, np.float32)), up(dev, np.zeros(k * n, np.float32))
        dev.call("axis_matmul_right_backward", lhs.vp, g.vp, pend.vp, *geo)
        assert _pending(dev) == 1
        table = (hip.AdamTensor * 1)(hip.AdamTensor(p0.ptr, pend.ptr, m0.ptr, v0.ptr, None, k * n))
        dev.call("axis_adam_multi", table, I32(1), F32(1e-3), F32(0.9), F32(0.999), F32(0.1), F32(0.001),
                 F32(1e-8), F32(0.0))
        assert _pending(dev) == 0
        # a pending output overwritten by another entry keeps the later values
        dev.call("axis_matmul_right_backward", lhs.vp, g.vp, pend.vp, *geo)
        dev.call("axis_relu", other_in.vp, VP(pend.ptr), I64(64))
        assert _pending(dev) == 0
        got = dev.read(pend, k * n)
        assert np.all(got[:64] == 1.0) and np.array_equal(got[64:], expected[64:])
    finally:
        dev.call("axis_finish_defer", I32(0))
    zero = np.zeros(k * n, np.float32)
    want_p, want_m, want_v = oracle.adam(zero, expected, zero, zero, 1e-3, 0.9, 0.999, 0.1, 0.001, 1e-8, 0.0)
    for buf, want in ((p0, want_p), (m0, want_m), (v0, want_v)):
        assert np.array_equal(dev.read(buf, k * n).view(np.uint32), want.view(np.uint32))


def test_deferred_finishing_sums_flush_past_the_held_byte_limit(dev):
    # large split weight gradients deferred one after another: the batch is launched once the
    # partial blocks it holds pass 256 MiB, well before the 24-task limit, with the same bits
    rng = np.random.default_rng(12)
    m, k, n = 65536, 1024, 1024
    lhs = up(dev, rng.standard_normal(m * k).astype(np.float32))
    g = up(dev, rng.standard_normal(m * n).astype(np.float32))
    geo = (I64(1), I64(m), I64(k), I64(n))
    ref = dev.empty(k * n)
    dev.call("axis_matmul_right_backward", lhs.vp, g.vp, ref.vp, *geo)
    expected = dev.read(ref, k * n)
    outs, most = [], 0
    dev.call("axis_finish_defer", I32(1))
    try:
        for _ in range(20):
            o = dev.empty(k * n)
            dev.call("axis_matmul_right_backward", lhs.vp, g.vp, o.vp, *geo)
            outs.append(o)
            most = max(most, _pending(dev))
    finally:
        dev.call("axis_finish_defer", I32(0))
    assert _pending(dev) == 0 and 1 <= most < 20, most
    for o in outs:
        assert np.array_equal(dev.read(o, k * n).view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("m,k,n", [(8192, 64, 48), (65536, 16, 20), (4096, 7, 9)])
def test_split_sums_vector_and_scalar_forms_agree(dev, m, k, n):
    # a split weight gradient into a 16-byte aligned output (four outputs per lane when k*n % 4 == 0)
    # and into one 4 bytes off (one output per lane): the same bits
    rng = np.random.default_rng(m + k + n)
    lhs = up(dev, rng.standard_normal(m * k).astype(np.float32))
    g = up(dev, rng.standard_normal(m * n).astype(np.float32))
    geo = (I64(1), I64(m), I64(k), I64(n))
    aligned, shifted = dev.empty(k * n), dev.empty(k * n + 1)
    dev.call("axis_matmul_right_backward", lhs.vp, g.vp, aligned.vp, *geo)
    dev.call("axis_matmul_right_backward", lhs.vp, g.vp, VP(shifted.ptr + 4), *geo)
    a = dev.read(aligned, k * n)
    b = dev.read(shifted, k * n + 1)[1:]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ref = np.asarray(dev.read(lhs, m * k), np.float64).reshape(m, k).T @ np.asarray(dev.read(g, m * n), np.float64).reshape(m, n)
    assert rel_err(a, ref.reshape(-1)) < 1e-5


@pytest.mark.parametrize("length", [4096 * 1000 + 3, 7, 1])
def test_muon_elementwise_entries_equal_the_op_sequence(dev, length):
    # model/optim.rs:644-669 as separate scale / add / sub launches against the fused passes: the
    # same bits, with and without a previous momentum and with and without Nesterov
    rng = np.random.default_rng(length)
    g = up(dev, rng.standard_normal(length).astype(np.float32))
    prev = up(dev, rng.standard_normal(length).astype(np.float32))
    p = up(dev, rng.standard_normal(length).astype(np.float32))
    o = up(dev, rng.standard_normal(length).astype(np.float32))
    momentum, n = np.float32(0.95), I64(length)
    observation = np.float32(1.0) - momentum

    def seq_scale(src, f):
        out = dev.empty(length)
        dev.call("axis_scale", src.vp, F32(f), out.vp, n)
        return out

    def seq_binary(a, b, op):
        out = dev.empty(length)
        dev.call("axis_binary", a.vp, b.vp, I32(op), out.vp, n)
        return out

    read = lambda b: dev.read(b, length).view(np.uint32)
    for has_prev in (True, False):
        t2 = seq_scale(g, observation)
        ref_next = seq_binary(seq_scale(prev, momentum), t2, 0) if has_prev else t2
        ref_dir = seq_binary(seq_scale(g, observation), seq_scale(ref_next, momentum), 0)
        for nesterov in (1, 0):
            nxt, d = dev.empty(length), dev.empty(length)
            dev.call("axis_muon_momentum", g.vp, prev.vp if has_prev else None, nxt.vp, d.vp if nesterov else None,
                     F32(momentum), I32(nesterov), n)
            assert np.array_equal(read(nxt), read(ref_next))
            if nesterov:
                assert np.array_equal(read(d), read(ref_dir))
    lr, wd, scaling = np.float32(0.02), np.float32(0.01), np.float32(np.sqrt(2.0))
    decay, rate = np.float32(1.0) - lr * wd, lr * scaling
    ref = seq_binary(seq_scale(p, decay), seq_scale(o, rate), 1)
    out = dev.empty(length)
    dev.call("axis_muon_apply", p.vp, o.vp, out.vp, F32(decay), F32(rate), n)
    assert np.array_equal(read(out), read(ref))
