"""Seeded random shapes through the fp32 product and convolution entries, against the CPU oracle.

The fixed cases elsewhere pin the tile shapes, partial depth steps and split schedules one at a
time; these draw extents from one seeded generator so that ragged tiles, short and long
reductions, every tile shape and the split-depth schedules meet in combinations nobody chose by
hand. Tolerance: relative 1e-5 of the largest reference value, as for the fixed cases.
"""
import numpy as np
import pytest

from axis_amd import hip
from axis_amd.hip import I32, I64

pytestmark = pytest.mark.gpu


def _product_shapes():
    rng = np.random.default_rng(20261202)
    shapes = []
    for i in range(48):
        kind = i % 4
        if kind == 0:    # everything below one tile
            m, k, n = rng.integers(1, 200, size=3)
        elif kind == 1:  # several tiles with ragged edges, short reductions
            m, k, n = rng.integers(100, 1300), rng.integers(1, 400), rng.integers(1, 700)
        elif kind == 2:  # few tiles over a long reduction: split-depth schedules
            m, k, n = rng.integers(1, 300), rng.integers(600, 6000), rng.integers(1, 300)
        else:            # widths that leave the 64-wide half of a 128 tile (64x128 tiles)
            m = 128 * rng.integers(1, 8) + rng.integers(1, 65)
            k, n = rng.integers(1, 600), rng.integers(64, 900)
        batch = int(rng.integers(1, 4)) if i % 6 == 5 else 1
        shapes.append((batch, int(m), int(k), int(n)))
    return shapes


def _conv_shapes():
    rng = np.random.default_rng(1202)
    shapes = []
    while len(shapes) < 32:
        k = int(rng.choice([1, 2, 3, 3, 3, 5]))
        s = int(rng.choice([1, 1, 2]))
        p = int(rng.integers(0, k // 2 + 1))
        b = int(rng.integers(1, 5))
        h, w = int(rng.integers(k, 41)), int(rng.integers(k, 41))
        c = int(rng.choice([int(rng.integers(1, 9)), int(rng.integers(9, 70)), 64]))
        n = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(40, 160)), 128]))
        channel_major = bool(rng.integers(0, 4) == 0)
        if (h + 2 * p - k) // s + 1 >= 1 and (w + 2 * p - k) // s + 1 >= 1:
            shapes.append((b, h, w, c, n, k, s, p, channel_major))
    return shapes


def _pool_shapes():
    rng = np.random.default_rng(2212)
    shapes = []
    while len(shapes) < 16:
        ph, pw = [(2, 2), (2, 2), (2, 2), (1, 2), (2, 4), (4, 4), (2, 1), (4, 2)][int(rng.integers(0, 8))]
        ow = int(rng.choice([w for w in (2, 4, 8, 16, 32, 64) if w % pw == 0 and 128 % (ph * w) == 0]))
        oh = ph * int(rng.integers(1, 9))
        k = int(rng.choice([1, 3, 3, 5]))
        b = int(rng.integers(1, 4))
        c = int(rng.choice([int(rng.integers(1, 9)), int(rng.integers(9, 70))]))
        n = int(rng.choice([int(rng.integers(1, 70)), int(rng.integers(70, 260))]))
        shapes.append((b, oh, ow, c, n, k, ph, pw, bool(rng.integers(0, 3) == 0)))
    return shapes


PRODUCT_SHAPES = _product_shapes()
CONV_SHAPES = _conv_shapes()
POOL_SHAPES = _pool_shapes()
# every kind of product shape: ragged below one tile, ragged multi-tile, split-depth, 64-wide halves
BF16_SHAPES = PRODUCT_SHAPES[::4] + PRODUCT_SHAPES[1::8] + PRODUCT_SHAPES[2::8] + PRODUCT_SHAPES[3::8]


@pytest.fixture(scope="module")
def dev():
    return hip.Device(0)


@pytest.fixture(scope="module")
def dev_bf16():
    return hip.Device(0, bf16_matmul=True)


def _up(dev, a):
    return dev.upload(np.ascontiguousarray(a, dtype=np.float32))


def _rel_err(actual, expected):
    e = np.asarray(expected, np.float64)
    return float(np.abs(np.asarray(actual, np.float64) - e).max() / max(np.abs(e).max(), 1e-30))


@pytest.mark.parametrize("batch,m,k,n", PRODUCT_SHAPES)
def test_random_product_shapes(dev, oracle, batch, m, k, n):
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    g = rng.standard_normal(batch * m * n).astype(np.float32)
    da, db, dg = _up(dev, a), _up(dev, b), _up(dev, g)
    out = dev.empty(batch * m * n)
    dev.call("axis_matmul", da.vp, db.vp, out.vp, I64(batch), I64(m), I64(k), I64(n))
    assert _rel_err(dev.read(out, batch * m * n), oracle.matmul(a, b, batch, m, k, n)) < 1e-5
    out = dev.empty(batch * m * k)
    dev.call("axis_matmul_left_backward", dg.vp, db.vp, out.vp, I64(batch), I64(m), I64(k), I64(n))
    assert _rel_err(dev.read(out, batch * m * k), oracle.matmul_left_backward(g, b, batch, m, k, n)) < 1e-5
    out = dev.empty(batch * k * n)
    dev.call("axis_matmul_right_backward", da.vp, dg.vp, out.vp, I64(batch), I64(m), I64(k), I64(n))
    assert _rel_err(dev.read(out, batch * k * n), oracle.matmul_right_backward(a, g, batch, m, k, n)) < 1e-5


@pytest.mark.parametrize("b,h,w,c,n,k,s,p,channel_major", CONV_SHAPES)
def test_random_convolution_shapes(dev, oracle, b, h, w, c, n, k, s, p, channel_major):
    rng = np.random.default_rng(b * 1000003 + h * 1009 + w * 101 + c * 11 + n)
    x = rng.standard_normal(b * h * w * c).astype(np.float32)
    weight = (rng.standard_normal(c * k * k * n) * 0.1).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    if channel_major:
        dims = [("batch", b), ("c", c), ("height", h), ("width", w)]
        strides = (I64 * 4)(c * h * w, h * w, w, 1)
    else:
        dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
        strides = None
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("group", 1),
                           ("patch", c * k * k), [k, k], [s, s], [p, p], 0.0)
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    m = b * oh * ow
    patches = oracle.unfold2d(x, u)
    ref = oracle.binary(oracle.matmul(patches, weight, 1, m, c * k * k, n), np.tile(bias, m), 0)
    geo = [(I32 * 2)(k, k), (I32 * 2)(s, s), (I32 * 2)(p, p)]
    dx, dw, dbias, out = _up(dev, x), _up(dev, weight), _up(dev, bias), dev.empty(m * n)
    dev.call("axis_conv2d_forward", dx.vp, strides, dw.vp, dbias.vp, out.vp, I64(b), I32(h), I32(w), I32(c),
             I32(n), *geo)
    assert _rel_err(dev.read(out, m * n), ref) < 1e-5
    g = rng.standard_normal(m * n).astype(np.float32)
    dg, gw = _up(dev, g), dev.empty(c * k * k * n)
    dev.call("axis_conv2d_backward_weight", dx.vp, strides, dg.vp, gw.vp, I64(b), I32(h), I32(w), I32(c),
             I32(n), *geo)
    assert _rel_err(dev.read(gw, c * k * k * n), oracle.matmul_right_backward(patches, g, 1, m, c * k * k, n)) < 1e-5
    if s == 1 and not channel_major:
        gx = dev.empty(b * h * w * c)
        dev.call("axis_conv2d_backward_data", dg.vp, dw.vp, gx.vp, I64(b), I32(h), I32(w), I32(c), I32(n), *geo)
        ref_dx = oracle.unfold2d_backward(oracle.matmul_left_backward(g, weight, 1, m, c * k * k, n), u, len(x))
        assert _rel_err(dev.read(gx, len(x)), ref_dx) < 1e-5


@pytest.mark.parametrize("batch,m,k,n", BF16_SHAPES)
def test_random_bf16_product_shapes(dev_bf16, oracle, batch, m, k, n):
    # a bf16 handle rounds each product's operands to bf16 and accumulates in fp32
    rng = np.random.default_rng(m * 7919 + k * 31 + n + 1)
    a = rng.standard_normal(batch * m * k).astype(np.float32)
    b = rng.standard_normal(batch * k * n).astype(np.float32)
    g = rng.standard_normal(batch * m * n).astype(np.float32)
    ra, rb, rg = oracle.bf16_round(a), oracle.bf16_round(b), oracle.bf16_round(g)
    da, db, dg = _up(dev_bf16, a), _up(dev_bf16, b), _up(dev_bf16, g)
    geo = (I64(batch), I64(m), I64(k), I64(n))
    out = dev_bf16.empty(batch * m * n)
    dev_bf16.call("axis_matmul", da.vp, db.vp, out.vp, *geo)
    assert _rel_err(dev_bf16.read(out, batch * m * n), oracle.matmul(ra, rb, batch, m, k, n)) < 1e-5
    out = dev_bf16.empty(batch * m * k)
    dev_bf16.call("axis_matmul_left_backward", dg.vp, db.vp, out.vp, *geo)
    assert _rel_err(dev_bf16.read(out, batch * m * k), oracle.matmul_left_backward(rg, rb, batch, m, k, n)) < 1e-5
    out = dev_bf16.empty(batch * k * n)
    dev_bf16.call("axis_matmul_right_backward", da.vp, dg.vp, out.vp, *geo)
    assert _rel_err(dev_bf16.read(out, batch * k * n), oracle.matmul_right_backward(ra, rg, batch, m, k, n)) < 1e-5


@pytest.mark.parametrize("b,h,w,c,n,k,ph,pw,channel_major", POOL_SHAPES)
def test_random_relu_pool_shapes(dev, oracle, b, h, w, c, n, k, ph, pw, channel_major):
    # "same" convolutions (stride 1, padding k // 2) whose output the pool windows tile exactly
    rng = np.random.default_rng(b * 100003 + h * 1009 + w * 101 + c * 11 + n)
    p = k // 2
    x = rng.standard_normal(b * h * w * c).astype(np.float32)
    weight = (rng.standard_normal(c * k * k * n) * 0.2).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    if channel_major:
        dims = [("batch", b), ("c", c), ("height", h), ("width", w)]
        strides = (I64 * 4)(c * h * w, h * w, w, 1)
    else:
        dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
        strides = None
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("group", 1),
                           ("patch", c * k * k), [k, k], [1, 1], [p, p], 0.0)
    m = b * h * w
    z = oracle.binary(oracle.matmul(oracle.unfold2d(x, u), weight, 1, m, c * k * k, n), np.tile(bias, m), 0)
    def window_rows(t):
        return t.reshape(b, h // ph, ph, w // pw, pw, n).transpose(0, 1, 3, 5, 2, 4).reshape(-1, ph * pw)

    windows = window_rows(np.maximum(z, np.float32(0)))
    pooled_len = len(windows)
    geo = [(I32 * 2)(k, k), (I32 * 2)(1, 1), (I32 * 2)(p, p)]
    dx, dw, dbias = _up(dev, x), _up(dev, weight), _up(dev, bias)
    pooled, arg = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
    dev.call("axis_conv2d_relu_pool_forward", dx.vp, strides, dw.vp, dbias.vp, pooled.vp, arg.vp, I64(b), I32(h),
             I32(w), I32(c), I32(n), *geo, (I32 * 2)(ph, pw))
    got, got_arg = dev.read(pooled, pooled_len), dev.read(arg, pooled_len, np.uint8)
    scale = max(float(np.abs(z).max()), 1e-30)
    assert np.abs(got - windows.max(axis=1)).max() <= 1e-5 * scale
    # the winner is the first position holding the window's largest value, wherever that largest
    # value beats the runner-up by more than rounding; windows negative beyond rounding before the
    # ReLU hold only zeros, and position 0 wins
    top2 = np.sort(windows, axis=1)[:, -2:]
    negative = (window_rows(z) < -1e-4 * scale).all(axis=1)
    clear = (top2[:, 1] - top2[:, 0] > 1e-4 * scale) | negative
    first = np.argmax(windows == windows.max(axis=1, keepdims=True), axis=1)
    assert clear.mean() > 0.5
    assert np.array_equal(got_arg[clear], first[clear])
    # the separate GPU entries (forward, ReLU, pool) give the same bits while the forward runs unsplit
    if c * k * k < 256:
        zz, yy = dev.empty(m * n), dev.empty(m * n)
        dev.call("axis_conv2d_forward", dx.vp, strides, dw.vp, dbias.vp, zz.vp, I64(b), I32(h), I32(w), I32(c),
                 I32(n), *geo)
        dev.call("axis_relu", zz.vp, yy.vp, I64(m * n))
        p2, a2 = dev.empty(pooled_len), dev.empty(pooled_len, np.uint8)
        dev.call("axis_max_pool2d", yy.vp, p2.vp, a2.vp, I64(b), I32(h), I32(w), I64(n), (I32 * 2)(ph, pw),
                 (I32 * 2)(ph, pw), (I32 * 2)(0, 0))
        assert np.array_equal(dev.read(p2, pooled_len), got)
        assert np.array_equal(dev.read(a2, pooled_len, np.uint8), got_arg)


# ---------------------------------------------------------------- bit-exact index and reduction kernels

def _unfold_cases():
    rng = np.random.default_rng(4242)
    cases = []
    while len(cases) < 16:
        kh, kw = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        sy, sx = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        py, px = int(rng.integers(0, kh)), int(rng.integers(0, kw))
        h, w = int(rng.integers(1, 20)), int(rng.integers(1, 20))
        if h + 2 * py < kh or w + 2 * px < kw:
            continue
        groups = int(rng.choice([1, 1, 2, 3]))
        c = groups * int(rng.integers(1, 6))
        b = int(rng.integers(1, 4))
        names = ["batch", "channel", "height", "width"]
        order = [names[i] for i in rng.permutation(4)]
        fill = float(rng.choice([0.0, -np.inf]))
        cases.append((b, c, h, w, groups, [kh, kw], [sy, sx], [py, px], order, fill))
    return cases


UNFOLD_RANDOM = _unfold_cases()


@pytest.mark.parametrize("b,c,h,w,groups,kernel,stride,padding,order,fill", UNFOLD_RANDOM)
def test_random_unfold_and_col2im(dev, oracle, b, c, h, w, groups, kernel, stride, padding, order, fill):
    import ctypes

    dims = [("batch", b), ("channel", c), ("height", h), ("width", w)]
    strides = oracle.layout_for(dims, order)
    u = oracle.unfold_spec(dims, strides, "channel", ["height", "width"], ("group", groups),
                           ("patch", c // groups * kernel[0] * kernel[1]), kernel, stride, padding, fill)
    spec = hip.UnfoldSpec()
    ctypes.memmove(ctypes.byref(spec), ctypes.byref(u.spec), ctypes.sizeof(spec))
    rng = np.random.default_rng(b * 1000 + c * 100 + h * 10 + w)
    x = rng.standard_normal(oracle.shape_len(dims)).astype(np.float32)
    dx, out = _up(dev, x), dev.empty(spec.output_len)
    dev.call("axis_unfold", dx.vp, out.vp, ctypes.byref(spec))
    assert np.array_equal(dev.read(out, spec.output_len), oracle.unfold2d(x, u))
    y = rng.standard_normal(spec.output_len).astype(np.float32)
    dy, back = _up(dev, y), dev.empty(spec.input_len)
    dev.call("axis_unfold_backward", dy.vp, back.vp, ctypes.byref(spec))
    assert np.array_equal(dev.read(back, spec.input_len), oracle.unfold2d_backward(y, u, len(x)))


def _pool_cases():
    rng = np.random.default_rng(777)
    cases = []
    while len(cases) < 12:
        kh, kw = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        sy, sx = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        py, px = int(rng.integers(0, (kh + 1) // 2)), int(rng.integers(0, (kw + 1) // 2))
        h, w = int(rng.integers(kh, 24)), int(rng.integers(kw, 24))
        cases.append((int(rng.integers(1, 4)), h, w, int(rng.integers(1, 70)), [kh, kw], [sy, sx], [py, px]))
    return cases


@pytest.mark.parametrize("b,h,w,c,kernel,stride,padding", _pool_cases())
def test_random_max_pool(dev, oracle, b, h, w, c, kernel, stride, padding):
    from axis_amd.hip import I64 as L

    rng = np.random.default_rng(b * 7 + h * 5 + w * 3 + c)
    x = rng.integers(-3, 4, b * h * w * c).astype(np.float32)  # ties everywhere
    x[::23] = np.nan
    x[::29] = np.inf
    dims = [("batch", b), ("height", h), ("width", w), ("c", c)]
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "c", ["height", "width"], ("c", c),
                           ("pool", kernel[0] * kernel[1]), kernel, stride, padding, float("-inf"))
    q = oracle.scale(oracle.unfold2d(x, u), -1.0)
    _, fwd, rev = oracle.min_plans(u.shape, u.strides, "pool")
    mn, mask, _ = oracle.grouped_minimum(q, fwd, rev)
    ref = oracle.scale(mn, -1.0)
    n_out = len(ref)
    gout = rng.standard_normal(n_out).astype(np.float32)
    gg = oracle.mask_gradient(oracle.grouped(oracle.scale(gout, -1.0), None, rev, 1.0), mask)
    ref_dx = oracle.unfold2d_backward(oracle.scale(gg, -1.0), u, len(x))
    k, s, p = (I32 * 2)(*kernel), (I32 * 2)(*stride), (I32 * 2)(*padding)
    dx, out, arg = _up(dev, x), dev.empty(n_out), dev.empty(n_out, np.uint8)
    dev.call("axis_max_pool2d", dx.vp, out.vp, arg.vp, L(b), I32(h), I32(w), L(c), k, s, p)
    got = dev.read(out, n_out)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    dg, back = _up(dev, gout), dev.empty(len(x))
    dev.call("axis_max_pool2d_backward", dg.vp, arg.vp, back.vp, L(b), I32(h), I32(w), L(c), k, s, p)
    assert np.array_equal(dev.read(back, len(x)), ref_dx)


def _axes_cases():
    rng = np.random.default_rng(99)
    cases = []
    for i in range(14):
        rank = int(rng.integers(1, 5))
        names = "abcd"[:rank]
        dims = [(names[j], int(rng.choice([1, int(rng.integers(2, 9)), int(rng.integers(9, 300))]))) for j in range(rank)]
        while int(np.prod([e for _, e in dims])) > 400000:
            dims = [(n_, max(1, e // 2)) for n_, e in dims]
        order = [names[j] for j in rng.permutation(rank)]
        k = int(rng.integers(1, rank + 1))
        axes = [names[j] for j in sorted(rng.choice(rank, size=k, replace=False))]
        cases.append((dims, order, axes, bool(i % 2)))
    return cases


@pytest.mark.parametrize("dims,order,axes,mean", _axes_cases())
def test_random_reduce_axes(dev, oracle, dims, order, axes, mean):
    from axis_amd.hip import F32, VP

    rng = np.random.default_rng(sum(e for _, e in dims) * 13 + len(axes))
    n = int(np.prod([e for _, e in dims]))
    a = rng.standard_normal(n).astype(np.float32)
    strides = oracle.layout_for(dims, order)
    out_dims, fwd, rev, factor = oracle.reduction_plans(dims, strides, axes, mean)
    olen = int(np.prod([e for _, e in out_dims])) if out_dims else 1
    ext = np.array([e for _, e in dims], np.int64)
    st = np.array(strides, np.int64)
    red = np.array([1 if name in axes else 0 for name, _ in dims], np.int32)
    geo = (I32(len(dims)), ext.ctypes.data_as(VP), st.ctypes.data_as(VP), red.ctypes.data_as(VP), F32(factor))
    da, out = _up(dev, a), dev.empty(olen)
    dev.call("axis_reduce_axes", da.vp, out.vp, *geo)
    got = dev.read(out, olen)
    assert np.array_equal(got, oracle.grouped(a, None, fwd, factor))
    back = dev.empty(n)
    dev.call("axis_reduce_axes_backward", out.vp, back.vp, *geo)
    assert np.array_equal(dev.read(back, n), oracle.grouped(got, None, rev, factor))


def _extreme_cases():
    rng = np.random.default_rng(31337)
    cases = []
    for i in range(12):
        rank = int(rng.integers(1, 5))
        names = "abcd"[:rank]
        dims = [(names[j], int(rng.choice([1, int(rng.integers(2, 10)), int(rng.integers(10, 200))]))) for j in range(rank)]
        while int(np.prod([e for _, e in dims])) > 300000:
            dims = [(n_, max(1, e // 2)) for n_, e in dims]
        order = [names[j] for j in rng.permutation(rank)]
        cases.append((dims, order, names[int(rng.integers(0, rank))], bool(i % 2)))
    return cases


@pytest.mark.parametrize("dims,order,axis,maximum", _extreme_cases())
def test_random_extreme_axis(dev, oracle, dims, order, axis, maximum):
    from axis_amd.hip import VP

    rng = np.random.default_rng(sum(e for _, e in dims) * 17 + int(maximum))
    n = int(np.prod([e for _, e in dims]))
    a = np.round(rng.standard_normal(n) * 3).astype(np.float32) / 3  # many ties
    a[::19] = np.inf
    a[::23] = -np.inf
    a[::29] = np.nan
    strides = oracle.layout_for(dims, order)
    out_dims, fwd, rev = oracle.min_plans(dims, strides, axis)
    olen = int(np.prod([e for _, e in out_dims])) if out_dims else 1
    ref, ref_mask, _ = oracle.grouped_minimum(a, fwd, rev, maximum)
    ext = np.array([e for _, e in dims], np.int64)
    st = np.array(strides, np.int64)
    geo = (I32(len(dims)), ext.ctypes.data_as(VP), st.ctypes.data_as(VP), I32([nm for nm, _ in dims].index(axis)))
    da, out, mask = _up(dev, a), dev.empty(olen), dev.empty(n)
    dev.call("axis_extreme_axis", da.vp, *geo, I32(1 if maximum else 0), out.vp, mask.vp)
    got = dev.read(out, olen)
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    assert np.array_equal(dev.read(mask, n), ref_mask)
    g = rng.standard_normal(olen).astype(np.float32)
    dg, back = _up(dev, g), dev.empty(n)
    dev.call("axis_extreme_axis_backward", dg.vp, mask.vp, *geo, back.vp)
    expect = oracle.mask_gradient(oracle.grouped(g, None, rev, 1.0), ref_mask)
    assert np.array_equal(dev.read(back, n).view(np.uint32), expect.view(np.uint32))


def _permute_cases():
    rng = np.random.default_rng(2718)
    cases = []
    for _ in range(16):
        rank = int(rng.integers(2, 6))
        shape = tuple(int(rng.choice([1, int(rng.integers(2, 8)), int(rng.integers(8, 90))])) for _ in range(rank))
        while int(np.prod(shape)) > 500000:
            shape = tuple(max(1, e // 2) for e in shape)
        cases.append((shape, tuple(int(p) for p in rng.permutation(rank))))
    return cases


@pytest.mark.parametrize("shape,perm", _permute_cases())
def test_random_permutations(dev, oracle, shape, perm):
    from axis_amd.hip import VP

    rng = np.random.default_rng(int(np.prod(shape)) + len(shape))
    n = int(np.prod(shape))
    x = rng.standard_normal(n).astype(np.float32)
    src = [int(np.prod(shape[i + 1:])) for i in range(len(shape))]
    dst_shape = [shape[p] for p in perm]
    dst_of_axis = {perm[k]: int(np.prod(dst_shape[k + 1:])) for k in range(len(perm))}
    md = np.array([v for i, e in enumerate(shape) for v in (e, src[i], dst_of_axis[i])], np.int32)
    dx, out, back = _up(dev, x), dev.empty(n), dev.empty(n)
    dev.call("axis_select_axis", dx.vp, out.vp, md.ctypes.data_as(VP), I32(len(shape)), I32(0), I64(n))
    got = dev.read(out, n)
    assert np.array_equal(got, x.reshape(shape).transpose(perm).reshape(-1))
    if n <= 1 << 16:
        assert np.array_equal(got, oracle.select_axis(x, md, len(shape), 0, n))
    dev.call("axis_select_axis_backward", out.vp, back.vp, md.ctypes.data_as(VP), I32(len(shape)), I32(0), I64(n))
    assert np.array_equal(dev.read(back, n), x)
