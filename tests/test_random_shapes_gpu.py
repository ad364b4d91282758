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
BF16_SHAPES = PRODUCT_SHAPES[::4]


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
