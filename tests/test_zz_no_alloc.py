"""axis_matmul_right_backward_noalloc: the weight-gradient product with its split partial sums in a
static device array.  Checked bit for bit against axis_matmul_right_backward (same kernels, same
split rule) on consecutive calls -- larger, then smaller, then one with more than 32 slices
(range sums) -- and the caching allocator's counters show the calls allocated nothing; calls from
two handles on the one GPU, enqueued back to back with no host wait, are ordered by the array's
event and each gives its own product's bits."""
import ctypes

import numpy as np
import pytest

from axis_amd import hip
from axis_amd.hip import I64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return hip.Device(0)


def stats(dev):
    in_use, cached = ctypes.c_size_t(), ctypes.c_size_t()
    dev.call("axis_memory_stats", ctypes.byref(in_use), ctypes.byref(cached))
    return in_use.value, cached.value


def test_noalloc_matches_allocating_entry_on_consecutive_calls(dev):
    # (m, k, n): 13 slices, then a smaller product, then 64 slices (the dense schedule's cap; more
    # than 32, so two range sums), then unsplit
    shapes = [(8192, 784, 1024), (2048, 300, 200), (262144, 64, 64), (100, 70, 50)]
    for m, k, n in shapes:
        print(f"noalloc case m={m} k={k} n={n}", flush=True)
        rng = np.random.default_rng(m + k + n)
        lhs = dev.upload(rng.standard_normal(m * k).astype(np.float32))
        grad = dev.upload(rng.standard_normal(m * n).astype(np.float32))
        want, got = dev.empty(k * n), dev.empty(k * n)
        geo = (I64(1), I64(m), I64(k), I64(n))
        dev.call("axis_matmul_right_backward", lhs.vp, grad.vp, want.vp, *geo)
        dev.synchronize()
        before = stats(dev)
        dev.call("axis_matmul_right_backward_noalloc", lhs.vp, grad.vp, got.vp, *geo)
        dev.synchronize()
        assert stats(dev) == before
        w, g = dev.read(want, k * n), dev.read(got, k * n)
        assert np.array_equal(w.view(np.uint32), g.view(np.uint32)), (m, k, n)


def test_noalloc_batched_product(dev):
    batch, m, k, n = 3, 4000, 96, 80
    rng = np.random.default_rng(5)
    lhs = dev.upload(rng.standard_normal(batch * m * k).astype(np.float32))
    grad = dev.upload(rng.standard_normal(batch * m * n).astype(np.float32))
    want, got = dev.empty(batch * k * n), dev.empty(batch * k * n)
    geo = (I64(batch), I64(m), I64(k), I64(n))
    dev.call("axis_matmul_right_backward", lhs.vp, grad.vp, want.vp, *geo)
    dev.call("axis_matmul_right_backward_noalloc", lhs.vp, grad.vp, got.vp, *geo)
    assert np.array_equal(dev.read(want, batch * k * n), dev.read(got, batch * k * n))


def test_noalloc_rejects_bf16_handles_and_bad_arguments(dev):
    buf = dev.empty(64)
    with pytest.raises(hip.AxisError, match="positive"):
        dev.call("axis_matmul_right_backward_noalloc", buf.vp, buf.vp, buf.vp, I64(1), I64(0), I64(4), I64(4))
    with pytest.raises(hip.AxisError, match="null"):
        dev.call("axis_matmul_right_backward_noalloc", None, buf.vp, buf.vp, I64(1), I64(4), I64(4), I64(4))
    bf = hip.Device(0, bf16_matmul=True)
    b2 = bf.empty(64)
    with pytest.raises(hip.AxisError, match="fp32 only"):
        bf.call("axis_matmul_right_backward_noalloc", b2.vp, b2.vp, b2.vp, I64(1), I64(4), I64(4), I64(4))


def test_noalloc_calls_from_two_handles_are_ordered(dev):
    # two handles (two streams) on one GPU share the array: a large product on the first handle,
    # then a different product on the second with no host wait between; each must equal its
    # allocating entry's result
    other = hip.Device(0)
    cases = [(dev, (65536, 576, 128), 1), (other, (16384, 1152, 256), 2), (dev, (8192, 784, 1024), 3)]
    made = []
    for d, (m, k, n), seed in cases:
        rng = np.random.default_rng(seed)
        lhs = d.upload(rng.standard_normal(m * k).astype(np.float32))
        grad = d.upload(rng.standard_normal(m * n).astype(np.float32))
        want, got = d.empty(k * n), d.empty(k * n)
        d.call("axis_matmul_right_backward", lhs.vp, grad.vp, want.vp, I64(1), I64(m), I64(k), I64(n))
        d.synchronize()
        made.append((d, lhs, grad, want, got, (m, k, n)))
    print("noalloc two handles: enqueue without waits", flush=True)
    for d, lhs, grad, want, got, (m, k, n) in made:
        d.call("axis_matmul_right_backward_noalloc", lhs.vp, grad.vp, got.vp, I64(1), I64(m), I64(k), I64(n))
    for d, lhs, grad, want, got, (m, k, n) in made:
        w, g = d.read(want, k * n), d.read(got, k * n)
        assert np.array_equal(w.view(np.uint32), g.view(np.uint32)), (m, k, n)
