"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is independent of the oracle's own formulas: literal fixtures from the reference's
tests (file:line cited), closed forms, invariants (col2im is the adjoint of im2col), brute force
in float64, and torch's CPU float64 autograd as an independent library.
"""
import math

import numpy as np
import pytest

from tests.conftest import close


# ---------------------------------------------------------------- RNG

def test_rng_literal_fixture(oracle):
    # src/library/src/tests.rs:5143-5184 (seed 7 uniform, seed 99 normal)
    close("uniform seed 7", oracle.uniform(7, 6), [
        0.0, 0.4375271201133728, 0.755250871181488, 0.4715511202812195, 0.459380567073822,
        0.7119333148002625])
    close("normal seed 99", oracle.normal(99, 6), [
        0.0, 0.0, -0.04610706669773621, 0.15413647086258625, 1.160083365411145,
        -1.2878684354641539])
    # small seeds draw exactly 0.0 first (tensor.rs:23-28)
    assert oracle.xorshift_unit_stream(1, 1)[0] == 0.0 and oracle.xorshift_unit_stream(0, 1)[0] == 0.0
    # the xorshift64 recurrence in plain Python integers
    rng, ref = 0xDEADBEEFCAFE, []
    for _ in range(5):
        rng ^= (rng << 13) & (2**64 - 1)
        rng ^= rng >> 7
        rng ^= (rng << 17) & (2**64 - 1)
        ref.append((rng >> 40) / float(1 << 24))
    assert np.array_equal(oracle.xorshift_unit_stream(0xDEADBEEFCAFE, 5), np.float32(ref))
    # odd count drops the final sine value
    assert np.array_equal(oracle.normal(5, 7), oracle.normal(5, 8)[:7])


def test_powi_matches_repeated_squaring(oracle):
    for t in range(1, 12):
        expected = np.float32(1.0)
        base, e = np.float32(0.999), t
        while True:
            if e & 1:
                expected = np.float32(expected * base)
            e //= 2
            if e == 0:
                break
            base = np.float32(base * base)
        assert oracle.powi(0.999, t) == float(expected)
    assert abs(oracle.powi(0.9, 10) - 0.9 ** 10) < 1e-6


# ---------------------------------------------------------------- contractions

def test_bf16_round_matches_torch(oracle):
    # The operand conversion of the reference's bf16 products (backend.rs:2209-2312) against an
    # independent implementation (torch's float32 -> bfloat16, round to nearest even), including
    # exact ties, overflow to infinity, subnormals, signed zeros, infinities and NaN.
    import torch
    rng = np.random.default_rng(12)
    values = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10) ** rng.integers(-30, 30, 100000).astype(np.float32),
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7FFFFF, 0x7F7F8000, 0x00018000, 0x00008000,
                  0x80000000, 0x00000000, 0x7F800000, 0xFF800000], np.uint32).view(np.float32),
    ]).astype(np.float32)
    got = oracle.bf16_round(values)
    ref = torch.from_numpy(values).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # ties go to the even bf16 neighbour
    assert got[-11:-9].view(np.uint32).tolist() == [0x3F800000, 0x3F820000]
    nan = oracle.bf16_round(np.array([np.nan, -np.nan], np.float32))
    assert np.all(np.isnan(nan)) and np.all((nan.view(np.uint32) & 0xFFFF) == 0)


def test_matmul_family_matches_float64(oracle):
    rng = np.random.default_rng(0)
    b, m, k, n = 2, 7, 5, 9
    a = rng.standard_normal((b, m, k)).astype(np.float32)
    w = rng.standard_normal((b, k, n)).astype(np.float32)
    g = rng.standard_normal((b, m, n)).astype(np.float32)
    close("matmul", oracle.matmul(a, w, b, m, k, n), (a.astype(np.float64) @ w).reshape(-1))
    close("dgrad", oracle.matmul_left_backward(g, w, b, m, k, n),
          (g.astype(np.float64) @ np.swapaxes(w, 1, 2)).reshape(-1))
    close("wgrad", oracle.matmul_right_backward(a, g, b, m, k, n),
          (np.swapaxes(a.astype(np.float64), 1, 2) @ g).reshape(-1))


# ---------------------------------------------------------------- unfold / col2im

def _conv_literal(oracle):
    dims = [("channel", 1), ("height", 3), ("width", 3)]
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "channel", ["height", "width"],
                           ("group", 1), ("patch", 4), [2, 2], [1, 1], [0, 0], 0.0)
    return dims, u


def test_conv2d_literal_fixture(oracle):
    # src/library/src/tests.rs:1372-1421: 3x3 input 1..9, kernel [1,0,0,-1], bias 0.5
    dims, u = _conv_literal(oracle)
    x = np.arange(1, 10, dtype=np.float32)
    w = np.array([1.0, 0.0, 0.0, -1.0], np.float32)
    patches = oracle.unfold2d(x, u)
    z = oracle.matmul(patches, w, 1, 4, 4, 1)
    y = oracle.binary(z, np.full(4, 0.5, np.float32), 0)
    close("Conv2d forward", y, [-3.5] * 4)
    g = np.full(4, 0.25, np.float32)  # mean over [height, width, output]
    close("bias gradient", oracle.bias_gradient(g, 4, 1), [1.0])
    close("weight gradient", oracle.matmul_right_backward(patches, g, 1, 4, 4, 1), [3, 4, 6, 7])
    dp = oracle.matmul_left_backward(g, w, 1, 4, 4, 1)
    close("input gradient", oracle.unfold2d_backward(dp, u, 9),
          [0.25, 0.25, 0.0, 0.25, 0.0, -0.25, 0.0, -0.25, -0.25])


def test_unfold_probe_fixture(oracle):
    # src/library/src/tests.rs:1427-1475: input 100y+10x+t, [height,width] vs [height,time]
    dims = [("channel", 1), ("height", 3), ("width", 3), ("time", 3)]
    x = np.array([100 * y + 10 * xx + t for y in range(3) for xx in range(3) for t in range(3)],
                 np.float32)
    probe = ((3 + 2) * 3) * 9 + 5
    hw = oracle.unfold_spec(dims, oracle.contiguous(dims), "channel", ["height", "width"],
                            ("group", 1), ("patch", 9), [3, 3], [1, 1], [1, 1], 0.0)
    ht = oracle.unfold_spec(dims, oracle.contiguous(dims), "channel", ["height", "time"],
                            ("group", 1), ("patch", 9), [3, 3], [1, 1], [1, 1], 0.0)
    a = oracle.to_logical(oracle.unfold2d(x, hw), hw.shape, hw.strides)
    b = oracle.to_logical(oracle.unfold2d(x, ht), ht.shape, ht.strides)
    assert a[probe] == 0.0
    assert b[probe] == 121.0


def _random_spec(oracle, rng, layout_perm, groups, kernel, stride, padding):
    cin = 2 * groups
    dims = [("batch", 2), ("channel", cin), ("height", 5), ("width", 4)]
    order = [dims[i][0] for i in layout_perm]
    strides = oracle.layout_for(dims, order)
    u = oracle.unfold_spec(dims, strides, "channel", ["height", "width"], ("group", groups),
                           ("patch", 2 * kernel[0] * kernel[1]), kernel, stride, padding, 0.0)
    return dims, strides, u


@pytest.mark.parametrize("perm,groups,kernel,stride,padding", [
    ((0, 1, 2, 3), 1, [3, 3], [1, 1], [1, 1]),
    ((0, 2, 3, 1), 1, [3, 2], [2, 1], [2, 3]),
    ((3, 1, 0, 2), 2, [2, 2], [2, 2], [0, 1]),
])
def test_col2im_is_adjoint_of_im2col(oracle, perm, groups, kernel, stride, padding):
    rng = np.random.default_rng(1)
    dims, strides, u = _random_spec(oracle, rng, perm, groups, kernel, stride, padding)
    x = rng.standard_normal(oracle.shape_len(dims)).astype(np.float32)
    y = rng.standard_normal(oracle.shape_len(u.shape)).astype(np.float32)
    lhs = float(np.dot(oracle.unfold2d(x, u).astype(np.float64), y.astype(np.float64)))
    rhs = float(np.dot(x.astype(np.float64), oracle.unfold2d_backward(y, u, len(x)).astype(np.float64)))
    assert abs(lhs - rhs) < 1e-4 * (1 + abs(lhs))


def test_im2col_matches_torch_unfold(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    n, c, h, w = 2, 3, 6, 5
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    dims = [("batch", n), ("channel", c), ("height", h), ("width", w)]
    u = oracle.unfold_spec(dims, oracle.contiguous(dims), "channel", ["height", "width"],
                           ("group", 1), ("patch", c * 9), [3, 3], [2, 1], [1, 1], 0.0)
    ours = oracle.unfold2d(x, u).reshape(n, -1, c * 9)  # [batch, oy*ox, patch]
    ref = torch.nn.functional.unfold(torch.from_numpy(x), 3, padding=1, stride=(2, 1))
    assert np.array_equal(ours, ref.numpy().transpose(0, 2, 1))


# ---------------------------------------------------------------- pooling

def _max_pool(oracle, x, dims, strides, channels, kernel, stride, padding):
    """MaxPool2d forward+backward through the oracle pieces (convolution.rs:1334-1370)."""
    c = dict(dims)[channels]
    u = oracle.unfold_spec(dims, strides, channels, ["height", "width"], (channels, c),
                           ("pool", kernel[0] * kernel[1]), kernel, stride, padding, float("-inf"))
    q = oracle.scale(oracle.unfold2d(x, u), -1.0)
    out_dims, fwd, rev = oracle.min_plans(u.shape, u.strides, "pool")
    mn, mask, _ = oracle.grouped_minimum(q, fwd, rev)
    out = oracle.scale(mn, -1.0)
    n_out = oracle.shape_len(out_dims)
    g = np.full(n_out, 1.0 / n_out, np.float32)
    g = oracle.scale(g, -1.0)
    g = oracle.mask_gradient(oracle.grouped(g, None, rev, 1.0), mask)
    g = oracle.unfold2d_backward(oracle.scale(g, -1.0), u, len(x))
    return out, out_dims, g


def test_max_pool_ties_fixture(oracle):
    # src/library/src/tests.rs:4004-4059
    x = np.array([1, 5, 2, 6, 5, 3, 6, 0.5, 9, 9, 9, 9,
                  -1, -2, -3, -4, -5, -0.5, -6, -7, 0, 0, 0, 0], np.float32)
    dims = [("channel", 2), ("height", 3), ("width", 4)]
    out, out_dims, g = _max_pool(oracle, x, dims, oracle.contiguous(dims), "channel", [2, 2],
                                 [2, 2], [0, 0])
    assert [a for a, _ in out_dims] == ["height", "width", "channel"]
    close("MaxPool2d forward", out, [5.0, -0.5, 6.0, -3.0])
    close("MaxPool2d gradient", g, [0, .25, 0, .25, 0, 0, 0, 0, 0, 0, 0, 0,
                                    0, 0, .25, 0, 0, .25, 0, 0, 0, 0, 0, 0])


def test_max_pool_padding_fixture(oracle):
    # src/library/src/tests.rs:4063-4114 (physical layout [width, height, channel])
    logical = np.array([-1, -9, -2, -8, -7, -9, -3, -9, -4], np.float32).reshape(3, 3)
    dims = [("channel", 1), ("height", 3), ("width", 3)]
    strides = oracle.layout_for(dims, ["width", "height", "channel"])
    physical = np.ascontiguousarray(logical.T).reshape(-1)
    out, out_dims, g = _max_pool(oracle, physical, dims, strides, "channel", [3, 3], [1, 1], [1, 1])
    close("padded forward", out, [-1, -1, -2, -1, -1, -2, -3, -3, -4])
    g_logical = oracle.to_logical(g, dims, strides)
    close("padded gradient", g_logical, [4 / 9, 0, 2 / 9, 0, 0, 0, 2 / 9, 0, 1 / 9])


# ---------------------------------------------------------------- loss, reductions, optimizers

def test_categorical_cross_entropy_fixture(oracle):
    # src/library/src/tests.rs:2384-2470: logits 1000/999/998 class-major, one-hot targets
    logits = np.array([[1000.0, 999.0, 998.0], [-1.0, 0.0, 1.0]], np.float32)  # [batch, class]
    y = np.array([[1, 0, 0], [0, 0, 1]], np.float32)
    p, per_row, loss = oracle.ce_loss(logits, y, 2, 3)
    expected = math.log(1 + math.exp(-1) + math.exp(-2))
    close("CE", per_row, [expected, expected])
    g = oracle.categorical_cross_entropy_backward(oracle.mean_rows_backward(2), p, y, 2, 3)
    p0 = 1 / (1 + math.exp(-1) + math.exp(-2))
    p1, p2 = math.exp(-1) * p0, math.exp(-2) * p0
    # logical [class, batch] order of the fixture
    close("CE gradient", g.reshape(2, 3).T.reshape(-1),
          [(p0 - 1) / 2, p2 / 2, p1 / 2, p1 / 2, p2 / 2, (p0 - 1) / 2])
    with pytest.raises(ValueError, match="row 1 must sum to 1"):
        oracle.check_targets(np.array([[1, 0, 0], [0, 0, 0.5]], np.float32), 3)


def test_adam_and_adamw_fixtures(oracle):
    # src/library/src/tests.rs:2470-2500: mean(p * [0.2, -0.4]) -> grad = c / 2
    p = {"w": np.array([1.0, -2.0], np.float32)}
    adam = oracle.AdamOracle(0.01)
    for expected in ([0.99, -1.99], [0.98, -1.98]):
        p = adam.step(p, {"w": np.array([0.1, -0.2], np.float32)})
        close("Adam", p["w"], expected)
    adamw = oracle.AdamOracle(0.1, wd=0.2)
    p = adamw.step(p, {"w": np.zeros(2, np.float32)})
    close("AdamW decay", p["w"], [0.9604, -1.9404])
    # src/library/src/tests.rs:5237-5275: beta (0.8, 0.9), lr = wd = 0.1, g = 0.4
    p = {"w": np.array([1.0], np.float32)}
    adamw = oracle.AdamOracle(0.1, b1=0.8, b2=0.9, wd=0.1)
    for expected in (0.89, 0.7811):
        p = adamw.step(p, {"w": np.array([0.4], np.float32)})
        close("AdamW two-step", p["w"], [expected])


def test_grouped_multi_chunk_fixture(oracle):
    # src/library/src/tests.rs:26955-27010: 600 x 2 field + bias; sum(batch) then sum(channel)
    field = np.array([(i % 97) * 0.01 - 0.3 for i in range(1200)], np.float32)
    bias = np.array([0.25, -0.75], np.float32)
    biased = oracle.binary(field, np.tile(bias, 600), 0)
    dims = [("batch", 600), ("channel", 2)]
    _, fwd, rev, factor = oracle.reduction_plans(dims, [2, 1], ["batch"], mean=False)
    summed = oracle.grouped(biased, None, fwd, factor)
    close("large-group sum", summed, biased.astype(np.float64).reshape(600, 2).sum(0))
    ones = oracle.grouped(np.ones(1, np.float32), None,
                          oracle.reduction_plans([("channel", 2)], [1], ["channel"], False)[2], 1.0)
    g = oracle.grouped(ones, None, rev, 1.0)
    assert np.array_equal(oracle.bias_gradient(g, 600, 2), [600.0, 600.0])


def test_grouped_chunk_order_is_the_reference_order(oracle):
    # 1300 contributions = chunks of 512 + 512 + 276 summed separately, then in chunk order
    rng = np.random.default_rng(3)
    a = rng.standard_normal(1300).astype(np.float32) * np.float32(1e3)
    plan = oracle.plan_groups([[(i, 0) for i in range(1300)]])
    parts = []
    for lo, hi in ((0, 512), (512, 1024), (1024, 1300)):
        s = np.float32(0)
        for v in a[lo:hi]:
            s = np.float32(s + v)
        parts.append(s)
    total = np.float32(np.float32(np.float32(np.float32(0) + parts[0]) + parts[1]) + parts[2])
    assert oracle.grouped(a, None, plan, 1.0)[0] == total
    with pytest.raises(ValueError):
        oracle.plan_gather(np.zeros(oracle.PLAN_CAP + 1, np.int64))


def test_normalized_l2_fixture(oracle):
    # model/optim.rs:1492-1503
    v = np.array([3.0, -4.0, 12.0], np.float32)
    close("L2 normalization", oracle.normalized_l2(v, 1e-7), v / (13.0 + 1e-7), rtol=2e-6)


def _scalar_muon(expected, momentum, gradient, rows, cols, fan_in_first, lr, mu, nesterov, wd):
    """Independent float64 Muon step in plain loops (the math of model/optim.rs:610-752)."""
    n = rows * cols
    m = [mu * momentum[i] + (1 - mu) * gradient[i] for i in range(n)]
    d = [(1 - mu) * gradient[i] + mu * m[i] for i in range(n)] if nesterov else list(m)
    norm = math.sqrt(sum(v * v for v in d))
    x = [[d[r * cols + c] / (norm + 1e-7) for c in range(cols)] for r in range(rows)]
    if rows > cols:
        x = [list(col) for col in zip(*x)]
    s, l = len(x), len(x[0])
    for _ in range(5):
        gram = [[sum(x[i][t] * x[j][t] for t in range(l)) for j in range(s)] for i in range(s)]
        g2 = [[sum(gram[i][t] * gram[t][j] for t in range(s)) for j in range(s)] for i in range(s)]
        b = [[-4.7750 * gram[i][j] + 2.0315 * g2[i][j] for j in range(s)] for i in range(s)]
        x = [[3.4445 * x[i][c] + sum(b[i][t] * x[t][c] for t in range(s)) for c in range(l)]
             for i in range(s)]
    if rows > cols:
        x = [list(col) for col in zip(*x)]
    fan_in, fan_out = (rows, cols) if fan_in_first else (cols, rows)
    scaling = math.sqrt(max(fan_out / fan_in, 1.0))
    new = [expected[r * cols + c] * (1 - lr * wd) - lr * scaling * x[r][c]
           for r in range(rows) for c in range(cols)]
    return new, m


@pytest.mark.parametrize("rows,cols,fan_in_first", [(3, 2, True), (2, 3, True), (3, 2, False)])
def test_muon_two_step_fixture(oracle, rows, cols, fan_in_first):
    # model/optim.rs:992-1073: initial (i-2)*0.11, gradients (i+1)*0.07-0.19 and 0.23-0.035i
    n = rows * cols
    p = {"w": np.array([(i - 2.0) * 0.11 for i in range(n)], np.float32)}
    grads = [[(i + 1.0) * 0.07 - 0.19 for i in range(n)], [0.23 - i * 0.035 for i in range(n)]]
    opt = oracle.MuonOracle(0.04, momentum=0.8, nesterov=True, wd=0.03)
    expected, momentum = [float(v) for v in p["w"]], [0.0] * n
    fans = (rows, cols) if fan_in_first else (cols, rows)
    for g in grads:
        g32 = np.array(g, np.float32)
        p = opt.step(p, {"w": g32}, {"w": (rows, cols)}, {"w": fans})
        expected, momentum = _scalar_muon(expected, momentum, [float(v) for v in g32], rows, cols,
                                          fan_in_first, 0.04, 0.8, True, 0.03)
        close("Muon momentum", opt.states["w"], momentum, rtol=2e-6)
        close("Muon value", p["w"], expected, rtol=3e-4)


# ---------------------------------------------------------------- whole steps

def _mlp_float64(x, y, params, batch, sizes):
    """Independent float64 backprop of the ReLU MLP + softmax cross-entropy."""
    acts, pres = [x.reshape(batch, -1).astype(np.float64)], []
    h = acts[0]
    L = len(sizes) - 1
    for j in range(L):
        z = h @ params[f"w{j}"].reshape(sizes[j], sizes[j + 1]).astype(np.float64) + params[f"b{j}"]
        pres.append(z)
        h = np.maximum(z, 0) if j < L - 1 else z
        acts.append(h)
    yy = y.reshape(batch, -1)
    z = h - h.max(1, keepdims=True)
    p = np.exp(z) / np.exp(z).sum(1, keepdims=True)
    loss = float(np.mean(-(yy * np.log(p)).sum(1)))
    g = (p - yy) / batch
    grads = {}
    for j in reversed(range(L)):
        if j < L - 1:
            g = g * (pres[j] > 0)
        grads[f"b{j}"] = g.sum(0)
        grads[f"w{j}"] = (acts[j].T @ g).reshape(-1)
        g = g @ params[f"w{j}"].reshape(sizes[j], sizes[j + 1]).astype(np.float64).T
    return loss, grads


def test_mlp_config1_matches_float64_backprop(oracle):
    sizes = (784, 256, 256, 10)
    out = oracle.mlp_step(128, sizes)
    loss, grads = _mlp_float64(out["x"], out["y"], out["initial"], 128, sizes)
    assert abs(out["loss"] - loss) < 1e-5 * max(1.0, abs(loss))
    for name, g in grads.items():
        scale = np.abs(g).max()
        assert np.abs(out["grads"][name] - g).max() <= 1e-4 * scale + 1e-7, name


def test_cnn_small_matches_torch_float64_autograd(oracle):
    torch = pytest.importorskip("torch")
    batch, size, classes, ch = 2, 16, 10, (3, 8, 16, 32)
    x, y, params = oracle.cnn_inputs(batch, size, classes, ch)
    loss, grads = oracle.cnn_forward_backward(x, y, params, batch, size, classes, ch)
    tp = {}
    for j in range(3):
        w = params[f"conv{j}.weight"].reshape(ch[j] * 9, ch[j + 1]).T.reshape(ch[j + 1], ch[j], 3, 3)
        tp[f"conv{j}.weight"] = torch.tensor(w, dtype=torch.float64, requires_grad=True)
        tp[f"conv{j}.bias"] = torch.tensor(params[f"conv{j}.bias"], dtype=torch.float64, requires_grad=True)
    tp["linear.weight"] = torch.tensor(params["linear.weight"].reshape(ch[3], classes), dtype=torch.float64, requires_grad=True)
    tp["linear.bias"] = torch.tensor(params["linear.bias"], dtype=torch.float64, requires_grad=True)
    h = torch.tensor(x.reshape(batch, 3, size, size), dtype=torch.float64)
    for j in range(3):
        h = torch.nn.functional.conv2d(h, tp[f"conv{j}.weight"], tp[f"conv{j}.bias"], padding=1)
        h = torch.nn.functional.max_pool2d(torch.relu(h), 2)
    logits = h.mean((2, 3)) @ tp["linear.weight"] + tp["linear.bias"]
    target = torch.tensor(y.reshape(batch, classes).argmax(1))
    tloss = torch.nn.functional.cross_entropy(logits, target)
    tloss.backward()
    assert abs(loss - tloss.item()) < 1e-5
    for j in range(3):
        g = tp[f"conv{j}.weight"].grad.numpy().reshape(ch[j + 1], ch[j] * 9).T.reshape(-1)
        assert np.abs(grads[f"conv{j}.weight"] - g).max() <= 1e-4 * np.abs(g).max()
        gb = tp[f"conv{j}.bias"].grad.numpy()
        assert np.abs(grads[f"conv{j}.bias"] - gb).max() <= 1e-4 * np.abs(gb).max() + 1e-7
    gl = tp["linear.weight"].grad.numpy().reshape(-1)
    assert np.abs(grads["linear.weight"] - gl).max() <= 1e-4 * np.abs(gl).max()


# ---------------------------------------------------------------- pins for the remaining oracle functions

def test_softmax_backward_matches_torch_autograd(oracle):
    # backend.rs:2529-2543 against torch's float64 softmax vector-Jacobian product (an independent
    # implementation): rows of logits with spread and with a dominant entry
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    rows, width = 37, 129
    z = torch.tensor(rng.standard_normal((rows, width)) * 3.0, dtype=torch.float64, requires_grad=True)
    with torch.no_grad():
        z[5, 7] += 40.0
    p = torch.softmax(z, dim=1)
    g = rng.standard_normal((rows, width))
    (vjp,) = torch.autograd.grad(p, z, torch.from_numpy(g))
    got = oracle.softmax_backward(g.astype(np.float32), p.detach().numpy().astype(np.float32), rows, width)
    ref = vjp.numpy()
    err = np.abs(got.reshape(rows, width) - ref)
    assert np.all(err <= 1e-6 + 1e-5 * np.abs(ref)), float(err.max())
    # a dropped "- sum(g p)" term or a sign error would not pass
    wrong = p.detach().numpy() * g
    assert np.abs(wrong - ref).max() > 1e-2


def _brute_extreme(values, groups, maximum):
    out, winners = [], []
    for members in groups:
        best, win = None, -1
        for i in members:
            v = values[i]
            if not np.isfinite(v):
                continue
            if best is None or (v > best if maximum else v < best):
                best, win = v, i
        out.append(np.nan if best is None else best)
        winners.append(win)
    return np.array(out, np.float32), np.array(winners, np.int32)


def test_grouped_maximum_first_strictly_greater_finite(oracle):
    # backend.rs:3059-3099: first strictly greater finite value in plan order, NaN and -1 for a group
    # with none; brute force over shuffled member orders with ties, NaN and infinities, and the
    # identity max(x) = -min(-x) with the minimum pinned by the max-pool fixtures
    rng = np.random.default_rng(8)
    n, count = 600, 97
    values = rng.integers(-4, 5, n).astype(np.float32)
    values[rng.choice(n, 40, replace=False)] = np.nan
    values[rng.choice(n, 20, replace=False)] = np.inf
    values[rng.choice(n, 20, replace=False)] = -np.inf
    owner = rng.integers(0, count, n)
    owner[:8] = count - 1  # a group whose members are all non-finite
    values[:8] = [np.nan, np.inf, -np.inf, np.nan, np.inf, np.nan, -np.inf, np.nan]
    values[np.isin(owner, [count - 1]) & (np.arange(n) >= 8)] = np.nan
    groups = [list(rng.permutation(np.flatnonzero(owner == gi))) for gi in range(count)]
    forward = oracle.plan_groups([[(int(i), 0) for i in members] for members in groups], cap=False)
    reverse = oracle.plan_gather(owner)
    out, mask, winners = oracle.grouped_minimum(values, forward, reverse, maximum=True)
    want, want_w = _brute_extreme(values, groups, True)
    assert np.array_equal(out, want, equal_nan=True)
    assert np.array_equal(winners, want_w)
    assert np.isnan(out[count - 1]) and winners[count - 1] == -1
    expect_mask = np.zeros(n, np.float32)
    expect_mask[want_w[want_w >= 0]] = 1.0
    assert np.array_equal(mask, expect_mask)
    mn, _, mn_w = oracle.grouped_minimum(-values, forward, reverse)
    assert np.array_equal(out, -mn, equal_nan=True) and np.array_equal(winners, mn_w)


def _select_metadata(extents, order, selected):
    """Dense input laid out in `order` (axis indices, outermost first); output row-major over the
    kept dims in dim order; (extent, input_stride, output_stride or -1) per dim."""
    strides = [0] * len(extents)
    s = 1
    for d in reversed(order):
        strides[d] = s
        s *= extents[d]
    kept = [d for d in range(len(extents)) if d != selected]
    out_strides, s = {}, 1
    for d in reversed(kept):
        out_strides[d] = s
        s *= extents[d]
    md = []
    for d, e in enumerate(extents):
        md += [e, strides[d], -1 if d == selected else out_strides[d]]
    return md, strides


@pytest.mark.parametrize("extents,order,selected,coordinate", [
    ((3, 4, 5), (0, 1, 2), 1, 2), ((3, 4, 5), (2, 0, 1), 0, 1), ((2, 3, 4, 5), (3, 1, 0, 2), 2, 3),
    ((6, 1, 7), (1, 2, 0), 2, 6)])
def test_select_axis_pair_against_numpy_and_adjoint(oracle, extents, order, selected, coordinate):
    # backend.rs:2057-2148: the forward copy against numpy's indexing of the same strided view; the
    # backward as its adjoint, <select(x), y> = <x, select_backward(y)> in float64, and zero off the
    # selected coordinate
    rng = np.random.default_rng(sum(extents) + selected)
    md, strides = _select_metadata(extents, order, selected)
    n = int(np.prod(extents))
    x = rng.standard_normal(n).astype(np.float32)
    view = np.lib.stride_tricks.as_strided(x, shape=extents, strides=[s * 4 for s in strides])
    out_len = n // extents[selected]
    got = oracle.select_axis(x, md, len(extents), coordinate, out_len)
    assert np.array_equal(got, np.take(view, coordinate, axis=selected).reshape(-1))
    y = rng.standard_normal(out_len).astype(np.float32)
    back = oracle.select_axis_backward(y, md, len(extents), coordinate, n)
    lhs = float(np.dot(got.astype(np.float64), y.astype(np.float64)))
    rhs = float(np.dot(x.astype(np.float64), back.astype(np.float64)))
    assert abs(lhs - rhs) <= 1e-12 * max(1.0, abs(lhs))
    bview = np.lib.stride_tricks.as_strided(back, shape=extents, strides=[s * 4 for s in strides])
    assert np.array_equal(np.take(bview, coordinate, axis=selected).reshape(-1), y)
    assert np.count_nonzero(back) == np.count_nonzero(y)


def _ns_bf16_float64(d, rows, cols, oracle):
    """Newton-Schulz with bf16 product operands in float64 arithmetic, every stored intermediate
    rounded to fp32 as the device's fp32 tensors hold them (optim.rs:728-752; convert_tile +
    mma of backend.rs:2209-2312).  The bf16 rounding itself is torch's."""
    import torch

    def f32(v):
        return np.asarray(v, np.float64).astype(np.float32).astype(np.float64)

    def r(v):
        return torch.from_numpy(np.asarray(v, np.float32)).to(torch.bfloat16).to(torch.float64).numpy()

    a, b, c = 3.4445, -4.7750, 2.0315
    x = oracle.normalized_l2(d, 1e-7).astype(np.float64).reshape(rows, cols)
    if rows > cols:
        x = x.T.copy()
    for _ in range(5):
        gram = f32(r(x) @ r(x).T)
        gram2 = f32(r(gram) @ r(gram))
        bm = f32(f32(np.float32(b) * gram.astype(np.float32)) + f32(np.float32(c) * gram2.astype(np.float32)))
        bx = f32(r(bm) @ r(x))
        x = f32(f32(np.float32(a) * x.astype(np.float32)) + bx)
    return (x.T if rows > cols else x).reshape(-1)


@pytest.mark.parametrize("rows,cols", [(24, 40), (40, 24)])
def test_bf16_zeroth_power_matches_float64_restatement(oracle, rows, cols):
    # the bf16 Newton-Schulz (zeroth_power(..., bf16=True)) against an independent float64
    # restatement; the fp32 zeroth power of the same input lies far from both, so a product whose
    # operands were not rounded would not pass
    rng = np.random.default_rng(rows * cols)
    d = rng.standard_normal(rows * cols).astype(np.float32)
    got = oracle.zeroth_power(d, rows, cols, bf16=True).astype(np.float64)
    want = _ns_bf16_float64(d, rows, cols, oracle)
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    gap = np.linalg.norm(oracle.zeroth_power(d, rows, cols, bf16=False) - want) / np.linalg.norm(want)
    assert err < 1e-5 and gap > 1e-3, (err, gap)


def test_cnn_decision_replay_is_exact_and_used(oracle):
    # a forward's own pool winners and ReLU signs, replayed, give bit-identical gradients (so the
    # window and activation layouts of the replay are the forward's); moving one winner changes them
    batch, size, classes, ch = 2, 16, 10, (3, 8, 16, 32)
    x, y, params = oracle.cnn_inputs(batch, size, classes, ch)
    loss, grads, made = oracle.cnn_forward_backward(x, y, params, batch, size, classes, ch,
                                                    return_decisions=True)
    assert [d[0].shape for d in made] == [(2, 8, 8, 8), (2, 4, 4, 16), (2, 2, 2, 32)]
    assert all(np.all(d[0] < 4) for d in made)
    loss2, grads2 = oracle.cnn_forward_backward(x, y, params, batch, size, classes, ch, decisions=made)
    assert loss2 == loss
    for name in grads:
        assert np.array_equal(grads[name], grads2[name]), name
    # the decision margins: winners sit where the window's best value is, the gap is that best
    # minus the runner-up, and the ReLU sign at the winner is the sign of the best pre-activation
    for a, p, gap, zmax in made:
        assert gap.shape == a.shape == zmax.shape and np.all(gap >= 0)
        assert np.array_equal(p > 0, zmax > 0)
        assert np.array_equal(p[p > 0], zmax[p > 0])
    moved = [(a.copy(), p.copy()) for a, p, *_ in made]
    pos = np.argwhere(moved[2][1] > 0)[0]
    moved[2][0][tuple(pos)] = (moved[2][0][tuple(pos)] + 1) % 4
    _, grads3 = oracle.cnn_forward_backward(x, y, params, batch, size, classes, ch, decisions=moved)
    assert not np.array_equal(grads3["conv2.weight"], grads["conv2.weight"])
    assert np.array_equal(grads3["linear.weight"], grads["linear.weight"])


def test_block_decision_check_accepts_own_and_catches_moved_winner(oracle):
    # the config-4 decision check (tests/test_configs_gpu.check_block_decisions) passes a forward's
    # own decisions and fails when one clearly decided winner moves or a clear ReLU sign flips
    from tests.test_configs_gpu import check_block_decisions
    batch, size, classes, ch = 4, 16, 10, (3, 8, 16, 32)
    x, y, params = oracle.cnn_inputs(batch, size, classes, ch)
    _, _, own = oracle.cnn_forward_backward(x, y, params, batch, size, classes, ch, return_decisions=True)
    made = [(a.reshape(-1).copy(), p.reshape(-1).copy()) for a, p, *_ in own]
    counts = check_block_decisions(made, own)
    assert [c[2:] for c in counts] == [(0, 0)] * 3 and all(c[1] > 0.9 * c[0] for c in counts)
    a, p, gap, z = own[1]
    tol = 1e-4 * np.abs(z).max()
    idx = tuple(np.argwhere((z > tol) & (gap > tol))[0])
    moved = [(m[0].copy(), m[1].copy()) for m in made]
    moved[1][0].reshape(a.shape)[idx] = (a[idx] + 1) % 4
    with pytest.raises(AssertionError):
        check_block_decisions(moved, own)
    flipped = [(m[0].copy(), m[1].copy()) for m in made]
    flipped[2][1].reshape(own[2][0].shape)[tuple(np.argwhere(own[2][3] > 1e-4 * np.abs(own[2][3]).max())[0])] = 0.0
    with pytest.raises(AssertionError):
        check_block_decisions(flipped, own)


def test_first_adam_step_bound_is_exact(oracle):
    # the whole-step parameter check (tests/test_host_gpu.check_first_adam_step) accepts an update
    # whose gradient differs from the oracle's, element by element, by what lr * |u(g) - u(g_ref)|
    # allows (u(x) = x / (|x| + eps)), and rejects a parameter moved past it
    from tests.test_host_gpu import check_first_adam_step
    rng = np.random.default_rng(3)
    p0 = (rng.standard_normal(4096) * 0.05).astype(np.float32)
    g_ref = (rng.standard_normal(4096) * 1e-3).astype(np.float32)
    g = g_ref.copy()
    g[:8] = -g[:8]                                   # sign flips: moves of ~2 lr are allowed there
    g[8:16] = (g[8:16] * np.float32(1.0 + 1e-6)).astype(np.float32)
    g_ref[100] = g[100] = np.float32(3e-6)           # too small a gradient for the 1%-agreement subset
    c1, c2 = 1 - oracle.powi(0.9, 1), 1 - oracle.powi(0.999, 1)
    zero = np.zeros_like(p0)
    p_ref = oracle.adam(p0, g_ref, zero, zero, 1e-3, 0.9, 0.999, c1, c2, 1e-8, 0.0)[0]
    v = oracle.adam(p0, g, zero, zero, 1e-3, 0.9, 0.999, c1, c2, 1e-8, 0.0)[0]
    outside, miss = check_first_adam_step(oracle, "w", v, g, p0, g_ref, p_ref)
    assert miss == 8 / 4096
    bad = p_ref.copy()
    bad[100] += np.float32(1e-4)                       # well inside 2 lr, but its gradients agree exactly
    with pytest.raises(AssertionError):
        check_first_adam_step(oracle, "w", v, g, p0, g_ref, bad)
