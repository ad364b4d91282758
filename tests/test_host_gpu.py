"""The reference's own hot-path tests, replayed through the C++ host layer (named-axis Tensor,
autograd tape, modules, optimizers) on the GPU, plus whole-step parity against the CPU oracle.

Fixture sources are cited per test (src/library/src/... of the reference).  Tolerances: the
reference's close() (3e-6 + 3e-5|e|) for literal fixtures; BASELINE's rel 1e-4 on gradients and
1e-5 on parameters after one step for the whole-model checks (relative to the tensor's max).
"""
import math

import numpy as np
import pytest

import axis_amd
from tests.conftest import close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ax():
    return axis_amd.host()


@pytest.fixture(scope="module")
def device(ax):
    return ax.Device.hip(0)


def rel_max(actual, expected):
    e = np.asarray(expected, np.float64)
    return float(np.abs(np.asarray(actual, np.float64) - e).max() / max(np.abs(e).max(), 1e-30))


# ---------------------------------------------------------------- literal fixtures

def test_seeded_tensors(ax, device):
    # tests.rs:5143-5184
    s, f = ax.Axis("sample"), ax.Axis("feature")
    u = ax.Tensor.uniform([s.of(2), f.of(3)], 7, 0.0, 1.0, device)
    close("uniform", u.to_vec(), [0.0, 0.4375271201133728, 0.755250871181488, 0.4715511202812195,
                                  0.459380567073822, 0.7119333148002625])
    assert not u.requires_grad
    nrm = ax.Tensor.normal([s.of(2), f.of(3)], 99, 0.0, 1.0, device)
    close("normal", nrm.to_vec(), [0.0, 0.0, -0.04610706669773621, 0.15413647086258625,
                                   1.160083365411145, -1.2878684354641539])


def test_conv2d_fixture(ax, device):
    # tests.rs:1372-1421
    ch, h, w, out = ax.Axis("channel"), ax.Axis("height"), ax.Axis("width"), ax.Axis("output")
    x = ax.Tensor.from_slice(np.arange(1, 10, dtype=np.float32), [ch.of(1), h.of(3), w.of(3)], device).with_grad()
    conv = ax.Conv2d(ch, out.of(1), [h, w], [2, 2])
    with pytest.raises(RuntimeError):
        conv.forward(x)
    assert conv.build(x.shape, device, 7) == ax.Shape([h.of(2), w.of(2), out.of(1)])
    conv.parameter("weight").set_values([1.0, 0.0, 0.0, -1.0])
    conv.parameter("bias").set_values([0.5])
    y = conv.forward(x)
    close("Conv2d forward", y.to_vec(), [-3.5] * 4)
    y.mean([h, w, out]).backward()
    close("input gradient", x.grad().to_vec(), [0.25, 0.25, 0.0, 0.25, 0.0, -0.25, 0.0, -0.25, -0.25])
    close("weight gradient", conv.parameter("weight").grad().to_vec(), [3.0, 4.0, 6.0, 7.0])
    close("bias gradient", conv.parameter("bias").grad().to_vec(), [1.0])
    with pytest.raises(RuntimeError):
        conv.output_shape(ax.Shape([ch.of(2), h.of(3), w.of(3)]))


def test_max_pool_ties_fixture(ax, device):
    # tests.rs:4004-4059 (channel-major input: the generic unfold/min lowering)
    ch, h, w = ax.Axis("channel"), ax.Axis("height"), ax.Axis("width")
    values = [1, 5, 2, 6, 5, 3, 6, 0.5, 9, 9, 9, 9, -1, -2, -3, -4, -5, -0.5, -6, -7, 0, 0, 0, 0]
    x = ax.Tensor.from_slice(values, [ch.of(2), h.of(3), w.of(4)], device).with_grad()
    pool = ax.MaxPool2d(ch, [h, w], [2, 2])
    assert pool.build(x.shape, device, 0) == ax.Shape([h.of(1), w.of(2), ch.of(2)])
    y = pool.forward(x)
    close("MaxPool2d forward", y.to_vec(), [5.0, -0.5, 6.0, -3.0])
    y.mean([ch, h, w]).backward()
    close("MaxPool2d gradient", x.grad().to_vec(),
          [0, .25, 0, .25, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, .25, 0, 0, .25, 0, 0, 0, 0, 0, 0])


def test_max_pool_padding_fixture(ax, device):
    # tests.rs:4063-4114 (physical layout [width, height, channel])
    ch, h, w = ax.Axis("channel"), ax.Axis("height"), ax.Axis("width")
    x = ax.Tensor.from_slice([-1, -9, -2, -8, -7, -9, -3, -9, -4], [ch.of(1), h.of(3), w.of(3)], device)
    x = x.with_layout([w, h, ch]).with_grad()
    pool = ax.MaxPool2d(ch, [h, w], [3, 3]).stride([1, 1]).padding([1, 1])
    assert pool.build(x.shape, device, 0) == ax.Shape([h.of(3), w.of(3), ch.of(1)])
    y = pool.forward(x)
    close("padded forward", y.to_vec(), [-1, -1, -2, -1, -1, -2, -3, -3, -4])
    y.mean([ch, h, w]).backward()
    close("padded gradient", x.grad().to_vec(), [4 / 9, 0, 2 / 9, 0, 0, 0, 2 / 9, 0, 1 / 9])


def test_fused_max_pool_matches_generic_lowering(ax, device):
    # channel-innermost input takes the fused kernel; the same values channel-major take the
    # reference's unfold/min path -- outputs and gradients must agree exactly.
    b, hh, ww, c = 2, 6, 7, 5
    rng = np.random.default_rng(0)
    data = rng.integers(-3, 4, b * hh * ww * c).astype(np.float32)
    bt, h, w, ch = ax.Axis("batch"), ax.Axis("height"), ax.Axis("width"), ax.Axis("channel")
    nhwc = ax.Tensor.from_slice(data, [bt.of(b), h.of(hh), w.of(ww), ch.of(c)], device).with_grad()
    nchw = ax.Tensor.from_slice(data.reshape(b, hh, ww, c).transpose(0, 3, 1, 2).copy(),
                                [bt.of(b), ch.of(c), h.of(hh), w.of(ww)], device).with_grad()
    pool = ax.MaxPool2d(ch, [h, w], [3, 3]).stride([2, 2]).padding([1, 1])
    y1, y2 = pool.forward(nhwc), pool.forward(nchw)
    assert y1.shape == y2.shape
    assert np.array_equal(y1.to_vec(), y2.to_vec())
    g = ax.Tensor.from_slice(rng.standard_normal(y1.shape.len).astype(np.float32), y1.shape.dims, device)
    y1.mul(g).sum(y1.shape.axes()).backward()
    y2.mul(g).sum(y2.shape.axes()).backward()
    g1 = nhwc.grad().to_vec().reshape(b, hh, ww, c)
    g2 = nchw.grad().to_vec().reshape(b, c, hh, ww).transpose(0, 2, 3, 1)
    assert np.array_equal(g1, g2)


def test_cross_entropy_and_adam_fixtures(ax, device):
    # tests.rs:2384-2500
    cls, batch = ax.Axis("class"), ax.Axis("batch")
    logits = ax.Tensor.from_slice([1000.0, -1.0, 999.0, 0.0, 998.0, 1.0], [cls.of(3), batch.of(2)], device).with_grad()
    targets = ax.Tensor.from_slice([1.0, 0.0, 0.0, 0.0, 0.0, 1.0], [cls.of(3), batch.of(2)], device)
    losses = logits.categorical_cross_entropy_with_logits(targets, cls)
    assert losses.shape == ax.Shape([batch.of(2)])
    expected = math.log(1 + math.exp(-1) + math.exp(-2))
    close("CE", losses.to_vec(), [expected, expected])
    losses.mean([batch]).backward()
    p0 = 1 / (1 + math.exp(-1) + math.exp(-2))
    p1, p2 = math.exp(-1) * p0, math.exp(-2) * p0
    close("CE gradient", logits.grad().to_vec(), [(p0 - 1) / 2, p2 / 2, p1 / 2, p1 / 2, p2 / 2, (p0 - 1) / 2])
    with pytest.raises(RuntimeError):
        logits.detach().categorical_cross_entropy_with_logits(targets.with_grad(), cls)
    bad = ax.Tensor.from_slice([1.0, 0.0, 0.0, 0.0, 0.0, 0.5], [cls.of(3), batch.of(2)], device)
    with pytest.raises(RuntimeError, match="row 1 must sum to 1"):
        logits.detach().categorical_cross_entropy_with_logits(bad, cls)

    feature = ax.Axis("feature")
    param = ax.Parameter(ax.Tensor.from_slice([1.0, -2.0], [feature.of(2)], device))
    coefficient = ax.Tensor.from_slice([0.2, -0.4], [feature.of(2)], device)
    adam = ax.Adam(0.01)
    for expected in ([0.99, -1.99], [0.98, -1.98]):
        param.tensor().mul(coefficient).mean([feature]).backward()
        adam.step_parameters([param, param])
        close("Adam", param.tensor().to_vec(), expected)
        param.zero_grad()
    assert adam.completed_steps() == 2
    with pytest.raises(RuntimeError):
        ax.Adam(0.1, 1.0, 0.999, 1e-8)
    param.tensor().scale(0.0).mean([feature]).backward()
    adamw = ax.AdamW(0.1, 0.2)
    adamw.step_parameters([param])
    close("AdamW decay", param.tensor().to_vec(), [0.9604, -1.9404])


def test_adamw_two_step_fixture(ax, device):
    # tests.rs:5237-5286
    unit = ax.Axis("unit")
    param = ax.Parameter(ax.Tensor.from_slice([1.0], [unit.of(1)], device))
    coefficient = ax.Tensor.from_slice([0.4], [unit.of(1)], device)
    adamw = ax.AdamW(0.1, 0.1, 0.8, 0.9, 1e-8)
    for expected in (0.89, 0.7811):
        param.tensor().mul(coefficient).mean([unit]).backward()
        adamw.step_parameters([param])
        close("AdamW", param.tensor().to_vec(), [expected])
        param.zero_grad()
    for args in [(0.0, 0.0), (float("nan"), 0.0), (0.1, -0.1)]:
        with pytest.raises(RuntimeError):
            ax.AdamW(*args)


def test_large_group_bias_gradient_fixture(ax, device):
    # tests.rs:26955-27010: 600 x 2 broadcast add, sums over both axes, exact gradient 600
    batch, ch = ax.Axis("batch"), ax.Axis("channel")
    field = [(i % 97) * 0.01 - 0.3 for i in range(1200)]
    f = ax.Tensor.from_slice(field, [batch.of(600), ch.of(2)], device).with_grad()
    bias = ax.Tensor.from_slice([0.25, -0.75], [ch.of(2)], device).with_grad()
    biased = f.add(bias)
    expected = np.float32(field).reshape(600, 2) + np.float32([0.25, -0.75])
    close("broadcast values", biased.to_vec(), expected.reshape(-1))
    summed = biased.sum([batch])
    close("sum", summed.to_vec(), expected.astype(np.float64).sum(0))
    summed.sum([ch]).backward()
    assert np.array_equal(bias.grad().to_vec(), [600.0, 600.0])
    assert np.array_equal(f.grad().to_vec(), np.ones(1200, np.float32))


@pytest.mark.parametrize("reduced,order,mean", [
    ((0, 2), (2, 0, 3, 1), True),
    ((1, 3), (0, 1, 2, 3), False),
    ((0, 3), (3, 1, 0, 2), True),
    ((1,), (2, 1, 3, 0), False),
    ((0, 1, 2, 3), (1, 3, 0, 2), True),
])
def test_reduce_any_axis_set_and_layout(ax, device, reduced, order, mean):
    """sum/mean over axis sets that are not one consecutive block of a contiguous tensor
    (tensor.rs:2755-2854), through a permuted layout; the gradient is factor * upstream at every
    element, exactly."""
    names = [ax.Axis(f"d{i}") for i in range(4)]
    extents = [6, 5, 7, 4]
    rng = np.random.default_rng(sum(reduced) * 10 + order[0])
    values = rng.standard_normal(int(np.prod(extents))).astype(np.float32)
    x = ax.Tensor.from_slice(values, [a.of(e) for a, e in zip(names, extents)], device).with_grad()
    y = x.with_layout([names[i] for i in order])
    axes = [names[i] for i in reduced]
    r = y.mean(axes) if mean else y.sum(axes)
    expect = values.reshape(extents).astype(np.float64).sum(axis=reduced)
    kept = int(np.prod([extents[i] for i in range(4) if i not in reduced]))
    factor = np.float32(kept) / np.float32(values.size) if mean else np.float32(1.0)
    close("reduce", r.to_vec(), (expect * float(factor)).reshape(-1))
    w = rng.standard_normal(kept).astype(np.float32)
    kept_dims = [names[i].of(extents[i]) for i in range(4) if i not in reduced]
    wt = ax.Tensor.from_slice(w, kept_dims, device) if kept_dims else None
    (r.mul(wt).sum([d for d in r.shape.axes()]) if wt is not None else r).backward()
    wk = w.reshape([extents[i] for i in range(4) if i not in reduced]) if kept_dims else np.float32(1.0)
    grad = np.broadcast_to(np.expand_dims(np.float32(wk) * factor, axis=reduced), extents)
    assert np.array_equal(x.grad().to_vec(), grad.reshape(-1))


def test_reduce_past_the_plan_cap(ax, device):
    """17.8M elements summed over two non-adjacent axes: the reference's plan path rejects this
    (16,777,216 contributions, backend.rs:1588-1596); the strided reduction does not need a plan."""
    names = [ax.Axis(n) for n in ("b", "h", "w", "c")]
    extents = [17, 64, 32, 512]
    rng = np.random.default_rng(3)
    values = rng.standard_normal(int(np.prod(extents))).astype(np.float32)
    x = ax.Tensor.from_slice(values, [a.of(e) for a, e in zip(names, extents)], device)
    r = x.mean([names[0], names[2]])
    expect = values.reshape(extents).astype(np.float64).mean(axis=(0, 2))
    close("mean", r.to_vec(), expect.reshape(-1))


@pytest.mark.parametrize("extents", [(3, 700, 5), (17, 2048, 512)])
def test_align_backward_without_plan(ax, device, oracle, extents):
    """A [a, c] operand broadcast over a middle axis: its gradient is the reverse plan's grouped sum
    (tensor.rs:679-698), taken by the strided reduction -- bit-identical, and past the plan's
    16,777,216 cap for the second shape."""
    A, B, C = extents
    a, b, c = ax.Axis("a"), ax.Axis("b"), ax.Axis("c")
    rng = np.random.default_rng(A)
    n = A * B * C
    xv = rng.standard_normal(n).astype(np.float32)
    wv = rng.standard_normal(n).astype(np.float32)
    tv = rng.standard_normal(A * C).astype(np.float32)
    x = ax.Tensor.from_slice(xv, [a.of(A), b.of(B), c.of(C)], device)
    w = ax.Tensor.from_slice(wv, [a.of(A), b.of(B), c.of(C)], device)
    t = ax.Tensor.from_slice(tv, [a.of(A), c.of(C)], device).with_grad()
    y = x.add(t)
    close("broadcast add", y.to_vec(), (xv.reshape(A, B, C) + tv.reshape(A, 1, C)).reshape(-1))
    y.mul(w).sum([a, b, c]).backward()
    got = t.grad().to_vec()
    if n <= 16777216:
        small = [("a", A), ("c", C)]
        rev = oracle.align_reverse_plan(small, oracle.contiguous(small), [("a", A), ("b", B), ("c", C)])
        assert np.array_equal(got, oracle.grouped(wv, None, rev, 1.0))
    else:
        # a 2048-term fp32 sum against float64
        close("broadcast gradient", got, wv.reshape(A, B, C).astype(np.float64).sum(axis=1).reshape(-1),
              atol=5e-4, rtol=1e-5)


@pytest.mark.parametrize("extents", [(3, 700, 5), (6, 9, 4), (17, 2048, 512)])
def test_align_backward_permuted_operand(ax, device, oracle, extents):
    """A [c, a] operand (axes in the other order than the output's [a, b, c]) broadcast over b: the
    reverse plan's grouped sum lands in the operand's own c-major layout -- bit-identical to the
    plan, and past the plan's 16,777,216 cap for the last shape."""
    A, B, C = extents
    a, b, c = ax.Axis("a"), ax.Axis("b"), ax.Axis("c")
    rng = np.random.default_rng(A + 1)
    n = A * B * C
    xv = rng.standard_normal(n).astype(np.float32)
    wv = rng.standard_normal(n).astype(np.float32)
    tv = rng.standard_normal(A * C).astype(np.float32)
    x = ax.Tensor.from_slice(xv, [a.of(A), b.of(B), c.of(C)], device)
    w = ax.Tensor.from_slice(wv, [a.of(A), b.of(B), c.of(C)], device)
    t = ax.Tensor.from_slice(tv, [c.of(C), a.of(A)], device).with_grad()
    y = x.add(t)
    close("broadcast add", y.to_vec(), (xv.reshape(A, B, C) + tv.reshape(C, A).T.reshape(A, 1, C)).reshape(-1))
    y.mul(w).sum([a, b, c]).backward()
    got = t.grad().to_vec()
    if n <= 16777216:
        small = [("c", C), ("a", A)]
        rev = oracle.align_reverse_plan(small, oracle.contiguous(small), [("a", A), ("b", B), ("c", C)])
        assert np.array_equal(got, oracle.grouped(wv, None, rev, 1.0))
    else:
        close("broadcast gradient", got, wv.reshape(A, B, C).astype(np.float64).sum(axis=1).T.reshape(-1),
              atol=5e-4, rtol=1e-5)


def test_normalized_l2_fixture(ax, device):
    # model/optim.rs:1492-1503
    v = ax.Axis("value")
    t = ax.Tensor.from_slice([3.0, -4.0, 12.0], [v.of(3)], device)
    close("L2", t.normalized_l2(1e-7).to_vec(), np.float32([3, -4, 12]) / (13 + 1e-7), rtol=2e-6)


@pytest.mark.parametrize("rows,cols,fan_in_first", [(3, 2, True), (2, 3, True), (3, 2, False)])
def test_muon_two_step_fixture(ax, device, oracle, rows, cols, fan_in_first):
    # model/optim.rs:992-1073, checked against the oracle (itself pinned by a float64 scalar
    # restatement in test_oracle.py)
    from tests.test_oracle import _scalar_muon
    r, c = ax.Axis("row"), ax.Axis("column")
    n = rows * cols
    initial = np.array([(i - 2.0) * 0.11 for i in range(n)], np.float32)
    grads = [np.array([(i + 1.0) * 0.07 - 0.19 for i in range(n)], np.float32),
             np.array([0.23 - i * 0.035 for i in range(n)], np.float32)]
    param = ax.Parameter(ax.Tensor.from_slice(initial, [r.of(rows), c.of(cols)], device))
    matrix = ax.MuonMatrix.fan_in_fan_out(param) if fan_in_first else ax.MuonMatrix.fan_out_fan_in(param)
    model = ax.ParameterList([("weight", param), ("tied_weight", param)])
    opt = ax.Muon([matrix], 0.04, 0.8, True, 0.03)
    expected, momentum = [float(v) for v in initial], [0.0] * n
    for step, g in enumerate(grads):
        param.zero_grad()
        # set the gradient: d/dp mean(p * g * n) = g
        gt = ax.Tensor.from_slice(g * n, [r.of(rows), c.of(cols)], device)
        param.tensor().mul(gt).mean([r, c]).backward()
        g_now = [float(v) for v in param.grad().to_vec()]
        opt.step(model)
        expected, momentum = _scalar_muon(expected, momentum, g_now,
                                          rows, cols, fan_in_first, 0.04, 0.8, True, 0.03)
        close("Muon momentum", opt.momentum_state(param), momentum, rtol=2e-6)
        close("Muon value", param.tensor().to_vec(), expected, rtol=3e-4)
        assert opt.completed_steps() == step + 1


def test_failures_leave_no_partial_commit(ax, device):
    # tensor.rs:5569-5576 and optim.rs:97-99: double backward, stale parameter, missing gradient
    u = ax.Axis("u")
    p = ax.Parameter(ax.Tensor.from_slice([1.0, 2.0], [u.of(2)], device))
    q = ax.Parameter(ax.Tensor.from_slice([3.0, 4.0], [u.of(2)], device))
    loss = p.tensor().mul(p.tensor()).sum([u])
    loss.backward()
    with pytest.raises(RuntimeError, match="already consumed"):
        loss.backward()
    stale = p.tensor().sum([u])
    p.set_values([5.0, 6.0])
    with pytest.raises(RuntimeError, match="parameter changed"):
        stale.backward()
    adam = ax.Adam(0.1)
    p.tensor().sum([u]).backward()
    with pytest.raises(RuntimeError, match="no gradient"):
        adam.step_parameters([p, q])
    assert adam.completed_steps() == 0
    assert np.array_equal(p.tensor().to_vec(), [5.0, 6.0])


# ---------------------------------------------------------------- whole-step parity

def _set_all(model, named):
    for name, values in named.items():
        model.parameter(name).set_values(values)


def build_mlp(ax, device, batch, sizes):
    bt, feats = ax.Axis("batch"), [ax.Axis(f"f{i}") for i in range(len(sizes))]
    layers = []
    for j in range(len(sizes) - 1):
        layers.append(ax.Linear(feats[j], feats[j + 1].of(sizes[j + 1])))
        if j < len(sizes) - 2:
            layers.append(ax.ReLU())
    model = ax.Sequential(layers)
    model.build(ax.Shape([bt.of(batch), feats[0].of(sizes[0])]), device, 7)
    return model, bt, feats


def check_first_adam_step(oracle, name, v, g, p0, g_ref, p_ref, lr=1e-3):
    """Parameters v after one Adam(lr) step from p0 with our gradients g, against the oracle's whole
    step (p_ref from its gradients g_ref)."""
    # The update is the reference's Adam arithmetic, bit for bit, given these gradients.
    c1, c2 = 1 - oracle.powi(0.9, 1), 1 - oracle.powi(0.999, 1)
    zero = np.zeros_like(p0)
    exact = oracle.adam(p0, g, zero, zero, lr, 0.9, 0.999, c1, c2, 1e-8, 0.0)[0]
    assert np.array_equal(v, exact), name
    # Against the whole oracle step: from zero moments Adam's first update is p0 - lr * u(g) with
    # u(g) = g / (|g| + eps) up to a few ulps (m / c1 = g and sqrt(v / c2) = |g| after one step), so
    # v and the oracle's p_ref differ by exactly lr * |u(g) - u(g_ref)| plus rounding.  That is the
    # bound for every element: an element whose gradient nearly cancels may move by up to 2 lr when
    # its gradient's sign or size differs, and by no more than the difference in u its gradient
    # gives, anywhere.
    g64, gr = np.asarray(g, np.float64), np.asarray(g_ref, np.float64)
    u, u_ref = g64 / (np.abs(g64) + 1e-8), gr / (np.abs(gr) + 1e-8)
    span = np.abs(np.asarray(p_ref, np.float64)).max()
    diff = np.abs(np.asarray(v, np.float64) - p_ref)
    bound = lr * np.abs(u - u_ref) * (1.0 + 1e-3) + 1e-5 * span
    excess = diff > bound
    assert not excess.any(), (name, int(excess.sum()), float((diff - bound).max()))
    # Returned for the record: the fraction of parameters whose gradient is not within 1% of the
    # oracle's (where the bound above exceeds 1e-5 of the tensor's range noticeably), and the
    # fraction that actually miss 1e-5 of the tensor's range.
    sure = (np.abs(gr) >= 100.0 * np.abs(g64 - gr)) & (np.abs(gr) >= 1e-5)
    miss = diff > 1e-5 * span
    assert not (miss & sure).any(), name
    return float(1.0 - sure.mean()), float(miss.mean())


def test_mlp_config1_step_matches_oracle(ax, device, oracle):
    sizes, batch = (784, 256, 256, 10), 128
    ref = oracle.mlp_step(batch, sizes)
    model, bt, feats = build_mlp(ax, device, batch, sizes)
    names = {}
    for j in range(len(sizes) - 1):
        names[f"{2 * j}.weight"] = ref["initial"][f"w{j}"]
        names[f"{2 * j}.bias"] = ref["initial"][f"b{j}"]
    _set_all(model, names)
    x = ax.Tensor.from_slice(ref["x"], [bt.of(batch), feats[0].of(784)], device)
    y = ax.Tensor.from_slice(ref["y"], [bt.of(batch), feats[-1].of(10)], device)
    loss = model.forward(x).categorical_cross_entropy_with_logits(y, feats[-1]).mean([bt])
    loss.backward()
    assert abs(loss.item() - ref["loss"]) <= 1e-5 * max(1, abs(ref["loss"]))
    grads = {name: model.parameter(name).grad().to_vec() for name in names}
    ax.Adam(1e-3).step(model)
    for j in range(len(sizes) - 1):
        for kind, key in (("weight", f"w{j}"), ("bias", f"b{j}")):
            g = grads[f"{2 * j}.{kind}"]
            assert rel_max(g, ref["grads"][key]) < 1e-4, (key, rel_max(g, ref["grads"][key]))
            v = model.parameter(f"{2 * j}.{kind}").tensor().to_vec()
            check_first_adam_step(oracle, key, v, g, ref["initial"][key], ref["grads"][key], ref["params"][key])


def test_mlp_config1_step_bf16_device(ax, oracle):
    """Config 1 on a Device.hip_bf16 handle against the oracle's step with bf16-rounded product
    operands (Device::cuda_bf16: parameters, activations and optimizer state stay fp32)."""
    device = ax.Device.hip_bf16(0)
    assert device.bf16_matmul()
    sizes, batch = (784, 256, 256, 10), 128
    ref = oracle.mlp_step(batch, sizes, bf16=True)
    model, bt, feats = build_mlp(ax, device, batch, sizes)
    names = {}
    for j in range(len(sizes) - 1):
        names[f"{2 * j}.weight"] = ref["initial"][f"w{j}"]
        names[f"{2 * j}.bias"] = ref["initial"][f"b{j}"]
    _set_all(model, names)
    x = ax.Tensor.from_slice(ref["x"], [bt.of(batch), feats[0].of(784)], device)
    y = ax.Tensor.from_slice(ref["y"], [bt.of(batch), feats[-1].of(10)], device)
    loss = model.forward(x).categorical_cross_entropy_with_logits(y, feats[-1]).mean([bt])
    loss.backward()
    assert abs(loss.item() - ref["loss"]) <= 1e-5 * max(1, abs(ref["loss"]))
    fp32 = oracle.mlp_step(batch, sizes)
    assert abs(ref["loss"] - fp32["loss"]) > 1e-6  # bf16 operands change the loss
    grads = {name: model.parameter(name).grad().to_vec() for name in names}
    ax.Adam(1e-3).step(model)
    for j in range(len(sizes) - 1):
        for kind, key in (("weight", f"w{j}"), ("bias", f"b{j}")):
            g = grads[f"{2 * j}.{kind}"]
            assert rel_max(g, ref["grads"][key]) < 1e-4, (key, rel_max(g, ref["grads"][key]))
            v = model.parameter(f"{2 * j}.{kind}").tensor().to_vec()
            check_first_adam_step(oracle, key, v, g, ref["initial"][key], ref["grads"][key], ref["params"][key])


@pytest.mark.parametrize("rows,cols", [(64, 96), (160, 48)])
def test_muon_steps_bf16_device(ax, oracle, rows, cols):
    """Two Muon steps (optim.rs:610-678) on a Device.hip_bf16 handle: every Newton-Schulz product
    runs on the bf16 matrix-core path with bf16-rounded operands; the scale-and-add terms, momentum
    and the update stay fp32.  Five bf16 iterations amplify single operand rounding flips (the
    quintic keeps singular values oscillating in a band): the oracle's own result moves by 0.1-2%
    when its input changes by one ulp, so two accumulation orders agree only to that level.  Hence:
    the momentum exactly; the update exactly as the oracle's formula applied to this device's own
    zeroth power of the same direction; that zeroth power nearer the oracle's bf16 restatement
    than the fp32 products are.  test_bf16_newton_schulz_iterations pins each iteration to 2e-4."""
    device = ax.Device.hip_bf16(0)
    r, c = ax.Axis("row"), ax.Axis("column")
    n = rows * cols
    rng = np.random.default_rng(rows * cols)
    initial = rng.standard_normal(n).astype(np.float32) * np.float32(0.05)
    grads = [rng.standard_normal(n).astype(np.float32) for _ in range(2)]
    param = ax.Parameter(ax.Tensor.from_slice(initial, [r.of(rows), c.of(cols)], device))
    model = ax.ParameterList([("weight", param)])
    lr, mu, wd = 0.04, 0.8, 0.03
    opt = ax.Muon([ax.MuonMatrix.fan_in_fan_out(param)], lr, mu, True, wd)
    ref = oracle.MuonOracle(lr, mu, True, wd, bf16=True)
    w = float(np.float32(1.0) - np.float32(mu))
    scaling = float(np.sqrt(max(np.float32(cols) / np.float32(rows), np.float32(1.0)), dtype=np.float32))
    for g in grads:
        param.zero_grad()
        # a gradient of about g: d/dp mean(p * g * n); the oracle takes the gradient the tape produced
        gt = ax.Tensor.from_slice(g * np.float32(n), [r.of(rows), c.of(cols)], device)
        param.tensor().mul(gt).mean([r, c]).backward()
        g_now = param.grad().to_vec()
        before = param.tensor().to_vec()
        opt.step(model)
        got = param.tensor().to_vec()
        ref.step({"w": before}, {"w": g_now}, {"w": (rows, cols)}, {"w": (rows, cols)})
        m = ref.states["w"]
        assert np.array_equal(np.asarray(opt.momentum_state(param), np.float32), m)
        d = oracle.binary(oracle.scale(g_now, w), oracle.scale(m, mu), 0)
        ns = ax.zeroth_power(ax.Tensor.from_slice(d, [r.of(rows), c.of(cols)], device)).to_vec()
        decayed = oracle.scale(before, float(np.float32(1.0) - np.float32(lr) * np.float32(wd)))
        expect = oracle.binary(decayed, oracle.scale(ns, float(np.float32(lr) * np.float32(scaling))), 1)
        assert np.array_equal(got, expect)
        ns_bf, ns_32 = oracle.zeroth_power(d, rows, cols, True), oracle.zeroth_power(d, rows, cols, False)
        err = np.linalg.norm(ns - ns_bf) / np.linalg.norm(ns_bf)
        gap = np.linalg.norm(ns_32 - ns_bf) / np.linalg.norm(ns_bf)
        assert err < gap, (err, gap)


def build_cnn(ax, device, batch, size, classes, ch):
    bt, c0, h, w = ax.Axis("batch"), ax.Axis("channel"), ax.Axis("height"), ax.Axis("width")
    cs = [c0] + [ax.Axis(f"c{j + 1}") for j in range(3)]
    cls = ax.Axis("class")
    layers = []
    for j in range(3):
        layers += [ax.Conv2d(cs[j], cs[j + 1].of(ch[j + 1]), [h, w], [3, 3]).padding([1, 1]), ax.ReLU(),
                   ax.MaxPool2d(cs[j + 1], [h, w], [2, 2])]
    features = ax.Sequential(layers)
    features.build(ax.Shape([bt.of(batch), c0.of(ch[0]), h.of(size), w.of(size)]), device, 1)
    head = ax.Linear(cs[3], cls.of(classes))
    head.build(ax.Shape([bt.of(batch), cs[3].of(ch[3])]), device, 4)
    model = ax.Sequential([features, head])  # parameters: 0.{0,3,6}.{weight,bias}, 1.{weight,bias}
    return model, features, head, bt, c0, h, w, cls


def cnn_names(j):
    return {"conv": [f"0.{3 * i}" for i in range(3)]}


def test_cnn_small_batch_step_matches_oracle(ax, device, oracle):
    batch, size, classes, ch = 8, 32, 1000, (3, 64, 128, 256)
    ref = oracle.cnn_step(batch, size, classes, 1e-3, ch)
    model, features, head, bt, c0, h, w, cls = build_cnn(ax, device, batch, size, classes, ch)
    mapping = {}
    for j in range(3):
        mapping[f"0.{3 * j}.weight"] = f"conv{j}.weight"
        mapping[f"0.{3 * j}.bias"] = f"conv{j}.bias"
    mapping["1.weight"], mapping["1.bias"] = "linear.weight", "linear.bias"
    for ours, theirs in mapping.items():
        model.parameter(ours).set_values(ref["initial"][theirs])
    x = ax.Tensor.from_slice(ref["x"], [bt.of(batch), c0.of(3), h.of(size), w.of(size)], device)
    y = ax.Tensor.from_slice(ref["y"], [bt.of(batch), cls.of(classes)], device)

    def loss_fn(m):
        feats = features.forward(x).mean([h, w])
        return head.forward(feats).categorical_cross_entropy_with_logits(y, cls).mean([bt])

    loss = loss_fn(model)
    loss.backward()
    assert abs(loss.item() - ref["loss"]) <= 1e-5 * max(1, abs(ref["loss"]))
    grads = {ours: model.parameter(ours).grad().to_vec() for ours in mapping}
    ax.Adam(1e-3).step(model)
    for ours, theirs in mapping.items():
        g = grads[ours]
        assert rel_max(g, ref["grads"][theirs]) < 1e-4, (theirs, rel_max(g, ref["grads"][theirs]))
        v = model.parameter(ours).tensor().to_vec()
        check_first_adam_step(oracle, theirs, v, g, ref["initial"][theirs], ref["grads"][theirs],
                              ref["params"][theirs])


def test_cnn_small_batch_step_on_bf16_device_near_fp32_oracle(ax, oracle):
    # The CNN step on a Device.hip_bf16 handle (backend.rs:274-283: every convolution and matrix
    # product rounds its operands to bf16): the implicit-GEMM conv1 path, the deferred bias sums and
    # the bf16 dense products together, held to bf16 operand precision of the fp32 oracle step
    # (measured: gradients 0.6-2.0% of each tensor's max away, loss 1.5e-5 relative)
    device = ax.Device.hip_bf16(0)
    batch, size, classes, ch = 8, 32, 1000, (3, 64, 128, 256)
    ref = oracle.cnn_step(batch, size, classes, 1e-3, ch)
    model, features, head, bt, c0, h, w, cls = build_cnn(ax, device, batch, size, classes, ch)
    mapping = {}
    for j in range(3):
        mapping[f"0.{3 * j}.weight"] = f"conv{j}.weight"
        mapping[f"0.{3 * j}.bias"] = f"conv{j}.bias"
    mapping["1.weight"], mapping["1.bias"] = "linear.weight", "linear.bias"
    for ours, theirs in mapping.items():
        model.parameter(ours).set_values(ref["initial"][theirs])
    x = ax.Tensor.from_slice(ref["x"], [bt.of(batch), c0.of(3), h.of(size), w.of(size)], device)
    y = ax.Tensor.from_slice(ref["y"], [bt.of(batch), cls.of(classes)], device)
    loss = head.forward(features.forward(x).mean([h, w])).categorical_cross_entropy_with_logits(y, cls).mean([bt])
    loss.backward()
    assert abs(loss.item() - ref["loss"]) <= 1e-2 * max(1, abs(ref["loss"]))
    for ours, theirs in mapping.items():
        g = model.parameter(ours).grad().to_vec()
        assert np.all(np.isfinite(g)), theirs
        assert rel_max(g, ref["grads"][theirs]) < 5e-2, (theirs, rel_max(g, ref["grads"][theirs]))


def test_cnn_fused_mean_backwards_match_materialised_broadcasts(ax, device):
    # The CNN step takes three fused backward paths that each fold a launch away: the loss's
    # mean over the batch into the cross-entropy backward (with the classifier's bias gradient), and
    # the mean over [height, width] into conv3's ReLU/pool backward.  A second reader of each mean's
    # input (a zero-weighted sum) keeps the plain rules; every gradient must agree in value.
    batch, size, classes, ch = 4, 16, 50, (3, 8, 16, 32)
    model, features, head, bt, c0, h, w, cls = build_cnn(ax, device, batch, size, classes, ch)
    rng = np.random.default_rng(11)
    x = ax.Tensor.from_slice(rng.uniform(0, 1, batch * 3 * size * size).astype(np.float32),
                             [bt.of(batch), c0.of(3), h.of(size), w.of(size)], device)
    labels = np.zeros((batch, classes), np.float32)
    labels[np.arange(batch), rng.integers(0, classes, batch)] = 1.0
    y = ax.Tensor.from_slice(labels.reshape(-1), [bt.of(batch), cls.of(classes)], device)
    names = [n for n, _ in model.named_parameters()]

    def grads(plain):
        for n in names:
            model.parameter(n).zero_grad()
        pooled = features.forward(x)
        feats = pooled.mean([h, w])
        per_row = head.forward(feats).categorical_cross_entropy_with_logits(y, cls)
        loss = per_row.mean([bt])
        if plain:  # second readers: the means' inputs no longer feed one rule only
            loss = loss.add(pooled.sum(list(pooled.shape.axes())).scale(0.0)).add(per_row.sum([bt]).scale(0.0))
        loss.backward()
        return {n: np.asarray(model.parameter(n).grad().to_vec()) for n in names}

    fused, plain = grads(False), grads(True)
    for n in names:
        assert np.array_equal(fused[n], plain[n]), n


# ---------------------------------------------------------------- convolution block lowerings

def _torch_block(x_nchw, weight, bias, kh, kw, stride, pad, pool):
    """Reference forward in float64 on the CPU: conv2d -> relu -> optional max pool."""
    import torch
    xt = torch.tensor(x_nchw, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(weight, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(bias, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.conv2d(xt, wt, bt, stride=stride, padding=pad).relu()
    if pool is not None:
        k, s, p = pool
        y = torch.nn.functional.max_pool2d(y, k, s, p)
    return xt, wt, bt, y


BLOCK_CASES = [
    # input layout, x requires grad, conv stride, pool (kernel, stride, padding) -- and which lowering runs
    ("nhwc", True, 1, (2, 2, 0)),   # fused Conv2d+ReLU+MaxPool2d
    ("nhwc", True, 1, (3, 2, 1)),   # implicit conv, then separate ReLU and overlapping pool
    ("nhwc", True, 2, (2, 2, 0)),   # strided conv with an input gradient: the explicit unfold lowering
    ("nhwc", False, 2, (2, 2, 0)),  # strided conv without one: implicit forward + wgrad, fused block
    ("nchw", True, 1, (2, 2, 0)),   # channel-major input needing its gradient: explicit lowering
    ("nchw", False, 1, (2, 2, 0)),  # channel-major input without one: repacked implicit conv, fused
]


def _random_mlps():
    rng = np.random.default_rng(4321)
    cases = []
    for _ in range(10):
        depth = int(rng.integers(1, 4))
        sizes = [int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(40, 700))])) for _ in range(depth + 1)]
        sizes[-1] = max(sizes[-1], 2)  # classes
        cases.append((int(rng.choice([1, int(rng.integers(2, 64)), int(rng.integers(64, 700))])), tuple(sizes)))
    return cases


@pytest.mark.parametrize("batch,sizes", _random_mlps())
def test_random_mlp_step_against_torch(ax, device, batch, sizes):
    # Linear (bias in the product) -> ReLU ... -> mean softmax cross-entropy: every fused rule of
    # the MLP path (bias with the ReLU mask, the mean folded into the cross-entropy backward with the
    # last bias gradient) against torch float64 autograd
    import torch
    model, bt, feats = build_mlp(ax, device, batch, list(sizes))
    rng = np.random.default_rng(batch + sum(sizes))
    xv = rng.standard_normal((batch, sizes[0])).astype(np.float32)
    labels = rng.integers(0, sizes[-1], batch)
    yv = np.zeros((batch, sizes[-1]), np.float32)
    yv[np.arange(batch), labels] = 1.0
    x = ax.Tensor.from_slice(xv.reshape(-1), [bt.of(batch), feats[0].of(sizes[0])], device)
    y = ax.Tensor.from_slice(yv.reshape(-1), [bt.of(batch), feats[-1].of(sizes[-1])], device)
    loss = model.forward(x).categorical_cross_entropy_with_logits(y, feats[-1]).mean([bt])
    loss.backward()
    h = torch.tensor(xv, dtype=torch.float64)
    params = []
    for j in range(len(sizes) - 1):
        wv = np.asarray(model.parameter(f"{2 * j}.weight").tensor().to_vec(), np.float64).reshape(sizes[j], sizes[j + 1])
        bv = np.asarray(model.parameter(f"{2 * j}.bias").tensor().to_vec(), np.float64)
        wt = torch.tensor(wv, requires_grad=True)
        bt_ = torch.tensor(bv, requires_grad=True)
        params.append((f"{2 * j}", wt, bt_))
        h = h @ wt + bt_
        if j < len(sizes) - 2:
            h = h.relu()
    ref = torch.nn.functional.cross_entropy(h, torch.tensor(labels))
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-5 * max(1.0, abs(ref.item()))
    for name, wt, bt_ in params:
        assert rel_max(model.parameter(name + ".weight").grad().to_vec(), wt.grad.numpy().reshape(-1)) < 1e-4, name
        assert rel_max(model.parameter(name + ".bias").grad().to_vec(), bt_.grad.numpy()) < 1e-4, name


def _random_blocks():
    rng = np.random.default_rng(777)
    cases = []
    while len(cases) < 16:
        k = int(rng.choice([1, 3, 3, 5]))
        stride = int(rng.choice([1, 1, 2]))
        pool = [(2, 2, 0), (2, 2, 0), (3, 2, 1), (2, 1, 0), None][int(rng.integers(0, 5))]
        c = int(rng.choice([int(rng.integers(1, 9)), 16, 32, 64]))
        out = int(rng.choice([int(rng.integers(1, 40)), 64, 128]))
        hh, ww = int(rng.integers(4, 21)), int(rng.integers(4, 21))
        layout = "nhwc" if rng.integers(0, 3) else "nchw"
        cases.append((layout, bool(rng.integers(0, 2)), int(rng.integers(1, 4)), c, hh, ww, out, k, stride, pool))
    return cases


@pytest.mark.parametrize("layout,needs_grad,b,c,hh,ww,out,k,stride,pool", _random_blocks())
def test_random_conv_blocks_against_torch(ax, device, layout, needs_grad, b, c, hh, ww, out, k, stride, pool):
    # seeded random geometries through whichever lowering the tape picks (fused block, implicit
    # convolution + separate pool, explicit unfold) against torch float64 on the CPU
    import torch
    rng = np.random.default_rng(b * 1000 + c * 100 + hh * 10 + ww + out + k)
    pad = k // 2
    x_nchw = rng.standard_normal((b, c, hh, ww))
    weight = rng.standard_normal((out, c, k, k)) * 0.3
    bias = rng.standard_normal(out) * 0.1
    bt_, ch, h, w, o = ax.Axis("batch"), ax.Axis("channel"), ax.Axis("height"), ax.Axis("width"), ax.Axis("out")
    if layout == "nhwc":
        dims, x_host = [bt_.of(b), h.of(hh), w.of(ww), ch.of(c)], x_nchw.transpose(0, 2, 3, 1)
    else:
        dims, x_host = [bt_.of(b), ch.of(c), h.of(hh), w.of(ww)], x_nchw
    x = ax.Tensor.from_slice(np.ascontiguousarray(x_host, np.float32).reshape(-1), dims, device)
    if needs_grad:
        x = x.with_grad()
    conv = ax.Conv2d(ch, o.of(out), [h, w], [k, k]).padding([pad, pad]).stride([stride, stride])
    layers = [conv, ax.ReLU()]
    if pool is not None:
        layers.append(ax.MaxPool2d(o, [h, w], [pool[0], pool[0]]).stride([pool[1], pool[1]]).padding([pool[2], pool[2]]))
    model = ax.Sequential(layers)
    model.build(x.shape, device, 3)
    conv.parameter("weight").set_values(np.ascontiguousarray(weight.transpose(1, 2, 3, 0), np.float32).reshape(-1))
    conv.parameter("bias").set_values(bias.astype(np.float32))
    y = model.forward(x)
    xt, wt, btt, yt = _torch_block(x_nchw, weight, bias, k, k, stride, pad, pool)
    y_ref = yt.detach().numpy().transpose(0, 2, 3, 1)
    assert rel_max(y.to_vec(), y_ref.reshape(-1)) < 1e-5
    r = rng.standard_normal(y_ref.shape)
    rt = ax.Tensor.from_slice(r.astype(np.float32).reshape(-1), [bt_.of(b), h.of(r.shape[1]), w.of(r.shape[2]), o.of(out)],
                              device)
    y.mul(rt).sum([bt_, h, w, o]).backward()
    (yt * torch.tensor(r.transpose(0, 3, 1, 2), dtype=torch.float64)).sum().backward()
    assert rel_max(conv.parameter("weight").grad().to_vec(), wt.grad.numpy().transpose(1, 2, 3, 0).reshape(-1)) < 1e-4
    assert rel_max(conv.parameter("bias").grad().to_vec(), btt.grad.numpy()) < 1e-4
    if needs_grad:
        gx = xt.grad.numpy()
        gx = gx.transpose(0, 2, 3, 1) if layout == "nhwc" else gx
        assert rel_max(x.grad().to_vec(), gx.reshape(-1)) < 1e-4


@pytest.mark.parametrize("case", range(len(BLOCK_CASES)))
def test_conv_relu_pool_block_lowerings(ax, device, case):
    layout, needs_grad, stride, pool = BLOCK_CASES[case]
    b, c, hh, ww, out, k = 2, 5, 16, 16, 16, 3
    rng = np.random.default_rng(100 + case)
    x_nchw = rng.standard_normal((b, c, hh, ww))
    weight = rng.standard_normal((out, c, k, k)) * 0.3
    bias = rng.standard_normal(out) * 0.1
    bt_, ch, h, w, o = ax.Axis("batch"), ax.Axis("channel"), ax.Axis("height"), ax.Axis("width"), ax.Axis("out")
    if layout == "nhwc":
        dims = [bt_.of(b), h.of(hh), w.of(ww), ch.of(c)]
        x_host = x_nchw.transpose(0, 2, 3, 1)
    else:
        dims = [bt_.of(b), ch.of(c), h.of(hh), w.of(ww)]
        x_host = x_nchw
    x = ax.Tensor.from_slice(np.ascontiguousarray(x_host, np.float32).reshape(-1), dims, device)
    if needs_grad:
        x = x.with_grad()
    conv = ax.Conv2d(ch, o.of(out), [h, w], [k, k]).padding([1, 1]).stride([stride, stride])
    mp = ax.MaxPool2d(o, [h, w], [pool[0], pool[0]]).stride([pool[1], pool[1]]).padding([pool[2], pool[2]])
    model = ax.Sequential([conv, ax.ReLU(), mp])
    model.build(x.shape, device, 3)
    # the reference's weight layout [(c, ky, kx), out]
    conv.parameter("weight").set_values(np.ascontiguousarray(weight.transpose(1, 2, 3, 0), np.float32).reshape(-1))
    conv.parameter("bias").set_values(bias.astype(np.float32))
    y = model.forward(x)
    xt, wt, btt, yt = _torch_block(x_nchw, weight, bias, k, k, stride, 1, pool)
    y_ref = yt.detach().numpy().transpose(0, 2, 3, 1)  # outputs are channel-innermost
    assert y.shape == ax.Shape([bt_.of(b), h.of(y_ref.shape[1]), w.of(y_ref.shape[2]), o.of(out)])
    assert rel_max(y.to_vec(), y_ref.reshape(-1)) < 1e-5
    r = rng.standard_normal(y_ref.shape)
    rt = ax.Tensor.from_slice(r.astype(np.float32).reshape(-1), [bt_.of(b), h.of(r.shape[1]), w.of(r.shape[2]), o.of(out)],
                              device)
    y.mul(rt).sum([bt_, h, w, o]).backward()
    import torch
    (yt * torch.tensor(r.transpose(0, 3, 1, 2), dtype=torch.float64)).sum().backward()
    gw = np.asarray(conv.parameter("weight").grad().to_vec())
    assert rel_max(gw, wt.grad.numpy().transpose(1, 2, 3, 0).reshape(-1)) < 1e-4
    assert rel_max(conv.parameter("bias").grad().to_vec(), btt.grad.numpy()) < 1e-4
    if needs_grad:
        gx = xt.grad.numpy()
        gx = gx.transpose(0, 2, 3, 1) if layout == "nhwc" else gx
        assert rel_max(x.grad().to_vec(), gx.reshape(-1)) < 1e-4
    else:
        assert x.grad() is None


@pytest.mark.parametrize("batch,fin,fout,relu", [(256, 256, 1000, False), (64, 300, 70, True), (5, 3000, 9, False)])
def test_linear_bias_in_product_matches_contract_then_add(ax, device, batch, fin, fout, relu):
    # Linear with a bias runs one product with the bias in its epilogue (or its split-K sum); the
    # reference's lowering is contract then add.  Same values and the same three gradients, bit for
    # bit, including when a ReLU reads the output (the bias gradient then comes from the masked pass)
    bt, fi, fo = ax.Axis("batch"), ax.Axis("fin"), ax.Axis("fout")
    rng = np.random.default_rng(batch + fin + fout)
    xv = rng.standard_normal(batch * fin).astype(np.float32)
    gv = rng.standard_normal(batch * fout).astype(np.float32)
    layer = ax.Linear(fi, fo.of(fout))
    layer.build(ax.Shape([bt.of(batch), fi.of(fin)]), device, 3)
    w = np.asarray(layer.parameter("weight").tensor().to_vec(), np.float32)
    bvals = rng.standard_normal(fout).astype(np.float32)
    layer.parameter("bias").set_values(bvals)
    x1 = ax.Tensor.from_slice(xv, [bt.of(batch), fi.of(fin)], device).with_grad()
    x2 = ax.Tensor.from_slice(xv, [bt.of(batch), fi.of(fin)], device).with_grad()
    wt = ax.Tensor.from_slice(w, layer.parameter("weight").tensor().shape.dims, device).with_grad()
    wi, wo = [d.axis for d in layer.parameter("weight").tensor().shape.dims]
    bb = ax.Tensor.from_slice(bvals, [wo.of(fout)], device).with_grad()
    g = ax.Tensor.from_slice(gv, [bt.of(batch), fo.of(fout)], device)
    fused = layer.forward(x1)
    sep = x2.rename(fi, wi).contract(wt, [wi]).add(bb).rename(wo, fo)
    if relu:
        fused, sep = fused.relu(), sep.relu()
    assert np.array_equal(np.asarray(fused.to_vec()).view(np.uint32), np.asarray(sep.to_vec()).view(np.uint32))
    fused.mul(g).sum([bt, fo]).backward()
    sep.mul(g).sum([bt, fo]).backward()
    pairs = [(x1.grad(), x2.grad()), (layer.parameter("weight").grad(), wt.grad()),
             (layer.parameter("bias").grad(), bb.grad())]
    for got, ref in pairs:
        assert np.array_equal(np.asarray(got.to_vec()).view(np.uint32), np.asarray(ref.to_vec()).view(np.uint32))


@pytest.mark.parametrize("lhs_t,rhs_t,tracked", [(False, True, False), (True, False, False), (True, True, False),
                                                 (False, True, True), (True, False, True)])
def test_contract_reads_transposed_operands(ax, device, lhs_t, rhs_t, tracked):
    # untracked products read a transposed operand in place (NT / TN kernels); tracked ones keep the
    # reference's operand layouts for their saved rules -- same values either way
    i, kk, j = ax.Axis("i"), ax.Axis("k"), ax.Axis("j")
    m, k, n = 96, 80, 72
    rng = np.random.default_rng(7)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    la = ax.Tensor.from_slice(a.reshape(-1), [i.of(m), kk.of(k)], device)
    lb = ax.Tensor.from_slice(b.reshape(-1), [kk.of(k), j.of(n)], device)
    if tracked:
        la, lb = la.with_grad(), lb.with_grad()
    ta = la.with_layout([kk, i]) if lhs_t else la
    tb = lb.with_layout([j, kk]) if rhs_t else lb
    y = ta.contract(tb, [kk])
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert y.shape == ax.Shape([i.of(m), j.of(n)])
    assert rel_max(y.to_vec(), ref.reshape(-1)) < 1e-5
    if tracked:
        g = rng.standard_normal((m, n)).astype(np.float32)
        tg = ax.Tensor.from_slice(g.reshape(-1), [i.of(m), j.of(n)], device)
        y.mul(tg).sum([i, j]).backward()
        assert rel_max(la.grad().to_vec(), (g.astype(np.float64) @ b.T.astype(np.float64)).reshape(-1)) < 1e-4
        assert rel_max(lb.grad().to_vec(), (a.T.astype(np.float64) @ g.astype(np.float64)).reshape(-1)) < 1e-4


@pytest.mark.parametrize("batch,n", [(4096, 64), (3000, 40)])
def test_tied_weight_gradients_accumulate_after_deferred_sums(ax, device, batch, n):
    # one weight used by two products: each product's weight gradient is a split-K sum the backward
    # defers, and adding the two reads the first, which must run before the add; against torch
    # float64 (the batch makes both weight gradients split their reductions)
    import torch
    rng = np.random.default_rng(batch + n)
    bt, a, b = ax.Axis("batch"), ax.Axis("a"), ax.Axis("b")
    wv = (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float32)
    xv = rng.standard_normal((batch, n)).astype(np.float32)
    cv = rng.standard_normal((batch, n)).astype(np.float32)
    w = ax.Parameter(ax.Tensor.from_slice(wv.reshape(-1), [a.of(n), b.of(n)], device))
    x = ax.Tensor.from_slice(xv.reshape(-1), [bt.of(batch), a.of(n)], device)
    coefficient = ax.Tensor.from_slice(cv.reshape(-1), [bt.of(batch), b.of(n)], device)
    h = x.contract(w.tensor(), [a]).relu().rename(b, a)
    out = h.contract(w.tensor(), [a])
    loss = out.mul(coefficient).mean([bt, b])
    loss.backward()
    wt = torch.tensor(wv.astype(np.float64), requires_grad=True)
    ref = ((torch.tensor(xv, dtype=torch.float64) @ wt).relu() @ wt * torch.tensor(cv, dtype=torch.float64)).mean()
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-5 * max(1.0, abs(ref.item()))
    assert rel_max(w.grad().to_vec(), wt.grad.numpy().reshape(-1)) < 1e-4
    # a second backward accumulates into the stored gradient
    h = x.contract(w.tensor(), [a]).relu().rename(b, a)
    h.contract(w.tensor(), [a]).mul(coefficient).mean([bt, b]).backward()
    assert rel_max(w.grad().to_vec(), 2.0 * wt.grad.numpy().reshape(-1)) < 1e-4
