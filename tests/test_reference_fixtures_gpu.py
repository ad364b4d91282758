"""More of the reference's own hot-path tests replayed through the C++ host layer on the GPU, with
the reference's literals, scalar oracles and tolerances.  Each test cites the reference test it
replays (src/library/src/...).

Tolerances: tests.rs's close() is |a - e| < 3e-6 + 3e-5 |e|; optim.rs's close(tol) is
|a - e| <= tol + tol |e|.
"""
import numpy as np
import pytest

import axis_amd
from tests.conftest import close
from tests.test_oracle import _scalar_muon

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ax():
    return axis_amd.host()


@pytest.fixture(scope="module")
def device(ax):
    return ax.Device.hip(0)


def close_tol(name, actual, expected, tol):
    """model/optim.rs:860-869."""
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    assert a.shape == e.shape, name
    err = np.abs(a - e)
    assert np.all(err <= tol + tol * np.abs(e)), (name, a, e)


def set_gradient(ax, param, gradient):
    """optim.rs:954-968: gradient g through mean(p * (g * len))."""
    t = param.tensor()
    n = t.shape.len
    coefficient = np.asarray(gradient, np.float32) * np.float32(n)
    t.mul(ax.Tensor.from_slice(coefficient, t.shape.dims, t.device())).mean(t.shape.axes()).backward()


def weight_and_bias(ax, device):
    row, column, bias_axis = ax.Axis("row"), ax.Axis("column"), ax.Axis("bias")
    weight = ax.Parameter(ax.Tensor.from_slice([0.2, -0.1, 0.3, 0.5], [row.of(2), column.of(2)], device))
    bias = ax.Parameter(ax.Tensor.from_slice([0.4, -0.6], [bias_axis.of(2)], device))
    return weight, bias, row, column


# ---------------------------------------------------------------- MuonWithAuxAdamW (optim.rs:1155-1441)

def test_hybrid_partitions_deduplicates_ties_and_is_atomic(ax, device):
    # optim.rs:1155-1250
    weight, bias, row, column = weight_and_bias(ax, device)
    model = ax.ParameterList([("weight", weight), ("tied_weight", weight), ("bias", bias), ("tied_bias", bias)])
    wg, bg = [0.3, -0.2, 0.1, 0.4], [0.25, -0.5]
    set_gradient(ax, weight, wg)
    set_gradient(ax, bias, bg)
    opt = ax.MuonWithAuxAdamW([ax.MuonMatrix.axis_linear(weight), ax.MuonMatrix.axis_linear(weight)], 0.02, 0.01, 0.05)
    opt.step(model)
    assert opt.completed_steps() == 1
    expected, _ = _scalar_muon([0.2, -0.1, 0.3, 0.5], [0.0] * 4, [float(np.float32(v)) for v in wg],
                               2, 2, True, 0.02, 0.95, True, 0.05)
    close_tol("hybrid Muon arm", weight.tensor().to_vec(), expected, 3e-4)
    v0 = np.array([0.4, -0.6], np.float32)
    g = np.array(bg, np.float32)
    expected_bias = v0 - np.float32(0.01) * (g / (np.abs(g) + np.float32(1e-8)) + np.float32(0.05) * v0)
    close_tol("hybrid exact AdamW remainder", bias.tensor().to_vec(), expected_bias, 2e-5)

    foreign = ax.Parameter(ax.Tensor.from_slice([1.0, 2.0, 3.0, 4.0], [row.of(2), column.of(2)], device))
    missing = ax.MuonWithAuxAdamW([ax.MuonMatrix.axis_linear(foreign)], 0.02, 0.01, 0.0)
    before_w, before_b = weight.tensor().to_vec(), bias.tensor().to_vec()
    with pytest.raises(RuntimeError, match="do not belong to this model"):
        missing.step(model)
    assert missing.completed_steps() == 0
    assert np.array_equal(weight.tensor().to_vec(), before_w)
    assert np.array_equal(bias.tensor().to_vec(), before_b)


def test_hybrid_rejects_rank_and_auxiliary_failures_without_committing(ax, device):
    # optim.rs:1254-1334
    weight, bias, _, _ = weight_and_bias(ax, device)
    model = ax.ParameterList([("weight", weight), ("bias", bias)])
    with pytest.raises(RuntimeError, match="conflicting matrix orientations"):
        ax.MuonWithAuxAdamW([ax.MuonMatrix.fan_in_fan_out(weight), ax.MuonMatrix.fan_out_fan_in(weight)],
                            0.02, 0.01, 0.0)
    set_gradient(ax, bias, [0.25, -0.5])
    before_w, before_b = weight.tensor().to_vec(), bias.tensor().to_vec()
    wrong_rank = ax.MuonWithAuxAdamW([ax.MuonMatrix.axis_linear(bias)], 0.02, 0.01, 0.0)
    with pytest.raises(RuntimeError, match="must have rank 2"):
        wrong_rank.step(model)
    assert wrong_rank.completed_steps() == 0
    assert np.array_equal(weight.tensor().to_vec(), before_w)
    assert np.array_equal(bias.tensor().to_vec(), before_b)

    weight.zero_grad()
    bias.zero_grad()
    set_gradient(ax, weight, [0.3, -0.2, 0.1, 0.4])
    missing_aux = ax.MuonWithAuxAdamW([ax.MuonMatrix.axis_linear(weight)], 0.02, 0.01, 0.0)
    with pytest.raises(RuntimeError, match="parameter has no gradient"):
        missing_aux.step(model)
    assert missing_aux.completed_steps() == 0
    assert missing_aux.muon.completed_steps() == 0 and missing_aux.adamw.completed_steps() == 0
    assert np.array_equal(weight.tensor().to_vec(), before_w)
    assert np.array_equal(bias.tensor().to_vec(), before_b)


def test_hybrid_failure_after_a_success_is_atomic_against_control(ax, device):
    # optim.rs:1338-1421
    def make():
        weight, bias, _, _ = weight_and_bias(ax, device)
        return ax.ParameterList([("weight", weight), ("bias", bias)]), weight, bias

    subject, sw, sb = make()
    control, cw, cb = make()
    subject_opt = ax.MuonWithAuxAdamW([ax.MuonMatrix.axis_linear(sw)], 0.02, 0.01, 0.01)
    control_opt = ax.MuonWithAuxAdamW([ax.MuonMatrix.axis_linear(cw)], 0.02, 0.01, 0.01)
    for w, b in ((sw, sb), (cw, cb)):
        set_gradient(ax, w, [0.3, -0.2, 0.1, 0.4])
        set_gradient(ax, b, [0.25, -0.5])
    subject_opt.step(subject)
    control_opt.step(control)

    sw.zero_grad()
    sb.zero_grad()
    set_gradient(ax, sw, [-0.12, 0.31, 0.08, -0.27])
    with pytest.raises(RuntimeError, match="parameter has no gradient"):
        subject_opt.step(subject)
    assert subject_opt.completed_steps() == 1
    assert subject_opt.muon.completed_steps() == 1 and subject_opt.adamw.completed_steps() == 1
    assert np.array_equal(sw.tensor().to_vec(), cw.tensor().to_vec())
    assert np.array_equal(sb.tensor().to_vec(), cb.tensor().to_vec())
    # the failed step left both arms' state as the control's: same moments, same momentum
    for a, b in zip(subject_opt.adamw.moments(sb), control_opt.adamw.moments(cb)):
        assert np.array_equal(a, b)
    assert np.array_equal(subject_opt.muon.momentum_state(sw), control_opt.muon.momentum_state(cw))

    cw.zero_grad()
    cb.zero_grad()
    set_gradient(ax, cw, [-0.12, 0.31, 0.08, -0.27])
    set_gradient(ax, cb, [-0.2, 0.15])
    set_gradient(ax, sb, [-0.2, 0.15])
    subject_opt.step(subject)
    control_opt.step(control)
    assert subject_opt.completed_steps() == 2
    close_tol("recovered weight matches control state", sw.tensor().to_vec(), cw.tensor().to_vec(), 3e-5)
    close_tol("recovered bias matches control state", sb.tensor().to_vec(), cb.tensor().to_vec(), 3e-5)


def test_hybrid_allows_an_empty_auxiliary_partition(ax, device):
    # optim.rs:1425-1441
    weight, _, _, _ = weight_and_bias(ax, device)
    model = ax.ParameterList([("weight", weight)])
    set_gradient(ax, weight, [0.3, -0.2, 0.1, 0.4])
    opt = ax.MuonWithAuxAdamW([ax.MuonMatrix.axis_linear(weight)], 0.02, 0.01, 0.0)
    opt.step(model)
    assert opt.completed_steps() == 1
    assert opt.adamw.completed_steps() == 1


def test_muon_without_nesterov_two_gradient_fixture(ax, device):
    # optim.rs:1076-1131
    weight, _, _, _ = weight_and_bias(ax, device)
    model = ax.ParameterList([("weight", weight)])
    opt = ax.Muon([ax.MuonMatrix.axis_linear(weight)], 0.02, 0.7, False, 0.01)
    expected, momentum = [0.2, -0.1, 0.3, 0.5], [0.0] * 4
    for step, g in enumerate(([0.3, -0.2, 0.1, 0.4], [-0.12, 0.31, 0.08, -0.27])):
        weight.zero_grad()
        set_gradient(ax, weight, g)
        opt.step(model)
        expected, momentum = _scalar_muon(expected, momentum, [float(np.float32(v)) for v in g],
                                          2, 2, True, 0.02, 0.7, False, 0.01)
        close_tol("Muon without Nesterov state", opt.momentum_state(weight), momentum, 2e-6)
        close_tol("Muon without Nesterov value", weight.tensor().to_vec(), expected, 3e-4)
        assert opt.completed_steps() == step + 1


# ---------------------------------------------------------------- contractions (tests.rs:575-757)

def test_shared_axes_contract_and_both_input_derivatives(ax, device):
    # tests.rs:575-636: shared batch and head axes, permuted operand layouts, both derivatives
    b, h, f, time = ax.Axis("batch"), ax.Axis("head"), ax.Axis("feature"), ax.Axis("time")
    q, k = time.role("query"), time.role("key")
    av = np.array([(i - 25.0) / 30.0 for i in range(60)], np.float32)
    bv = np.array([(i - 35.0) / 40.0 for i in range(80)], np.float32)
    a = ax.Tensor.from_slice(av, [b.of(2), q.of(3), h.of(2), f.of(5)], device).with_layout([f, b, h, q]).with_grad()
    rhs = ax.Tensor.from_slice(bv, [b.of(2), k.of(4), h.of(2), f.of(5)], device).with_layout([h, f, k, b]).with_grad()
    out = a.contract(rhs, [f])
    assert out.shape == ax.Shape([b.of(2), q.of(3), h.of(2), k.of(4)])
    A = av.astype(np.float64).reshape(2, 3, 2, 5)
    B = bv.astype(np.float64).reshape(2, 4, 2, 5)
    close("shared-axis contraction", out.to_vec(), np.einsum("bqhf,bkhf->bqhk", A, B))
    out.mean([q, k, b, h]).backward()
    da = np.einsum("bkhf->bhf", B)[:, None, :, :].repeat(3, axis=1) / 48.0
    db = np.einsum("bqhf->bhf", A)[:, None, :, :].repeat(4, axis=1) / 48.0
    close("contraction left gradient", a.grad().to_vec(), da)
    close("contraction right gradient", rhs.grad().to_vec(), db)


def test_multiple_axis_contraction_exceeds_plan_limit_with_both_gradients(ax, device):
    # tests.rs:638-712: integer operands, so every sum is exact; both layouts
    batch, row, a_ax, b_ax, column = (ax.Axis(n) for n in ("batch", "row", "a", "b", "column"))
    B, M, A, K, N = 2, 129, 16, 16, 257
    assert B * M * A * K * N > 16_777_216
    lv = (np.arange(B * M * A * K) % 19 - 9).astype(np.float32)
    rv = (np.arange(B * A * K * N) % 17 - 8).astype(np.float32)
    wv = (np.arange(B * M * N) % 5 - 2).astype(np.float32)
    L = lv.astype(np.float64).reshape(B, M, A, K)
    R = rv.astype(np.float64).reshape(B, A, K, N)
    W = wv.astype(np.float64).reshape(B, M, N)
    expected = np.einsum("bmak,bakn->bmn", L, R)
    dl = np.einsum("bmn,bakn->bmak", W, R)
    dr = np.einsum("bmn,bmak->bakn", W, L)
    for reordered in (False, True):
        left = ax.Tensor.from_slice(lv, [batch.of(B), row.of(M), a_ax.of(A), b_ax.of(K)], device)
        right = ax.Tensor.from_slice(rv, [batch.of(B), a_ax.of(A), b_ax.of(K), column.of(N)], device)
        if reordered:
            left = left.with_layout([b_ax, row, batch, a_ax])
            right = right.with_layout([column, b_ax, a_ax, batch])
        left, right = left.with_grad(), right.with_grad()
        output = left.contract(right, [b_ax, a_ax] if reordered else [a_ax, b_ax])
        assert output.shape == ax.Shape([batch.of(B), row.of(M), column.of(N)])
        close("large multi-axis contraction", output.to_vec(), expected)
        weight = ax.Tensor.from_slice(wv, output.shape.dims, device)
        output.mul(weight).sum([batch, row, column]).backward()
        close("large multi-axis left gradient", left.grad().to_vec(), dl)
        close("large multi-axis right gradient", right.grad().to_vec(), dr)
        device.synchronize()


def test_multiple_axis_contraction_literals(ax, device):
    # tests.rs:714-757
    row, ia, ib, column = ax.Axis("row"), ax.Axis("inner_a"), ax.Axis("inner_b"), ax.Axis("column")
    vals = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0]
    left = ax.Tensor.from_slice(vals, [row.of(2), ia.of(2), ib.of(2)], device).with_layout([ib, row, ia]).with_grad()
    right = ax.Tensor.from_slice(vals, [ia.of(2), ib.of(2), column.of(2)], device).with_layout([column, ia, ib]).with_grad()
    output = left.contract(right, [ia, ib])
    assert output.shape == ax.Shape([row.of(2), column.of(2)])
    close("multiple-axis contraction", output.to_vec(), [50.0, 60.0, 114.0, 140.0])
    output.mean([row, column]).backward()
    close("multiple-axis left gradient", left.grad().to_vec(), [0.75, 1.75, 2.75, 3.75, 0.75, 1.75, 2.75, 3.75])
    close("multiple-axis right gradient", right.grad().to_vec(), [1.5, 1.5, 2.0, 2.0, 2.5, 2.5, 3.0, 3.0])


# ---------------------------------------------------------------- ReLU at zero, im2col probe

def test_relu_derivative_including_zero(ax, device):
    # tests.rs:950-956
    f = ax.Axis("feature")
    x = ax.Tensor.from_slice([-1.0, 0.0, 1.0], [f.of(3)], device).with_grad()
    x.relu().mean([f]).backward()
    close("ReLU derivative including zero", x.grad().to_vec(), [0.0, 0.0, 1.0 / 3.0])


def test_unfold2d_distinguishes_equal_extent_spatial_axes(ax, device):
    # tests.rs:1427-1475: the same input unfolded over [height, width] and over [height, time]
    channel, height, width, time = ax.Axis("channel"), ax.Axis("height"), ax.Axis("width"), ax.Axis("time")
    group, patch = ax.Axis("conv_group"), ax.Axis("conv_patch")
    values = [100 * y + 10 * x + t for y in range(3) for x in range(3) for t in range(3)]
    inp = ax.Tensor.from_slice(values, [channel.of(1), height.of(3), width.of(3), time.of(3)], device)
    hw = inp.unfold_grouped(channel, [height, width], group.of(1), patch.of(9), [3, 3], [1, 1], [1, 1], 0.0)
    ht = inp.unfold_grouped(channel, [height, time], group.of(1), patch.of(9), [3, 3], [1, 1], [1, 1], 0.0)
    probe = ((3 + 2) * 3) * 9 + 5  # output h=1, w=2, t=0, patch (ky=1, kx=2)
    assert hw.to_vec()[probe] == 0.0
    assert ht.to_vec()[probe] == 121.0
    again = inp.unfold_grouped(channel, [height, width], group.of(1), patch.of(9), [3, 3], [1, 1], [1, 1], 0.0)
    assert np.array_equal(again.to_vec(), hw.to_vec())


# ---------------------------------------------------------------- grouped convolution (tests.rs:1570-1751)

def test_configured_grouped_conv2d_matches_scalar_forward_and_all_gradients(ax, device):
    BATCHES, CHANNELS, HEIGHT, WIDTH, OUTPUTS, GROUPS = 1, 4, 4, 5, 6, 2
    KERNEL, STRIDE, PADDING = (2, 3), (2, 1), (2, 3)
    OH, OW = 4, 9
    CPG, OPG = CHANNELS // GROUPS, OUTPUTS // GROUPS
    PATCH = CPG * KERNEL[0] * KERNEL[1]
    batch, channel, height, width, output = (ax.Axis(n) for n in ("batch", "channel", "height", "width", "output"))
    inputs = np.array([(i - 31.0) / 17.0 for i in range(BATCHES * CHANNELS * HEIGHT * WIDTH)], np.float32)
    weights = np.array([((i * 7 % 29) - 14.0) / 19.0 for i in range(GROUPS * PATCH * OPG)], np.float32)
    biases = np.array([(i - 2.0) / 11.0 for i in range(OUTPUTS)], np.float32)
    x = ax.Tensor.from_slice(inputs, [batch.of(BATCHES), channel.of(CHANNELS), height.of(HEIGHT), width.of(WIDTH)],
                             device).with_layout([width, batch, channel, height]).with_grad()
    conv = ax.Conv2d(channel, output.of(OUTPUTS), [height, width], list(KERNEL)).stride(list(STRIDE)) \
        .padding(list(PADDING)).groups(GROUPS)
    assert conv.build(x.shape, device, 19) == ax.Shape([batch.of(BATCHES), height.of(OH), width.of(OW), output.of(OUTPUTS)])
    conv.parameter("weight").set_values(weights)
    conv.parameter("bias").set_values(biases)
    # the reference's scalar oracle, in float64
    expected = np.zeros(BATCHES * OH * OW * OUTPUTS)
    din = np.zeros(inputs.size)
    dw = np.zeros(weights.size)
    db = np.zeros(biases.size)
    up = 1.0 / expected.size
    for n in range(BATCHES):
        for oy in range(OH):
            for ox in range(OW):
                for oc in range(OUTPUTS):
                    g, og = oc // OPG, oc % OPG
                    value = float(biases[oc])
                    db[oc] += up
                    for cg in range(CPG):
                        ic = g * CPG + cg
                        for ky in range(KERNEL[0]):
                            for kx in range(KERNEL[1]):
                                iy = oy * STRIDE[0] + ky - PADDING[0]
                                ix = ox * STRIDE[1] + kx - PADDING[1]
                                if iy < 0 or ix < 0 or iy >= HEIGHT or ix >= WIDTH:
                                    continue
                                ii = ((n * CHANNELS + ic) * HEIGHT + iy) * WIDTH + ix
                                wi = (g * PATCH + (cg * KERNEL[0] + ky) * KERNEL[1] + kx) * OPG + og
                                value += float(inputs[ii]) * float(weights[wi])
                                din[ii] += up * float(weights[wi])
                                dw[wi] += up * float(inputs[ii])
                    expected[((n * OH + oy) * OW + ox) * OUTPUTS + oc] = value
    actual = conv.forward(x)
    close("configured grouped Conv2d forward", actual.to_vec(), expected)
    close("cached configured grouped Conv2d forward", conv.forward(x).to_vec(), expected)
    actual.mean([batch, height, width, output]).backward()
    close("configured grouped Conv2d input gradient", x.grad().to_vec(), din)
    close("configured grouped Conv2d weight gradient", conv.parameter("weight").grad().to_vec(), dw)
    close("configured grouped Conv2d bias gradient", conv.parameter("bias").grad().to_vec(), db)
    with pytest.raises(RuntimeError, match="built parameters"):
        conv.groups(1).output_shape(x.shape)

    # a legal strided window wholly in padding: zero before the bias, zero input/weight derivatives
    isolated = ax.Tensor.from_slice([3.0], [channel.of(1), height.of(1), width.of(1)], device).with_grad()
    padded = ax.Conv2d(channel, output.of(1), [height, width], [1, 1]).stride([100, 100]).padding([10, 10])
    padded.build(isolated.shape, device, 23)
    padded.parameter("weight").set_values([2.0])
    padded.parameter("bias").set_values([0.25])
    result = padded.forward(isolated)
    close("all-padding Conv2d forward", result.to_vec(), [0.25])
    result.mean([height, width, output]).backward()
    close("all-padding Conv2d input gradient", isolated.grad().to_vec(), [0.0])
    close("all-padding Conv2d weight gradient", padded.parameter("weight").grad().to_vec(), [0.0])
    close("all-padding Conv2d bias gradient", padded.parameter("bias").grad().to_vec(), [1.0])
