// Immutable named-axis Tensor and its autograd tape (algebra/tensor.rs).  Each op validates
// before any launch, records the reference's Rule for its inputs that require gradients, and
// lowers to libaxis_hip.  Where a hot-path op has a dedicated fused entry (bias broadcast-add,
// contiguous mean, channel-innermost max pooling, softmax + cross-entropy) the op takes it when
// the layouts match and records the rule of that entry; otherwise it takes the reference's
// generic lowering (select_axis copies, CSR plans, unfold + min).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>
#include <unordered_set>

#include "axis.hpp"

namespace axis {

namespace {

std::atomic<uint64_t> next_node{1};
constexpr int64_t kPlanCap = 16777216;  // runtime/backend.rs:1588-1596

void check_plan_size(int64_t count) {
    if (count == 0 || count > kPlanCap)
        raise("index plan must have 1..=16777216 contributions (experimental backend limit)");
}

int32_t to_i32(int64_t v) {
    if (v < std::numeric_limits<int32_t>::min() || v > std::numeric_limits<int32_t>::max())
        raise("value exceeds the i32 kernel index range");
    return (int32_t)v;
}

// Plan::groups / gather (runtime/backend.rs:1549-1583) as host vectors.
struct HostPlan {
    std::vector<int32_t> offsets{0}, left, right;
};

HostPlan plan_gather(const std::vector<int64_t> &map) {
    check_plan_size((int64_t)map.size());
    HostPlan p;
    p.offsets.resize(map.size() + 1);
    for (size_t i = 0; i <= map.size(); ++i) p.offsets[i] = (int32_t)i;
    p.left.reserve(map.size());
    for (int64_t v : map) p.left.push_back(to_i32(v));
    return p;
}

Plan upload(const Device &d, const HostPlan &p) { return d.plan(p.offsets, p.left, p.right); }

std::vector<Edge> one_edge(const Tensor &input, Rule rule) {
    std::vector<Edge> e;
    e.push_back(Edge{input, std::move(rule)});
    return e;
}

Rule rule(Rule::Kind kind) {
    Rule r;
    r.kind = kind;
    return r;
}

void require_same_device(const Tensor &a, const Tensor &b) {
    if (!a.device().same(b.device())) raise("tensors must use the same Device handle");
}

void shared_extents(const Tensor &a, const Tensor &b) {
    for (auto &d : a.shape().dims)
        if (b.shape().contains(d.axis) && b.extent(d.axis) != d.extent)
            raise("extent mismatch for " + d.axis.debug());
}

std::vector<Axis> select_axes(const Shape &shape, const std::vector<Axis> &axes) {
    for (size_t i = 0; i < axes.size(); ++i) {
        shape.index(axes[i]);
        for (size_t j = 0; j < i; ++j)
            if (axes[j] == axes[i]) raise("duplicate selected axis " + axes[i].debug());
    }
    return axes;
}

bool contains(const std::vector<Axis> &axes, const Axis &a) {
    return std::find(axes.begin(), axes.end(), a) != axes.end();
}

// `small` (contiguous) broadcasts along leading axes of `big` (contiguous): its axes are the
// trailing axes of big, in order.  Returns the broadcast width (small's length) or 0.
int64_t trailing_broadcast(const Tensor &small, const Shape &big) {
    const Shape &s = small.shape();
    if (s.rank() == 0 || s.rank() >= big.rank() || !small.is_contiguous()) return 0;
    size_t off = big.rank() - s.rank();
    for (size_t i = 0; i < s.rank(); ++i)
        if (big.dims[off + i].axis != s.dims[i].axis || big.dims[off + i].extent != s.dims[i].extent)
            return 0;
    return s.len;
}

}  // namespace

// ------------------------------------------------------------------ construction

Tensor Tensor::node(const Shape &shape, const Layout &layout, const Buffer &value,
                    const Device &device, std::vector<Edge> edges, bool leaf,
                    std::shared_ptr<uint64_t> version) {
    auto nd = std::make_shared<Node>();
    nd->id = next_node.fetch_add(1);
    nd->shape = shape;
    nd->layout = layout;
    nd->value = value;
    nd->device = device;
    std::vector<Edge> kept;
    for (auto &e : edges)
        if (e.input.n->tracked) kept.push_back(std::move(e));
    nd->tracked = leaf || !kept.empty();
    if (!kept.empty()) nd->edges = std::make_shared<std::vector<Edge>>(std::move(kept));
    if (version) {
        nd->version = version;
        nd->expected_version = *version;
    }
    return Tensor(nd);
}

Tensor Tensor::from_slice(const std::vector<float> &values, const std::vector<Dim> &dims,
                          const Device &device) {
    Shape shape = Shape::make(dims);
    if ((int64_t)values.size() != shape.len) raise("data length does not match shape");
    Tensor t = node(shape, Layout::contiguous(shape), device.upload(values), device, {}, false);
    t.n->host = std::make_shared<std::vector<float>>(values);
    return t;
}

Tensor Tensor::zeros(const std::vector<Dim> &dims, const Device &device) {
    Shape shape = Shape::make(dims);
    return node(shape, Layout::contiguous(shape), device.zeros_buffer(shape.len), device, {}, false);
}

Tensor Tensor::uniform(const std::vector<Dim> &dims, uint64_t seed, float low, float high,
                       const Device &device) {
    if (!(std::isfinite(low) && std::isfinite(high) && low < high))
        raise("uniform requires finite low < high, got low=" + std::to_string(low) +
              " high=" + std::to_string(high));
    Shape shape = Shape::make(dims);
    return from_slice(uniform_host_values(seed, shape.len, low, high), dims, device);
}

Tensor Tensor::normal(const std::vector<Dim> &dims, uint64_t seed, float mean, float std,
                      const Device &device) {
    if (!(std::isfinite(mean) && std::isfinite(std) && std >= 0.0f))
        raise("normal requires finite mean and non-negative std");
    Shape shape = Shape::make(dims);
    return from_slice(normal_host_values(seed, shape.len, mean, std), dims, device);
}

Tensor Tensor::with_grad() const { return node(shape(), layout(), value(), device(), {}, true); }
Tensor Tensor::detach() const { return node(shape(), layout(), value(), device(), {}, false); }

Tensor Tensor::parameter_leaf(std::shared_ptr<uint64_t> version) const {
    return node(shape(), layout(), value(), device(), {}, true, std::move(version));
}

std::vector<float> Tensor::to_vec() const {
    std::vector<float> physical = device().read(value());
    if ((int64_t)physical.size() == shape().len && is_contiguous()) return physical;
    std::vector<float> out((size_t)shape().len);
    const auto &dims = shape().dims;
    std::vector<int64_t> coord(dims.size(), 0);
    int64_t offset = 0;
    for (int64_t i = 0; i < shape().len; ++i) {
        out[(size_t)i] = physical[(size_t)offset];
        for (size_t a = dims.size(); a-- > 0;) {
            ++coord[a];
            offset += layout().strides[a];
            if (coord[a] < dims[a].extent) break;
            offset -= layout().strides[a] * dims[a].extent;
            coord[a] = 0;
        }
    }
    return out;
}

float Tensor::item() const {
    if (shape().rank() != 0) raise("item requires a scalar tensor");
    return to_vec()[0];
}

std::optional<Tensor> Tensor::grad() const {
    if (!n->grad) return std::nullopt;
    return node(shape(), layout(), n->grad, device(), {}, false);
}

void Tensor::zero_grad() const { n->grad.reset(); }

// ------------------------------------------------------------------ elementwise

Tensor Tensor::scale(float factor) const {
    if (!std::isfinite(factor)) raise("scale must be finite");
    Rule r = rule(Rule::Scale);
    r.factor = factor;
    return node(shape(), layout(), device().scale(value(), factor), device(), one_edge(*this, r), false);
}

Tensor Tensor::relu() const {
    Rule r = rule(Rule::Relu);
    r.a = value();
    return node(shape(), layout(), device().relu(value()), device(), one_edge(*this, r), false);
}

Tensor Tensor::inverse_sqrt(float epsilon) const {
    // Rule::InverseSqrt is not on the training hot path; the result carries no edge here.
    if (requires_grad()) raise("inverse_sqrt gradients are not part of this backend");
    return node(shape(), layout(), device().inverse_sqrt(value(), epsilon), device(), {}, false);
}

// tensor.rs:779-818: elementwise ops align both operands to the larger axis set.
Tensor Tensor::binary(const Tensor &rhs, int op) const {
    require_same_device(*this, rhs);
    shared_extents(*this, rhs);
    bool a_in_b = true, b_in_a = true;
    for (auto &a : shape().axes()) a_in_b = a_in_b && rhs.shape().contains(a);
    for (auto &a : rhs.shape().axes()) b_in_a = b_in_a && shape().contains(a);
    if (!a_in_b && !b_in_a)
        raise("incomparable axis sets: elementwise broadcasting cannot introduce an implicit outer product");
    const Shape &target = b_in_a ? shape() : rhs.shape();
    // Fused broadcast add: a contiguous [.., width] operand plus a [width] bias
    // (align's select_axis + binary add in one pass; gradient = the bias's Group rule).
    if (op == 0) {
        const Tensor &big = b_in_a ? *this : rhs;
        const Tensor &small = b_in_a ? rhs : *this;
        int64_t width = big.is_contiguous() ? trailing_broadcast(small, big.shape()) : 0;
        if (width > 0) {
            int64_t rows = big.shape().len / width;
            Buffer out = device().alloc(big.shape().len);
            check(axis_bias_add(device().h(), big.value()->f32(), small.value()->f32(), out->f32(),
                                nullptr, rows, width),
                  "bias_add");
            Rule rb = rule(Rule::BiasBroadcast);
            rb.outer = rows;
            rb.inner = width;
            std::vector<Edge> edges;
            if (b_in_a) {
                edges.push_back(Edge{big, rule(Rule::Identity)});
                edges.push_back(Edge{small, rb});
            } else {
                edges.push_back(Edge{small, rb});
                edges.push_back(Edge{big, rule(Rule::Identity)});
            }
            return node(target, Layout::contiguous(target), out, device(), std::move(edges), false);
        }
    }
    Tensor a = align(target), b = rhs.align(target);
    Buffer value = device().binary(a.value(), b.value(), op);
    std::vector<Edge> edges;
    switch (op) {
    case 0:
        edges.push_back(Edge{a, rule(Rule::Identity)});
        edges.push_back(Edge{b, rule(Rule::Identity)});
        break;
    case 1: {
        edges.push_back(Edge{a, rule(Rule::Identity)});
        Rule s = rule(Rule::Scale);
        s.factor = -1.0f;
        edges.push_back(Edge{b, s});
        break;
    }
    case 2: {
        Rule ma = rule(Rule::Multiply), mb = rule(Rule::Multiply);
        ma.a = b.value();
        mb.a = a.value();
        edges.push_back(Edge{a, ma});
        edges.push_back(Edge{b, mb});
        break;
    }
    default:
        raise("division is not part of this backend's hot path");
    }
    return node(target, Layout::contiguous(target), value, device(), std::move(edges), false);
}

// tensor.rs:706-778
Tensor Tensor::align(const Shape &target) const {
    double started = now_seconds();
    Layout layout = Layout::contiguous(target);
    if (shape() == target && this->layout() == layout) return *this;
    std::vector<size_t> positions;
    for (auto &a : shape().axes()) positions.push_back(target.index(a));
    if (shape().rank() == target.rank()) {
        Tensor ordered = with_layout(target.axes());
        Tensor out = node(target, layout, ordered.value(), device(),
                          one_edge(ordered, rule(Rule::Identity)), false);
        profile("align", started);
        return out;
    }
    std::vector<int32_t> metadata;
    for (size_t index = 0; index < target.rank(); ++index) {
        int64_t input_stride = 0;
        for (size_t own = 0; own < positions.size(); ++own)
            if (positions[own] == index) input_stride = this->layout().strides[own];
        metadata.push_back(to_i32(target.dims[index].extent));
        metadata.push_back(to_i32(input_stride));
        metadata.push_back(to_i32(layout.strides[index]));
    }
    Buffer value = device().select_axis(this->value(), metadata, target.len);
    std::vector<Edge> edges;
    if (requires_grad()) {
        int64_t width = trailing_broadcast(*this, target);
        bool in_order = is_contiguous();
        for (size_t own = 1; own < positions.size() && in_order; ++own) in_order = positions[own] > positions[own - 1];
        if (width > 0) {
            Rule rb = rule(Rule::BiasBroadcast);
            rb.outer = target.len / width;
            rb.inner = width;
            edges.push_back(Edge{*this, rb});
        } else {
            // The reverse plan (tensor.rs:679-698, Plan::reverse) sums each input element's copies in
            // increasing output position: that is the strided reduction over the new axes, which
            // walks every group in increasing memory position of the output gradient and writes the
            // kept axes in the output's order.  An input whose axes run in another order (its
            // layout is a dense permutation) then takes one select_axis copy into its own layout.
            Rule rb = rule(Rule::BroadcastAxes);
            for (size_t index = 0; index < target.rank(); ++index) {
                rb.extents.push_back(target.dims[index].extent);
                rb.strides.push_back(layout.strides[index]);
                bool own = false;
                for (size_t p : positions) own = own || p == index;
                rb.metadata.push_back(own ? 0 : 1);
            }
            if (!in_order) {
                // stride of target axis `index` in the reduced buffer: extents of the kept axes after it
                for (size_t own = 0; own < positions.size(); ++own) {
                    int64_t reduced_stride = 1;
                    for (size_t index = positions[own] + 1; index < target.rank(); ++index)
                        if (!rb.metadata[index]) reduced_stride *= target.dims[index].extent;
                    rb.place.push_back(to_i32(shape().dims[own].extent));
                    rb.place.push_back(to_i32(reduced_stride));
                    rb.place.push_back(to_i32(this->layout().strides[own]));
                }
            }
            edges.push_back(Edge{*this, rb});
        }
    }
    Tensor out = node(target, layout, value, device(), std::move(edges), false);
    profile("align", started);
    return out;
}

// tensor.rs:5278-5333
Tensor Tensor::with_layout(const std::vector<Axis> &order) const {
    double started = now_seconds();
    Layout target = Layout::make(shape(), order);
    if (layout() == target) return *this;
    bool same = true;
    for (size_t i = 0; i < shape().rank(); ++i)
        same = same && (shape().dims[i].extent == 1 || layout().strides[i] == target.strides[i]);
    if (same) return node(shape(), target, value(), device(), one_edge(*this, rule(Rule::Identity)), false);
    std::vector<int32_t> metadata;
    for (size_t i = 0; i < shape().rank(); ++i) {
        metadata.push_back(to_i32(shape().dims[i].extent));
        metadata.push_back(to_i32(layout().strides[i]));
        metadata.push_back(to_i32(target.strides[i]));
    }
    Buffer v = device().select_axis(value(), metadata, shape().len);
    Rule r = rule(Rule::Select);
    r.metadata = metadata;
    r.n = shape().len;
    Tensor out = node(shape(), target, v, device(), one_edge(*this, r), false);
    profile("with_layout", started);
    return out;
}

Tensor Tensor::rename(const Axis &from, const Axis &to) const {
    shape().index(from);
    std::vector<Dim> dims = shape().dims;
    for (auto &d : dims)
        if (d.axis == from) d.axis = to;
    return node(Shape::make(dims), layout(), value(), device(), one_edge(*this, rule(Rule::Identity)),
                false);
}

// tensor.rs:5355-5399
Tensor Tensor::merge(const std::vector<Axis> &axes_in, const Axis &axis) const {
    double started = now_seconds();
    auto axes = select_axes(shape(), axes_in);
    if (axes.empty()) raise("merge requires at least one axis");
    int64_t parts = 1;
    for (auto &a : axes) parts *= extent(a);
    std::vector<Dim> dims;
    bool inserted = false;
    for (auto &d : shape().dims) {
        if (contains(axes, d.axis)) {
            if (!inserted) {
                dims.push_back(Dim{axis, parts});
                inserted = true;
            }
        } else {
            dims.push_back(d);
        }
    }
    Shape merged = Shape::make(dims);
    std::vector<Axis> order;
    for (auto &d : merged.dims) {
        if (d.axis == axis)
            order.insert(order.end(), axes.begin(), axes.end());
        else
            order.push_back(d.axis);
    }
    Tensor ordered = with_layout(order);
    Tensor out = node(merged, Layout::contiguous(merged), ordered.value(), device(),
                      one_edge(ordered, rule(Rule::Identity)), false);
    profile("merge", started);
    return out;
}

// ------------------------------------------------------------------ contraction (tensor.rs:4051-4172)

namespace {

// The batched-matmul reading of a contraction (tensor.rs contract): shared axes kept by both sides
// are batch axes, then the lhs's kept axes (m), the contracted axes (k) and the rhs's kept axes (n).
struct ContractPlan {
    std::vector<Axis> axes, batch_axes, left_axes, right_axes, left_order, right_order, output_order;
    Shape out_shape;
    int64_t batch = 1, m = 1, k = 1, n = 1;
};

ContractPlan plan_contract(const Tensor &lhs, const Tensor &rhs, const std::vector<Axis> &axes_in) {
    ContractPlan c;
    c.axes = select_axes(lhs.shape(), axes_in);
    select_axes(rhs.shape(), c.axes);
    if (c.axes.empty()) raise("outer products (contraction over no axes) are not part of this backend");
    for (auto &a : c.axes) c.k *= lhs.extent(a);
    std::vector<Dim> dims;
    for (auto &d : lhs.shape().dims)
        if (!contains(c.axes, d.axis)) dims.push_back(d);
    for (auto &d : rhs.shape().dims) {
        bool present = contains(c.axes, d.axis);
        for (auto &e : dims) present = present || e.axis == d.axis;
        if (!present) dims.push_back(d);
    }
    c.out_shape = Shape::make(dims);
    for (auto &a : lhs.shape().axes()) {
        if (contains(c.axes, a)) continue;
        if (rhs.shape().contains(a))
            c.batch_axes.push_back(a);
        else
            c.left_axes.push_back(a);
    }
    for (auto &a : rhs.shape().axes())
        if (!contains(c.axes, a) && !lhs.shape().contains(a)) c.right_axes.push_back(a);
    c.left_order = c.batch_axes;
    c.right_order = c.batch_axes;
    c.left_order.insert(c.left_order.end(), c.left_axes.begin(), c.left_axes.end());
    c.left_order.insert(c.left_order.end(), c.axes.begin(), c.axes.end());
    c.right_order.insert(c.right_order.end(), c.axes.begin(), c.axes.end());
    c.right_order.insert(c.right_order.end(), c.right_axes.begin(), c.right_axes.end());
    for (auto &a : c.batch_axes) c.batch *= lhs.extent(a);
    for (auto &a : c.left_axes) c.m *= lhs.extent(a);
    for (auto &a : c.right_axes) c.n *= rhs.extent(a);
    c.output_order = c.batch_axes;
    c.output_order.insert(c.output_order.end(), c.left_axes.begin(), c.left_axes.end());
    c.output_order.insert(c.output_order.end(), c.right_axes.begin(), c.right_axes.end());
    return c;
}

Tensor laid_out_as(const Tensor &t, const std::vector<Axis> &order) {
    Layout l = Layout::make(t.shape(), order);
    return t.layout() == l ? t : t.with_layout(order);
}

bool is_laid_out(const Tensor &t, const std::vector<Axis> &order) {
    return t.layout() == Layout::make(t.shape(), order);
}

// The product's gradient edges: rules save the other operand in its [batch, m, k] / [batch, k, n]
// layout.
void matmul_edges(const ContractPlan &c, const Tensor &left, const Tensor &right, std::vector<Edge> &edges) {
    if (left.requires_grad()) {
        Rule r = rule(Rule::MatmulLeft);
        r.a = right.value();
        r.batch = c.batch, r.m = c.m, r.k = c.k, r.n = c.n;
        edges.push_back(Edge{left, r});
    }
    if (right.requires_grad()) {
        Rule r = rule(Rule::MatmulRight);
        r.a = left.value();
        r.batch = c.batch, r.m = c.m, r.k = c.k, r.n = c.n;
        edges.push_back(Edge{right, r});
    }
}

}  // namespace

Tensor Tensor::contract(const Tensor &rhs, const std::vector<Axis> &axes_in) const {
    require_same_device(*this, rhs);
    shared_extents(*this, rhs);
    const ContractPlan c = plan_contract(*this, rhs, axes_in);
    // An untracked product (no gradient rules to save) reads a transposed operand in place: a
    // contraction-major lhs through the TN kernel, a contraction-minor rhs through the NT kernel
    // (matmul_right_backward / matmul_left_backward compute exactly those products, in the same
    // reduction order).  Tracked products keep the reference's [batch, m, k] x [batch, k, n] operands
    // because their saved rules assume that layout.
    if (!requires_grad() && !rhs.requires_grad()) {
        std::vector<Axis> left_t = c.batch_axes, right_t = c.batch_axes;
        left_t.insert(left_t.end(), c.axes.begin(), c.axes.end());
        left_t.insert(left_t.end(), c.left_axes.begin(), c.left_axes.end());
        right_t.insert(right_t.end(), c.right_axes.begin(), c.right_axes.end());
        right_t.insert(right_t.end(), c.axes.begin(), c.axes.end());
        const bool lhs_plain = is_laid_out(*this, c.left_order), rhs_plain = is_laid_out(rhs, c.right_order);
        Buffer value;
        if (!lhs_plain && is_laid_out(*this, left_t)) {
            Tensor right = laid_out_as(rhs, c.right_order);
            value = device().matmul_right_backward(this->value(), right.value(), c.batch, c.k, c.m, c.n);
        } else if (!rhs_plain && is_laid_out(rhs, right_t)) {
            Tensor left = laid_out_as(*this, c.left_order);
            value = device().matmul_left_backward(left.value(), rhs.value(), c.batch, c.m, c.n, c.k);
        }
        if (value)
            return node(c.out_shape, Layout::make(c.out_shape, c.output_order), value, device(), {}, false);
    }
    Tensor left = laid_out_as(*this, c.left_order), right = laid_out_as(rhs, c.right_order);
    Buffer value = device().matmul(left.value(), right.value(), c.batch, c.m, c.k, c.n);
    std::vector<Edge> edges;
    matmul_edges(c, left, right, edges);
    return node(c.out_shape, Layout::make(c.out_shape, c.output_order), value, device(), std::move(edges),
                false);
}

Tensor Tensor::contract_add(const Tensor &rhs, const std::vector<Axis> &axes_in, const Tensor &bias) const {
    require_same_device(*this, rhs);
    require_same_device(*this, bias);
    shared_extents(*this, rhs);
    const ContractPlan c = plan_contract(*this, rhs, axes_in);
    // The fused form is the separate add's own fused case: a contiguous product (its output order
    // is its shape's order) plus a contiguous bias over exactly its trailing (rhs-kept) axes.
    const bool fusable = (requires_grad() || rhs.requires_grad()) && bias.is_contiguous() &&
                         bias.shape().axes() == c.right_axes &&
                         Layout::make(c.out_shape, c.output_order) == Layout::contiguous(c.out_shape);
    if (!fusable) return contract(rhs, axes_in).add(bias);
    shared_extents(bias, rhs);
    Tensor left = laid_out_as(*this, c.left_order), right = laid_out_as(rhs, c.right_order);
    Buffer value = device().matmul_bias(left.value(), right.value(), bias.value(), c.batch, c.m, c.k, c.n);
    std::vector<Edge> edges;
    matmul_edges(c, left, right, edges);
    if (bias.requires_grad()) {
        Rule rb = rule(Rule::BiasBroadcast);
        rb.outer = c.batch * c.m;
        rb.inner = c.n;
        edges.push_back(Edge{bias, rb});
    }
    return node(c.out_shape, Layout::contiguous(c.out_shape), value, device(), std::move(edges), false);
}

// ------------------------------------------------------------------ reductions (tensor.rs:2755-2946)

Tensor Tensor::reduce(const std::vector<Axis> &axes_in, bool mean, const char *label) const {
    double started = now_seconds();
    auto axes = select_axes(shape(), axes_in);
    std::vector<Dim> out_dims;
    for (auto &d : shape().dims)
        if (!contains(axes, d.axis)) out_dims.push_back(d);
    Shape out_shape = Shape::make(out_dims);
    const float factor = mean ? (float)out_shape.len / (float)shape().len : 1.0f;
    // Fast path: contiguous input whose reduced axes form one consecutive block.  The group sum
    // then reads [outer, reduce, inner] and sums each group in increasing physical order, the
    // reference plan's order (Plan::reverse lists contributions by increasing position).
    std::vector<size_t> pos;
    for (auto &a : axes) pos.push_back(shape().index(a));
    std::sort(pos.begin(), pos.end());
    bool block = is_contiguous() && !pos.empty();
    for (size_t i = 1; i < pos.size() && block; ++i) block = pos[i] == pos[i - 1] + 1;
    Buffer value;
    Rule r;
    if (block) {
        int64_t outer = 1, red = 1, inner = 1;
        for (size_t i = 0; i < shape().rank(); ++i) {
            if (i < pos.front())
                outer *= shape().dims[i].extent;
            else if (i <= pos.back())
                red *= shape().dims[i].extent;
            else
                inner *= shape().dims[i].extent;
        }
        value = device().alloc(out_shape.len);
        check(axis_reduce_middle(device().h(), this->value()->f32(), value->f32(), outer, red, inner,
                                 factor),
              label);
        r.kind = Rule::MeanMiddle;
        r.outer = outer, r.reduce = red, r.inner = inner, r.factor = factor;
    } else {
        // Any other axis set: the strided reduction walks each group in increasing memory
        // position, the reverse plan's order, without building an element-sized plan.
        r.kind = Rule::ReduceAxes;
        for (size_t i = 0; i < shape().rank(); ++i) {
            r.extents.push_back(shape().dims[i].extent);
            r.strides.push_back(layout().strides[i]);
            r.metadata.push_back(contains(axes, shape().dims[i].axis) ? 1 : 0);
        }
        r.factor = factor;
        value = device().alloc(out_shape.len);
        check(axis_reduce_axes(device().h(), this->value()->f32(), value->f32(), (int32_t)shape().rank(),
                               r.extents.data(), r.strides.data(), r.metadata.data(), factor),
              label);
    }
    Tensor out = node(out_shape, Layout::contiguous(out_shape), value, device(), one_edge(*this, r), false);
    profile(label, started);
    return out;
}

Tensor Tensor::mean(const std::vector<Axis> &axes) const { return reduce(axes, true, "mean"); }
Tensor Tensor::sum(const std::vector<Axis> &axes) const { return reduce(axes, false, "sum"); }

Tensor Tensor::min(const Axis &axis) const {
    double started = now_seconds();
    size_t reduced = shape().index(axis);
    int64_t ext = extent(axis);
    std::vector<Dim> out_dims;
    for (auto &d : shape().dims)
        if (d.axis != axis) out_dims.push_back(d);
    Shape out_shape = Shape::make(out_dims);
    if (shape().len <= (int64_t)INT32_MAX - 256) {
        // The plans' order (each output's members by increasing coordinate along the axis) walked
        // through the strides: no element-sized plan and no 16,777,216 cap.
        Rule r = rule(Rule::MinimumAxis);
        for (size_t i = 0; i < shape().rank(); ++i) {
            r.extents.push_back(shape().dims[i].extent);
            r.strides.push_back(layout().strides[i]);
        }
        r.metadata.push_back((int32_t)reduced);
        Buffer value = device().alloc(out_shape.len);
        r.a = device().alloc(shape().len);
        check(axis_extreme_axis(device().h(), this->value()->f32(), (int32_t)shape().rank(), r.extents.data(),
                                r.strides.data(), (int32_t)reduced, 0, value->f32(), r.a->f32()),
              "min");
        Tensor out = node(out_shape, Layout::contiguous(out_shape), value, device(), one_edge(*this, r), false);
        profile("min", started);
        return out;
    }
    std::vector<int64_t> map((size_t)shape().len);
    HostPlan forward;
    check_plan_size(shape().len);
    forward.offsets.reserve((size_t)out_shape.len + 1);
    forward.left.reserve((size_t)shape().len);
    for (int64_t o = 0; o < out_shape.len; ++o) {
        auto oc = out_shape.coords(o);
        for (int64_t c = 0; c < ext; ++c) {
            auto ic = oc;
            ic.insert(ic.begin() + (long)reduced, c);
            int64_t physical = layout().offset(ic);
            map[(size_t)physical] = o;
            forward.left.push_back((int32_t)physical);
        }
        forward.offsets.push_back((int32_t)forward.left.size());
    }
    Plan fplan = upload(device(), forward);
    Plan rplan = upload(device(), plan_gather(map));
    auto [value, winners] = device().grouped_minimum(this->value(), fplan, rplan);
    Rule r = rule(Rule::Minimum);
    r.plan = rplan;
    r.a = winners;
    Tensor out = node(out_shape, Layout::contiguous(out_shape), value, device(), one_edge(*this, r), false);
    profile("min", started);
    return out;
}

// ------------------------------------------------------------------ unfold (tensor.rs:3654-3946)

Tensor Tensor::unfold_grouped(const Axis &channels, const std::vector<Axis> &spatial,
                              std::optional<Dim> group, const Dim &patch,
                              const std::vector<int64_t> &kernel, const std::vector<int64_t> &stride,
                              const std::vector<int64_t> &padding, float fill) const {
    const char *name = "unfold2d";
    if (spatial.size() != 2 || kernel.size() != 2 || stride.size() != 2 || padding.size() != 2)
        raise(std::string("Axis ") + name + " supports exactly two spatial axes on this backend");
    if (!std::isfinite(fill) && fill != -std::numeric_limits<float>::infinity())
        raise(std::string(name) + " fill must be finite or negative infinity");
    for (size_t i = 0; i < 2; ++i) {
        if (spatial[i] == channels || (i == 1 && spatial[0] == spatial[1]))
            raise(std::string(name) + " requires distinct channel and spatial axes");
    }
    if (kernel[0] <= 0 || kernel[1] <= 0) raise(std::string(name) + " kernel extents must be positive");
    if (stride[0] <= 0 || stride[1] <= 0) raise(std::string(name) + " stride extents must be positive");
    const Shape &image = shape();
    int64_t channel_extent = image.extent(channels);
    int64_t in_sp[2] = {image.extent(spatial[0]), image.extent(spatial[1])};
    int64_t groups = group ? group->extent : 1;
    if (groups <= 0) raise(std::string(name) + " groups must be positive");
    if (channel_extent % groups) raise(std::string(name) + " channels must be divisible by groups");
    int64_t out_sp[2];
    for (int i = 0; i < 2; ++i) {
        int64_t padded = in_sp[i] + 2 * padding[i];
        if (kernel[i] > padded) raise(std::string(name) + " kernel exceeds the padded spatial extent");
        out_sp[i] = (padded - kernel[i]) / stride[i] + 1;
    }
    int64_t cpg = channel_extent / groups;
    int64_t expected_patch = cpg * kernel[0] * kernel[1];
    if (patch.extent != expected_patch)
        raise(std::string(name) + " patch extent must equal channels per group * kernel volume");
    std::vector<Dim> dims;
    for (auto &d : image.dims) {
        if (d.axis == channels) {
            if (!group) dims.push_back(patch);
        } else if (d.axis == spatial[0]) {
            dims.push_back(Dim{d.axis, out_sp[0]});
        } else if (d.axis == spatial[1]) {
            dims.push_back(Dim{d.axis, out_sp[1]});
        } else {
            dims.push_back(d);
        }
    }
    if (group) {
        dims.push_back(*group);
        dims.push_back(patch);
    }
    Shape out_shape = Shape::make(dims);
    std::vector<Axis> order;
    if (group) order.push_back(group->axis);
    for (auto &a : out_shape.axes())
        if (!(group && a == group->axis) && a != patch.axis) order.push_back(a);
    order.push_back(patch.axis);
    Layout out_layout = Layout::make(out_shape, order);
    if (image.len > std::numeric_limits<int32_t>::max() - 127 ||
        out_shape.len > std::numeric_limits<int32_t>::max() - 127)
        raise(std::string(name) + " tensor is too large for its 32-bit index arithmetic");
    bool has_input = true;
    for (int d = 0; d < 2; ++d) {
        bool any = false;
        for (int64_t o = 0; o < out_sp[d] && !any; ++o)
            for (int64_t off = 0; off < kernel[d] && !any; ++off) {
                int64_t pos = o * stride[d] + off - padding[d];
                any = pos >= 0 && pos < in_sp[d];
            }
        has_input = has_input && any;
    }
    if (!has_input) {
        Rule z = rule(Rule::Zero);
        z.n = image.len;
        return node(out_shape, out_layout, device().zeros_buffer(out_shape.len), device(),
                    one_edge(*this, z), false);
    }
    auto spec = std::make_shared<axis_unfold_spec>();
    std::memset(spec.get(), 0, sizeof(axis_unfold_spec));
    spec->spatial_rank = 2;
    spec->input_len = image.len;
    spec->output_len = out_shape.len;
    spec->input_rank = (int32_t)image.rank();
    spec->output_rank = (int32_t)out_shape.rank();
    if (image.rank() > 8 || out_shape.rank() > 8) raise("unfold supports rank at most 8");
    for (size_t i = 0; i < out_shape.rank(); ++i) {
        const Dim &d = out_shape.dims[i];
        int32_t istride = 0, role = 0;
        if (d.axis == spatial[0])
            role = 1;
        else if (d.axis == spatial[1])
            role = 2;
        else if (group && d.axis == group->axis)
            role = 3;
        else if (d.axis == patch.axis)
            role = 4;
        else
            istride = to_i32(layout().strides[image.index(d.axis)]);
        int32_t *md = spec->forward_metadata + 4 * i;
        md[0] = to_i32(d.extent);
        md[1] = to_i32(out_layout.strides[i]);
        md[2] = istride;
        md[3] = role;
    }
    for (size_t i = 0; i < image.rank(); ++i) {
        const Dim &d = image.dims[i];
        int32_t ostride = 0, role = 0;
        if (d.axis == channels)
            role = 1;
        else if (d.axis == spatial[0])
            role = 2;
        else if (d.axis == spatial[1])
            role = 3;
        else
            ostride = to_i32(out_layout.strides[out_shape.index(d.axis)]);
        int32_t *md = spec->backward_metadata + 4 * i;
        md[0] = to_i32(d.extent);
        md[1] = to_i32(layout().strides[i]);
        md[2] = ostride;
        md[3] = role;
    }
    spec->channels_per_group = to_i32(cpg);
    spec->fill = fill;
    for (int i = 0; i < 2; ++i) {
        spec->kernel[i] = to_i32(kernel[i]);
        spec->stride[i] = to_i32(stride[i]);
        spec->padding[i] = to_i32(padding[i]);
        spec->input_spatial[i] = to_i32(in_sp[i]);
        spec->output_spatial[i] = to_i32(out_sp[i]);
        spec->input_special_strides[i + 1] = to_i32(layout().strides[image.index(spatial[i])]);
        spec->output_special_strides[i] = to_i32(out_layout.strides[out_shape.index(spatial[i])]);
    }
    spec->kernel[2] = spec->stride[2] = spec->input_spatial[2] = spec->output_spatial[2] = 1;
    spec->input_special_strides[0] = to_i32(layout().strides[image.index(channels)]);
    spec->output_special_strides[3] = group ? to_i32(out_layout.strides[out_shape.index(group->axis)]) : 0;
    spec->output_special_strides[4] = to_i32(out_layout.strides[out_shape.index(patch.axis)]);
    Buffer value = device().unfold(this->value(), *spec);
    Rule r = rule(Rule::Unfold);
    r.spec = spec;
    return node(out_shape, out_layout, value, device(), one_edge(*this, r), false);
}

// MaxPool2d forward (convolution.rs:1334-1370): -min(-unfold(x, -inf)) over each window.  A
// contiguous [.., spatial0, spatial1, channels] input takes the fused channel-innermost kernel;
// anything else takes the reference's generic lowering.
Tensor Tensor::max_pool2d(const Axis &channels, const std::vector<Axis> &spatial,
                          const std::vector<int64_t> &kernel, const std::vector<int64_t> &stride,
                          const std::vector<int64_t> &padding) const {
    const Shape &s = shape();
    if (spatial.size() != 2) raise("MaxPool2d needs two spatial axes");
    for (int i = 0; i < 2; ++i) {
        if (kernel[i] <= 0 || stride[i] <= 0) raise("MaxPool2d kernel and stride must be positive");
        if (padding[i] < 0 || 2 * padding[i] > kernel[i])
            raise("MaxPool2d padding must be at most half the kernel extent");
    }
    size_t r = s.rank();
    bool fused = r >= 3 && is_contiguous() && s.dims[r - 1].axis == channels &&
                 s.dims[r - 3].axis == spatial[0] && s.dims[r - 2].axis == spatial[1] &&
                 kernel[0] * kernel[1] < 255;
    int64_t channel_extent = s.extent(channels);
    if (!fused) {
        Axis pool_patch = Axis::make("pool_patch");
        Tensor patches = unfold_grouped(channels, spatial, Dim{channels, channel_extent},
                                        Dim{pool_patch, kernel[0] * kernel[1]}, kernel, stride,
                                        padding, -std::numeric_limits<float>::infinity());
        return patches.scale(-1.0f).min(pool_patch).scale(-1.0f);
    }
    PoolGeometry g;
    g.channels = channel_extent;
    g.height = (int32_t)s.dims[r - 3].extent;
    g.width = (int32_t)s.dims[r - 2].extent;
    g.outer = s.len / (g.channels * g.height * g.width);
    int64_t oh = 0, ow = 0;
    for (int i = 0; i < 2; ++i) {
        g.kernel[i] = (int32_t)kernel[i];
        g.stride[i] = (int32_t)stride[i];
        g.padding[i] = (int32_t)padding[i];
        int64_t padded = (i == 0 ? g.height : g.width) + 2 * padding[i];
        if (kernel[i] > padded) raise("MaxPool2d kernel exceeds the padded spatial extent");
    }
    oh = (g.height + 2 * padding[0] - kernel[0]) / stride[0] + 1;
    ow = (g.width + 2 * padding[1] - kernel[1]) / stride[1] + 1;
    std::vector<Dim> dims(s.dims.begin(), s.dims.end());
    dims[r - 3].extent = oh;
    dims[r - 2].extent = ow;
    Shape out_shape = Shape::make(dims);
    Buffer value = device().alloc(out_shape.len);
    Buffer argmax = device().alloc_bytes(out_shape.len);
    check(axis_max_pool2d(device().h(), this->value()->f32(), value->f32(),
                          static_cast<uint8_t *>(argmax->ptr), g.outer, g.height, g.width, g.channels,
                          g.kernel, g.stride, g.padding),
          "max_pool2d");
    Rule rp = rule(Rule::MaxPool);
    rp.a = argmax;
    rp.pool = g;
    return node(out_shape, Layout::contiguous(out_shape), value, device(), one_edge(*this, rp), false);
}

// ------------------------------------------------------------------ loss (tensor.rs:1485-1557)

Tensor Tensor::categorical_cross_entropy_with_logits(const Tensor &targets, const Axis &cls) const {
    if (targets.requires_grad()) raise("categorical cross-entropy targets cannot require gradients");
    bool ok = targets.shape().contains(cls);
    for (auto &a : targets.shape().axes()) ok = ok && shape().contains(a);
    if (!ok)
        raise("categorical_cross_entropy_with_logits targets must contain the class axis and may "
              "omit only broadcast axes");
    require_same_device(*this, targets);
    shared_extents(*this, targets);
    int64_t width = extent(cls);
    if (width < 2) raise("categorical cross-entropy requires at least two classes");
    std::vector<Dim> ordered_dims;
    for (auto &d : shape().dims)
        if (d.axis != cls) ordered_dims.push_back(d);
    Shape output = Shape::make(ordered_dims);
    ordered_dims.push_back(Dim{cls, width});
    Shape ordered = Shape::make(ordered_dims);
    Tensor logits = align(ordered);
    Tensor t = targets.align(ordered);
    // Target validation (tensor.rs:1520-1536), from the host copy when the targets came from host
    // data in this order (no device round trip), else read back.
    std::vector<float> host = (t.n->host && t.n == targets.n) ? *t.n->host : t.to_vec();
    int64_t rows = output.len;
    for (int64_t row = 0; row < rows; ++row) {
        float sum = 0.0f;
        for (int64_t j = 0; j < width; ++j) {
            float v = host[(size_t)(row * width + j)];
            if (!std::isfinite(v) || v < 0.0f)
                raise("categorical target row " + std::to_string(row) +
                      " must contain finite nonnegative probabilities");
            sum += v;
        }
        if (std::fabs(sum - 1.0f) > 1e-5f)
            raise("categorical target row " + std::to_string(row) + " must sum to 1; observed " +
                  std::to_string(sum));
    }
    Buffer probability = device().alloc(ordered.len);
    Buffer loss = device().alloc(rows);
    check(axis_softmax_cross_entropy(device().h(), logits.value()->f32(), t.value()->f32(),
                                     probability->f32(), loss->f32(), rows, width),
          "softmax_cross_entropy");
    Rule r = rule(Rule::CategoricalCrossEntropy);
    r.a = probability;
    r.b = t.value();
    r.n = width;
    r.m = rows;
    return node(output, Layout::contiguous(output), loss, device(), one_edge(logits, r), false);
}

// tensor.rs:2100-2134
Tensor Tensor::normalized_l2(float epsilon) const {
    if (!std::isfinite(epsilon) || epsilon <= 0.0f)
        raise("L2 normalization epsilon must be finite and positive");
    Shape scalar = Shape::make({});
    const float tiny = std::numeric_limits<float>::min();
    Tensor norm_squared = node(scalar, Layout::contiguous(scalar), device().sum_squares(value()),
                               device(), {}, false);
    Tensor inverse_root = norm_squared.inverse_sqrt(tiny);
    Tensor norm = norm_squared.mul(inverse_root);
    Tensor denominator = norm.add(from_slice({epsilon}, {}, device()));
    Tensor inverse_half = denominator.inverse_sqrt(tiny);
    Tensor inverse = inverse_half.mul(inverse_half);
    return node(shape(), layout(), device().multiply_scalar(value(), inverse.value()), device(), {},
                false);
}

// ------------------------------------------------------------------ backward (tensor.rs:5551-5738)

void Tensor::backward() const {
    if (shape().rank() != 0) raise("backward requires a scalar; reduce the loss axes explicitly");
    if (!requires_grad()) raise("tensor does not require gradients");
    double started = now_seconds();
    std::vector<Tensor> order;
    std::unordered_set<uint64_t> seen;
    std::unordered_map<uint64_t, int> uses;  // edges that read each node
    std::vector<std::pair<Tensor, bool>> stack{{*this, false}};
    while (!stack.empty()) {
        auto [node_t, expanded] = stack.back();
        stack.pop_back();
        if (expanded) {
            order.push_back(node_t);
            continue;
        }
        if (!seen.insert(node_t.id()).second) continue;
        if (node_t.n->consumed) raise("backward graph already consumed; run forward again");
        if (node_t.n->version && *node_t.n->version != node_t.n->expected_version)
            raise("parameter changed between forward and backward");
        stack.push_back({node_t, true});
        if (node_t.n->edges)
            for (auto &e : *node_t.n->edges) {
                ++uses[e.input.id()];
                stack.push_back({e.input, false});
            }
    }
    const Device &dev = device();
    // The last sums of weight and bias gradients (split-K slices, per-block partials) are recorded
    // and run in one launch before the commit; a rule about to read a buffer that such a sum may
    // still have to write asks for it first (finish_before_read).
    struct Deferral {
        const Device &dev;
        bool on = true;
        explicit Deferral(const Device &d) : dev(d) { dev.finish_defer(true); }
        void finish() {
            on = false;
            dev.finish_defer(false);
        }
        ~Deferral() {
            if (on) (void)axis_finish_defer(dev.h(), 0);
        }
    } deferral(dev);
    std::unordered_map<uint64_t, Buffer> adjoints;
    // Bias gradients produced together with a ReLU backward (one pass over the activation), keyed
    // by the bias-add node whose BiasBroadcast edge they answer.
    std::unordered_map<uint64_t, Buffer> fused_bias;
    // Weight gradients produced together with a ReLU/pool backward, keyed by the convolution's
    // pre-activation node: that node then carries no adjoint buffer.
    std::unordered_map<uint64_t, Buffer> fused_weight;
    // Means whose backward broadcast is left to their input's only rule: the input node's adjoint is
    // the mean's output gradient, and this factor (1 / reduced extent) goes with it.
    std::unordered_map<uint64_t, float> lazy_mean;
    // The seed is the device's shared 1.0 when every rule of the root reads it into a fresh buffer;
    // an Identity edge would hand the buffer itself on (possibly to a leaf's stored gradient).
    bool seed_shared = static_cast<bool>(n->edges);
    if (n->edges)
        for (auto &e : *n->edges) seed_shared = seed_shared && e.rule.kind != Rule::Identity;
    adjoints[id()] = seed_shared ? dev.seed_one() : dev.filled(1, 1.0f);
    std::vector<std::pair<Tensor, Buffer>> leaves;
    for (auto it = order.rbegin(); it != order.rend(); ++it) {
        const Tensor &nd = *it;
        auto found = adjoints.find(nd.id());
        if (found == adjoints.end()) raise("internal error: unreachable gradient");
        Buffer g = found->second;
        adjoints.erase(found);
        if (nd.n->edges) {
            dev.finish_before_read(g);
            for (auto &e : *nd.n->edges) {
                const Rule &r = e.rule;
                Buffer c;
                switch (r.kind) {
                case Rule::Identity: c = g; break;
                case Rule::Zero: c = dev.zeros_buffer(r.n); break;
                case Rule::Scale: c = dev.scale(g, r.factor); break;
                case Rule::Multiply: c = dev.binary(g, r.a, 2); break;
                case Rule::Relu: {
                    // relu(bias_add(z, b)) whose add feeds nothing else: mask the gradient and sum
                    // the bias gradient in one pass (same values, same summation order).
                    // Look through renames (single Identity edge, same buffer) to the add node.
                    std::shared_ptr<Node> x = e.input.n;
                    while (uses[x->id] == 1 && x->edges && x->edges->size() == 1 &&
                           (*x->edges)[0].rule.kind == Rule::Identity &&
                           (*x->edges)[0].input.n->value == x->value)
                        x = (*x->edges)[0].input.n;
                    // The add node's other edges all consume the same (masked) adjoint.
                    const Rule *bias_rule = nullptr;
                    if (uses[x->id] == 1 && x->edges) {
                        int biases = 0;
                        for (auto &xe : *x->edges)
                            if (xe.rule.kind == Rule::BiasBroadcast) bias_rule = &xe.rule, ++biases;
                        if (biases != 1) bias_rule = nullptr;
                    }
                    if (bias_rule && bias_rule->outer * bias_rule->inner == g->floats()) {
                        c = dev.alloc(g->floats());
                        Buffer db = dev.alloc(bias_rule->inner);
                        check(axis_bias_gradient(dev.h(), g->f32(), r.a->f32(), c->f32(), db->f32(),
                                                 bias_rule->outer, bias_rule->inner),
                              "bias_gradient");
                        fused_bias[x->id] = db;
                    } else {
                        c = dev.relu_backward(g, r.a);
                    }
                    break;
                }
                case Rule::CategoricalCrossEntropy: {
                    c = dev.alloc(r.m * r.n);
                    auto lazy = lazy_mean.find(nd.id());
                    if (lazy != lazy_mean.end()) {
                        // The logits' producer (through renames) read by nothing else, with one
                        // BiasBroadcast edge over the classes: its bias gradient comes out of this pass.
                        std::shared_ptr<Node> x = e.input.n;
                        while (uses[x->id] == 1 && x->edges && x->edges->size() == 1 &&
                               (*x->edges)[0].rule.kind == Rule::Identity &&
                               (*x->edges)[0].input.n->value == x->value)
                            x = (*x->edges)[0].input.n;
                        const Rule *bias_rule = nullptr;
                        if (uses[x->id] == 1 && x->edges) {
                            int biases = 0;
                            for (auto &xe : *x->edges)
                                if (xe.rule.kind == Rule::BiasBroadcast) bias_rule = &xe.rule, ++biases;
                            if (biases != 1) bias_rule = nullptr;
                        }
                        if (bias_rule && !(bias_rule->outer == r.m && bias_rule->inner == r.n)) bias_rule = nullptr;
                        Buffer db = bias_rule ? dev.alloc(r.n) : Buffer();
                        check(axis_categorical_cross_entropy_backward_mean(dev.h(), g->f32(), lazy->second,
                                                                           r.a->f32(), r.b->f32(), c->f32(),
                                                                           db ? db->f32() : nullptr, r.m, r.n),
                              "categorical_cross_entropy_backward");
                        if (db) fused_bias[x->id] = db;
                    } else
                        check(axis_categorical_cross_entropy_backward(dev.h(), g->f32(), r.a->f32(),
                                                                      r.b->f32(), c->f32(), r.m, r.n),
                              "categorical_cross_entropy_backward");
                    break;
                }
                case Rule::MatmulLeft: c = dev.matmul_left_backward(g, r.a, r.batch, r.m, r.k, r.n); break;
                case Rule::MatmulRight: c = dev.matmul_right_backward(r.a, g, r.batch, r.m, r.k, r.n); break;
                case Rule::Group: c = dev.grouped(g, r.b ? &r.b : nullptr, r.plan, r.factor); break;
                case Rule::Minimum: {
                    Buffer expanded = dev.grouped(g, nullptr, r.plan, 1.0f);
                    c = dev.mask_gradient(expanded, r.a);
                    break;
                }
                case Rule::Unfold: c = dev.unfold_backward(g, *r.spec); break;
                case Rule::Select: c = dev.select_axis_backward(g, r.metadata, r.n); break;
                case Rule::BiasBroadcast: {
                    auto fused = fused_bias.find(nd.id());
                    if (fused != fused_bias.end()) {
                        c = fused->second;
                        fused_bias.erase(fused);
                        break;
                    }
                    c = dev.alloc(r.inner);
                    check(axis_bias_gradient(dev.h(), g->f32(), nullptr, nullptr, c->f32(), r.outer,
                                             r.inner),
                          "bias_gradient");
                    break;
                }
                case Rule::ReduceAxes: {
                    int64_t len = 1;
                    for (int64_t e : r.extents) len *= e;
                    c = dev.alloc(len);
                    check(axis_reduce_axes_backward(dev.h(), g->f32(), c->f32(), (int32_t)r.extents.size(),
                                                    r.extents.data(), r.strides.data(), r.metadata.data(),
                                                    r.factor),
                          "reduce_axes_backward");
                    break;
                }
                case Rule::BroadcastAxes: {
                    int64_t len = 1;
                    for (size_t d = 0; d < r.extents.size(); ++d)
                        if (!r.metadata[d]) len *= r.extents[d];
                    c = dev.alloc(len);
                    check(axis_reduce_axes(dev.h(), g->f32(), c->f32(), (int32_t)r.extents.size(), r.extents.data(),
                                           r.strides.data(), r.metadata.data(), 1.0f),
                          "align_backward");
                    if (!r.place.empty()) c = dev.select_axis(c, r.place, len);
                    break;
                }
                case Rule::MinimumAxis: {
                    int64_t len = 1;
                    for (int64_t e : r.extents) len *= e;
                    c = dev.alloc(len);
                    check(axis_extreme_axis_backward(dev.h(), g->f32(), r.a->f32(), (int32_t)r.extents.size(),
                                                     r.extents.data(), r.strides.data(), r.metadata[0], c->f32()),
                          "min_backward");
                    break;
                }
                case Rule::MeanMiddle: {
                    // A mean read by exactly one rule that can take the broadcast itself (the
                    // cross-entropy of a mean over rows, the ReLU/pool backward of a mean over the
                    // pooled height and width): hand that rule the mean's gradient and factor.
                    const std::shared_ptr<Node> &x = e.input.n;
                    bool lazy = false;
                    if (uses[x->id] == 1 && x->edges && x->edges->size() == 1) {
                        const Rule &xr = (*x->edges)[0].rule;
                        if (xr.kind == Rule::CategoricalCrossEntropy)
                            lazy = r.outer == 1 && r.inner == 1 && r.reduce == xr.m;
                        else if (xr.kind == Rule::ReluPool)
                            lazy = r.outer == xr.pool.outer && r.inner == xr.pool.channels &&
                                   r.reduce == (int64_t)(xr.pool.height / xr.pool.kernel[0]) *
                                                   (xr.pool.width / xr.pool.kernel[1]);
                    }
                    if (lazy && g->floats() == r.outer * r.inner) {
                        c = g;
                        lazy_mean[x->id] = r.factor;
                        break;
                    }
                    c = dev.alloc(r.outer * r.reduce * r.inner);
                    check(axis_broadcast_middle(dev.h(), g->f32(), c->f32(), r.outer, r.reduce, r.inner,
                                                r.factor),
                          "broadcast_middle");
                    break;
                }
                case Rule::ConvData: {
                    const ConvGeometry &q = r.conv;
                    c = dev.alloc(q.batch * q.height * q.width * q.channels);
                    check(axis_conv2d_backward_data(dev.h(), g->f32(), r.a->f32(), c->f32(), q.batch,
                                                    q.height, q.width, q.channels, q.out_channels,
                                                    q.kernel, q.stride, q.padding),
                          "conv2d_backward_data");
                    break;
                }
                case Rule::ConvWeight: {
                    auto fused = fused_weight.find(nd.id());
                    if (fused != fused_weight.end()) {
                        c = fused->second;
                        fused_weight.erase(fused);
                        break;
                    }
                    const ConvGeometry &q = r.conv;
                    c = dev.alloc((int64_t)q.channels * q.kernel[0] * q.kernel[1] * q.out_channels);
                    check(axis_conv2d_backward_weight(dev.h(), r.a->f32(), q.strides(), g->f32(), c->f32(), q.batch,
                                                      q.height, q.width, q.channels, q.out_channels,
                                                      q.kernel, q.stride, q.padding),
                          "conv2d_backward_weight");
                    break;
                }
                case Rule::ReluPool: {
                    // The pre-activation node's bias gradient comes out of the same pass when that
                    // node has exactly one BiasBroadcast edge and no other reader.
                    const PoolGeometry &p = r.pool;
                    const int64_t pooled_len = p.outer * (p.height / p.kernel[0]) * (p.width / p.kernel[1]) * p.channels;
                    auto lazy = lazy_mean.find(nd.id());
                    const float mean_factor = lazy != lazy_mean.end() ? lazy->second : 0.0f;
                    const std::shared_ptr<Node> &x = e.input.n;
                    const Rule *bias_rule = nullptr;
                    const Rule *weight_rule = nullptr;
                    bool others = false;
                    if (uses[x->id] == 1 && x->edges) {
                        int biases = 0, weights = 0;
                        for (auto &xe : *x->edges) {
                            if (xe.rule.kind == Rule::BiasBroadcast) bias_rule = &xe.rule, ++biases;
                            else if (xe.rule.kind == Rule::ConvWeight) weight_rule = &xe.rule, ++weights;
                            else others = true;
                        }
                        if (biases != 1) bias_rule = nullptr;
                        if (weights != 1) weight_rule = nullptr, others = true;
                    }
                    if (bias_rule && !(bias_rule->inner == p.channels &&
                                       bias_rule->outer == p.outer * p.height * p.width))
                        bias_rule = nullptr, others = true;
                    if (weight_rule && !others && weight_rule->conv.out_channels == p.channels &&
                        weight_rule->conv.batch == p.outer) {
                        // The convolution's only gradients are its weight and bias (its input
                        // needs none): both straight from the pooled gradient, without the
                        // pre-activation gradient.
                        const ConvGeometry &q = weight_rule->conv;
                        if (mean_factor != 0.0f) {  // this path reads one gradient per pooled value
                            Buffer full = dev.alloc(pooled_len);
                            check(axis_broadcast_middle(dev.h(), g->f32(), full->f32(), p.outer,
                                                        pooled_len / (p.outer * p.channels), p.channels, mean_factor),
                                  "broadcast_middle");
                            g = full;
                        }
                        Buffer dw = dev.alloc((int64_t)q.channels * q.kernel[0] * q.kernel[1] * q.out_channels);
                        Buffer db = bias_rule ? dev.alloc(p.channels) : Buffer();
                        check(axis_conv2d_relu_pool_backward_weight(
                                  dev.h(), weight_rule->a->f32(), q.strides(), g->f32(), r.b->f32(),
                                  static_cast<const uint8_t *>(r.a->ptr), dw->f32(), db ? db->f32() : nullptr,
                                  q.batch, q.height, q.width, q.channels, q.out_channels, q.kernel, q.stride,
                                  q.padding, p.kernel),
                              "conv2d_relu_pool_backward_weight");
                        fused_weight[x->id] = dw;
                        if (db) fused_bias[x->id] = db;
                        break;  // c stays empty: every edge of x is answered from the maps
                    }
                    c = dev.alloc(p.outer * p.height * p.width * p.channels);
                    Buffer db;
                    if (bias_rule) db = dev.alloc(p.channels);
                    if (mean_factor != 0.0f)
                        check(axis_relu_pool_backward_mean(dev.h(), g->f32(), mean_factor, r.b->f32(),
                                                           static_cast<const uint8_t *>(r.a->ptr), c->f32(),
                                                           db ? db->f32() : nullptr, p.outer, p.height, p.width,
                                                           (int32_t)p.channels, p.kernel),
                              "relu_pool_backward");
                    else
                        check(axis_relu_pool_backward(dev.h(), g->f32(), r.b->f32(),
                                                      static_cast<const uint8_t *>(r.a->ptr), c->f32(),
                                                      db ? db->f32() : nullptr, p.outer, p.height, p.width,
                                                      (int32_t)p.channels, p.kernel),
                              "relu_pool_backward");
                    if (db) fused_bias[x->id] = db;
                    break;
                }
                case Rule::MaxPool: {
                    const PoolGeometry &p = r.pool;
                    c = dev.alloc(p.outer * p.height * p.width * p.channels);
                    check(axis_max_pool2d_backward(dev.h(), g->f32(), static_cast<uint8_t *>(r.a->ptr),
                                                   c->f32(), p.outer, p.height, p.width, p.channels,
                                                   p.kernel, p.stride, p.padding),
                          "max_pool2d_backward");
                    break;
                }
                }
                uint64_t input_id = e.input.id();
                auto existing = adjoints.find(input_id);
                if (existing != adjoints.end()) {
                    dev.finish_before_read(existing->second);
                    dev.finish_before_read(c);
                    existing->second = dev.binary(existing->second, c, 0);
                } else
                    adjoints.emplace(input_id, c);
            }
        } else {
            if (nd.n->grad) dev.finish_before_read(g);
            Buffer sum = nd.n->grad ? dev.binary(nd.n->grad, g, 0) : g;
            leaves.emplace_back(nd, sum);
        }
    }
    deferral.finish();
    // Commit only after every device operation was enqueued successfully.
    for (auto &[leaf, gradient] : leaves) leaf.n->grad = gradient;
    for (auto &nd : order) {
        if (nd.n->edges) {
            nd.n->edges.reset();
            nd.n->consumed = true;
        }
    }
    profile("backward", started);
}

}  // namespace axis
