// Parameters and the hot-path modules: Linear (model/nn.rs:186-295), Conv2d
// (model/convolution.rs:38-305), MaxPool2d (convolution.rs:1334-1556), ReLU and Sequential
// (nn.rs:1885-1896, :3731-3790).
#include <atomic>
#include <cmath>

#include "axis.hpp"

namespace axis {

namespace {
std::atomic<uint64_t> next_parameter{1};
}

// ------------------------------------------------------------------ Parameter (nn.rs:14-65)

Parameter Parameter::make(const Tensor &tensor) {
    Parameter p;
    p.s = std::make_shared<ParamState>();
    p.s->id = next_parameter.fetch_add(1);
    p.s->version = std::make_shared<uint64_t>(0);
    p.s->tensor = tensor.parameter_leaf(p.s->version);
    return p;
}

void Parameter::set_values(const std::vector<float> &values) const {
    Tensor current = tensor();
    replace(Tensor::from_slice(values, current.shape().dims, current.device()));
}

void Parameter::replace(const Tensor &t) const {
    *s->version += 1;
    s->tensor = t.parameter_leaf(s->version);
}

std::vector<Parameter> Module::parameters() {
    std::vector<Parameter> out;
    for (auto &kv : named_parameters()) out.push_back(kv.second);
    return out;
}

Parameter Module::parameter(const std::string &name) {
    std::optional<Parameter> found;
    for (auto &kv : named_parameters()) {
        if (kv.first != name) continue;
        if (found) raise("ambiguous parameter path \"" + name + "\"");
        found = kv.second;
    }
    if (!found) raise("unknown parameter \"" + name + "\"; build the model before accessing parameters");
    return *found;
}

void Module::zero_grad() {
    for (auto &p : parameters()) p.zero_grad();
}

// ------------------------------------------------------------------ Linear

Linear::Linear(const Axis &input_axis, const Dim &out)
    : input(input_axis),
      input_role(input_axis.role("linear_input")),
      output_role(out.axis.role("linear_output")),
      output(out) {}

Shape Linear::output_shape(const Shape &in) {
    int64_t extent = in.extent(input);
    if (bound && std::get<0>(*bound) != extent) raise("Linear input extent differs from its built extent");
    std::vector<Dim> dims;
    for (auto &d : in.dims)
        if (d.axis != input) dims.push_back(d);
    dims.push_back(output);
    return Shape::make(dims);
}

Shape Linear::build(const Shape &in, const Device &device, uint64_t seed) {
    Shape shape = output_shape(in);
    if (bound) {
        if (!std::get<1>(*bound).tensor().device().same(device))
            raise("Linear is already built on a different Device");
        return shape;
    }
    int64_t extent = in.extent(input);
    Shape weight_shape = Shape::make({Dim{input_role, extent}, Dim{output_role, output.extent}});
    const float scale = std::sqrt(6.0f / (float)(extent + output.extent));
    auto values = xorshift_unit_stream(seed, weight_shape.len);
    for (auto &v : values) v = (v * 2.0f - 1.0f) * scale;
    Parameter weight = Parameter::make(Tensor::from_slice(values, weight_shape.dims, device));
    std::optional<Parameter> b;
    if (bias)
        b = Parameter::make(Tensor::from_slice(std::vector<float>((size_t)output.extent, 0.0f),
                                               {Dim{output_role, output.extent}}, device));
    bound = std::make_tuple(extent, weight, b);
    return shape;
}

Tensor Linear::forward(const Tensor &x) {
    output_shape(x.shape());
    if (!bound) raise("Linear must be built before forward");
    auto &[extent, weight, b] = *bound;
    (void)extent;
    const Tensor renamed = x.rename(input, input_role);
    Tensor projected = b ? renamed.contract_add(weight.tensor(), {input_role}, b->tensor())
                         : renamed.contract(weight.tensor(), {input_role});
    return projected.rename(output_role, output.axis);
}

std::vector<std::pair<std::string, Parameter>> Linear::named_parameters() {
    std::vector<std::pair<std::string, Parameter>> out;
    if (!bound) return out;
    out.emplace_back("weight", std::get<1>(*bound));
    if (std::get<2>(*bound)) out.emplace_back("bias", *std::get<2>(*bound));
    return out;
}

// ------------------------------------------------------------------ Conv2d

Conv2d::Conv2d(const Axis &input_axis, const Dim &out, const std::vector<Axis> &spatial_axes,
               const std::vector<int64_t> &kernel_extents)
    : input(input_axis),
      group(input_axis.role("conv_group")),
      patch(input_axis.role("conv_patch_in_group")),
      output_in_group(out.axis.role("conv_output_in_group")),
      output_role(out.axis.role("conv_output")),
      output(out),
      spatial(spatial_axes),
      kernel(kernel_extents) {
    if (spatial.size() != 2 || kernel.size() != 2) raise("Conv2d needs two spatial axes and kernel extents");
}

Shape Conv2d::output_shape(const Shape &in) {
    for (size_t i = 0; i < 2; ++i)
        if (spatial[i] == input || (i == 1 && spatial[0] == spatial[1]))
            raise("Conv2d requires distinct input-channel and spatial axes");
    int64_t channels = in.extent(input);
    if (groups <= 0 || channels % groups || output.extent % groups)
        raise("Conv2d channels and outputs must be divisible by groups");
    if (kernel[0] <= 0 || kernel[1] <= 0 || stride[0] <= 0 || stride[1] <= 0)
        raise("Conv2d kernel and stride must be positive");
    int64_t out_sp[2];
    for (int i = 0; i < 2; ++i) {
        int64_t padded = in.extent(spatial[i]) + 2 * padding[i];
        if (kernel[i] > padded) raise("Conv2d kernel must fit the padded spatial axes");
        out_sp[i] = (padded - kernel[i]) / stride[i] + 1;
    }
    int64_t patch_extent = channels / groups * kernel[0] * kernel[1];
    if (bound) {
        if (bound->channels != channels) raise("Conv2d input channels differ from its built extent");
        if (bound->patch != patch_extent || bound->output_in_group != output.extent / groups)
            raise("Conv2d group geometry differs from its built parameters");
    }
    std::vector<Dim> dims;
    for (auto &d : in.dims) {
        if (d.axis == input) continue;
        if (d.axis == spatial[0])
            dims.push_back(Dim{d.axis, out_sp[0]});
        else if (d.axis == spatial[1])
            dims.push_back(Dim{d.axis, out_sp[1]});
        else
            dims.push_back(d);
    }
    dims.push_back(output);
    return Shape::make(dims);
}

Shape Conv2d::build(const Shape &in, const Device &device, uint64_t seed) {
    Shape shape = output_shape(in);
    if (bound) {
        if (!bound->weight.tensor().device().same(device))
            raise("Conv2d is already built on a different Device");
        return shape;
    }
    int64_t channels = in.extent(input);
    int64_t patch_extent = channels / groups * kernel[0] * kernel[1];
    int64_t out_in_group = output.extent / groups;
    Shape weight_shape = Shape::make(
        {Dim{group, groups}, Dim{patch, patch_extent}, Dim{output_in_group, out_in_group}});
    // convolution.rs:176-186: xavier-uniform from an inline xorshift stream
    uint64_t rng = seed > 1 ? seed : 1;
    const float scale = std::sqrt(6.0f / (float)(patch_extent + out_in_group));
    std::vector<float> values((size_t)weight_shape.len);
    for (auto &v : values) {
        rng ^= rng << 13;
        rng ^= rng >> 7;
        rng ^= rng << 17;
        v = (((float)(rng >> 40) / (float)(1u << 24)) * 2.0f - 1.0f) * scale;
    }
    Bound b{channels, patch_extent, out_in_group,
            Parameter::make(Tensor::from_slice(values, weight_shape.dims, device)), std::nullopt};
    if (bias)
        b.bias = Parameter::make(Tensor::from_slice(std::vector<float>((size_t)output.extent, 0.0f),
                                                    {Dim{output_role, output.extent}}, device));
    bound = b;
    return shape;
}

// Geometry of an implicit-GEMM launch for x (one group), or false when x needs the reference's
// explicit lowering.  A channel-innermost contiguous [.., height, width, channels] input takes
// every rule (stride 1 and padding < kernel when x needs its gradient, which the data-gradient
// kernel writes channel-innermost); any other rank-4 layout, e.g. channel-major, is gathered
// through its strides and is accepted only when x needs no gradient.
bool Conv2d::implicit_geometry(const Tensor &x, ConvGeometry &q) const {
    if (groups != 1) return false;
    const Shape &in = x.shape();
    const size_t r = in.rank();
    if (r < 3 || in.len >= (int64_t(1) << 31)) return false;
    const bool channels_last = x.is_contiguous() && in.dims[r - 1].axis == input &&
                               in.dims[r - 3].axis == spatial[0] && in.dims[r - 2].axis == spatial[1];
    q = ConvGeometry{};
    for (int i = 0; i < 2; ++i) {
        q.kernel[i] = (int32_t)kernel[i];
        q.stride[i] = (int32_t)stride[i];
        q.padding[i] = (int32_t)padding[i];
    }
    q.out_channels = (int32_t)output.extent;
    if (channels_last) {
        q.channels = (int32_t)in.dims[r - 1].extent;
        q.height = (int32_t)in.dims[r - 3].extent;
        q.width = (int32_t)in.dims[r - 2].extent;
        q.batch = in.len / ((int64_t)q.channels * q.height * q.width);
        if (!x.requires_grad()) return true;
        return stride[0] == 1 && stride[1] == 1 && padding[0] <= kernel[0] - 1 && padding[1] <= kernel[1] - 1;
    }
    if (r != 4 || x.requires_grad()) return false;
    int ci = -1, hi = -1, wi = -1, bi = -1;
    for (int i = 0; i < 4; ++i) {
        const Axis &a = in.dims[i].axis;
        if (a == input) ci = i;
        else if (a == spatial[0]) hi = i;
        else if (a == spatial[1]) wi = i;
        else bi = i;
    }
    if (ci < 0 || hi < 0 || wi < 0 || bi < 0) return false;
    const std::vector<int64_t> &st = x.layout().strides;
    q.batch = in.dims[bi].extent;
    q.channels = (int32_t)in.dims[ci].extent;
    q.height = (int32_t)in.dims[hi].extent;
    q.width = (int32_t)in.dims[wi].extent;
    q.strided = true;
    q.input_strides[0] = st[bi];
    q.input_strides[1] = st[ci];
    q.input_strides[2] = st[hi];
    q.input_strides[3] = st[wi];
    return true;
}

// Rules of the implicit convolution: data and weight gradients through the implicit-GEMM
// kernels, bias gradient as the column sum of the output gradient.
std::vector<Edge> Conv2d::implicit_edges(const Tensor &x, const ConvGeometry &q, int64_t out_len) const {
    std::vector<Edge> edges;
    Rule data;
    data.kind = Rule::ConvData;
    data.a = bound->weight.tensor().value();
    data.conv = q;
    edges.push_back(Edge{x, data});
    Rule weight_rule;
    weight_rule.kind = Rule::ConvWeight;
    weight_rule.a = x.value();
    weight_rule.conv = q;
    edges.push_back(Edge{bound->weight.tensor(), weight_rule});
    if (bound->bias) {
        Rule rb;
        rb.kind = Rule::BiasBroadcast;
        rb.outer = out_len / output.extent;
        rb.inner = output.extent;
        edges.push_back(Edge{bound->bias->tensor(), rb});
    }
    return edges;
}

Tensor Conv2d::forward(const Tensor &x) {
    Shape out_shape = output_shape(x.shape());
    if (!bound) raise("Conv2d must be built before forward");
    // The implicit-GEMM path adds the bias in the epilogue; its rules are the derivatives of
    // exactly that composition.  Every other geometry takes the reference's unfold -> contract ->
    // merge -> add lowering below.
    ConvGeometry q;
    if (out_shape.len < (int64_t(1) << 31) && implicit_geometry(x, q)) {
        const Device &dev = x.device();
        Tensor w = bound->weight.tensor();
        Buffer out = dev.alloc(out_shape.len);
        const float *bias_ptr = bound->bias ? bound->bias->tensor().value()->f32() : nullptr;
        check(axis_conv2d_forward(dev.h(), x.value()->f32(), q.strides(), w.value()->f32(), bias_ptr,
                                  out->f32(), q.batch, q.height, q.width, q.channels, q.out_channels,
                                  q.kernel, q.stride, q.padding),
              "conv2d_forward");
        return Tensor::node(out_shape, Layout::contiguous(out_shape), out, dev,
                            implicit_edges(x, q, out_shape.len), false);
    }
    Tensor projected = x.unfold_grouped(input, spatial, Dim{group, groups}, Dim{patch, bound->patch},
                                        kernel, stride, padding, 0.0f)
                           .contract(bound->weight.tensor(), {patch})
                           .merge({group, output_in_group}, output_role);
    if (bound->bias) projected = projected.add(bound->bias->tensor());
    return projected.rename(output_role, output.axis);
}

// Conv2d -> ReLU -> MaxPool2d in one launch: the GEMM epilogue adds the bias, applies ReLU and
// pools whole windows, so the pre-activation is never stored.  The graph gets an internal
// pre-activation node (no value) carrying the convolution's rules and the pooled node with a
// ReluPool rule; backward scatters the pooled gradient through the winners and the ReLU mask in
// one pass.  Returns nothing when the shapes need the separate modules.
std::optional<Tensor> Conv2d::forward_relu_pool(const Tensor &x, const MaxPool2d &pool) {
    if (!bound) raise("Conv2d must be built before forward");
    Shape conv_shape = output_shape(x.shape());
    const size_t r = conv_shape.rank();
    if (pool.channels != output.axis || pool.spatial.size() != 2 || pool.spatial[0] != spatial[0] ||
        pool.spatial[1] != spatial[1] || r < 3 || conv_shape.dims[r - 1].axis != output.axis ||
        conv_shape.dims[r - 3].axis != spatial[0] || conv_shape.dims[r - 2].axis != spatial[1])
        return std::nullopt;
    for (int i = 0; i < 2; ++i)
        if (pool.stride[i] != pool.kernel[i] || pool.padding[i] != 0 || pool.kernel[i] < 1)
            return std::nullopt;
    const int64_t oh = conv_shape.dims[r - 3].extent, ow = conv_shape.dims[r - 2].extent;
    const int64_t kh = pool.kernel[0], kw = pool.kernel[1];
    if (kh * kw >= 255 || oh % kh || ow % kw || 128 % (kh * ow) || conv_shape.len >= (int64_t(1) << 31))
        return std::nullopt;
    ConvGeometry q;
    if (!implicit_geometry(x, q)) return std::nullopt;
    Shape pooled_shape = const_cast<MaxPool2d &>(pool).output_shape(conv_shape);
    const Device &dev = x.device();
    Buffer pooled = dev.alloc(pooled_shape.len);
    Buffer argmax = dev.alloc_bytes(pooled_shape.len);
    const float *bias_ptr = bound->bias ? bound->bias->tensor().value()->f32() : nullptr;
    const int32_t window[2] = {(int32_t)kh, (int32_t)kw};
    check(axis_conv2d_relu_pool_forward(dev.h(), x.value()->f32(), q.strides(),
                                        bound->weight.tensor().value()->f32(), bias_ptr, pooled->f32(),
                                        static_cast<uint8_t *>(argmax->ptr), q.batch, q.height, q.width,
                                        q.channels, q.out_channels, q.kernel, q.stride, q.padding, window),
          "conv2d_relu_pool_forward");
    Tensor pre = Tensor::node(conv_shape, Layout::contiguous(conv_shape), nullptr, dev,
                              implicit_edges(x, q, conv_shape.len), false);
    Rule rp;
    rp.kind = Rule::ReluPool;
    rp.a = argmax;
    rp.b = pooled;
    rp.pool.outer = conv_shape.len / (oh * ow * output.extent);
    rp.pool.height = (int32_t)oh;
    rp.pool.width = (int32_t)ow;
    rp.pool.channels = output.extent;
    rp.pool.kernel[0] = rp.pool.stride[0] = (int32_t)kh;
    rp.pool.kernel[1] = rp.pool.stride[1] = (int32_t)kw;
    return Tensor::node(pooled_shape, Layout::contiguous(pooled_shape), pooled, dev, {Edge{pre, rp}}, false);
}

std::vector<std::pair<std::string, Parameter>> Conv2d::named_parameters() {
    std::vector<std::pair<std::string, Parameter>> out;
    if (!bound) return out;
    out.emplace_back("weight", bound->weight);
    if (bound->bias) out.emplace_back("bias", *bound->bias);
    return out;
}

// ------------------------------------------------------------------ MaxPool2d

MaxPool2d::MaxPool2d(const Axis &channel_axis, const std::vector<Axis> &spatial_axes,
                     const std::vector<int64_t> &kernel_extents)
    : channels(channel_axis),
      patch(channel_axis.role("pool_patch")),
      spatial(spatial_axes),
      kernel(kernel_extents),
      stride(kernel_extents) {
    if (spatial.size() != 2 || kernel.size() != 2) raise("MaxPool2d needs two spatial axes and kernel extents");
}

// Spatial axes keep their position at the pooled extent; the channel axis is appended.
Shape MaxPool2d::output_shape(const Shape &in) {
    in.extent(channels);
    std::vector<Dim> dims;
    for (auto &d : in.dims) {
        if (d.axis == channels) continue;
        bool found = false;
        for (int i = 0; i < 2; ++i) {
            if (d.axis != spatial[i]) continue;
            int64_t padded = d.extent + 2 * padding[i];
            if (kernel[i] <= 0 || stride[i] <= 0) raise("MaxPool2d kernel and stride must be positive");
            if (kernel[i] > padded) raise("MaxPool2d kernel exceeds the padded spatial extent");
            dims.push_back(Dim{d.axis, (padded - kernel[i]) / stride[i] + 1});
            found = true;
        }
        if (!found) dims.push_back(d);
    }
    dims.push_back(Dim{channels, in.extent(channels)});
    return Shape::make(dims);
}

Tensor MaxPool2d::forward(const Tensor &x) {
    Shape expected = output_shape(x.shape());
    Tensor out = x.max_pool2d(channels, spatial, kernel, stride, padding);
    if (!(out.shape() == expected)) {
        // The fused path keeps the input's axis order; present the reference's order.
        std::vector<Axis> order = expected.axes();
        Tensor aligned = out.with_layout(order);
        std::vector<Dim> dims = expected.dims;
        return Tensor::node(expected, Layout::contiguous(expected), aligned.value(), aligned.device(),
                            {Edge{aligned, Rule{}}}, false);
    }
    return out;
}

// ------------------------------------------------------------------ Sequential

Shape Sequential::output_shape(const Shape &in) {
    Shape s = in;
    for (auto &l : layers) s = l->output_shape(s);
    return s;
}

Shape Sequential::build(const Shape &in, const Device &device, uint64_t seed) {
    output_shape(in);
    Shape s = in;
    for (size_t i = 0; i < layers.size(); ++i) s = layers[i]->build(s, device, seed + i);
    return s;
}

Tensor Sequential::forward(const Tensor &x) {
    output_shape(x.shape());
    Tensor v = x;
    for (size_t i = 0; i < layers.size(); ++i) {
        // Conv2d -> ReLU -> MaxPool2d runs as one fused launch when its geometry allows.
        if (i + 2 < layers.size()) {
            auto conv = std::dynamic_pointer_cast<Conv2d>(layers[i]);
            auto relu = std::dynamic_pointer_cast<ReLU>(layers[i + 1]);
            auto pool = std::dynamic_pointer_cast<MaxPool2d>(layers[i + 2]);
            if (conv && relu && pool) {
                if (auto fused = conv->forward_relu_pool(v, *pool)) {
                    v = *fused;
                    i += 2;
                    continue;
                }
            }
        }
        v = layers[i]->forward(v);
    }
    return v;
}

std::vector<std::pair<std::string, Parameter>> Sequential::named_parameters() {
    std::vector<std::pair<std::string, Parameter>> out;
    for (size_t i = 0; i < layers.size(); ++i)
        for (auto &kv : layers[i]->named_parameters())
            out.emplace_back(std::to_string(i) + "." + kv.first, kv.second);
    return out;
}

}  // namespace axis
