// C++ host layer over the C ABI of include/axis_hip.h: named axes, shapes and layouts
// (algebra/axis.rs), the device handle and its buffers (runtime/backend.rs:113-392), the
// immutable Tensor with its autograd tape (algebra/tensor.rs:126-238, :5551-5738), modules
// (model/nn.rs, model/convolution.rs), optimizers (model/optim.rs) and the Trainer
// (runtime/train.rs).  Names, argument meaning and error behaviour follow the reference; every
// device operation goes through libaxis_hip (there is no other compute path).
#pragma once

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "axis_hip.h"

namespace axis {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void raise(const std::string &message);
void check(int status, const char *what);
void profile(const char *label, double started_seconds);
double now_seconds();

// ------------------------------------------------------------------ axes (algebra/axis.rs:11-176)

struct Axis {
    uint64_t id = 0;
    std::string name;
    uint64_t parent = 0;
    static Axis make(const std::string &name);
    Axis role(const std::string &role_name) const;
    bool operator==(const Axis &o) const { return id == o.id; }
    bool operator!=(const Axis &o) const { return id != o.id; }
    bool operator<(const Axis &o) const { return id < o.id; }
    std::string debug() const { return name + "#" + std::to_string(id); }
};

struct Dim {
    Axis axis;
    int64_t extent = 0;
};

struct Shape {
    std::vector<Dim> dims;
    int64_t len = 1;
    static Shape make(const std::vector<Dim> &dims);
    size_t rank() const { return dims.size(); }
    size_t index(const Axis &a) const;
    bool contains(const Axis &a) const;
    int64_t extent(const Axis &a) const { return dims[index(a)].extent; }
    std::vector<Axis> axes() const;
    std::vector<int64_t> coords(int64_t flat) const;
    bool operator==(const Shape &o) const;
    std::string debug() const;
};

struct Layout {
    std::vector<int64_t> strides;
    static Layout make(const Shape &shape, const std::vector<Axis> &order);
    static Layout contiguous(const Shape &shape);
    int64_t offset(const std::vector<int64_t> &coords) const;
    bool operator==(const Layout &o) const { return strides == o.strides; }
};

// ------------------------------------------------------------------ device and buffers

struct DeviceImpl {
    axis_device handle = nullptr;
    int ordinal = 0;
    // One float holding 1.0, written once: the seed adjoint of backward() (read-only by every rule).
    void *one = nullptr;
    ~DeviceImpl();
};

struct BufferImpl {
    std::shared_ptr<DeviceImpl> device;
    void *ptr = nullptr;
    int64_t bytes = 0;
    bool owned = true;  // false for views of device-held memory (the seed)
    ~BufferImpl();
    float *f32() const { return static_cast<float *>(ptr); }
    int64_t floats() const { return bytes / 4; }
};
using Buffer = std::shared_ptr<BufferImpl>;

// A CSR plan uploaded once (the reference's device_plan cache, backend.rs:1449-1475).
struct PlanImpl {
    std::shared_ptr<DeviceImpl> device;
    axis_plan handle = nullptr;
    int64_t groups = 0;
    ~PlanImpl();
};
using Plan = std::shared_ptr<PlanImpl>;

struct PoolGeometry {
    int64_t outer = 0, channels = 0;
    int32_t height = 0, width = 0;
    int32_t kernel[2] = {1, 1}, stride[2] = {1, 1}, padding[2] = {0, 0};
};

// A one-group convolution of a channel-innermost [batch, height, width, channels] input.
struct ConvGeometry {
    int64_t batch = 0;
    int32_t height = 0, width = 0, channels = 0, out_channels = 0;
    int32_t kernel[2] = {1, 1}, stride[2] = {1, 1}, padding[2] = {0, 0};
    // Element strides {batch, channel, row, column} of the input when it is not channel-innermost
    // contiguous.
    bool strided = false;
    int64_t input_strides[4] = {0, 0, 0, 0};
    const int64_t *strides() const { return strided ? input_strides : nullptr; }
};

// Device (runtime/backend.rs:116-392): one GPU, one stream, out-of-place ops returning fresh
// buffers, exactly the reference's method surface for the hot path.
class Device {
  public:
    std::shared_ptr<DeviceImpl> impl;

    static Device hip(int ordinal);
    static Device hip_bf16(int ordinal);
    bool bf16_matmul() const;
    bool same(const Device &o) const { return impl == o.impl; }
    axis_device h() const { return impl->handle; }

    Buffer alloc_bytes(int64_t bytes) const;
    Buffer alloc(int64_t floats) const { return alloc_bytes(floats * 4); }
    Buffer upload(const std::vector<float> &values) const;
    Buffer upload_i32(const std::vector<int32_t> &values) const;
    std::vector<float> read(const Buffer &b) const;
    void synchronize() const;
    // Weight and bias gradients' last sums recorded and run in one launch (axis_finish_*): on /
    // off (off runs what is recorded), and the flush a read of a possibly pending buffer needs.
    void finish_defer(bool on) const;
    void finish_before_read(const Buffer &b) const;
    Buffer zeros_buffer(int64_t len) const;
    Buffer filled(int64_t len, float value) const;
    // A read-only [1] buffer holding 1.0, filled once per device.
    Buffer seed_one() const;
    Plan plan(const std::vector<int32_t> &offsets, const std::vector<int32_t> &left,
              const std::vector<int32_t> &right, bool uncapped = false) const;

    Buffer scale(const Buffer &a, float f) const;
    Buffer binary(const Buffer &a, const Buffer &b, int op) const;
    Buffer relu(const Buffer &a) const;
    Buffer relu_backward(const Buffer &g, const Buffer &a) const;
    Buffer mask_gradient(const Buffer &g, const Buffer &winners) const;
    Buffer matmul(const Buffer &a, const Buffer &b, int64_t batch, int64_t m, int64_t k, int64_t n) const;
    Buffer matmul_bias(const Buffer &a, const Buffer &b, const Buffer &bias, int64_t batch, int64_t m, int64_t k,
                       int64_t n) const;
    Buffer matmul_left_backward(const Buffer &g, const Buffer &rhs, int64_t batch, int64_t m,
                                int64_t k, int64_t n) const;
    // beta * d + alpha * (a . b), each product and the sum rounded once (Newton-Schulz steps)
    Buffer matmul_axpby(const Buffer &a, const Buffer &b, const Buffer &d, int64_t batch, int64_t m,
                        int64_t k, int64_t n, float alpha, float beta) const;
    Buffer matmul_right_backward(const Buffer &lhs, const Buffer &g, int64_t batch, int64_t m,
                                 int64_t k, int64_t n) const;
    Buffer unfold(const Buffer &input, const axis_unfold_spec &spec) const;
    Buffer unfold_backward(const Buffer &g, const axis_unfold_spec &spec) const;
    Buffer grouped(const Buffer &a, const Buffer *b, const Plan &plan, float scale) const;
    std::pair<Buffer, Buffer> grouped_minimum(const Buffer &a, const Plan &forward,
                                              const Plan &reverse) const;
    Buffer select_axis(const Buffer &input, const std::vector<int32_t> &metadata, int64_t out_len) const;
    Buffer select_axis_backward(const Buffer &g, const std::vector<int32_t> &metadata,
                                int64_t in_len) const;
    Buffer sum_squares(const Buffer &a) const;
    Buffer inverse_sqrt(const Buffer &a, float eps) const;
    Buffer multiply_scalar(const Buffer &a, const Buffer &scalar) const;
};

// ------------------------------------------------------------------ tensor and tape

struct Node;
class Tensor;

// One saved backward rule (algebra/tensor.rs:143-238), plus the rules of this backend's fused
// lowerings (BiasBroadcast, MeanMiddle, MaxPool, ConvData, ConvWeight), each the exact
// derivative of the composition it replaces.
struct Rule {
    enum Kind {
        Identity,
        Zero,
        Scale,
        Multiply,
        Relu,
        CategoricalCrossEntropy,
        MatmulLeft,
        MatmulRight,
        Group,
        Minimum,
        Unfold,
        Select,
        BiasBroadcast,
        MeanMiddle,
        MaxPool,
        ConvData,    // input gradient of an implicit-GEMM convolution (a = weight)
        ConvWeight,  // weight gradient of an implicit-GEMM convolution (a = input)
        ReluPool,    // ReLU then non-overlapping max pool (a = argmax bytes, b = pooled values)
        ReduceAxes,  // sum over any axis set (extents/strides of the input, metadata = reduced flags)
        BroadcastAxes,  // broadcast into new axes (extents/strides of the output, metadata = new-axis flags)
        MinimumAxis,    // min over one axis without plans (a = winner mask; input geometry; metadata = {axis})
    } kind = Identity;
    float factor = 1.0f;
    Buffer a, b;  // saved operands (rhs / lhs / probability / input / winners / argmax)
    int64_t batch = 0, m = 0, k = 0, n = 0;  // matmul extents; Zero: n = length
    Plan plan;
    std::shared_ptr<axis_unfold_spec> spec;
    std::vector<int32_t> metadata;  // select_axis metadata; ReduceAxes: reduced flags
    std::vector<int64_t> extents, strides;  // ReduceAxes input geometry
    // BroadcastAxes: select_axis metadata that moves the reduced gradient (kept axes in the output's
    // order, contiguous) into the input's own layout; empty when it is already in that layout
    std::vector<int32_t> place;
    int64_t outer = 0, reduce = 0, inner = 0;
    PoolGeometry pool;
    ConvGeometry conv;
};

struct Edge;

struct Node {
    uint64_t id = 0;
    Shape shape;
    Layout layout;
    Buffer value;
    Device device;
    bool tracked = false;
    std::shared_ptr<std::vector<Edge>> edges;  // null: leaf or consumed
    bool consumed = false;
    Buffer grad;
    std::shared_ptr<uint64_t> version;  // parameter leaves only
    uint64_t expected_version = 0;
    std::shared_ptr<std::vector<float>> host;  // host copy of values created from host data
};

class Tensor {
  public:
    std::shared_ptr<Node> n;

    Tensor() = default;
    explicit Tensor(std::shared_ptr<Node> node) : n(std::move(node)) {}

    static Tensor node(const Shape &shape, const Layout &layout, const Buffer &value,
                       const Device &device, std::vector<Edge> edges, bool leaf,
                       std::shared_ptr<uint64_t> version = nullptr);
    static Tensor from_slice(const std::vector<float> &values, const std::vector<Dim> &dims,
                             const Device &device);
    static Tensor zeros(const std::vector<Dim> &dims, const Device &device);
    static Tensor uniform(const std::vector<Dim> &dims, uint64_t seed, float low, float high,
                          const Device &device);
    static Tensor normal(const std::vector<Dim> &dims, uint64_t seed, float mean, float std,
                         const Device &device);

    const Shape &shape() const { return n->shape; }
    const Layout &layout() const { return n->layout; }
    const Device &device() const { return n->device; }
    const Buffer &value() const { return n->value; }
    bool requires_grad() const { return n->tracked; }
    uint64_t id() const { return n->id; }
    int64_t extent(const Axis &a) const { return n->shape.extent(a); }

    Tensor with_grad() const;
    Tensor detach() const;
    std::vector<float> to_vec() const;
    float item() const;
    std::optional<Tensor> grad() const;
    void zero_grad() const;
    Tensor parameter_leaf(std::shared_ptr<uint64_t> version) const;

    Tensor add(const Tensor &rhs) const { return binary(rhs, 0); }
    Tensor sub(const Tensor &rhs) const { return binary(rhs, 1); }
    Tensor mul(const Tensor &rhs) const { return binary(rhs, 2); }
    Tensor scale(float factor) const;
    Tensor relu() const;
    Tensor contract(const Tensor &rhs, const std::vector<Axis> &axes) const;
    // contract(rhs, axes).add(bias) for a bias over exactly the rhs's kept axes: one product with
    // the bias added in its epilogue (same values; falls back to the two operations otherwise).
    Tensor contract_add(const Tensor &rhs, const std::vector<Axis> &axes, const Tensor &bias) const;
    Tensor rename(const Axis &from, const Axis &to) const;
    Tensor merge(const std::vector<Axis> &axes, const Axis &axis) const;
    Tensor with_layout(const std::vector<Axis> &order) const;
    Tensor mean(const std::vector<Axis> &axes) const;
    Tensor sum(const std::vector<Axis> &axes) const;
    Tensor min(const Axis &axis) const;
    Tensor unfold_grouped(const Axis &channels, const std::vector<Axis> &spatial,
                          std::optional<Dim> group, const Dim &patch,
                          const std::vector<int64_t> &kernel, const std::vector<int64_t> &stride,
                          const std::vector<int64_t> &padding, float fill) const;
    Tensor max_pool2d(const Axis &channels, const std::vector<Axis> &spatial,
                      const std::vector<int64_t> &kernel, const std::vector<int64_t> &stride,
                      const std::vector<int64_t> &padding) const;
    Tensor categorical_cross_entropy_with_logits(const Tensor &targets, const Axis &cls) const;
    Tensor normalized_l2(float epsilon) const;
    Tensor inverse_sqrt(float epsilon) const;
    void backward() const;

    // Internal helpers shared by the ops.
    Tensor binary(const Tensor &rhs, int op) const;
    Tensor align(const Shape &shape) const;
    Tensor reduce(const std::vector<Axis> &axes, bool mean, const char *label) const;
    bool is_contiguous() const { return n->layout == Layout::contiguous(n->shape); }
};

struct Edge {
    Tensor input;
    Rule rule;
};

// RNG (algebra/tensor.rs:29-71).
std::vector<float> xorshift_unit_stream(uint64_t seed, int64_t count);
std::vector<float> uniform_host_values(uint64_t seed, int64_t count, float low, float high);
std::vector<float> normal_host_values(uint64_t seed, int64_t count, float mean, float std);
float powi(float base, int32_t exponent);

// ------------------------------------------------------------------ parameters and modules

struct ParamState {
    uint64_t id = 0;
    Tensor tensor;
    std::shared_ptr<uint64_t> version;
};

// model/nn.rs:14-65: cloning shares the parameter, including its accumulated gradient.
class Parameter {
  public:
    std::shared_ptr<ParamState> s;
    static Parameter make(const Tensor &tensor);
    uint64_t id() const { return s->id; }
    Tensor tensor() const { return s->tensor; }
    std::optional<Tensor> grad() const { return s->tensor.grad(); }
    void zero_grad() const { s->tensor.zero_grad(); }
    void set_values(const std::vector<float> &values) const;
    void replace(const Tensor &tensor) const;
};

class Module {
  public:
    virtual ~Module() = default;
    virtual Shape output_shape(const Shape &input) = 0;
    virtual Shape build(const Shape &input, const Device &device, uint64_t seed) = 0;
    virtual Tensor forward(const Tensor &input) = 0;
    virtual std::vector<std::pair<std::string, Parameter>> named_parameters() { return {}; }
    std::vector<Parameter> parameters();
    Parameter parameter(const std::string &name);
    void zero_grad();
};
using ModulePtr = std::shared_ptr<Module>;

class Linear : public Module {
  public:
    Axis input, input_role, output_role;
    Dim output;
    bool bias = true;
    std::optional<std::tuple<int64_t, Parameter, std::optional<Parameter>>> bound;
    Linear(const Axis &input, const Dim &output);
    Shape output_shape(const Shape &in) override;
    Shape build(const Shape &in, const Device &device, uint64_t seed) override;
    Tensor forward(const Tensor &x) override;
    std::vector<std::pair<std::string, Parameter>> named_parameters() override;
};

class Conv2d : public Module {
  public:
    Axis input, group, patch, output_in_group, output_role;
    Dim output;
    std::vector<Axis> spatial;
    std::vector<int64_t> kernel, stride{1, 1}, padding{0, 0};
    int64_t groups = 1;
    bool bias = true;
    struct Bound {
        int64_t channels, patch, output_in_group;
        Parameter weight;
        std::optional<Parameter> bias;
    };
    std::optional<Bound> bound;
    Conv2d(const Axis &input, const Dim &output, const std::vector<Axis> &spatial,
           const std::vector<int64_t> &kernel);
    Shape output_shape(const Shape &in) override;
    Shape build(const Shape &in, const Device &device, uint64_t seed) override;
    Tensor forward(const Tensor &x) override;
    // Conv2d -> ReLU -> pool as one launch when the geometry allows it (Sequential uses this).
    std::optional<Tensor> forward_relu_pool(const Tensor &x, const class MaxPool2d &pool);
    std::vector<std::pair<std::string, Parameter>> named_parameters() override;

  private:
    bool implicit_geometry(const Tensor &x, ConvGeometry &q) const;
    std::vector<Edge> implicit_edges(const Tensor &x, const ConvGeometry &q, int64_t out_len) const;
};

class MaxPool2d : public Module {
  public:
    Axis channels, patch;
    std::vector<Axis> spatial;
    std::vector<int64_t> kernel, stride, padding{0, 0};
    MaxPool2d(const Axis &channels, const std::vector<Axis> &spatial, const std::vector<int64_t> &kernel);
    Shape output_shape(const Shape &in) override;
    Shape build(const Shape &in, const Device &, uint64_t) override { return output_shape(in); }
    Tensor forward(const Tensor &x) override;
};

class ReLU : public Module {
  public:
    Shape output_shape(const Shape &in) override { return in; }
    Shape build(const Shape &in, const Device &, uint64_t) override { return in; }
    Tensor forward(const Tensor &x) override { return x.relu(); }
};

class Sequential : public Module {
  public:
    std::vector<ModulePtr> layers;
    Shape output_shape(const Shape &in) override;
    Shape build(const Shape &in, const Device &device, uint64_t seed) override;
    Tensor forward(const Tensor &x) override;
    std::vector<std::pair<std::string, Parameter>> named_parameters() override;
};

// A module whose parameters are given explicitly (the tests' `Parameters` helper).
class ParameterList : public Module {
  public:
    std::vector<std::pair<std::string, Parameter>> params;
    Shape output_shape(const Shape &in) override { return in; }
    Shape build(const Shape &in, const Device &, uint64_t) override { return in; }
    Tensor forward(const Tensor &x) override { return x; }
    std::vector<std::pair<std::string, Parameter>> named_parameters() override { return params; }
};

// ------------------------------------------------------------------ optimizers (model/optim.rs)

class Optimizer {
  public:
    virtual ~Optimizer() = default;
    virtual void step(Module &model) = 0;
    virtual int32_t completed_steps() const = 0;
};

class Adam : public Optimizer {
  public:
    float learning_rate, beta1, beta2, epsilon, weight_decay = 0.0f;
    int32_t step_count = 0;
    struct State {
        Buffer first, second;
    };
    std::unordered_map<uint64_t, State> states;
    Adam(float lr, float beta1 = 0.9f, float beta2 = 0.999f, float epsilon = 1e-8f);
    void step(Module &model) override { step_parameters(model.parameters()); }
    void step_parameters(const std::vector<Parameter> &parameters);
    int32_t completed_steps() const override { return step_count; }
    void set_learning_rate(float lr);

    struct Update {
        Parameter parameter;
        Tensor tensor;
        State state;
    };
    struct Prepared {
        int32_t next_step;
        std::vector<Update> updates;
    };
    Prepared prepare(const std::vector<Parameter> &parameters) const;
    void commit(Prepared &&prepared);
};

class AdamW : public Adam {
  public:
    AdamW(float lr, float weight_decay, float beta1 = 0.9f, float beta2 = 0.999f,
          float epsilon = 1e-8f);
};

enum class MuonOrientation { FanInFanOut, FanOutFanIn };

struct MuonMatrix {
    uint64_t id;
    MuonOrientation orientation;
};

class Muon : public Optimizer {
  public:
    std::map<uint64_t, MuonOrientation> selected;
    float learning_rate, momentum;
    bool nesterov;
    float weight_decay;
    int32_t step_count = 0;
    std::unordered_map<uint64_t, Tensor> states;
    Muon(const std::vector<MuonMatrix> &selected, float lr, float momentum, bool nesterov,
         float weight_decay);
    void step(Module &model) override;
    int32_t completed_steps() const override { return step_count; }

    struct Selected {
        Parameter parameter;
        MuonOrientation orientation;
    };
    struct Update {
        Parameter parameter;
        Tensor tensor, momentum;
    };
    struct Prepared {
        int32_t next_step;
        std::vector<Update> updates;
    };
    Prepared prepare(const std::vector<Selected> &parameters) const;
    void commit(Prepared &&prepared);
    std::pair<std::vector<Selected>, std::vector<Parameter>> partition(Module &model) const;
};

class MuonWithAuxAdamW : public Optimizer {
  public:
    Muon muon;
    AdamW adamw;
    MuonWithAuxAdamW(const std::vector<MuonMatrix> &selected, float muon_lr, float adamw_lr,
                     float weight_decay);
    void step(Module &model) override;
    int32_t completed_steps() const override { return muon.completed_steps(); }
};

Tensor zeroth_power(const Tensor &matrix);

// ------------------------------------------------------------------ trainer (runtime/train.rs)

struct TrainStep {
    uint64_t step;
    Tensor pre_update_loss;
};

class Trainer {
  public:
    std::shared_ptr<Optimizer> optimizer;
    uint64_t completed = 0;
    explicit Trainer(std::shared_ptr<Optimizer> optimizer) : optimizer(std::move(optimizer)) {}
    TrainStep step(Module &model, const std::function<Tensor(Module &)> &loss);
};

}  // namespace axis
