// Axes, shapes, layouts (algebra/axis.rs), the device handle and its out-of-place operations
// (runtime/backend.rs:203-1476), and the host RNG (algebra/tensor.rs:29-71).
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <limits>

#include "axis.hpp"

namespace axis {

[[noreturn]] void raise(const std::string &message) { throw Error(message); }

void check(int status, const char *what) {
    if (status != AXIS_OK) raise(std::string(what) + ": " + axis_last_error());
}

double now_seconds() {
    using namespace std::chrono;
    return duration<double>(steady_clock::now().time_since_epoch()).count();
}

// AXIS_PROFILE=1 prints `axis_profile <label> <seconds>` to stderr (train.rs:31-38,
// backend.rs:15-22, tensor.rs:14-21).
void profile(const char *label, double started) {
    static const bool enabled = std::getenv("AXIS_PROFILE") != nullptr;
    if (enabled) std::fprintf(stderr, "axis_profile %s %.6f\n", label, now_seconds() - started);
}

// ------------------------------------------------------------------ axes

namespace {
std::atomic<uint64_t> next_axis{1};
}

Axis Axis::make(const std::string &name) {
    Axis a;
    a.id = next_axis.fetch_add(1);
    a.name = name;
    return a;
}

Axis Axis::role(const std::string &role_name) const {
    Axis a = make(role_name);
    a.parent = id;
    return a;
}

Shape Shape::make(const std::vector<Dim> &dims) {
    Shape s;
    s.dims = dims;
    int64_t len = 1;
    for (size_t i = 0; i < dims.size(); ++i) {
        if (dims[i].extent <= 0) raise("zero extent for " + dims[i].axis.debug());
        for (size_t j = 0; j < i; ++j)
            if (dims[j].axis == dims[i].axis) raise("duplicate axis " + dims[i].axis.debug());
        if (len > std::numeric_limits<int64_t>::max() / dims[i].extent) raise("shape size overflow");
        len *= dims[i].extent;
    }
    if (len > std::numeric_limits<int32_t>::max()) raise("tensor exceeds the 32-bit index range");
    s.len = len;
    return s;
}

size_t Shape::index(const Axis &a) const {
    for (size_t i = 0; i < dims.size(); ++i)
        if (dims[i].axis == a) return i;
    raise("missing axis " + a.debug() + " in " + debug());
}

bool Shape::contains(const Axis &a) const {
    for (auto &d : dims)
        if (d.axis == a) return true;
    return false;
}

std::vector<Axis> Shape::axes() const {
    std::vector<Axis> out;
    for (auto &d : dims) out.push_back(d.axis);
    return out;
}

std::vector<int64_t> Shape::coords(int64_t flat) const {
    std::vector<int64_t> out(dims.size());
    for (size_t i = dims.size(); i-- > 0;) {
        out[i] = flat % dims[i].extent;
        flat /= dims[i].extent;
    }
    return out;
}

bool Shape::operator==(const Shape &o) const {
    if (dims.size() != o.dims.size()) return false;
    for (size_t i = 0; i < dims.size(); ++i)
        if (dims[i].axis != o.dims[i].axis || dims[i].extent != o.dims[i].extent) return false;
    return true;
}

std::string Shape::debug() const {
    std::string s = "[";
    for (size_t i = 0; i < dims.size(); ++i) {
        if (i) s += ", ";
        s += dims[i].axis.debug() + ":" + std::to_string(dims[i].extent);
    }
    return s + "]";
}

Layout Layout::make(const Shape &shape, const std::vector<Axis> &order) {
    if (order.size() != shape.rank()) raise("layout must contain every axis exactly once");
    for (size_t i = 0; i < order.size(); ++i) {
        shape.index(order[i]);
        for (size_t j = 0; j < i; ++j)
            if (order[j] == order[i]) raise("duplicate selected axis " + order[i].debug());
    }
    Layout l;
    l.strides.assign(shape.rank(), 0);
    int64_t stride = 1;
    for (size_t i = order.size(); i-- > 0;) {
        size_t idx = shape.index(order[i]);
        l.strides[idx] = stride;
        stride *= shape.dims[idx].extent;
    }
    return l;
}

Layout Layout::contiguous(const Shape &shape) { return make(shape, shape.axes()); }

int64_t Layout::offset(const std::vector<int64_t> &coords) const {
    int64_t o = 0;
    for (size_t i = 0; i < coords.size(); ++i) o += coords[i] * strides[i];
    return o;
}

// ------------------------------------------------------------------ device

DeviceImpl::~DeviceImpl() {
    if (handle) {
        if (one) axis_free(handle, one);
        axis_device_destroy(handle);
    }
}

BufferImpl::~BufferImpl() {
    if (owned && ptr && device && device->handle) axis_free(device->handle, ptr);
}

PlanImpl::~PlanImpl() {
    if (handle && device && device->handle) axis_plan_destroy(device->handle, handle);
}

Device Device::hip(int ordinal) {
    Device d;
    d.impl = std::make_shared<DeviceImpl>();
    d.impl->ordinal = ordinal;
    check(axis_device_create(ordinal, &d.impl->handle), "Device::hip");
    return d;
}

// Device::cuda_bf16 (backend.rs:274-283): bf16 operands, fp32 accumulation in matrix products.
Device Device::hip_bf16(int ordinal) {
    Device d;
    d.impl = std::make_shared<DeviceImpl>();
    d.impl->ordinal = ordinal;
    check(axis_device_create_bf16(ordinal, &d.impl->handle), "Device::hip_bf16");
    return d;
}

bool Device::bf16_matmul() const {
    int enabled = 0;
    check(axis_device_bf16_matmul(h(), &enabled), "Device::bf16_matmul");
    return enabled != 0;
}

Buffer Device::alloc_bytes(int64_t bytes) const {
    auto b = std::make_shared<BufferImpl>();
    b->device = impl;
    b->bytes = bytes;
    check(axis_alloc(h(), (size_t)std::max<int64_t>(bytes, 4), &b->ptr), "allocate");
    return b;
}

Buffer Device::upload(const std::vector<float> &values) const {
    Buffer b = alloc((int64_t)values.size());
    check(axis_upload(h(), b->ptr, values.data(), values.size() * 4), "upload");
    return b;
}

Buffer Device::upload_i32(const std::vector<int32_t> &values) const {
    Buffer b = alloc_bytes((int64_t)values.size() * 4);
    check(axis_upload(h(), b->ptr, values.data(), values.size() * 4), "upload");
    return b;
}

std::vector<float> Device::read(const Buffer &b) const {
    std::vector<float> out((size_t)b->floats());
    check(axis_read(h(), out.data(), b->ptr, out.size() * 4), "read");
    return out;
}

void Device::synchronize() const { check(axis_device_synchronize(h()), "synchronize"); }

void Device::finish_defer(bool on) const { check(axis_finish_defer(h(), on ? 1 : 0), "finish_defer"); }

void Device::finish_before_read(const Buffer &b) const {
    if (b) check(axis_finish_before_read(h(), b->ptr, (size_t)b->bytes), "finish_before_read");
}

Buffer Device::zeros_buffer(int64_t len) const { return filled(len, 0.0f); }

Buffer Device::filled(int64_t len, float value) const {
    Buffer b = alloc(len);
    check(axis_fill(h(), b->f32(), value, len), "fill");
    return b;
}

Buffer Device::seed_one() const {
    if (!impl->one) {
        void *p = nullptr;
        check(axis_alloc(h(), 4, &p), "allocate");
        if (int st = axis_fill(h(), static_cast<float *>(p), 1.0f, 1)) {
            axis_free(h(), p);
            check(st, "fill");
        }
        impl->one = p;
    }
    auto b = std::make_shared<BufferImpl>();
    b->device = impl;
    b->ptr = impl->one;
    b->bytes = 4;
    b->owned = false;
    return b;
}

Plan Device::plan(const std::vector<int32_t> &offsets, const std::vector<int32_t> &left,
                  const std::vector<int32_t> &right, bool uncapped) const {
    auto p = std::make_shared<PlanImpl>();
    p->device = impl;
    p->groups = (int64_t)offsets.size() - 1;
    check(axis_plan_create(h(), offsets.data(), left.data(), right.empty() ? nullptr : right.data(),
                           p->groups, uncapped ? 1 : 0, &p->handle),
          "plan");
    return p;
}

Buffer Device::scale(const Buffer &a, float f) const {
    Buffer out = alloc(a->floats());
    check(axis_scale(h(), a->f32(), f, out->f32(), a->floats()), "scale");
    return out;
}

Buffer Device::binary(const Buffer &a, const Buffer &b, int op) const {
    Buffer out = alloc(a->floats());
    check(axis_binary(h(), a->f32(), b->f32(), op, out->f32(), a->floats()), "binary");
    return out;
}

Buffer Device::relu(const Buffer &a) const {
    Buffer out = alloc(a->floats());
    check(axis_relu(h(), a->f32(), out->f32(), a->floats()), "relu");
    return out;
}

Buffer Device::relu_backward(const Buffer &g, const Buffer &a) const {
    Buffer out = alloc(a->floats());
    check(axis_relu_backward(h(), g->f32(), a->f32(), out->f32(), a->floats()), "relu_backward");
    return out;
}

Buffer Device::mask_gradient(const Buffer &g, const Buffer &winners) const {
    Buffer out = alloc(g->floats());
    check(axis_mask_gradient(h(), g->f32(), winners->f32(), out->f32(), g->floats()), "mask_gradient");
    return out;
}

Buffer Device::matmul(const Buffer &a, const Buffer &b, int64_t batch, int64_t m, int64_t k,
                      int64_t n) const {
    Buffer out = alloc(batch * m * n);
    check(axis_matmul(h(), a->f32(), b->f32(), out->f32(), batch, m, k, n), "matmul");
    return out;
}

Buffer Device::matmul_bias(const Buffer &a, const Buffer &b, const Buffer &bias, int64_t batch, int64_t m,
                           int64_t k, int64_t n) const {
    Buffer out = alloc(batch * m * n);
    check(axis_matmul_bias(h(), a->f32(), b->f32(), bias->f32(), out->f32(), batch, m, k, n), "matmul_bias");
    return out;
}

Buffer Device::matmul_left_backward(const Buffer &g, const Buffer &rhs, int64_t batch, int64_t m,
                                    int64_t k, int64_t n) const {
    Buffer out = alloc(batch * m * k);
    check(axis_matmul_left_backward(h(), g->f32(), rhs->f32(), out->f32(), batch, m, k, n),
          "matmul_left_backward");
    return out;
}

Buffer Device::matmul_axpby(const Buffer &a, const Buffer &b, const Buffer &d, int64_t batch, int64_t m,
                            int64_t k, int64_t n, float alpha, float beta) const {
    Buffer out = alloc(batch * m * n);
    check(axis_matmul_axpby(h(), a->f32(), b->f32(), d->f32(), out->f32(), batch, m, k, n, alpha, beta),
          "matmul_axpby");
    return out;
}

Buffer Device::matmul_right_backward(const Buffer &lhs, const Buffer &g, int64_t batch, int64_t m,
                                     int64_t k, int64_t n) const {
    Buffer out = alloc(batch * k * n);
    check(axis_matmul_right_backward(h(), lhs->f32(), g->f32(), out->f32(), batch, m, k, n),
          "matmul_right_backward");
    return out;
}

Buffer Device::unfold(const Buffer &input, const axis_unfold_spec &spec) const {
    Buffer out = alloc(spec.output_len);
    check(axis_unfold(h(), input->f32(), out->f32(), &spec), "unfold");
    return out;
}

Buffer Device::unfold_backward(const Buffer &g, const axis_unfold_spec &spec) const {
    Buffer out = alloc(spec.input_len);
    check(axis_unfold_backward(h(), g->f32(), out->f32(), &spec), "unfold_backward");
    return out;
}

Buffer Device::grouped(const Buffer &a, const Buffer *b, const Plan &plan, float scale) const {
    Buffer out = alloc(plan->groups);
    check(axis_grouped(h(), a->f32(), b ? (*b)->f32() : nullptr, plan->handle, scale, out->f32()),
          "grouped");
    return out;
}

std::pair<Buffer, Buffer> Device::grouped_minimum(const Buffer &a, const Plan &forward,
                                                  const Plan &reverse) const {
    Buffer out = alloc(forward->groups);
    Buffer mask = alloc(a->floats());
    check(axis_grouped_minimum(h(), a->f32(), a->floats(), forward->handle, reverse->handle,
                               out->f32(), nullptr, mask->f32()),
          "grouped_minimum");
    return {out, mask};
}

Buffer Device::select_axis(const Buffer &input, const std::vector<int32_t> &metadata,
                           int64_t out_len) const {
    Buffer out = alloc(out_len);
    check(axis_select_axis(h(), input->f32(), out->f32(), metadata.data(),
                           (int32_t)(metadata.size() / 3), 0, out_len),
          "select_axis");
    return out;
}

Buffer Device::select_axis_backward(const Buffer &g, const std::vector<int32_t> &metadata,
                                    int64_t in_len) const {
    Buffer out = alloc(in_len);
    check(axis_select_axis_backward(h(), g->f32(), out->f32(), metadata.data(),
                                    (int32_t)(metadata.size() / 3), 0, in_len),
          "select_axis_backward");
    return out;
}

Buffer Device::sum_squares(const Buffer &a) const {
    Buffer out = alloc(1);
    check(axis_sum_squares(h(), a->f32(), a->floats(), out->f32()), "sum_squares");
    return out;
}

Buffer Device::inverse_sqrt(const Buffer &a, float eps) const {
    Buffer out = alloc(a->floats());
    check(axis_inverse_sqrt(h(), a->f32(), eps, out->f32(), a->floats()), "inverse_sqrt");
    return out;
}

Buffer Device::multiply_scalar(const Buffer &a, const Buffer &scalar) const {
    Buffer out = alloc(a->floats());
    check(axis_multiply_scalar(h(), a->f32(), scalar->f32(), out->f32(), a->floats()),
          "multiply_scalar");
    return out;
}

// ------------------------------------------------------------------ RNG

std::vector<float> xorshift_unit_stream(uint64_t seed, int64_t count) {
    uint64_t rng = seed > 1 ? seed : 1;
    std::vector<float> out((size_t)count);
    for (auto &v : out) {
        rng ^= rng << 13;
        rng ^= rng >> 7;
        rng ^= rng << 17;
        v = (float)(rng >> 40) / (float)(1u << 24);
    }
    return out;
}

std::vector<float> uniform_host_values(uint64_t seed, int64_t count, float low, float high) {
    auto v = xorshift_unit_stream(seed, count);
    const float span = high - low;
    for (auto &x : v) x = low + x * span;
    return v;
}

std::vector<float> normal_host_values(uint64_t seed, int64_t count, float mean, float std) {
    auto raw = xorshift_unit_stream(seed, (count + 1) / 2 * 2);
    std::vector<float> out;
    out.reserve((size_t)count);
    const float two_pi = 2.0f * 3.14159265358979323846f;
    for (size_t p = 0; p + 1 < raw.size(); p += 2) {
        volatile float one_minus = 1.0f - raw[p];
        float radius = std::sqrt(-2.0f * std::log((float)one_minus));
        float angle = two_pi * raw[p + 1];
        out.push_back(mean + std * (radius * std::cos(angle)));
        if ((int64_t)out.size() < count) out.push_back(mean + std * (radius * std::sin(angle)));
    }
    return out;
}

float powi(float base, int32_t exponent) {
    bool recip = exponent < 0;
    float r = 1.0f;
    for (;;) {
        if (exponent & 1) r *= base;
        exponent /= 2;
        if (exponent == 0) break;
        base *= base;
    }
    return recip ? 1.0f / r : r;
}

}  // namespace axis
