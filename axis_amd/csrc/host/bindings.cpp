// Python view of the C++ host layer (module axis_amd._axis).  Names follow the reference's
// public API (Axis, Dim, Shape, Device, Tensor, Parameter, Linear, Conv2d, MaxPool2d, ReLU,
// Sequential, Adam, AdamW, Muon, MuonMatrix, MuonWithAuxAdamW, Trainer) so tests read like the
// reference's own.
#include <pybind11/functional.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "axis.hpp"

namespace py = pybind11;
using namespace axis;

namespace {

std::vector<float> as_floats(py::object values) {
    auto arr = py::array_t<float, py::array::c_style | py::array::forcecast>::ensure(values);
    if (!arr) throw Error("values must be convertible to a float32 array");
    return std::vector<float>(arr.data(), arr.data() + arr.size());
}

py::array_t<float> to_numpy(const std::vector<float> &v) {
    py::array_t<float> out((py::ssize_t)v.size());
    std::copy(v.begin(), v.end(), out.mutable_data());
    return out;
}

std::vector<float> read_buffer(const Buffer &b) {
    std::vector<float> out((size_t)b->floats());
    check(axis_read(b->device->handle, out.data(), b->ptr, out.size() * 4), "read");
    return out;
}

template <class M, class... Bases>
py::class_<M, Bases..., std::shared_ptr<M>> module_class(py::module_ &m, const char *name) {
    return py::class_<M, Bases..., std::shared_ptr<M>>(m, name)
        .def("output_shape", &M::output_shape)
        .def("build", &M::build, py::arg("input"), py::arg("device"), py::arg("seed"))
        .def("forward", &M::forward)
        .def("__call__", &M::forward)
        .def("named_parameters", &M::named_parameters);
}

}  // namespace

PYBIND11_MODULE(_axis, m) {
    m.doc() = "C++ host layer of the MI355X backend: named-axis tensors, tape, modules, optimizers";
    py::register_exception<Error>(m, "AxisError", PyExc_RuntimeError);

    py::class_<Axis>(m, "Axis")
        .def(py::init([](const std::string &name) { return Axis::make(name); }))
        .def("role", &Axis::role)
        .def("of", [](const Axis &a, int64_t extent) { return Dim{a, extent}; })
        .def_property_readonly("name", [](const Axis &a) { return a.name; })
        .def_property_readonly("id", [](const Axis &a) { return a.id; })
        .def_property_readonly("parent_id", [](const Axis &a) -> py::object {
            return a.parent ? py::object(py::int_(a.parent)) : py::object(py::none());
        })
        .def("__eq__", [](const Axis &a, const Axis &b) { return a == b; })
        .def("__hash__", [](const Axis &a) { return std::hash<uint64_t>()(a.id); })
        .def("__repr__", &Axis::debug);

    py::class_<Dim>(m, "Dim")
        .def_readonly("axis", &Dim::axis)
        .def_readonly("extent", &Dim::extent)
        .def("__repr__", [](const Dim &d) { return d.axis.debug() + ":" + std::to_string(d.extent); });

    py::class_<Shape>(m, "Shape")
        .def(py::init([](const std::vector<Dim> &dims) { return Shape::make(dims); }))
        .def_readonly("dims", &Shape::dims)
        .def_readonly("len", &Shape::len)
        .def("rank", &Shape::rank)
        .def("extent", &Shape::extent)
        .def("axes", &Shape::axes)
        .def("__eq__", [](const Shape &a, const Shape &b) { return a == b; })
        .def("__repr__", &Shape::debug);

    py::class_<Device>(m, "Device")
        .def_static("hip", &Device::hip, py::arg("ordinal") = 0)
        .def_static("hip_bf16", &Device::hip_bf16, py::arg("ordinal") = 0)
        .def("bf16_matmul", &Device::bf16_matmul)
        .def("synchronize", &Device::synchronize)
        .def("same", &Device::same)
        .def("memory_stats", [](const Device &d) {
            size_t in_use = 0, cached = 0;
            check(axis_memory_stats(d.h(), &in_use, &cached), "memory_stats");
            return py::make_tuple(in_use, cached);
        })
        .def("stream", [](const Device &d) {
            void *s = nullptr;
            check(axis_device_stream(d.h(), &s), "stream");
            return (uintptr_t)s;
        });

    py::class_<Tensor>(m, "Tensor")
        .def_static("from_slice", [](py::object values, const std::vector<Dim> &dims, const Device &d) {
            return Tensor::from_slice(as_floats(values), dims, d);
        })
        .def_static("zeros", &Tensor::zeros)
        .def_static("uniform", &Tensor::uniform)
        .def_static("normal", &Tensor::normal)
        .def_property_readonly("shape", &Tensor::shape)
        .def_property_readonly("requires_grad", &Tensor::requires_grad)
        .def_property_readonly("layout_strides", [](const Tensor &t) { return t.layout().strides; })
        .def_property_readonly("node_id", &Tensor::id)
        .def("extent", &Tensor::extent)
        .def("device", &Tensor::device)
        .def("with_grad", &Tensor::with_grad)
        .def("detach", &Tensor::detach)
        .def("to_vec", [](const Tensor &t) { return to_numpy(t.to_vec()); })
        .def("item", &Tensor::item)
        .def("grad", &Tensor::grad)
        .def("zero_grad", &Tensor::zero_grad)
        .def("add", &Tensor::add)
        .def("sub", &Tensor::sub)
        .def("mul", &Tensor::mul)
        .def("scale", &Tensor::scale)
        .def("relu", &Tensor::relu)
        .def("contract", &Tensor::contract)
        .def("rename", &Tensor::rename)
        .def("merge", &Tensor::merge)
        .def("with_layout", &Tensor::with_layout)
        .def("mean", &Tensor::mean)
        .def("sum", &Tensor::sum)
        .def("min", &Tensor::min)
        .def("unfold_grouped", &Tensor::unfold_grouped)
        .def("max_pool2d", &Tensor::max_pool2d)
        .def("categorical_cross_entropy_with_logits", &Tensor::categorical_cross_entropy_with_logits)
        .def("normalized_l2", &Tensor::normalized_l2)
        .def("backward", &Tensor::backward)
        .def("shares_buffer", [](const Tensor &a, const Tensor &b) { return a.value() == b.value(); });

    py::class_<Parameter>(m, "Parameter")
        .def(py::init(&Parameter::make))
        .def_property_readonly("id", &Parameter::id)
        .def("tensor", &Parameter::tensor)
        .def("grad", &Parameter::grad)
        .def("zero_grad", &Parameter::zero_grad)
        .def("set_values", [](const Parameter &p, py::object v) { p.set_values(as_floats(v)); })
        .def("__eq__", [](const Parameter &a, const Parameter &b) { return a.s == b.s; });

    py::class_<Module, std::shared_ptr<Module>>(m, "Module")
        .def("parameters", &Module::parameters)
        .def("parameter", &Module::parameter)
        .def("zero_grad", &Module::zero_grad);

    module_class<Linear, Module>(m, "Linear")
        .def(py::init<const Axis &, const Dim &>())
        .def("bias", [](std::shared_ptr<Linear> l, bool b) { l->bias = b; return l; });

    module_class<Conv2d, Module>(m, "Conv2d")
        .def(py::init<const Axis &, const Dim &, const std::vector<Axis> &, const std::vector<int64_t> &>())
        .def("stride", [](std::shared_ptr<Conv2d> c, std::vector<int64_t> s) { c->stride = s; return c; })
        .def("padding", [](std::shared_ptr<Conv2d> c, std::vector<int64_t> p) { c->padding = p; return c; })
        .def("groups", [](std::shared_ptr<Conv2d> c, int64_t g) { c->groups = g; return c; })
        .def("bias", [](std::shared_ptr<Conv2d> c, bool b) { c->bias = b; return c; });

    module_class<MaxPool2d, Module>(m, "MaxPool2d")
        .def(py::init<const Axis &, const std::vector<Axis> &, const std::vector<int64_t> &>())
        .def("stride", [](std::shared_ptr<MaxPool2d> p, std::vector<int64_t> s) { p->stride = s; return p; })
        .def("padding", [](std::shared_ptr<MaxPool2d> p, std::vector<int64_t> s) { p->padding = s; return p; });

    module_class<ReLU, Module>(m, "ReLU").def(py::init<>());

    module_class<Sequential, Module>(m, "Sequential")
        .def(py::init([](const std::vector<ModulePtr> &layers) {
            auto s = std::make_shared<Sequential>();
            s->layers = layers;
            return s;
        }));

    module_class<ParameterList, Module>(m, "ParameterList")
        .def(py::init([](const std::vector<std::pair<std::string, Parameter>> &params) {
            auto s = std::make_shared<ParameterList>();
            s->params = params;
            return s;
        }));

    py::class_<Optimizer, std::shared_ptr<Optimizer>>(m, "Optimizer")
        .def("step", &Optimizer::step)
        .def("completed_steps", &Optimizer::completed_steps);

    py::class_<Adam, Optimizer, std::shared_ptr<Adam>>(m, "Adam")
        .def(py::init<float, float, float, float>(), py::arg("learning_rate"), py::arg("beta1") = 0.9f,
             py::arg("beta2") = 0.999f, py::arg("epsilon") = 1e-8f)
        .def("step_parameters", &Adam::step_parameters)
        .def("set_learning_rate", &Adam::set_learning_rate)
        .def("moments", [](const Adam &a, const Parameter &p) {
            auto it = a.states.find(p.id());
            if (it == a.states.end()) throw Error("no Adam state for this parameter");
            return py::make_tuple(to_numpy(read_buffer(it->second.first)),
                                  to_numpy(read_buffer(it->second.second)));
        });

    py::class_<AdamW, Adam, std::shared_ptr<AdamW>>(m, "AdamW")
        .def(py::init<float, float, float, float, float>(), py::arg("learning_rate"),
             py::arg("weight_decay"), py::arg("beta1") = 0.9f, py::arg("beta2") = 0.999f,
             py::arg("epsilon") = 1e-8f);

    py::enum_<MuonOrientation>(m, "MuonMatrixOrientation")
        .value("FanInFanOut", MuonOrientation::FanInFanOut)
        .value("FanOutFanIn", MuonOrientation::FanOutFanIn);

    py::class_<MuonMatrix>(m, "MuonMatrix")
        .def_static("axis_linear", [](const Parameter &p) { return MuonMatrix{p.id(), MuonOrientation::FanInFanOut}; })
        .def_static("fan_in_fan_out", [](const Parameter &p) { return MuonMatrix{p.id(), MuonOrientation::FanInFanOut}; })
        .def_static("fan_out_fan_in", [](const Parameter &p) { return MuonMatrix{p.id(), MuonOrientation::FanOutFanIn}; })
        .def_readonly("orientation", &MuonMatrix::orientation);

    py::class_<Muon, Optimizer, std::shared_ptr<Muon>>(m, "Muon")
        .def(py::init<const std::vector<MuonMatrix> &, float, float, bool, float>(), py::arg("selected"),
             py::arg("learning_rate"), py::arg("momentum") = 0.95f, py::arg("nesterov") = true,
             py::arg("weight_decay") = 0.0f)
        .def("momentum_state", [](const Muon &mu, const Parameter &p) {
            auto it = mu.states.find(p.id());
            if (it == mu.states.end()) throw Error("no Muon state for this parameter");
            return to_numpy(it->second.to_vec());
        });

    py::class_<MuonWithAuxAdamW, Optimizer, std::shared_ptr<MuonWithAuxAdamW>>(m, "MuonWithAuxAdamW")
        .def(py::init<const std::vector<MuonMatrix> &, float, float, float>(), py::arg("selected"),
             py::arg("muon_learning_rate"), py::arg("adamw_learning_rate"), py::arg("weight_decay"))
        .def_property_readonly("muon", [](MuonWithAuxAdamW &o) -> Muon & { return o.muon; },
                               py::return_value_policy::reference_internal)
        .def_property_readonly("adamw", [](MuonWithAuxAdamW &o) -> AdamW & { return o.adamw; },
                               py::return_value_policy::reference_internal);

    py::class_<Trainer>(m, "Trainer")
        .def(py::init<std::shared_ptr<Optimizer>>())
        .def("step", [](Trainer &t, Module &model, const std::function<Tensor(Module &)> &loss) {
            TrainStep s = t.step(model, loss);
            return py::make_tuple(s.step, s.pre_update_loss);
        })
        .def_property_readonly("completed_steps", [](const Trainer &t) { return t.completed; });

    m.def("device_handle", [](const Device &d) { return (uintptr_t)d.h(); },
          "The axis_device (C ABI handle) behind a Device, for calls made through the C ABI.");
    m.def("zeroth_power", &zeroth_power);
    m.def("xorshift_unit_stream", [](uint64_t seed, int64_t n) { return to_numpy(xorshift_unit_stream(seed, n)); });
    m.def("uniform_host_values", [](uint64_t seed, int64_t n, float lo, float hi) {
        return to_numpy(uniform_host_values(seed, n, lo, hi));
    });
    m.def("normal_host_values", [](uint64_t seed, int64_t n, float mean, float std) {
        return to_numpy(normal_host_values(seed, n, mean, std));
    });
    m.def("powi", &powi);
}
