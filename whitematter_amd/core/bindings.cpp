// bindings.cpp -- Python view of the C++ Tensor (whitematter_amd/_tensor).
//
// Used by the parity tests to drive the drop-in Tensor API the way the
// reference's own C++ tests do (tests/test_tensor.cpp, test_autograd.cpp):
// build tensors, call ops, run backward(), read data and grad.  data/grad are
// copied to and from numpy; everything else stays on the device.
#include <cstring>

#include <pybind11/functional.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "amp.h"
#include "layer.h"
#include "serialize.h"
#include "loss.h"
#include "optimizer.h"
#include "tensor.h"
#include "wm_hip.h"

namespace py = pybind11;

namespace {

py::array_t<float> to_numpy(const wm::DeviceVector& v, const std::vector<size_t>& shape) {
    std::vector<py::ssize_t> s(shape.begin(), shape.end());
    size_t n = 1;
    for (auto d : shape) n *= d;
    if (n != v.size()) s = {(py::ssize_t)v.size()};
    py::array_t<float> out(s);
    if (v.size()) std::memcpy(out.mutable_data(), v.data(), v.size() * sizeof(float));
    return out;
}

std::vector<float> from_numpy(py::array_t<float, py::array::c_style | py::array::forcecast> a) {
    return std::vector<float>(a.data(), a.data() + a.size());
}

std::vector<size_t> shape_of(py::array_t<float, py::array::c_style | py::array::forcecast> a) {
    std::vector<size_t> s;
    for (py::ssize_t i = 0; i < a.ndim(); ++i) s.push_back((size_t)a.shape(i));
    return s;
}

}  // namespace

PYBIND11_MODULE(_tensor, m) {
    m.doc() = "whitematter Tensor with device-resident storage on MI355X";
    m.def("init", [](int device) {
        if (wm_init(device) != WM_OK) throw std::runtime_error(wm_last_error());
    });

    py::class_<GradMode>(m, "GradMode")
        .def_static("is_enabled", &GradMode::is_enabled)
        .def_static("set_enabled", &GradMode::set_enabled);

    py::class_<Tensor, TensorPtr>(m, "Tensor")
        .def_static("create", [](const std::vector<size_t>& shape, bool rg) { return Tensor::create(shape, rg); },
                    py::arg("shape"), py::arg("requires_grad") = false)
        .def_static("from_array",
                    [](py::array_t<float, py::array::c_style | py::array::forcecast> a, py::object shape, bool rg) {
                        std::vector<size_t> s = shape.is_none() ? shape_of(a) : shape.cast<std::vector<size_t>>();
                        return Tensor::create(from_numpy(a), s, rg);
                    },
                    py::arg("data"), py::arg("shape") = py::none(), py::arg("requires_grad") = false)
        .def_static("zeros", &Tensor::zeros, py::arg("shape"), py::arg("requires_grad") = false)
        .def_static("ones", &Tensor::ones, py::arg("shape"), py::arg("requires_grad") = false)
        .def_static("randn", &Tensor::randn, py::arg("shape"), py::arg("requires_grad") = false)
        .def_readwrite("shape", &Tensor::shape)
        .def_readwrite("requires_grad", &Tensor::requires_grad)
        .def_property(
            "data", [](const Tensor& t) { return to_numpy(t.data, t.shape); },
            [](Tensor& t, py::array_t<float, py::array::c_style | py::array::forcecast> a) { t.data = from_numpy(a); })
        .def_property(
            "grad",
            [](const Tensor& t) -> py::object {
                if (t.grad.empty()) return py::none();
                return to_numpy(t.grad, t.shape);
            },
            [](Tensor& t, py::array_t<float, py::array::c_style | py::array::forcecast> a) { t.grad = from_numpy(a); })
        .def_property_readonly("grad_known_zero", [](const Tensor& t) { return t.grad.known_zero(); })
        .def_property_readonly("has_grad_fn", [](const Tensor& t) { return (bool)t.grad_fn; })
        .def_property_readonly("num_parents", [](const Tensor& t) { return t.parents.size(); })
        .def("size", &Tensor::size)
        .def("ndim", &Tensor::ndim)
        .def("item", &Tensor::item)
        .def("zero_grad", &Tensor::zero_grad)
        .def("backward", &Tensor::backward)
        // Inject an upstream gradient and run this node's closure only.
        .def("run_grad_fn",
             [](Tensor& t, py::array_t<float, py::array::c_style | py::array::forcecast> g) {
                 t.grad = from_numpy(g);
                 if (t.grad_fn) t.grad_fn();
             })
        // This node's closure alone, on the gradient it holds.
        .def("call_grad_fn", [](Tensor& t) { if (t.grad_fn) t.grad_fn(); })
        // The gradient as a device copy of another tensor's values.
        .def("set_grad_from", [](Tensor& t, const TensorPtr& src) { t.grad = src->data; })
        .def("add", &Tensor::add)
        .def("sub", &Tensor::sub)
        .def("mul", py::overload_cast<const TensorPtr&>(&Tensor::mul, py::const_))
        .def("mul", py::overload_cast<float>(&Tensor::mul, py::const_))
        .def("div", py::overload_cast<const TensorPtr&>(&Tensor::div, py::const_))
        .def("div", py::overload_cast<float>(&Tensor::div, py::const_))
        .def("neg", &Tensor::neg)
        .def("relu", &Tensor::relu)
        .def("sigmoid", &Tensor::sigmoid)
        .def("tanh_", &Tensor::tanh_)
        .def("log_", &Tensor::log_)
        .def("exp_", &Tensor::exp_)
        .def("pow", py::overload_cast<const TensorPtr&>(&Tensor::pow, py::const_))
        .def("pow", py::overload_cast<float>(&Tensor::pow, py::const_))
        .def("sqrt", &Tensor::sqrt)
        .def("abs", &Tensor::abs)
        .def("clamp", &Tensor::clamp)
        .def("softmax", &Tensor::softmax, py::arg("dim") = -1)
        .def("log_softmax", &Tensor::log_softmax, py::arg("dim") = -1)
        .def("sum", &Tensor::sum, py::arg("dim") = -1, py::arg("keepdim") = false)
        .def("mean", &Tensor::mean, py::arg("dim") = -1, py::arg("keepdim") = false)
        .def("max", py::overload_cast<int, bool>(&Tensor::max, py::const_), py::arg("dim"),
             py::arg("keepdim") = false)
        .def("min", py::overload_cast<int, bool>(&Tensor::min, py::const_), py::arg("dim"),
             py::arg("keepdim") = false)
        .def("maximum", py::overload_cast<const TensorPtr&>(&Tensor::max, py::const_))
        .def("minimum", py::overload_cast<const TensorPtr&>(&Tensor::min, py::const_))
        .def("argmax", &Tensor::argmax, py::arg("dim") = -1, py::arg("keepdim") = false)
        .def("argmin", &Tensor::argmin, py::arg("dim") = -1, py::arg("keepdim") = false)
        .def("reshape", &Tensor::reshape)
        .def("flatten", &Tensor::flatten, py::arg("start_dim") = 1)
        .def("squeeze", &Tensor::squeeze, py::arg("dim") = -1)
        .def("unsqueeze", &Tensor::unsqueeze)
        .def("matmul", &Tensor::matmul)
        .def("bmm", &Tensor::bmm)
        .def("transpose", &Tensor::transpose)
        .def("__add__", [](const TensorPtr& a, const TensorPtr& b) { return *a + b; })
        .def("__sub__", [](const TensorPtr& a, const TensorPtr& b) { return *a - b; })
        .def("__mul__", [](const TensorPtr& a, const TensorPtr& b) { return *a * b; })
        .def("__mul__", [](const TensorPtr& a, float s) { return *a * s; })
        .def("__rmul__", [](const TensorPtr& a, float s) { return s * a; })
        .def("__truediv__", [](const TensorPtr& a, const TensorPtr& b) { return *a / b; })
        .def("__truediv__", [](const TensorPtr& a, float s) { return *a / s; })
        .def("__neg__", [](const TensorPtr& a) { return -(*a); });

    m.def("set_grad_enabled", &GradMode::set_enabled);

    // Drop-in optimizers (optimizer.h): steps and clipping run on the device;
    // state(i) copies one parameter's state buffers to numpy.
    py::class_<Optimizer>(m, "Optimizer")
        .def("step", &Optimizer::step)
        .def("zero_grad", &Optimizer::zero_grad)
        .def_readwrite("lr", &Optimizer::lr);
    auto states = [](const std::vector<wm::DeviceVector>& a, const std::vector<wm::DeviceVector>& b, size_t i) {
        py::list out;
        if (i < a.size()) out.append(to_numpy(a[i], {a[i].size()}));
        if (i < b.size()) out.append(to_numpy(b[i], {b[i].size()}));
        return out;
    };
    py::class_<SGD, Optimizer>(m, "SGD")
        .def(py::init<const std::vector<TensorPtr>&, float, float>(), py::arg("params"), py::arg("lr"),
             py::arg("momentum") = 0.0f)
        .def_readwrite("momentum", &SGD::momentum)
        .def("state", [states](const SGD& o, size_t i) { return states(o.velocity, {}, i); });
    py::class_<Adam, Optimizer>(m, "Adam")
        .def(py::init<const std::vector<TensorPtr>&, float, float, float, float>(), py::arg("params"),
             py::arg("lr") = 0.001f, py::arg("beta1") = 0.9f, py::arg("beta2") = 0.999f, py::arg("eps") = 1e-8f)
        .def_readonly("t", &Adam::t)
        .def("state", [states](const Adam& o, size_t i) { return states(o.m, o.v, i); });
    py::class_<AdamW, Optimizer>(m, "AdamW")
        .def(py::init<const std::vector<TensorPtr>&, float, float, float, float, float>(), py::arg("params"),
             py::arg("lr") = 0.001f, py::arg("beta1") = 0.9f, py::arg("beta2") = 0.999f, py::arg("eps") = 1e-8f,
             py::arg("weight_decay") = 0.01f)
        .def_readonly("t", &AdamW::t)
        .def("state", [states](const AdamW& o, size_t i) { return states(o.m, o.v, i); });
    py::class_<RMSprop, Optimizer>(m, "RMSprop")
        .def(py::init<const std::vector<TensorPtr>&, float, float, float, float, float>(), py::arg("params"),
             py::arg("lr") = 0.01f, py::arg("alpha") = 0.99f, py::arg("eps") = 1e-8f, py::arg("momentum") = 0.0f,
             py::arg("weight_decay") = 0.0f)
        .def("state", [states](const RMSprop& o, size_t i) { return states(o.v, o.buffer, i); });
    m.def("clip_grad_norm_", [](std::vector<TensorPtr> ps, float max_norm) { clip_grad_norm_(ps, max_norm); });

    // Mixed precision (amp.h): fp16 storage and loss scaling.
    m.def("float_to_half", &float_to_half);
    m.def("half_to_float", &half_to_float);
    m.def("to_half", [](py::array_t<float, py::array::c_style | py::array::forcecast> x) {
        std::vector<float> v(x.data(), x.data() + x.size());
        const std::vector<uint16_t> h = to_half(v);
        py::array_t<uint16_t> out(h.size());
        if (!h.empty()) std::memcpy(out.mutable_data(), h.data(), h.size() * sizeof(uint16_t));
        return out;
    });
    m.def("from_half", [](py::array_t<uint16_t, py::array::c_style | py::array::forcecast> x) {
        std::vector<uint16_t> v(x.data(), x.data() + x.size());
        const std::vector<float> f = from_half(v);
        py::array_t<float> out(f.size());
        if (!f.empty()) std::memcpy(out.mutable_data(), f.data(), f.size() * sizeof(float));
        return out;
    });
    py::class_<HalfTensor>(m, "HalfTensor")
        .def(py::init<const TensorPtr&>())
        .def_property_readonly("data", [](const HalfTensor& h) {
            py::array_t<uint16_t> a(h.data.size());
            if (!h.data.empty()) std::memcpy(a.mutable_data(), h.data.data(), h.data.size() * sizeof(uint16_t));
            return a;
        })
        .def_readonly("shape", &HalfTensor::shape)
        .def("to_float", &HalfTensor::to_float, py::arg("requires_grad") = false)
        .def("size", &HalfTensor::size)
        .def("memory_saved", &HalfTensor::memory_saved);
    py::class_<GradScaler>(m, "GradScaler")
        .def(py::init<float, float, float, int, bool>(), py::arg("init_scale") = 65536.0f,
             py::arg("growth_factor") = 2.0f, py::arg("backoff_factor") = 0.5f, py::arg("growth_interval") = 2000,
             py::arg("enabled") = true)
        .def("get_scale", &GradScaler::get_scale)
        .def("scale", py::overload_cast<const TensorPtr&>(&GradScaler::scale, py::const_))
        .def("unscale", &GradScaler::unscale)
        .def("step", &GradScaler::step, py::arg("optimizer"), py::arg("already_unscaled") = false)
        .def("update", &GradScaler::update)
        .def("growth_tracker", &GradScaler::growth_tracker)
        .def("set_scale", &GradScaler::set_scale);
    m.def("check_gradients_finite", &check_gradients_finite);
    m.def("clip_grad_norm_amp", &clip_grad_norm_amp, py::arg("params"), py::arg("max_norm"), py::arg("scale") = 1.0f);
    m.def("clip_grad_value_", [](std::vector<TensorPtr> ps, float c) { clip_grad_value_(ps, c); });
    m.def("get_grad_norm", &get_grad_norm);

    // Modules whose bodies run on the device (core/layer.h).
    py::class_<Module>(m, "Module")
        .def("forward", &Module::forward)
        .def("__call__", [](Module& mod, const TensorPtr& x) { return mod(x); })
        .def("parameters", &Module::parameters)
        .def("num_parameters", &Module::num_parameters);
    py::class_<LayerNorm, Module>(m, "LayerNorm")
        .def(py::init<size_t, float>(), py::arg("normalized_shape"), py::arg("eps") = 1e-5f)
        .def(py::init<std::vector<size_t>, float>(), py::arg("normalized_shape"), py::arg("eps") = 1e-5f)
        .def_readwrite("gamma", &LayerNorm::gamma)
        .def_readwrite("beta", &LayerNorm::beta);
    py::class_<BatchNorm2d, Module>(m, "BatchNorm2d")
        .def(py::init<size_t, float, float>(), py::arg("num_features"), py::arg("eps") = 1e-5f,
             py::arg("momentum") = 0.1f)
        .def("train", &BatchNorm2d::train)
        .def("eval", &BatchNorm2d::eval)
        .def_readwrite("training", &BatchNorm2d::training)
        .def_readwrite("gamma", &BatchNorm2d::gamma)
        .def_readwrite("beta", &BatchNorm2d::beta)
        .def_readwrite("running_mean", &BatchNorm2d::running_mean)
        .def_readwrite("running_var", &BatchNorm2d::running_var);
    py::class_<Linear, Module>(m, "Linear")
        .def(py::init<size_t, size_t>(), py::arg("in_features"), py::arg("out_features"))
        .def_readwrite("weight", &Linear::weight)
        .def_readwrite("bias", &Linear::bias);
    py::class_<MultiHeadAttention, Module>(m, "MultiHeadAttention")
        .def(py::init<size_t, size_t>(), py::arg("embed_dim"), py::arg("num_heads"))
        .def("attend",
             [](MultiHeadAttention& a, const TensorPtr& q, const TensorPtr& k, const TensorPtr& v,
                const TensorPtr& mask) { return a.forward(q, k, v, mask); },
             py::arg("query"), py::arg("key"), py::arg("value"), py::arg("mask") = TensorPtr())
        .def_static("causal_mask", &MultiHeadAttention::causal_mask)
        .def_readwrite("attn_weights", &MultiHeadAttention::attn_weights)
        .def_readwrite("W_q", &MultiHeadAttention::W_q)
        .def_readwrite("W_k", &MultiHeadAttention::W_k)
        .def_readwrite("W_v", &MultiHeadAttention::W_v)
        .def_readwrite("W_o", &MultiHeadAttention::W_o)
        .def_readwrite("b_q", &MultiHeadAttention::b_q)
        .def_readwrite("b_k", &MultiHeadAttention::b_k)
        .def_readwrite("b_v", &MultiHeadAttention::b_v)
        .def_readwrite("b_o", &MultiHeadAttention::b_o);
    py::class_<Dropout, Module>(m, "Dropout")
        .def(py::init<float>(), py::arg("p") = 0.5f)
        .def("train", &Dropout::train)
        .def("eval", &Dropout::eval);

    // WMT / WMM / WMO / checkpoint files (core/serialize.h), device-direct.
    m.def("save_tensor", py::overload_cast<const TensorPtr&, const std::string&>(&save_tensor));
    m.def("load_tensor", py::overload_cast<const std::string&>(&load_tensor));
    m.def("save_model", [](Module* mod, const std::string& p) { return save_model(mod, p); });
    m.def("load_model", [](Module* mod, const std::string& p) { return load_model(mod, p); });
    m.def("save_optimizer", [](Optimizer* o, const std::string& p) { return save_optimizer(o, p); });
    m.def("load_optimizer", [](Optimizer* o, const std::string& p) { return load_optimizer(o, p); });
    m.def("save_checkpoint",
          [](const std::string& p, Module* mod, Optimizer* o, int epoch, float loss, float acc) {
              return save_checkpoint(p, mod, o, epoch, loss, acc);
          },
          py::arg("path"), py::arg("model"), py::arg("optimizer"), py::arg("epoch"), py::arg("loss") = 0.0f,
          py::arg("accuracy") = 0.0f);
    m.def("load_checkpoint", [](const std::string& p, Module* mod, Optimizer* o) {
        Checkpoint info{0, 0.0f, 0.0f};
        const bool ok = load_checkpoint(p, mod, o, info);
        return py::make_tuple(ok, info.epoch, info.loss, info.accuracy);
    });

    py::class_<LossFunction>(m, "LossFunction")
        .def("forward", &LossFunction::forward)
        .def("__call__", [](LossFunction& l, const TensorPtr& p, const TensorPtr& t) { return l(p, t); });
    py::class_<MSELoss, LossFunction>(m, "MSELoss").def(py::init<>());
    py::class_<L1Loss, LossFunction>(m, "L1Loss").def(py::init<>());
    py::class_<SmoothL1Loss, LossFunction>(m, "SmoothL1Loss")
        .def(py::init<float>(), py::arg("beta") = 1.0f)
        .def_readwrite("beta", &SmoothL1Loss::beta);
    py::class_<CrossEntropyLoss, LossFunction>(m, "CrossEntropyLoss").def(py::init<>());
    py::class_<NLLLoss, LossFunction>(m, "NLLLoss").def(py::init<>());
    py::class_<BCELoss, LossFunction>(m, "BCELoss").def(py::init<>());
    py::class_<BCEWithLogitsLoss, LossFunction>(m, "BCEWithLogitsLoss").def(py::init<>());
    py::class_<KLDivLoss, LossFunction>(m, "KLDivLoss")
        .def(py::init<bool>(), py::arg("log_target") = false)
        .def_readwrite("log_target", &KLDivLoss::log_target);
    py::class_<FocalLoss, LossFunction>(m, "FocalLoss")
        .def(py::init<float, float>(), py::arg("gamma") = 2.0f, py::arg("alpha") = -1.0f)
        .def_readwrite("gamma", &FocalLoss::gamma)
        .def_readwrite("alpha", &FocalLoss::alpha);
    py::class_<BinaryFocalLoss, LossFunction>(m, "BinaryFocalLoss")
        .def(py::init<float, float>(), py::arg("gamma") = 2.0f, py::arg("alpha") = 0.25f)
        .def_readwrite("gamma", &BinaryFocalLoss::gamma)
        .def_readwrite("alpha", &BinaryFocalLoss::alpha);
}
