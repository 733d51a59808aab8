// Python binding of the host library (spar_amd._spar) for tests, benchmarks
// and Python users.  It exposes the same names as the C++ API; exceptions map
// to Python as: std::invalid_argument -> ValueError, std::out_of_range ->
// IndexError, std::overflow_error -> OverflowError, other std::logic_error ->
// spar_amd._spar.LogicError, std::runtime_error -> RuntimeError.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>

#include "spar/spar.hpp"

namespace py = pybind11;
using spar::Device;
using spar::DType;
using spar::Shape;
using spar::Tensor;

namespace {

Shape to_shape(const std::vector<std::int64_t>& dims) { return Shape{dims}; }

py::tuple shape_tuple(const Shape& shape) {
  py::tuple t(shape.rank());
  for (std::size_t i = 0; i < shape.rank(); ++i) t[i] = shape[i];
  return t;
}

py::dtype numpy_dtype(DType dtype) {
  switch (dtype) {
    case DType::Float32: return py::dtype::of<float>();
    case DType::Float64: return py::dtype::of<double>();
    case DType::Int32: return py::dtype::of<std::int32_t>();
    case DType::Int64: return py::dtype::of<std::int64_t>();
  }
  throw std::logic_error{"unknown dtype"};
}

template <typename T>
Tensor tensor_from(py::array_t<T, py::array::c_style | py::array::forcecast> array) {
  std::vector<std::int64_t> dims(array.shape(), array.shape() + array.ndim());
  const auto* begin = array.data();
  return spar::from_values<T>(Shape{dims}, std::span<const T>{begin, static_cast<std::size_t>(array.size())});
}

Tensor from_numpy(py::array array) {
  const auto kind = array.dtype().kind();
  const auto size = array.dtype().itemsize();
  if (kind == 'f' && size == 4) return tensor_from<float>(array);
  if (kind == 'f' && size == 8) return tensor_from<double>(array);
  if (kind == 'i' && size == 4) return tensor_from<std::int32_t>(array);
  if (kind == 'i' && size == 8) return tensor_from<std::int64_t>(array);
  throw std::invalid_argument{"from_numpy supports float32, float64, int32 and int64 arrays"};
}

// Copies a CPU tensor's logical values into a new numpy array.
py::array to_numpy(const Tensor& tensor) {
  if (!tensor.device().is_cpu()) {
    throw std::logic_error{"numpy() requires a CPU tensor; call to(Device.cpu()) first"};
  }
  const Tensor contiguous{tensor.detach().contiguous()};
  std::vector<py::ssize_t> dims(contiguous.shape().dimensions().begin(),
                                contiguous.shape().dimensions().end());
  py::array out(numpy_dtype(contiguous.dtype()), dims);
  if (contiguous.nbytes() == 0) return out;
  switch (contiguous.dtype()) {
    case DType::Float32:
      std::memcpy(out.mutable_data(), contiguous.span<float>().data(), contiguous.nbytes());
      break;
    case DType::Float64:
      std::memcpy(out.mutable_data(), contiguous.span<double>().data(), contiguous.nbytes());
      break;
    case DType::Int32:
      std::memcpy(out.mutable_data(), contiguous.span<std::int32_t>().data(), contiguous.nbytes());
      break;
    case DType::Int64:
      std::memcpy(out.mutable_data(), contiguous.span<std::int64_t>().data(), contiguous.nbytes());
      break;
  }
  return out;
}

std::vector<std::size_t> axes_of(py::object axes) {
  if (py::isinstance<py::int_>(axes)) return {axes.cast<std::size_t>()};
  return axes.cast<std::vector<std::size_t>>();
}

}  // namespace

PYBIND11_MODULE(_spar, m) {
  m.doc() = "Spar tensor/ops API on the MI355X HIP backend";

  static py::exception<std::logic_error> logic_error(m, "LogicError", PyExc_RuntimeError);
  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const std::invalid_argument& e) {
      PyErr_SetString(PyExc_ValueError, e.what());
    } catch (const std::out_of_range& e) {
      PyErr_SetString(PyExc_IndexError, e.what());
    } catch (const std::overflow_error& e) {
      PyErr_SetString(PyExc_OverflowError, e.what());
    } catch (const std::logic_error& e) {
      logic_error(e.what());
    }
  });

  py::enum_<DType>(m, "DType")
      .value("float32", DType::Float32)
      .value("float64", DType::Float64)
      .value("int32", DType::Int32)
      .value("int64", DType::Int64);

  py::class_<Device>(m, "Device")
      .def_static("cpu", &Device::cpu)
      .def_static("hip", &Device::hip, py::arg("index") = 0)
      .def_property_readonly("index", &Device::index)
      .def_property_readonly("is_cpu", &Device::is_cpu)
      .def_property_readonly("is_hip", &Device::is_hip)
      .def("__eq__", [](const Device& a, const Device& b) { return a == b; })
      .def("__repr__", &Device::to_string);

  py::class_<Tensor>(m, "Tensor")
      .def(py::init([](const std::vector<std::int64_t>& shape, DType dtype, Device device) {
             return Tensor{to_shape(shape), dtype, device};
           }),
           py::arg("shape"), py::arg("dtype"), py::arg("device") = Device::cpu())
      .def_static("from_numpy", &from_numpy)
      .def("numpy", &to_numpy)
      .def_property_readonly("shape", [](const Tensor& t) { return shape_tuple(t.shape()); })
      .def_property_readonly("strides", [](const Tensor& t) {
        return std::vector<std::size_t>(t.strides().begin(), t.strides().end());
      })
      .def_property_readonly("storage_offset", &Tensor::storage_offset)
      .def_property_readonly("dtype", &Tensor::dtype)
      .def_property_readonly("device", &Tensor::device)
      .def_property_readonly("numel", &Tensor::numel)
      .def_property_readonly("nbytes", &Tensor::nbytes)
      .def_property_readonly("rank", &Tensor::rank)
      .def("is_contiguous", &Tensor::is_contiguous)
      .def_property_readonly("requires_grad", &Tensor::requires_grad)
      .def_property_readonly("is_leaf", &Tensor::is_leaf)
      .def_property_readonly("has_grad", &Tensor::has_grad)
      .def("set_requires_grad", &Tensor::set_requires_grad, py::arg("enabled") = true)
      .def("grad", &Tensor::grad)
      .def("zero_grad", &Tensor::zero_grad)
      .def("backward", &Tensor::backward, py::call_guard<py::gil_scoped_release>())
      .def("detach", &Tensor::detach)
      .def("to", &Tensor::to)
      .def("clone", &Tensor::clone)
      .def("contiguous", &Tensor::contiguous)
      .def("reshape", [](const Tensor& t, const std::vector<std::int64_t>& s) { return t.reshape(to_shape(s)); })
      .def("transpose", &Tensor::transpose)
      .def("permute", [](const Tensor& t, const std::vector<std::size_t>& axes) {
        return t.permute(std::span<const std::size_t>{axes.data(), axes.size()});
      })
      .def("expand", [](const Tensor& t, const std::vector<std::int64_t>& s) { return t.expand(to_shape(s)); })
      .def("narrow", &Tensor::narrow);

  py::class_<spar::Random>(m, "Random")
      .def(py::init<std::uint64_t>())
      .def_property("state", &spar::Random::state, &spar::Random::set_state)
      .def("next_u64", &spar::Random::next_u64)
      .def("uniform_float", &spar::Random::uniform_float)
      .def("uniform_double", &spar::Random::uniform_double);

  m.def("random_uniform",
        [](const std::vector<std::int64_t>& shape, DType dtype, spar::Random& random, double low,
           double high, Device device) {
          return spar::random_uniform(to_shape(shape), dtype, random, low, high, device);
        },
        py::arg("shape"), py::arg("dtype"), py::arg("random"), py::arg("low") = 0.0,
        py::arg("high") = 1.0, py::arg("device") = Device::cpu());
  m.def("random_normal",
        [](const std::vector<std::int64_t>& shape, DType dtype, spar::Random& random, double mean,
           double stddev, Device device) {
          return spar::random_normal(to_shape(shape), dtype, random, mean, stddev, device);
        },
        py::arg("shape"), py::arg("dtype"), py::arg("random"), py::arg("mean") = 0.0,
        py::arg("stddev") = 1.0, py::arg("device") = Device::cpu());

  m.def("set_exact_gradient_zero_signs", &spar::set_exact_gradient_zero_signs, py::arg("enabled"));
  m.def("exact_gradient_zero_signs", &spar::exact_gradient_zero_signs);
  m.def("zeros", [](const std::vector<std::int64_t>& s, DType d, Device dev) { return spar::zeros(to_shape(s), d, dev); },
        py::arg("shape"), py::arg("dtype"), py::arg("device") = Device::cpu());
  m.def("ones", [](const std::vector<std::int64_t>& s, DType d, Device dev) { return spar::ones(to_shape(s), d, dev); },
        py::arg("shape"), py::arg("dtype"), py::arg("device") = Device::cpu());
  m.def("full", [](const std::vector<std::int64_t>& s, double v, DType d, Device dev) {
          return spar::full_value(to_shape(s), d, v, dev);
        },
        py::arg("shape"), py::arg("value"), py::arg("dtype"), py::arg("device") = Device::cpu());

#define SPAR_BINARY(name) m.def(#name, &spar::name, py::call_guard<py::gil_scoped_release>());
  SPAR_BINARY(add)
  SPAR_BINARY(subtract)
  SPAR_BINARY(multiply)
  SPAR_BINARY(divide)
  SPAR_BINARY(equal)
  SPAR_BINARY(not_equal)
  SPAR_BINARY(less)
  SPAR_BINARY(less_equal)
  SPAR_BINARY(greater)
  SPAR_BINARY(greater_equal)
  SPAR_BINARY(add_scalar)
  SPAR_BINARY(subtract_scalar)
  SPAR_BINARY(multiply_scalar)
  SPAR_BINARY(divide_scalar)
  SPAR_BINARY(negate)
  SPAR_BINARY(square)
  SPAR_BINARY(reciprocal)
  SPAR_BINARY(exp)
  SPAR_BINARY(log)
  SPAR_BINARY(sqrt)
  SPAR_BINARY(sigmoid)
  SPAR_BINARY(silu)
  SPAR_BINARY(tanh)
  SPAR_BINARY(gelu)
  SPAR_BINARY(reduce_max)
#undef SPAR_BINARY

  m.def("sum", [](const Tensor& x, py::object axes, bool keepdim) {
          if (axes.is_none()) return spar::sum(x);
          const auto a = axes_of(axes);
          return spar::sum(x, std::span<const std::size_t>{a.data(), a.size()}, keepdim);
        },
        py::arg("input"), py::arg("axes") = py::none(), py::arg("keepdim") = false);
  m.def("mean", [](const Tensor& x, py::object axes, bool keepdim) {
          if (axes.is_none()) return spar::mean(x);
          const auto a = axes_of(axes);
          return spar::mean(x, std::span<const std::size_t>{a.data(), a.size()}, keepdim);
        },
        py::arg("input"), py::arg("axes") = py::none(), py::arg("keepdim") = false);
  m.def("max", &spar::max, py::arg("input"), py::arg("axis"), py::arg("keepdim") = false);
  m.def("argmax", &spar::argmax, py::arg("input"), py::arg("axis"), py::arg("keepdim") = false);
  m.def("softmax", [](const Tensor& x, py::object axis) {
          return axis.is_none() ? spar::softmax(x) : spar::softmax(x, axis.cast<std::size_t>());
        },
        py::arg("input"), py::arg("axis") = py::none());
  m.def("log_softmax", [](const Tensor& x, py::object axis) {
          return axis.is_none() ? spar::log_softmax(x) : spar::log_softmax(x, axis.cast<std::size_t>());
        },
        py::arg("input"), py::arg("axis") = py::none());
  auto loss = m.def_submodule("loss", "spar::loss (src/loss/cross_entropy.cppm)");
  py::enum_<spar::loss::Reduction>(loss, "Reduction")
      .value("None_", spar::loss::Reduction::None)
      .value("Sum", spar::loss::Reduction::Sum)
      .value("Mean", spar::loss::Reduction::Mean);
  loss.def("cross_entropy", &spar::loss::cross_entropy, py::arg("logits"), py::arg("targets"),
           py::arg("reduction") = spar::loss::Reduction::Mean,
           py::call_guard<py::gil_scoped_release>());
  loss.def("language_model_cross_entropy", &spar::loss::language_model_cross_entropy,
           py::arg("logits"), py::arg("token_ids"),
           py::arg("reduction") = spar::loss::Reduction::Mean,
           py::call_guard<py::gil_scoped_release>());
  auto nn = m.def_submodule("nn", "spar::nn::Parameter (src/nn/parameter.cppm)");
  py::class_<spar::nn::Parameter>(nn, "Parameter")
      .def(py::init<Tensor>(), py::arg("initial_value"))
      .def("tensor", &spar::nn::Parameter::tensor)
      .def("requires_grad", &spar::nn::Parameter::requires_grad)
      .def("shares_identity_with", &spar::nn::Parameter::shares_identity_with)
      .def("set_requires_grad", &spar::nn::Parameter::set_requires_grad, py::arg("enabled"))
      .def("has_grad", &spar::nn::Parameter::has_grad)
      .def("grad", &spar::nn::Parameter::grad)
      .def("zero_grad", &spar::nn::Parameter::zero_grad)
      .def("clone", &spar::nn::Parameter::clone);
  // Parameter copies share their Tensor and Storage, so moving the copies
  // in this list moves the caller's Parameters.
  nn.def("move_to", [](std::vector<spar::nn::Parameter> parameters, Device target) {
    py::gil_scoped_release release;
    spar::nn::move_to(std::span<spar::nn::Parameter>{parameters}, target);
  }, py::arg("parameters"), py::arg("target"));
  auto training = m.def_submodule("training", "spar::training (src/training/gradients.cppm)");
  py::class_<spar::training::ClipGradNormResult>(training, "ClipGradNormResult")
      .def_readonly("total_norm", &spar::training::ClipGradNormResult::total_norm)
      .def_readonly("scale", &spar::training::ClipGradNormResult::scale)
      .def_readonly("clipped", &spar::training::ClipGradNormResult::clipped);
  training.def("global_grad_norm", [](std::vector<spar::nn::Parameter> parameters) {
    py::gil_scoped_release release;
    return spar::training::global_grad_norm(parameters);
  }, py::arg("parameters"));
  training.def("scale_gradients", [](std::vector<spar::nn::Parameter> parameters, double factor) {
    py::gil_scoped_release release;
    spar::training::scale_gradients(parameters, factor);
  }, py::arg("parameters"), py::arg("factor"));
  training.def("clip_grad_norm", [](std::vector<spar::nn::Parameter> parameters, double max_norm) {
    py::gil_scoped_release release;
    return spar::training::clip_grad_norm(parameters, max_norm);
  }, py::arg("parameters"), py::arg("max_norm"));
  auto optim = m.def_submodule("optim", "spar::optim::AdamW (src/optim/adamw.cppm)");
  py::class_<spar::optim::AdamWParameterState>(optim, "AdamWParameterState")
      .def(py::init([](Tensor first, Tensor second, std::uint64_t step) {
             return spar::optim::AdamWParameterState{std::move(first), std::move(second), step};
           }),
           py::arg("first_moment"), py::arg("second_moment"), py::arg("step"))
      .def_readwrite("first_moment", &spar::optim::AdamWParameterState::first_moment)
      .def_readwrite("second_moment", &spar::optim::AdamWParameterState::second_moment)
      .def_readwrite("step", &spar::optim::AdamWParameterState::step);
  py::class_<spar::optim::AdamW>(optim, "AdamW")
      .def(py::init<std::vector<spar::nn::Parameter>, double, double, double, double, double>(),
           py::arg("parameters") = std::vector<spar::nn::Parameter>{},
           py::arg("learning_rate") = 1.0e-3, py::arg("beta1") = 0.9, py::arg("beta2") = 0.999,
           py::arg("epsilon") = 1.0e-8, py::arg("weight_decay") = 0.01)
      .def("step", &spar::optim::AdamW::step, py::call_guard<py::gil_scoped_release>())
      .def("zero_grad", &spar::optim::AdamW::zero_grad)
      .def("move_to", &spar::optim::AdamW::move_to, py::arg("target"),
           py::call_guard<py::gil_scoped_release>())
      .def("parameter_count", &spar::optim::AdamW::parameter_count)
      .def("learning_rate", &spar::optim::AdamW::learning_rate)
      .def("set_learning_rate", &spar::optim::AdamW::set_learning_rate, py::arg("learning_rate"))
      .def("beta1", &spar::optim::AdamW::beta1)
      .def("beta2", &spar::optim::AdamW::beta2)
      .def("epsilon", &spar::optim::AdamW::epsilon)
      .def("weight_decay", &spar::optim::AdamW::weight_decay)
      .def("tracks", &spar::optim::AdamW::tracks, py::arg("parameter"))
      .def("parameter_state", &spar::optim::AdamW::parameter_state, py::arg("parameter"))
      .def("set_parameter_state", &spar::optim::AdamW::set_parameter_state, py::arg("parameter"),
           py::arg("state"));
  m.def("rms_norm", &spar::rms_norm, py::arg("input"), py::arg("weight"),
        py::arg("epsilon") = 1.0e-5, py::call_guard<py::gil_scoped_release>());
  m.def("layer_norm", &spar::layer_norm, py::arg("input"), py::arg("weight"), py::arg("bias"),
        py::arg("epsilon") = 1.0e-5, py::call_guard<py::gil_scoped_release>());
  m.def("reduce_gradient_to_shape", [](const Tensor& g, const std::vector<std::int64_t>& s) {
    return spar::detail::reduce_gradient_to_shape(g, to_shape(s));
  });
  m.def("broadcast_shape", [](const std::vector<std::int64_t>& a, const std::vector<std::int64_t>& b) {
    return shape_tuple(spar::detail::broadcast_shape(to_shape(a), to_shape(b)));
  });
  m.def("copy_values", [](Tensor& destination, const Tensor& source) {
    spar::detail::copy_tensor_values(destination, source);
  });
  m.def("synchronize", &spar::synchronize, py::arg("device") = Device::hip(0));
  m.def("hip_device_count", &spar::hip_device_count);
  m.def("set_autograd_hand_overs", &spar::detail::set_autograd_hand_overs, py::arg("enabled"));
  m.def("autograd_counters", [] {
    const auto c = spar::detail::autograd_counters();
    py::dict d;
    d["backward_calls"] = c.backward_calls;
    d["leaf_copies"] = c.leaf_copies;
    d["in_place_adds"] = c.in_place_adds;
    d["out_of_place_adds"] = c.out_of_place_adds;
    d["window_fusions"] = c.window_fusions;
    d["placed_gradients"] = c.placed_gradients;
    d["scaled_gradients"] = c.scaled_gradients;
    return d;
  });
}
