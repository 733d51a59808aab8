// softmax / log_softmax forward and backward (src/ops/softmax.cpp:13-516)
// through the probability kernels.  The undefined-slice flags of the forward
// pass (Int32, one per slice) drive the NaN derivatives of the backward pass,
// as on the reference's device path (softmax.cpp:245-261, :285-312, :456-485).
#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"

namespace spar {
namespace {

using detail::HipTensorAccess;
namespace hip = detail::hip;

struct Geometry {
  std::size_t outer;
  std::size_t axis_extent;
  std::size_t inner;
};

Geometry axis_geometry(const Tensor& input, std::size_t axis) {
  Geometry g{1, static_cast<std::size_t>(input.shape()[axis]), 1};
  for (std::size_t index{0}; index < axis; ++index) g.outer *= static_cast<std::size_t>(input.shape()[index]);
  for (std::size_t index{axis + 1}; index < input.rank(); ++index) {
    g.inner *= static_cast<std::size_t>(input.shape()[index]);
  }
  return g;
}

Tensor probability(const Tensor& input, const Geometry& g, bool logarithmic) {
  const char* name{logarithmic ? "log_softmax" : "softmax"};
  detail::require_hip(input, name);
  const Tensor contiguous_input{input.is_contiguous() ? input.detach() : input.detach().contiguous()};
  Tensor output{input.shape(), input.dtype(), input.device()};
  Tensor undefined_slices{Shape{static_cast<Shape::dimension_type>(g.outer * g.inner)},
                          DType::Int32, input.device()};
  hip::check(spar_hip_launch_probability_forward(
                 HipTensorAccess::mutable_data(output),
                 static_cast<std::int32_t*>(HipTensorAccess::mutable_data(undefined_slices)),
                 HipTensorAccess::data(contiguous_input), g.outer, g.axis_extent, g.inner,
                 hip::dtype_tag(input.dtype()), logarithmic ? 1 : 0, input.device().index()),
             name, input.device());
  if (input.requires_grad()) {
    const Tensor saved_output{output.detach()};
    detail::record_operation(
        output, {input}, [saved_output, undefined_slices, g, logarithmic](const Tensor& gradient) {
          const Tensor contiguous_gradient{gradient.is_contiguous() ? gradient.detach()
                                                                    : gradient.detach().contiguous()};
          Tensor contribution{saved_output.shape(), saved_output.dtype(), saved_output.device()};
          hip::check(spar_hip_launch_probability_backward(
                         HipTensorAccess::mutable_data(contribution),
                         HipTensorAccess::data(contiguous_gradient),
                         HipTensorAccess::data(saved_output),
                         static_cast<const std::int32_t*>(HipTensorAccess::data(undefined_slices)),
                         g.outer, g.axis_extent, g.inner, hip::dtype_tag(saved_output.dtype()),
                         logarithmic ? 1 : 0, saved_output.device().index()),
                     logarithmic ? "log_softmax backward" : "softmax backward",
                     saved_output.device());
          return std::vector<Tensor>{contribution};
        });
  }
  return output;
}

// softmax.cpp:13-23 (full) and :25-35 (axis)
void validate_softmax_input(const Tensor& input, const char* name) {
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{std::string{name} + " currently supports floating-point dtypes only"};
  }
  if (input.numel() == 0) throw std::invalid_argument{std::string{name} + " is undefined for an empty tensor"};
}

}  // namespace

Tensor softmax(const Tensor& input) {
  validate_softmax_input(input, "softmax");
  if (!input.is_contiguous()) throw std::invalid_argument{"softmax currently requires a contiguous tensor"};
  return probability(input, Geometry{1, input.numel(), 1}, false);
}

Tensor softmax(const Tensor& input, std::size_t axis) {
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{"softmax currently supports floating-point dtypes only"};
  }
  if (axis >= input.rank()) throw std::out_of_range{"softmax axis is out of range"};
  if (input.numel() == 0) throw std::invalid_argument{"softmax is undefined for an empty tensor"};
  return probability(input, axis_geometry(input, axis), false);
}

// softmax.cpp:446-455
Tensor log_softmax(const Tensor& input) {
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{"log_softmax supports floating-point dtypes only"};
  }
  if (input.numel() == 0) throw std::invalid_argument{"log_softmax is undefined for an empty tensor"};
  return probability(input, Geometry{1, input.numel(), 1}, true);
}

Tensor log_softmax(const Tensor& input, std::size_t axis) {
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{"log_softmax supports floating-point dtypes only"};
  }
  if (input.numel() == 0) throw std::invalid_argument{"log_softmax is undefined for an empty tensor"};
  if (axis >= input.rank()) throw std::out_of_range{"log_softmax axis is out of range"};
  return probability(input, axis_geometry(input, axis), true);
}

}  // namespace spar
