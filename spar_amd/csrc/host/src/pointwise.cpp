// Elementwise, comparison, scalar and unary ops with their backward rules.
// Forward semantics and errors: src/ops/elementwise.cpp:15-220,
// src/ops/scalar.cpp:13-103, src/ops/unary.cpp:15-164.  Broadcast operands
// are read in place through zero strides (no expand().contiguous() copies).
#include <cmath>
#include <limits>
#include <optional>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"

namespace spar {
namespace {

using detail::HipTensorAccess;
namespace hip = detail::hip;

// elementwise.cpp:15-24
Shape validate_binary_inputs(const Tensor& a, const Tensor& b) {
  detail::validate_same_device(a, b, "Elementwise operation");
  if (a.dtype() != b.dtype()) throw std::invalid_argument{"Elementwise operations require identical dtypes"};
  if (!is_floating(a.dtype())) {
    throw std::invalid_argument{"Elementwise operations currently support floating-point dtypes only"};
  }
  return detail::broadcast_shape(a.shape(), b.shape());
}

const char* binary_name(int operation) {
  switch (operation) {
    case SPAR_HIP_ADD: return "add";
    case SPAR_HIP_SUBTRACT: return "subtract";
    case SPAR_HIP_MULTIPLY: return "multiply";
    case SPAR_HIP_DIVIDE: return "divide";
    case SPAR_HIP_EQUAL: return "equal";
    case SPAR_HIP_NOT_EQUAL: return "not_equal";
    case SPAR_HIP_LESS: return "less";
    case SPAR_HIP_LESS_EQUAL: return "less_equal";
    case SPAR_HIP_GREATER: return "greater";
    default: return "greater_equal";
  }
}

// One device pass over the broadcast shape.  Same-shape contiguous operands
// take the flat kernel; anything else is read through its (expanded) view.
Tensor binary_device(const Tensor& a, const Tensor& b, const Shape& output_shape, int operation) {
  const char* name = binary_name(operation);
  detail::require_hip(a, name);
  Tensor output{output_shape, a.dtype(), a.device()};
  if (output.numel() == 0) return output;
  const int device = a.device().index();
  if (a.shape() == output_shape && b.shape() == output_shape && a.is_contiguous() &&
      b.is_contiguous()) {
    hip::check(spar_hip_launch_binary(HipTensorAccess::mutable_data(output), HipTensorAccess::data(a),
                                      HipTensorAccess::data(b), output.numel(),
                                      hip::dtype_tag(a.dtype()), operation, device),
               name, a.device());
    return output;
  }
  const auto left{hip::expanded_view(a, output_shape)};
  const auto right{hip::expanded_view(b, output_shape)};
  hip::check(spar_hip_launch_strided_binary(HipTensorAccess::mutable_data(output),
                                            HipTensorAccess::storage_base(a), left.strides.data(),
                                            left.offset, HipTensorAccess::storage_base(b),
                                            right.strides.data(), right.offset,
                                            left.extents.size(), left.extents.data(),
                                            hip::dtype_tag(a.dtype()), operation, device),
             name, a.device());
  return output;
}

// An incoming gradient may be a view (a reduction's gradient is a stride-0
// broadcast); the scalar ops, like the reference's, take contiguous inputs.
Tensor dense_gradient(const Tensor& gradient) {
  return gradient.is_contiguous() ? gradient.detach() : gradient.detach().contiguous();
}

bool full_contiguous(const Tensor& t, const Shape& shape) {
  return t.shape() == shape && t.is_contiguous();
}

// reduce_gradient_to_shape(multiply(gradient, factor), shape) in one pass
// when both operands span the full output; the products are rounded exactly
// as multiply() would store them.
Tensor multiply_then_reduce(const Tensor& gradient, const Tensor& factor, const Shape& shape) {
  if (gradient.shape() != shape && full_contiguous(gradient, gradient.shape()) &&
      full_contiguous(factor, gradient.shape()) &&
      gradient.shape() == detail::broadcast_shape(gradient.shape(), shape)) {
    Tensor result{shape, gradient.dtype(), gradient.device()};
    const auto gradient_extents{hip::extents_of(gradient.shape())};
    const auto original_extents{hip::extents_of(shape)};
    hip::check(spar_hip_launch_multiply_reduce(
                   HipTensorAccess::mutable_data(result), HipTensorAccess::data(gradient),
                   HipTensorAccess::data(factor), gradient_extents.size(), gradient_extents.data(),
                   original_extents.size(), original_extents.data(), gradient.numel(),
                   hip::dtype_tag(gradient.dtype()), gradient.device().index()),
               "multiply backward", gradient.device());
    return result;
  }
  return detail::reduce_gradient_to_shape(multiply(gradient, factor), shape);
}

std::vector<Tensor> requiring(const Tensor& a, const Tensor& b, bool grad_a, bool grad_b) {
  std::vector<Tensor> parents;
  if (grad_a) parents.push_back(a);
  if (grad_b) parents.push_back(b);
  return parents;
}

Tensor compare(const Tensor& a, const Tensor& b, int operation) {
  const Shape output_shape{validate_binary_inputs(a, b)};
  if (a.requires_grad() || b.requires_grad()) {
    throw std::logic_error{std::string{"autograd for "} + binary_name(operation) +
                           " is not implemented"};
  }
  return binary_device(a, b, output_shape, operation);
}

// scalar.cpp:13-22
void validate_scalar_input(const Tensor& input) {
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{"Scalar operations currently support floating-point dtypes only"};
  }
  if (!input.is_contiguous()) {
    throw std::invalid_argument{"Scalar operations currently require contiguous tensors"};
  }
}

// scalar.cpp:36-81: float32 scalars must be representable (finite values
// beyond FLT_MAX are rejected); the device rounds the double to T.
Tensor dispatch_scalar(const Tensor& input, double value, int operation) {
  validate_scalar_input(input);
  if (input.dtype() == DType::Float32) {
    constexpr double float_limit{static_cast<double>(std::numeric_limits<float>::max())};
    if (std::isfinite(value) && (value > float_limit || value < -float_limit)) {
      throw std::overflow_error{"Scalar value is outside the finite Float32 range"};
    }
  }
  detail::require_hip(input, binary_name(operation));
  Tensor output{input.shape(), input.dtype(), input.device()};
  if (output.numel() == 0) return output;
  hip::check(spar_hip_launch_scalar(HipTensorAccess::mutable_data(output),
                                    HipTensorAccess::data(input), output.numel(),
                                    hip::dtype_tag(input.dtype()), operation, value,
                                    input.device().index()),
             binary_name(operation), input.device());
  return output;
}

// unary.cpp:15-22
void validate_unary_input(const Tensor& input) {
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{"Unary operations currently support floating-point dtypes only"};
  }
  if (!input.is_contiguous()) {
    throw std::invalid_argument{"Unary operations currently require contiguous tensors"};
  }
}

Tensor dispatch_unary(const Tensor& input, int operation, const char* name) {
  validate_unary_input(input);
  detail::require_hip(input, name);
  Tensor output{input.shape(), input.dtype(), input.device()};
  if (output.numel() == 0) return output;
  hip::check(spar_hip_launch_unary(HipTensorAccess::mutable_data(output),
                                   HipTensorAccess::data(input), output.numel(),
                                   hip::dtype_tag(input.dtype()), operation,
                                   input.device().index()),
             name, input.device());
  return output;
}

}  // namespace

// ------------------------------------------------------------ elementwise

Tensor add(const Tensor& a, const Tensor& b) {
  const Shape output_shape{validate_binary_inputs(a, b)};
  Tensor output{binary_device(a, b, output_shape, SPAR_HIP_ADD)};
  if (a.requires_grad() || b.requires_grad()) {
    const bool grad_a{a.requires_grad()}, grad_b{b.requires_grad()};
    const Shape shape_a{a.shape()}, shape_b{b.shape()};
    detail::record_operation(output, requiring(a, b, grad_a, grad_b),
                             [grad_a, grad_b, shape_a, shape_b](const Tensor& gradient) {
                               std::vector<Tensor> contributions;
                               if (grad_a) contributions.push_back(detail::reduce_gradient_to_shape(gradient, shape_a));
                               if (grad_b) contributions.push_back(detail::reduce_gradient_to_shape(gradient, shape_b));
                               return contributions;
                             });
  }
  return output;
}

Tensor subtract(const Tensor& a, const Tensor& b) {
  const Shape output_shape{validate_binary_inputs(a, b)};
  Tensor output{binary_device(a, b, output_shape, SPAR_HIP_SUBTRACT)};
  if (a.requires_grad() || b.requires_grad()) {
    const bool grad_a{a.requires_grad()}, grad_b{b.requires_grad()};
    const Shape shape_a{a.shape()}, shape_b{b.shape()};
    detail::record_operation(
        output, requiring(a, b, grad_a, grad_b),
        [grad_a, grad_b, shape_a, shape_b](const Tensor& gradient) {
          std::vector<Tensor> contributions;
          if (grad_a) contributions.push_back(detail::reduce_gradient_to_shape(gradient, shape_a));
          if (grad_b) {
            const auto negative{multiply_scalar(dense_gradient(gradient), -1.0)};
            contributions.push_back(detail::reduce_gradient_to_shape(negative, shape_b));
          }
          return contributions;
        });
  }
  return output;
}

// Saved operands alias the inputs (detach, no copy): device tensors are
// never modified in place by this backend's ops, so a saved alias holds the
// same values a clone would (elementwise.cpp:140-147 cloned them).
Tensor multiply(const Tensor& a, const Tensor& b) {
  const Shape output_shape{validate_binary_inputs(a, b)};
  Tensor output{binary_device(a, b, output_shape, SPAR_HIP_MULTIPLY)};
  if (a.requires_grad() || b.requires_grad()) {
    const bool grad_a{a.requires_grad()}, grad_b{b.requires_grad()};
    const Shape shape_a{a.shape()}, shape_b{b.shape()};
    std::optional<Tensor> saved_a, saved_b;
    if (grad_b) saved_a.emplace(a.detach());
    if (grad_a) saved_b.emplace(b.detach());
    detail::record_operation(
        output, requiring(a, b, grad_a, grad_b),
        [grad_a, grad_b, shape_a, shape_b, saved_a, saved_b](const Tensor& gradient) {
          std::vector<Tensor> contributions;
          if (grad_a) contributions.push_back(multiply_then_reduce(gradient, *saved_b, shape_a));
          if (grad_b) contributions.push_back(multiply_then_reduce(gradient, *saved_a, shape_b));
          return contributions;
        });
    // One tracked operand of the output's shape: its gradient is the output
    // gradient times the other operand, with no reduction, which a scaled
    // rule downstream can take as (other operand, value).
    const Tensor& factor{grad_a ? b : a};
    if (grad_a != grad_b && (grad_a ? shape_a : shape_b) == output_shape &&
        factor.shape() == output_shape && factor.is_contiguous()) {
      detail::set_product_factor(output, grad_a ? *saved_b : *saved_a);
    }
  }
  return output;
}

Tensor divide(const Tensor& a, const Tensor& b) {
  const Shape output_shape{validate_binary_inputs(a, b)};
  Tensor output{binary_device(a, b, output_shape, SPAR_HIP_DIVIDE)};
  if (a.requires_grad() || b.requires_grad()) {
    const bool grad_a{a.requires_grad()}, grad_b{b.requires_grad()};
    const Shape shape_a{a.shape()}, shape_b{b.shape()};
    std::optional<Tensor> saved_a;
    if (grad_b) saved_a.emplace(a.detach());
    const Tensor saved_b{b.detach()};
    detail::record_operation(
        output, requiring(a, b, grad_a, grad_b),
        [grad_a, grad_b, shape_a, shape_b, saved_a, saved_b](const Tensor& gradient) {
          // elementwise.cpp:204-217
          std::vector<Tensor> contributions;
          if (grad_a) {
            const auto local{divide(gradient, saved_b)};
            contributions.push_back(detail::reduce_gradient_to_shape(local, shape_a));
          }
          if (grad_b) {
            // -(g a / (b b)), negated through the denominator: x / -y is
            // -(x / y) bit for bit (division rounds symmetrically), and the
            // denominator has b's shape, which a broadcast b keeps small, where
            // the reference negates the full quotient.
            const auto denominator{multiply_scalar(multiply(saved_b, saved_b), -1.0)};
            const auto numerator{multiply(gradient, *saved_a)};
            const auto local{divide(numerator, denominator)};
            contributions.push_back(detail::reduce_gradient_to_shape(local, shape_b));
          }
          return contributions;
        });
  }
  return output;
}

Tensor equal(const Tensor& a, const Tensor& b) { return compare(a, b, SPAR_HIP_EQUAL); }
Tensor not_equal(const Tensor& a, const Tensor& b) { return compare(a, b, SPAR_HIP_NOT_EQUAL); }
Tensor less(const Tensor& a, const Tensor& b) { return compare(a, b, SPAR_HIP_LESS); }
Tensor less_equal(const Tensor& a, const Tensor& b) { return compare(a, b, SPAR_HIP_LESS_EQUAL); }
Tensor greater(const Tensor& a, const Tensor& b) { return compare(a, b, SPAR_HIP_GREATER); }
Tensor greater_equal(const Tensor& a, const Tensor& b) {
  return compare(a, b, SPAR_HIP_GREATER_EQUAL);
}

// ----------------------------------------------------------------- scalar

Tensor add_scalar(const Tensor& input, double value) {
  Tensor output{dispatch_scalar(input, value, SPAR_HIP_ADD)};
  if (input.requires_grad()) {
    detail::record_operation(output, {input},
                             [](const Tensor& gradient) { return std::vector<Tensor>{gradient}; });
  }
  return output;
}

Tensor subtract_scalar(const Tensor& input, double value) {
  Tensor output{dispatch_scalar(input, value, SPAR_HIP_SUBTRACT)};
  if (input.requires_grad()) {
    detail::record_operation(output, {input},
                             [](const Tensor& gradient) { return std::vector<Tensor>{gradient}; });
  }
  return output;
}

Tensor multiply_scalar(const Tensor& input, double value) {
  Tensor output{dispatch_scalar(input, value, SPAR_HIP_MULTIPLY)};
  if (input.requires_grad()) {
    detail::record_operation(output, {input}, [value](const Tensor& gradient) {
      return std::vector<Tensor>{multiply_scalar(dense_gradient(gradient), value)};
    });
  }
  return output;
}

Tensor divide_scalar(const Tensor& input, double value) {
  Tensor output{dispatch_scalar(input, value, SPAR_HIP_DIVIDE)};
  if (input.requires_grad()) {
    detail::record_operation(output, {input}, [value](const Tensor& gradient) {
      return std::vector<Tensor>{divide_scalar(dense_gradient(gradient), value)};
    });
  }
  return output;
}

// ------------------------------------------------------------------ unary

Tensor negate(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_NEGATE, "negate")};
  if (input.requires_grad()) {
    detail::record_operation(output, {input}, [](const Tensor& gradient) {
      return std::vector<Tensor>{multiply_scalar(dense_gradient(gradient), -1.0)};
    });
  }
  return output;
}

Tensor square(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_SQUARE, "square")};
  if (input.requires_grad()) {
    const Tensor saved_input{input.detach()};
    detail::record_operation(output, {input}, [saved_input](const Tensor& gradient) {
      return std::vector<Tensor>{multiply(gradient, multiply_scalar(saved_input, 2.0))};
    });
  }
  return output;
}

Tensor reciprocal(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_RECIPROCAL, "reciprocal")};
  if (input.requires_grad()) {
    const Tensor saved_input{input.detach()};
    detail::record_operation(output, {input}, [saved_input](const Tensor& gradient) {
      const auto denominator{multiply(saved_input, saved_input)};
      return std::vector<Tensor>{multiply_scalar(divide(gradient, denominator), -1.0)};
    });
  }
  return output;
}

Tensor exp(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_EXP, "exp")};
  if (input.requires_grad()) {
    const Tensor saved_output{output.detach()};
    detail::record_operation(output, {input}, [saved_output](const Tensor& gradient) {
      return std::vector<Tensor>{multiply(gradient, saved_output)};
    });
  }
  return output;
}

Tensor log(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_LOG, "log")};
  if (input.requires_grad()) {
    const Tensor saved_input{input.detach()};
    detail::record_operation(output, {input}, [saved_input](const Tensor& gradient) {
      return std::vector<Tensor>{divide(gradient, saved_input)};
    });
  }
  return output;
}

Tensor sqrt(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_SQRT, "sqrt")};
  if (input.requires_grad()) {
    const Tensor saved_output{output.detach()};
    detail::record_operation(output, {input}, [saved_output](const Tensor& gradient) {
      return std::vector<Tensor>{divide(gradient, multiply_scalar(saved_output, 2.0))};
    });
  }
  return output;
}

Tensor sigmoid(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_SIGMOID, "sigmoid")};
  if (input.requires_grad()) {
    const Tensor saved_output{output.detach()};
    detail::record_operation(output, {input}, [saved_output](const Tensor& gradient) {
      const auto one_minus_output{add_scalar(multiply_scalar(saved_output, -1.0), 1.0)};
      return std::vector<Tensor>{multiply(gradient, multiply(saved_output, one_minus_output))};
    });
  }
  return output;
}

Tensor silu(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_SILU, "silu")};
  if (input.requires_grad()) {
    const Tensor saved_input{input.detach()};
    detail::record_operation(output, {input}, [saved_input](const Tensor& gradient) {
      // unary.cpp:155-160
      const auto sigmoid_value{sigmoid(saved_input)};
      const auto one_minus_sigmoid{add_scalar(multiply_scalar(sigmoid_value, -1.0), 1.0)};
      const auto sigmoid_slope{multiply(sigmoid_value, one_minus_sigmoid)};
      const auto local_derivative{add(sigmoid_value, multiply(saved_input, sigmoid_slope))};
      return std::vector<Tensor>{multiply(gradient, local_derivative)};
    });
  }
  return output;
}

// d tanh / dx = 1 - tanh(x)^2, composed from ops on the saved output.
Tensor tanh(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_TANH, "tanh")};
  if (input.requires_grad()) {
    const Tensor saved_output{output.detach()};
    detail::record_operation(output, {input}, [saved_output](const Tensor& gradient) {
      const auto one_minus_square{
          add_scalar(multiply_scalar(multiply(saved_output, saved_output), -1.0), 1.0)};
      return std::vector<Tensor>{multiply(gradient, one_minus_square)};
    });
  }
  return output;
}

// d gelu / dx = Phi(x) + x phi(x), evaluated by the GELU_DERIVATIVE kernel.
Tensor gelu(const Tensor& input) {
  Tensor output{dispatch_unary(input, SPAR_HIP_GELU, "gelu")};
  if (input.requires_grad()) {
    const Tensor saved_input{input.detach()};
    detail::record_operation(output, {input}, [saved_input](const Tensor& gradient) {
      const auto slope{dispatch_unary(saved_input, SPAR_HIP_GELU_DERIVATIVE, "gelu backward")};
      return std::vector<Tensor>{multiply(gradient, slope)};
    });
  }
  return output;
}

}  // namespace spar
