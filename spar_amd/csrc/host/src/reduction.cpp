// Reductions and their backward rules (src/ops/reduction.cpp:15-347).
// Axis reductions read the input view in place (no permute().contiguous()
// staging); full reductions of contiguous tensors take the split-grid
// kernel.  max/argmax over an axis are additions with the first-occurrence /
// NaN-first rule of reduce_max.
#include <algorithm>
#include <limits>
#include <optional>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"

namespace spar {
namespace {

using detail::HipTensorAccess;
namespace hip = detail::hip;

void validate_reduction_input(const Tensor& input) {
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{"Reductions currently support floating-point dtypes only"};
  }
}

// reduction.cpp:62-77
std::vector<std::size_t> validate_axes(const Tensor& input, std::span<const std::size_t> axes) {
  if (axes.empty()) throw std::invalid_argument{"Reduction axes must not be empty"};
  std::vector<std::size_t> normalized{axes.begin(), axes.end()};
  std::sort(normalized.begin(), normalized.end());
  for (std::size_t index{0}; index < normalized.size(); ++index) {
    if (normalized[index] >= input.rank()) throw std::out_of_range{"Reduction axis is out of range"};
    if (index != 0 && normalized[index] == normalized[index - 1]) {
      throw std::invalid_argument{"Reduction axes must not contain duplicates"};
    }
  }
  return normalized;
}

// reduction.cpp:79-96
Shape reduced_shape(const Tensor& input, std::span<const std::size_t> axes, bool keepdim) {
  std::vector<bool> reduced(input.rank(), false);
  for (const std::size_t axis : axes) reduced[axis] = true;
  std::vector<Shape::dimension_type> dimensions;
  for (std::size_t axis{0}; axis < input.rank(); ++axis) {
    if (reduced[axis]) {
      if (keepdim) dimensions.push_back(1);
    } else {
      dimensions.push_back(input.shape()[axis]);
    }
  }
  return Shape{std::move(dimensions)};
}

// reduction.cpp:98-108
std::size_t reduced_element_count(const Tensor& input, std::span<const std::size_t> axes) {
  std::size_t count{1};
  for (const std::size_t axis : axes) {
    const auto extent{static_cast<std::size_t>(input.shape()[axis])};
    if (extent != 0 && count > std::numeric_limits<std::size_t>::max() / extent) {
      throw std::overflow_error{"Reduction element count overflow"};
    }
    count *= extent;
  }
  return count;
}

// One device reduction of `input` over `axes` into a new tensor of
// `output_shape` (whose layout is the kept axes in order).
Tensor axis_reduce(const Tensor& input, std::span<const std::size_t> axes,
                   const Shape& output_shape, int operation, const char* name) {
  detail::require_hip(input, name);
  const DType out_dtype{operation == SPAR_HIP_ARGMAX ? DType::Int64 : input.dtype()};
  Tensor output{output_shape, out_dtype, input.device()};
  if (output.numel() == 0) return output;
  if (input.rank() > SPAR_HIP_MAX_RANK) {
    throw std::invalid_argument{std::string{name} + " supports tensors of rank <= 8 on HIP"};
  }
  std::uint32_t mask{0};
  for (const std::size_t axis : axes) mask |= 1U << axis;
  const auto view{hip::view_of(input)};
  hip::check(spar_hip_launch_axis_reduction(
                 HipTensorAccess::mutable_data(output),
                 input.numel() == 0 ? nullptr : HipTensorAccess::storage_base(input),
                 view.extents.size(), view.extents.data(), view.strides.data(), view.offset, mask,
                 hip::dtype_tag(input.dtype()), operation, input.device().index()),
             name, input.device());
  return output;
}

// Full reduction to a rank-0 tensor; contiguous inputs take the flat kernel.
Tensor full_reduce(const Tensor& input, int operation, const char* name) {
  detail::require_hip(input, name);
  if (!input.is_contiguous()) {
    const Tensor contiguous_input{input.detach().contiguous()};
    return full_reduce(contiguous_input, operation, name);
  }
  const DType out_dtype{operation == SPAR_HIP_ARGMAX ? DType::Int64 : input.dtype()};
  Tensor output{Shape{}, out_dtype, input.device()};
  hip::check(spar_hip_launch_reduction(HipTensorAccess::mutable_data(output),
                                       HipTensorAccess::data(input), input.numel(),
                                       hip::dtype_tag(input.dtype()), operation,
                                       input.device().index()),
             name, input.device());
  return output;
}

// The gradient of a reduction is the output gradient broadcast back over the
// reduced axes (reduction.cpp:147-165, :200-212, :263-277).  It is returned
// as a stride-0 view of the output gradient instead of a filled tensor: the
// values are the same, and no pass over the input's extent is made here.
// Consumers read views in place (an elementwise product then reads one value
// per row instead of a filled tensor), and the engine makes a leaf's gradient
// dense.  A mean's gradient is divided by (T)n on the reduced tensor before
// the broadcast, which gives each element the same quotient as dividing the
// broadcast values one by one (the CPU path's g / (T)n, reduction.cpp:271).
Tensor dense(const Tensor& tensor) {
  return tensor.is_contiguous() ? tensor.detach() : tensor.detach().contiguous();
}

Tensor broadcast_full_gradient(const Shape& input_shape, const Tensor& gradient,
                               std::optional<double> divisor) {
  Tensor value{dense(gradient)};
  if (divisor) value = divide_scalar(value, *divisor);
  return value.expand(input_shape);
}

// reduction.cpp:147-165
Tensor restore_and_expand_gradient(const Tensor& gradient, const Shape& input_shape,
                                   std::span<const std::size_t> axes, bool keepdim,
                                   std::optional<double> divisor) {
  Tensor restored{dense(gradient)};
  if (!keepdim) {
    std::vector<bool> reduced(input_shape.rank(), false);
    for (const std::size_t axis : axes) reduced[axis] = true;
    std::vector<Shape::dimension_type> dimensions(input_shape.rank(), 1);
    std::size_t gradient_axis{0};
    for (std::size_t axis{0}; axis < input_shape.rank(); ++axis) {
      if (!reduced[axis]) dimensions[axis] = gradient.shape()[gradient_axis++];
    }
    restored = restored.reshape(Shape{std::move(dimensions)});
  }
  if (divisor) restored = divide_scalar(restored, *divisor);
  return restored.expand(input_shape);
}

}  // namespace

Tensor sum(const Tensor& input) {
  validate_reduction_input(input);
  Tensor output{full_reduce(input, SPAR_HIP_SUM, "sum")};
  if (input.requires_grad()) {
    const Shape input_shape{input.shape()};
    detail::record_operation(output, {input}, [input_shape](const Tensor& gradient) {
      return std::vector<Tensor>{broadcast_full_gradient(input_shape, gradient, std::nullopt)};
    });
  }
  return output;
}

Tensor sum(const Tensor& input, std::span<const std::size_t> axes, bool keepdim) {
  validate_reduction_input(input);
  std::vector<std::size_t> normalized_axes{validate_axes(input, axes)};
  const Shape output_shape{reduced_shape(input, normalized_axes, keepdim)};
  Tensor output{axis_reduce(input, normalized_axes, output_shape, SPAR_HIP_SUM, "sum")};
  if (input.requires_grad()) {
    const Shape input_shape{input.shape()};
    detail::record_operation(output, {input},
                             [input_shape, normalized_axes, keepdim](const Tensor& gradient) {
                               return std::vector<Tensor>{restore_and_expand_gradient(
                                   gradient, input_shape, normalized_axes, keepdim,
                                   std::nullopt)};
                             });
  }
  return output;
}

Tensor sum(const Tensor& input, std::size_t axis, bool keepdim) {
  return sum(input, std::span<const std::size_t>{&axis, 1}, keepdim);
}

Tensor sum(const Tensor& input, std::initializer_list<std::size_t> axes, bool keepdim) {
  return sum(input, std::span<const std::size_t>{axes.begin(), axes.size()}, keepdim);
}

Tensor mean(const Tensor& input) {
  validate_reduction_input(input);
  if (input.numel() == 0) throw std::invalid_argument{"mean is undefined for an empty tensor"};
  Tensor output{full_reduce(input, SPAR_HIP_MEAN, "mean")};
  if (input.requires_grad()) {
    const Shape input_shape{input.shape()};
    const std::size_t input_numel{input.numel()};
    detail::record_operation(
        output, {input}, [input_shape, input_numel](const Tensor& gradient) {
          return std::vector<Tensor>{broadcast_full_gradient(
              input_shape, gradient, static_cast<double>(input_numel))};
        });
  }
  return output;
}

Tensor mean(const Tensor& input, std::span<const std::size_t> axes, bool keepdim) {
  validate_reduction_input(input);
  std::vector<std::size_t> normalized_axes{validate_axes(input, axes)};
  const std::size_t element_count{reduced_element_count(input, normalized_axes)};
  if (element_count == 0) {
    throw std::invalid_argument{"mean is undefined for an empty reduction domain"};
  }
  const Shape output_shape{reduced_shape(input, normalized_axes, keepdim)};
  Tensor output{axis_reduce(input, normalized_axes, output_shape, SPAR_HIP_MEAN, "mean")};
  if (input.requires_grad()) {
    const Shape input_shape{input.shape()};
    detail::record_operation(
        output, {input},
        [input_shape, normalized_axes, keepdim, element_count](const Tensor& gradient) {
          return std::vector<Tensor>{restore_and_expand_gradient(
              gradient, input_shape, normalized_axes, keepdim,
              static_cast<double>(element_count))};
        });
  }
  return output;
}

Tensor mean(const Tensor& input, std::size_t axis, bool keepdim) {
  return mean(input, std::span<const std::size_t>{&axis, 1}, keepdim);
}

Tensor mean(const Tensor& input, std::initializer_list<std::size_t> axes, bool keepdim) {
  return mean(input, std::span<const std::size_t>{axes.begin(), axes.size()}, keepdim);
}

// reduction.cpp:321-347
Tensor reduce_max(const Tensor& input) {
  validate_reduction_input(input);
  if (input.requires_grad()) throw std::logic_error{"autograd for reduce_max is not implemented yet"};
  if (input.numel() == 0) throw std::invalid_argument{"reduce_max is undefined for an empty tensor"};
  return full_reduce(input, SPAR_HIP_MAX, "reduce_max");
}

Tensor max(const Tensor& input, std::size_t axis, bool keepdim) {
  validate_reduction_input(input);
  if (input.requires_grad()) throw std::logic_error{"autograd for max is not implemented"};
  const std::vector<std::size_t> axes{validate_axes(input, std::span<const std::size_t>{&axis, 1})};
  if (input.shape()[axis] == 0) throw std::invalid_argument{"max is undefined for an empty axis"};
  return axis_reduce(input, axes, reduced_shape(input, axes, keepdim), SPAR_HIP_MAX, "max");
}

Tensor argmax(const Tensor& input, std::size_t axis, bool keepdim) {
  validate_reduction_input(input);
  if (input.requires_grad()) throw std::logic_error{"autograd for argmax is not implemented"};
  const std::vector<std::size_t> axes{validate_axes(input, std::span<const std::size_t>{&axis, 1})};
  if (input.shape()[axis] == 0) throw std::invalid_argument{"argmax is undefined for an empty axis"};
  return axis_reduce(input, axes, reduced_shape(input, axes, keepdim), SPAR_HIP_ARGMAX, "argmax");
}

}  // namespace spar
