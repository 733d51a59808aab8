// Fused LayerNorm and RMSNorm over the last axis (additions; the reference
// composes RMSNorm from ops in RMSNorm::forward, src/nn/rmsnorm.cpp:41-53, and
// has no LayerNorm).  The forward and backward each run one fused kernel pair
// (spar_hip_launch_norm_forward / _backward); rows longer than the fused
// kernels accept take the composed ops, which compute the same function.
#include <cmath>
#include <memory>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"

namespace spar {
namespace {

using detail::HipTensorAccess;
namespace hip = detail::hip;

// Mirrors the argument checks of RMSNorm (rmsnorm.cpp:18-32, :41-49).
void validate(const Tensor& input, const Tensor& weight, const Tensor* bias, double epsilon,
              const char* name) {
  if (input.rank() == 0) throw std::invalid_argument{std::string{name} + " input must have rank at least 1"};
  if (!is_floating(input.dtype())) {
    throw std::invalid_argument{std::string{name} + " requires a floating-point dtype"};
  }
  detail::require_hip(input, name);
  if (!std::isfinite(epsilon) || epsilon <= 0.0) {
    throw std::invalid_argument{std::string{name} + " epsilon must be finite and positive"};
  }
  const auto extent{input.shape()[input.rank() - 1]};
  for (const Tensor* parameter : {&weight, bias}) {
    if (parameter == nullptr) continue;
    if (parameter->rank() != 1 || parameter->shape()[0] != extent) {
      throw std::invalid_argument{std::string{name} +
                                  " input final dimension does not match its parameters"};
    }
    if (parameter->dtype() != input.dtype()) {
      throw std::invalid_argument{std::string{name} + " input dtype does not match its parameters"};
    }
    if (parameter->device() != input.device()) {
      throw std::invalid_argument{std::string{name} + " input and parameters are on different devices"};
    }
  }
}

// The composed computation (rmsnorm.cpp:50-52 for RMSNorm; the same chain
// with centring and a bias for LayerNorm), for rows the fused kernels do not
// take.
Tensor composed(const Tensor& input, const Tensor& weight, const Tensor* bias, double epsilon) {
  const std::size_t axis{input.rank() - 1};
  if (bias == nullptr) {
    const Tensor mean_square{mean(square(input), axis, true)};
    const Tensor denominator{sqrt(add_scalar(mean_square, epsilon))};
    return multiply(divide(input, denominator), weight);
  }
  const Tensor centred{subtract(input, mean(input, axis, true))};
  const Tensor denominator{sqrt(add_scalar(mean(square(centred), axis, true), epsilon))};
  return add(multiply(divide(centred, denominator), weight), *bias);
}

// Rows of `input` as the fused kernels read them, in place where the view
// allows:
//   row layout: the last axis contiguous and the leading axes stepping
//     uniformly from row to row (a contiguous tensor, or a block of a wider
//     one such as a narrowed view): rows `row_stride` elements apart;
//   column layout: the leading axes contiguous among themselves and the
//     last axis `column_stride` >= rows elements apart (a transposed matrix):
//     forward and backward read x without a transposing copy;
// otherwise the input is made contiguous first.
struct Rows {
  Tensor source;              // the tensor whose storage the kernels read
  const void* first;          // its first element
  std::size_t row_stride;     // elements between row starts
  std::size_t column_stride;  // elements between neighbours in a row
};

std::optional<std::size_t> uniform_row_stride(const Shape& shape,
                                              std::span<const Shape::stride_type> strides) {
  const std::size_t rank{shape.rank()};
  if (strides[rank - 1] != 1 && shape[rank - 1] != 1) return std::nullopt;
  std::optional<std::size_t> stride;
  std::size_t inner_rows{1};  // rows spanned by the axes inside the current one
  for (std::size_t axis{rank - 1}; axis-- > 0;) {
    const auto extent{static_cast<std::size_t>(shape[axis])};
    if (extent == 1) continue;
    if (!stride) {
      stride = strides[axis];
    } else if (strides[axis] != *stride * inner_rows) {
      return std::nullopt;
    }
    inner_rows *= extent;
  }
  const auto extent{static_cast<std::size_t>(shape[rank - 1])};
  if (!stride) return extent;  // one row
  if (*stride < extent) return std::nullopt;
  return stride;
}

std::optional<std::size_t> uniform_row_stride(const Tensor& input) {
  return uniform_row_stride(input.shape(), input.strides());
}

std::optional<std::size_t> column_stride_of(const Tensor& input) {
  const std::size_t rank{input.rank()};
  if (rank < 2 || input.shape()[rank - 1] == 1) return std::nullopt;
  std::size_t rows{1};  // row-major over the leading axes, innermost stride 1
  for (std::size_t axis{rank - 1}; axis-- > 0;) {
    const auto extent{static_cast<std::size_t>(input.shape()[axis])};
    if (extent == 1) continue;
    if (input.strides()[axis] != rows) return std::nullopt;
    rows *= extent;
  }
  const std::size_t stride{input.strides()[rank - 1]};
  if (stride == 1 || stride < rows) return std::nullopt;
  return stride;
}

const void* first_element(const Tensor& tensor) {
  const auto* base{static_cast<const std::byte*>(HipTensorAccess::storage_base(tensor))};
  return base + tensor.storage_offset() * size_of(tensor.dtype());
}

Rows rows_of(const Tensor& input) {
  const auto extent{static_cast<std::size_t>(input.shape()[input.rank() - 1])};
  if (input.is_contiguous()) return Rows{input, HipTensorAccess::data(input), extent, 1};
  if (const auto stride{uniform_row_stride(input)}) {
    return Rows{input, first_element(input), *stride, 1};
  }
  if (const auto stride{column_stride_of(input)}) {
    return Rows{input, first_element(input), 1, *stride};
  }
  Tensor packed{input.contiguous()};
  const void* first{HipTensorAccess::data(packed)};
  return Rows{packed, first, extent, 1};
}

// Storage for a gradient of `shape` in the packed column layout: a
// contiguous [last, leading...] block viewed with the last axis moved back
// to the end (for a matrix, the transpose of a contiguous [n, rows] block).
struct PackedColumns {
  Tensor storage;  // contiguous: the kernels write here
  Tensor view;     // `shape`, the gradient handed to autograd
};

PackedColumns packed_columns(const Shape& shape, DType dtype, const Device& device) {
  const std::size_t rank{shape.rank()};
  std::vector<Shape::dimension_type> outer{shape[rank - 1]};
  std::vector<std::size_t> order;
  for (std::size_t axis{0}; axis + 1 < rank; ++axis) {
    outer.push_back(shape[axis]);
    order.push_back(axis + 1);
  }
  order.push_back(0);
  Tensor storage{Shape{std::move(outer)}, dtype, device};
  Tensor view{storage.permute(std::span<const std::size_t>{order})};
  return PackedColumns{std::move(storage), std::move(view)};
}

PackedColumns input_gradient(const Tensor& input, bool columns) {
  if (columns) return packed_columns(input.shape(), input.dtype(), input.device());
  Tensor storage{input.shape(), input.dtype(), input.device()};
  Tensor view{storage};
  return PackedColumns{std::move(storage), std::move(view)};
}

// What the backward keeps of a fused forward.
struct SavedNorm {
  Tensor x;  // the tensor whose rows the forward read (detached)
  std::size_t row_stride;
  std::size_t column_stride;
  Tensor w;
  std::optional<Tensor> mean_rows;  // LayerNorm only
  Tensor denominator;
  std::size_t rows;
  std::size_t extent;
  bool center;
  bool grad_x;
  bool grad_w;
  bool grad_b;
  Shape weight_shape;
  const char* name;
};

// The backward kernels with dx written at `dx` (rows `dx_stride` elements
// apart in the row layout; element (p, q) at dx[p + q * dx_stride] in the
// column layout); `dx_view` is the gradient handed to autograd for x.  With
// `scale` (one element), the output gradient is *scale * gradient, each
// product formed in the kernels.
std::vector<Tensor> norm_backward(const SavedNorm& saved, const Tensor& gradient,
                                  const Tensor* scale, void* dx, std::size_t dx_stride,
                                  const Tensor& dx_view) {
  const Tensor dy{gradient.is_contiguous() ? gradient.detach() : gradient.detach().contiguous()};
  Tensor dw{saved.weight_shape, saved.x.dtype(), saved.x.device()};
  std::optional<Tensor> db;
  if (saved.center) db.emplace(saved.weight_shape, saved.x.dtype(), saved.x.device());
  void* dbias{saved.center ? HipTensorAccess::mutable_data(*db) : nullptr};
  const void* mean{saved.center ? HipTensorAccess::data(*saved.mean_rows) : nullptr};
  const int dtype{hip::dtype_tag(saved.x.dtype())};
  const SparHipStatus status{
      scale == nullptr
          ? spar_hip_launch_norm_backward(
                dx, dx_stride, HipTensorAccess::mutable_data(dw), dbias, HipTensorAccess::data(dy),
                first_element(saved.x), saved.row_stride, saved.column_stride,
                HipTensorAccess::data(saved.w), mean, HipTensorAccess::data(saved.denominator),
                saved.rows, saved.extent, saved.center ? 1 : 0, dtype, saved.x.device().index())
          : spar_hip_launch_norm_backward_scaled(
                dx, dx_stride, HipTensorAccess::mutable_data(dw), dbias, HipTensorAccess::data(dy),
                first_element(*scale), first_element(saved.x), saved.row_stride,
                saved.column_stride, HipTensorAccess::data(saved.w), mean,
                HipTensorAccess::data(saved.denominator), saved.rows, saved.extent,
                saved.center ? 1 : 0, dtype, saved.x.device().index())};
  hip::check(status, std::string{saved.name} + " backward", saved.x.device());
  std::vector<Tensor> contributions;
  if (saved.grad_x) contributions.push_back(dx_view);
  if (saved.grad_w) contributions.push_back(dw);
  if (saved.grad_b) contributions.push_back(*db);
  return contributions;
}

// The backward rule in all its forms: dx into a fresh gradient (in x's
// layout: packed columns for an input read in the column layout, so that
// the gradient of a transposed view is the transpose of a contiguous block
// passed on without a copy; contiguous for one read in rows), or into the
// engine's `destination`; the output gradient `gradient`, or *scale *
// gradient.
std::vector<Tensor> norm_rule(const SavedNorm& saved, const Tensor& gradient, const Tensor* scale,
                              const Tensor* destination) {
  if (destination != nullptr) {
    void* first{const_cast<void*>(first_element(*destination))};
    return norm_backward(saved, gradient, scale, first, *uniform_row_stride(*destination),
                         *destination);
  }
  const bool columns{saved.column_stride != 1};
  PackedColumns dx{input_gradient(saved.x, columns)};
  return norm_backward(saved, gradient, scale, HipTensorAccess::mutable_data(dx.storage),
                       columns ? saved.rows : saved.extent, dx.view);
}

Tensor fused(const Tensor& input, const Tensor& weight, const Tensor* bias, double epsilon,
             const char* name) {
  const bool center{bias != nullptr};
  const std::size_t extent{static_cast<std::size_t>(input.shape()[input.rank() - 1])};
  if (extent > spar_hip_norm_max_extent(hip::dtype_tag(input.dtype())) || input.numel() == 0) {
    return composed(input, weight, bias, epsilon);
  }
  const std::size_t rows{input.numel() / extent};
  const Rows x{rows_of(input)};
  const Tensor w{weight.is_contiguous() ? weight : weight.contiguous()};
  std::optional<Tensor> b;
  if (center) b = bias->is_contiguous() ? *bias : bias->contiguous();
  const Shape row_shape{static_cast<Shape::dimension_type>(rows)};
  Tensor output{input.shape(), input.dtype(), input.device()};
  std::optional<Tensor> mean_rows;
  if (center) mean_rows.emplace(row_shape, input.dtype(), input.device());
  Tensor denominator{row_shape, input.dtype(), input.device()};
  const int device{input.device().index()};
  hip::check(spar_hip_launch_norm_forward(
                 HipTensorAccess::mutable_data(output),
                 center ? HipTensorAccess::mutable_data(*mean_rows) : nullptr,
                 HipTensorAccess::mutable_data(denominator), x.first, x.row_stride,
                 x.column_stride,
                 HipTensorAccess::data(w), center ? HipTensorAccess::data(*b) : nullptr, rows,
                 extent, epsilon, center ? 1 : 0, hip::dtype_tag(input.dtype()), device),
             name, input.device());

  // The parent is x.source: the input itself when its rows are read in
  // place (its gradient then has the input's shape, contiguous), else its
  // contiguous copy, whose node passes the gradient on to the input.
  const bool grad_x{x.source.requires_grad()}, grad_w{weight.requires_grad()};
  const bool grad_b{center && bias->requires_grad()};
  if (grad_x || grad_w || grad_b) {
    std::vector<Tensor> parents;
    if (grad_x) parents.push_back(x.source);
    if (grad_w) parents.push_back(weight);
    if (grad_b) parents.push_back(*bias);
    auto saved{std::make_shared<const SavedNorm>(SavedNorm{
        x.source.detach(), x.row_stride, x.column_stride, w.detach(), mean_rows, denominator,
        rows, extent, center, grad_x, grad_w, grad_b, weight.shape(), name})};
    detail::BackwardFunction rule{[saved](const Tensor& gradient) {
      return norm_rule(*saved, gradient, nullptr, nullptr);
    }};
    // The output gradient of loss = sum(y * c) is c times one value: the
    // kernels take (c, value) and form the products themselves.
    detail::ScaledBackward scaled{
        [saved](const Tensor& factor, const Tensor& value, const Tensor* destination) {
          return norm_rule(*saved, factor, &value, destination);
        }};
    if (!grad_x || x.column_stride != 1) {
      detail::record_operation(output, std::move(parents), std::move(rule));
    } else {
      // Rows read in place may also write their gradient in place, into a
      // block of a wider gradient whose rows are a uniform stride apart (the
      // gradient of a narrowed view's base).
      detail::PlacedBackward placed{
          [saved](const detail::PlacedLayout& destination) {
            return destination.device == saved->x.device() &&
                   destination.dtype == saved->x.dtype() &&
                   destination.shape == saved->x.shape() &&
                   uniform_row_stride(destination.shape, destination.strides).has_value();
          },
          [saved](const Tensor& gradient, const Tensor& destination) {
            return norm_rule(*saved, gradient, nullptr, &destination);
          }};
      detail::record_operation(output, std::move(parents), std::move(rule), std::move(placed));
    }
    detail::set_scaled_backward(output, std::move(scaled));
  }
  return output;
}

}  // namespace

Tensor layer_norm(const Tensor& input, const Tensor& weight, const Tensor& bias, double epsilon) {
  validate(input, weight, &bias, epsilon, "layer_norm");
  return fused(input, weight, &bias, epsilon, "layer_norm");
}

Tensor rms_norm(const Tensor& input, const Tensor& weight, double epsilon) {
  validate(input, weight, nullptr, epsilon, "rms_norm");
  // The composed forward starts with square(input), and unary ops reject
  // non-contiguous inputs (unary.cpp:19-21); the fused op keeps that error.
  if (!input.is_contiguous()) {
    throw std::invalid_argument{"Unary operations currently require contiguous tensors"};
  }
  return fused(input, weight, nullptr, epsilon, "rms_norm");
}

}  // namespace spar
