// Spar's elementwise, broadcast, reduction and softmax ops on HIP tensors.
//
// Same signatures and error behaviour as the reference's op modules:
// spar.ops.elementwise (src/ops/elementwise.cppm:7-10), spar.ops.scalar
// (src/ops/scalar.cppm:7-10), spar.ops.unary (src/ops/unary.cppm:7-15),
// spar.ops.reduction (src/ops/reduction.cppm:8-20) and spar.ops.softmax
// (src/ops/softmax.cppm:11-17).  Additions the reference lacks are marked.
// Inputs must be HIP tensors; the device work is enqueued on the backend's
// stream and results are complete when read back with `to(Device::cpu())`.
#pragma once

#include <cstddef>
#include <initializer_list>
#include <span>

#include "spar/tensor.hpp"

namespace spar {

// ---------------------------------------------------------- elementwise
[[nodiscard]] Tensor add(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor subtract(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor multiply(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor divide(const Tensor& a, const Tensor& b);

// Comparisons (addition): broadcast like add, 1 or 0 in the input dtype,
// IEEE semantics (NaN unequal to everything); not differentiable.
[[nodiscard]] Tensor equal(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor not_equal(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor less(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor less_equal(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor greater(const Tensor& a, const Tensor& b);
[[nodiscard]] Tensor greater_equal(const Tensor& a, const Tensor& b);

// --------------------------------------------------------------- scalar
[[nodiscard]] Tensor add_scalar(const Tensor& input, double value);
[[nodiscard]] Tensor subtract_scalar(const Tensor& input, double value);
[[nodiscard]] Tensor multiply_scalar(const Tensor& input, double value);
[[nodiscard]] Tensor divide_scalar(const Tensor& input, double value);

// ---------------------------------------------------------------- unary
[[nodiscard]] Tensor negate(const Tensor& input);
[[nodiscard]] Tensor square(const Tensor& input);
[[nodiscard]] Tensor reciprocal(const Tensor& input);
[[nodiscard]] Tensor exp(const Tensor& input);
[[nodiscard]] Tensor log(const Tensor& input);
[[nodiscard]] Tensor sqrt(const Tensor& input);
[[nodiscard]] Tensor sigmoid(const Tensor& input);
[[nodiscard]] Tensor silu(const Tensor& input);
/// addition: hyperbolic tangent.
[[nodiscard]] Tensor tanh(const Tensor& input);
/// addition: gelu(x) = 0.5 x erfc(-x / sqrt 2).
[[nodiscard]] Tensor gelu(const Tensor& input);

// ----------------------------------------------------------- reductions
[[nodiscard]] Tensor sum(const Tensor& input);
[[nodiscard]] Tensor sum(const Tensor& input, std::span<const std::size_t> axes,
                         bool keepdim = false);
[[nodiscard]] Tensor sum(const Tensor& input, std::size_t axis, bool keepdim = false);
[[nodiscard]] Tensor sum(const Tensor& input, std::initializer_list<std::size_t> axes,
                         bool keepdim = false);
[[nodiscard]] Tensor mean(const Tensor& input);
[[nodiscard]] Tensor mean(const Tensor& input, std::span<const std::size_t> axes,
                          bool keepdim = false);
[[nodiscard]] Tensor mean(const Tensor& input, std::size_t axis, bool keepdim = false);
[[nodiscard]] Tensor mean(const Tensor& input, std::initializer_list<std::size_t> axes,
                          bool keepdim = false);
[[nodiscard]] Tensor reduce_max(const Tensor& input);
/// addition: maximum over one axis (NaN wins, first occurrence on ties).
[[nodiscard]] Tensor max(const Tensor& input, std::size_t axis, bool keepdim = false);
/// addition: Int64 index of the first maximum over one axis (first NaN wins).
[[nodiscard]] Tensor argmax(const Tensor& input, std::size_t axis, bool keepdim = false);

// -------------------------------------------------------------- softmax
[[nodiscard]] Tensor softmax(const Tensor& input);
[[nodiscard]] Tensor softmax(const Tensor& input, std::size_t axis);
[[nodiscard]] Tensor log_softmax(const Tensor& input);
[[nodiscard]] Tensor log_softmax(const Tensor& input, std::size_t axis);

// ------------------------------------------------------- normalisation
/// addition: fused RMSNorm over the last axis, the computation of
/// nn::RMSNorm::forward (src/nn/rmsnorm.cpp:41-53):
/// (x / sqrt(mean(x*x, -1) + eps)) * weight, weight of the last extent.
[[nodiscard]] Tensor rms_norm(const Tensor& input, const Tensor& weight, double epsilon = 1.0e-5);
/// addition: fused LayerNorm over the last axis:
/// ((x - mean(x)) / sqrt(mean((x - mean(x))^2) + eps)) * weight + bias.
[[nodiscard]] Tensor layer_norm(const Tensor& input, const Tensor& weight, const Tensor& bias,
                                double epsilon = 1.0e-5);

}  // namespace spar
