// Private autograd and tensor-internals types of the host library.
//
// Every Tensor handle carries a shared GradState.  Copies of a handle share
// it (they are the same autograd identity); detach() and fresh outputs get
// their own.  An op output that depends on tracked inputs also owns a
// GradFunction: the inputs' identities with the shape, dtype and device each
// gradient must have, and the rule that maps the output's gradient to one
// gradient per input (the reference keeps the same information in its
// AutogradMeta/AutogradNode/AutogradEdge, src/autograd/autograd.cpp:13-41).
#pragma once

#include <memory>
#include <optional>
#include <vector>

#include "spar/tensor.hpp"

namespace spar::detail {

struct GradState;

/// One input of a recorded operation.
struct GradInput final {
  std::shared_ptr<GradState> identity;
  Shape shape;
  DType dtype;
  Device device;
};

/// One axis of the box a narrowed view takes of its input.
struct WindowAxis final {
  std::size_t start;
  std::size_t length;
};

/// A recorded operation: its tracked inputs, in recording order, and the
/// rule producing one gradient per input.
struct GradFunction final {
  std::vector<GradInput> inputs;
  BackwardFunction rule;
  /// Set (one entry per input axis) when the output is a narrowed view of
  /// its one input, inputs[0] restricted to this box: the rule then embeds
  /// the gradient in zeros of the input's shape, and the engine may compose
  /// a chain of such nodes into one embedding.
  std::vector<WindowAxis> window;
  /// Optional: the rule's form that writes inputs[0]'s gradient into a
  /// destination the engine provides (empty functions when absent).
  PlacedBackward placed;
  /// Optional: the rule's form that takes its gradient as factor x value.
  ScaledBackward scaled;
  /// Set for a product with one tracked input: the other operand, which
  /// times the output gradient is that input's gradient.
  std::optional<Tensor> product_factor;
};

struct GradState final {
  bool tracked{false};
  /// null for a leaf.
  std::shared_ptr<GradFunction> producer;
  /// the leaf's accumulated gradient, once backward() has reached it.
  std::optional<Tensor> accumulated;
};

/// Access to Tensor internals for the engine and the layout helpers.
struct TensorInternals final {
  [[nodiscard]] static std::shared_ptr<GradState>& grad_state(Tensor& tensor) {
    return tensor.grad_state_;
  }
  [[nodiscard]] static const std::shared_ptr<GradState>& grad_state(const Tensor& tensor) {
    return tensor.grad_state_;
  }
  [[nodiscard]] static const std::shared_ptr<Storage>& storage(const Tensor& tensor) {
    return tensor.storage_;
  }
  /// host address of a contiguous CPU tensor's first element.
  [[nodiscard]] static std::byte* host_bytes(Tensor& tensor) {
    return tensor.storage_->host_data() + tensor.storage_offset_ * size_of(tensor.dtype_);
  }
  [[nodiscard]] static const std::byte* host_bytes(const Tensor& tensor) {
    return tensor.storage_->host_data() + tensor.storage_offset_ * size_of(tensor.dtype_);
  }
  /// true when this handle is the only one on its storage and covers all of
  /// it contiguously, so the engine may add into it in place.
  [[nodiscard]] static bool sole_owner(const Tensor& tensor) {
    return tensor.storage_ != nullptr && tensor.storage_.use_count() == 1 &&
           tensor.storage_offset_ == 0 && tensor.is_contiguous() &&
           tensor.nbytes_ == tensor.storage_->nbytes();
  }
};

}  // namespace spar::detail
