// Private autograd graph types (src/autograd/autograd.cpp:13-41).
#pragma once

#include <memory>
#include <optional>
#include <vector>

#include "spar/tensor.hpp"

namespace spar::detail {

struct AutogradMeta;

struct AutogradEdge final {
  std::shared_ptr<AutogradMeta> identity;
  Shape expected_shape;
  DType expected_dtype;
  Device expected_device;
};

struct AutogradNode final {
  std::vector<AutogradEdge> parents;
  BackwardFunction backward;
};

struct AutogradMeta final {
  bool requires_grad{false};
  std::shared_ptr<AutogradNode> grad_fn;
  std::optional<Tensor> leaf_grad;
};

struct AutogradAccess final {
  [[nodiscard]] static std::shared_ptr<AutogradMeta>& meta(Tensor& tensor) {
    return tensor.autograd_;
  }
  [[nodiscard]] static const std::shared_ptr<AutogradMeta>& meta(const Tensor& tensor) {
    return tensor.autograd_;
  }
  [[nodiscard]] static const std::shared_ptr<Storage>& storage(const Tensor& tensor) {
    return tensor.storage_;
  }
  /// host bytes of a contiguous CPU tensor's first element
  [[nodiscard]] static std::byte* host_bytes(Tensor& tensor) {
    return tensor.storage_->host_data() + tensor.storage_offset_ * size_of(tensor.dtype_);
  }
  [[nodiscard]] static const std::byte* host_bytes(const Tensor& tensor) {
    return tensor.storage_->host_data() + tensor.storage_offset_ * size_of(tensor.dtype_);
  }
  /// true when no other Tensor handle shares this tensor's storage and the
  /// tensor covers the whole allocation contiguously.
  [[nodiscard]] static bool exclusively_owned(const Tensor& tensor) {
    return tensor.storage_ != nullptr && tensor.storage_.use_count() == 1 &&
           tensor.is_contiguous() && tensor.storage_offset_ == 0 &&
           tensor.nbytes_ == tensor.storage_->nbytes();
  }
};

}  // namespace spar::detail
