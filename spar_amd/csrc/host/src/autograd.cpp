// Reverse-mode autograd engine (src/autograd/autograd.cpp:43-265).
//
// Graph recording, the DFS topological order, the `ones` seed and the
// reverse sweep are the reference's.  Two differences keep the device path
// lean without changing any value:
//   * contributions are not cloned: a backward rule's result is kept as is
//     when it owns its storage outright; otherwise the first in-place
//     accumulation into it is done out of place (same additions, same order);
//   * a node's gradient is released once its backward rule has run.
// Gradient accumulation is the elementwise `dst += src` of the reference
// (add_gradient_values, :99-133), in the same order, so gradients are
// bit-identical given identical contributions.
#include <unordered_map>
#include <unordered_set>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"
#include "spar/tensor.hpp"

namespace spar::detail {

void record_operation(Tensor& output, std::vector<Tensor> requiring_parents,
                      BackwardFunction backward) {
  if (requiring_parents.empty()) {
    throw std::logic_error{"Cannot record an autograd operation without requiring-grad parents"};
  }
  for (const Tensor& parent : requiring_parents) {
    if (!parent.requires_grad()) {
      throw std::logic_error{"Autograd nodes may retain only requiring-grad parents"};
    }
    if (parent.device() != output.device()) {
      throw std::logic_error{"Autograd output and parent Device mismatch"};
    }
  }
  std::vector<AutogradEdge> edges;
  edges.reserve(requiring_parents.size());
  for (const Tensor& parent : requiring_parents) {
    edges.push_back(AutogradEdge{AutogradAccess::meta(parent), parent.shape(), parent.dtype(),
                                 parent.device()});
  }
  auto& output_meta{AutogradAccess::meta(output)};
  output_meta = std::make_shared<AutogradMeta>();
  output_meta->requires_grad = true;
  output_meta->grad_fn =
      std::make_shared<AutogradNode>(AutogradNode{std::move(edges), std::move(backward)});
}

void record_transfer_operation(Tensor& output, Tensor requiring_parent, BackwardFunction backward) {
  if (!requiring_parent.requires_grad()) {
    throw std::logic_error{"Cannot record a transfer from a non-requiring parent"};
  }
  if (requiring_parent.device() == output.device()) {
    throw std::logic_error{"Transfer autograd nodes require different source and destination Devices"};
  }
  std::vector<AutogradEdge> edges;
  edges.push_back(AutogradEdge{AutogradAccess::meta(requiring_parent), requiring_parent.shape(),
                               requiring_parent.dtype(), requiring_parent.device()});
  auto& output_meta{AutogradAccess::meta(output)};
  output_meta = std::make_shared<AutogradMeta>();
  output_meta->requires_grad = true;
  output_meta->grad_fn =
      std::make_shared<AutogradNode>(AutogradNode{std::move(edges), std::move(backward)});
}

bool shares_autograd_identity(const Tensor& left, const Tensor& right) noexcept {
  const auto& left_meta{AutogradAccess::meta(left)};
  const auto& right_meta{AutogradAccess::meta(right)};
  return left_meta != nullptr && left_meta == right_meta;
}

}  // namespace spar::detail

namespace spar {
namespace {

// destination += contribution (autograd.cpp:99-133).  An engine-internal
// accumulator whose storage is shared with another handle is replaced by a
// new tensor instead; a leaf gradient (`in_place`) is always updated in place
// so handles returned by grad() observe the accumulation, as in the reference.
void add_gradient_values(Tensor& destination, const Tensor& contribution, bool in_place = false) {
  if (destination.shape() != contribution.shape() || destination.dtype() != contribution.dtype() ||
      destination.device() != contribution.device()) {
    throw std::logic_error{"Internal gradient accumulation shape, dtype, or Device mismatch"};
  }
  if (!is_floating(destination.dtype())) throw std::logic_error{"Integer gradients are not supported"};
  detail::require_hip(destination, "gradient accumulation");
  const Tensor source{contribution.is_contiguous() ? contribution : contribution.contiguous()};
  if (!in_place && !detail::AutogradAccess::exclusively_owned(destination)) {
    destination = add(destination.detach(), source.detach());
    return;
  }
  detail::hip::check(
      spar_hip_launch_add_in_place(detail::HipTensorAccess::mutable_data(destination),
                                   detail::HipTensorAccess::data(source), destination.numel(),
                                   detail::hip::dtype_tag(destination.dtype()),
                                   destination.device().index()),
      "gradient accumulation", destination.device());
}

// autograd.cpp:135-146 without the clone.
void validate_contribution(const Tensor& contribution, const detail::AutogradEdge& parent) {
  if (contribution.shape() != parent.expected_shape ||
      contribution.dtype() != parent.expected_dtype ||
      contribution.device() != parent.expected_device) {
    throw std::logic_error{"Backward rule produced a gradient with incorrect shape, dtype, or Device"};
  }
  if (contribution.requires_grad()) {
    throw std::logic_error{"Backward rule produced a higher-order gradient"};
  }
}

}  // namespace

void Tensor::initialize_autograd() { autograd_ = std::make_shared<detail::AutogradMeta>(); }

bool Tensor::requires_grad() const noexcept {
  return autograd_ != nullptr && autograd_->requires_grad;
}

bool Tensor::is_leaf() const noexcept { return autograd_ == nullptr || autograd_->grad_fn == nullptr; }

bool Tensor::has_grad() const noexcept {
  return autograd_ != nullptr && autograd_->leaf_grad.has_value();
}

void Tensor::set_requires_grad(bool enabled) {
  if (!is_leaf()) throw std::invalid_argument{"requires_grad may only be changed on leaf tensors"};
  if (enabled && !is_floating(dtype_)) {
    throw std::invalid_argument{"Only Float32 and Float64 tensors may require gradients"};
  }
  if (autograd_ == nullptr) initialize_autograd();
  autograd_->requires_grad = enabled;
  if (!enabled) autograd_->leaf_grad.reset();
}

Tensor Tensor::grad() const {
  if (!is_leaf()) throw std::invalid_argument{"Gradients are retained for leaf tensors only"};
  if (!has_grad()) throw std::logic_error{"Tensor has no accumulated gradient"};
  return autograd_->leaf_grad->detach();
}

void Tensor::zero_grad() {
  if (!is_leaf()) throw std::invalid_argument{"zero_grad is supported for leaf tensors only"};
  if (autograd_ != nullptr) autograd_->leaf_grad.reset();
}

void Tensor::backward() {
  if (!requires_grad()) throw std::invalid_argument{"backward requires a Tensor that tracks gradients"};
  if (numel() != 1) {
    throw std::invalid_argument{"backward without an explicit gradient requires a one-element Tensor"};
  }
  if (!is_floating(dtype_)) throw std::invalid_argument{"backward supports Float32 and Float64 losses only"};

  std::vector<std::shared_ptr<detail::AutogradMeta>> topological_order;
  std::unordered_set<detail::AutogradMeta*> visited;
  const auto visit = [&topological_order, &visited](
                         const auto& self, const std::shared_ptr<detail::AutogradMeta>& meta) -> void {
    if (meta == nullptr || !meta->requires_grad || !visited.insert(meta.get()).second) return;
    if (meta->grad_fn != nullptr) {
      for (const detail::AutogradEdge& parent : meta->grad_fn->parents) self(self, parent.identity);
    }
    topological_order.push_back(meta);
  };
  visit(visit, autograd_);

  std::unordered_map<detail::AutogradMeta*, Tensor> gradients;
  gradients.emplace(autograd_.get(), ones(shape_, dtype_, device()));

  for (auto iterator{topological_order.rbegin()}; iterator != topological_order.rend(); ++iterator) {
    const auto& meta{*iterator};
    auto gradient_iterator{gradients.find(meta.get())};
    if (gradient_iterator == gradients.end()) {
      throw std::logic_error{"Reachable autograd identity did not receive a gradient"};
    }
    Tensor gradient{std::move(gradient_iterator->second)};
    gradients.erase(gradient_iterator);

    if (meta->grad_fn == nullptr) {
      if (meta->leaf_grad.has_value()) {
        add_gradient_values(*meta->leaf_grad, gradient, /*in_place=*/true);
      } else if (detail::AutogradAccess::exclusively_owned(gradient)) {
        meta->leaf_grad = gradient.detach();
      } else {
        meta->leaf_grad = gradient.detach().clone();
      }
      continue;
    }

    auto contributions{meta->grad_fn->backward(gradient)};
    if (contributions.size() != meta->grad_fn->parents.size()) {
      throw std::logic_error{"Backward rule returned an incorrect number of gradients"};
    }
    gradient = Tensor{Shape{}, dtype_, Device::cpu()};  // release this node's gradient
    for (std::size_t index{0}; index < contributions.size(); ++index) {
      const detail::AutogradEdge& parent{meta->grad_fn->parents[index]};
      validate_contribution(contributions[index], parent);
      Tensor contribution{contributions[index].detach()};
      contributions[index] = Tensor{Shape{}, dtype_, Device::cpu()};
      auto existing{gradients.find(parent.identity.get())};
      if (existing == gradients.end()) {
        gradients.emplace(parent.identity.get(), std::move(contribution));
      } else {
        add_gradient_values(existing->second, contribution);
      }
    }
  }
}

}  // namespace spar
