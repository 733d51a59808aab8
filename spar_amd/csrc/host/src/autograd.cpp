// Reverse-mode autograd engine of the host library.
//
// Public behaviour, messages and exception types follow Spar's engine
// (src/autograd/autograd.cpp:43-265).  The structure is this library's own:
// an explicit-stack graph walk, a slot per reachable identity, and gradients
// that are moved, not cloned, through the sweep.
//
// Accumulation-order contract.  It fixes every gradient bit, so it is the
// same as the reference's:
//   1. The reachable identities are ordered by a depth-first post-order walk
//      from the loss that visits each operation's inputs in the order they
//      were recorded and enters each identity once.
//   2. The sweep runs that order backwards, seeded with ones for the loss.
//   3. An identity's first incoming gradient is kept as it is; every later
//      one is added elementwise, `held += incoming`, in sweep order.
//   4. A leaf keeps the gradient it is handed on its first backward() and
//      adds later ones in place (`accumulated += incoming`).
//   5. A narrow whose input is itself a narrow with no other incoming
//      gradient hands its gradient down unembedded, with the composed box.
//      The last narrow of such a chain embeds it once, at its own turn, so
//      every identity the chain feeds receives the same values in the same
//      order as if each narrow had embedded its own.  A rule with a placed
//      form (the fused norms) whose first input heads such a chain writes
//      that gradient straight into the box of a buffer shaped like the
//      chain's base, its border zeroed; the buffer travels down the same
//      chain and is delivered at the same turn, with the same values.
//   6. A product whose one tracked input x receives value * factor (the
//      output gradient is one value broadcast, the factor the other
//      operand), where x's producer has a scaled form and this is the only
//      gradient x receives, hands that producer (factor, value) at x's own
//      turn; its kernels form value * factor[i] with the product's one
//      rounding and operand order, so x's producer computes what it would
//      from the materialised product, and every identity still receives its
//      gradients in the same order.
// Given identical contributions, the gradients are therefore identical to
// the reference's.  The reference also cloned each contribution
// (autograd.cpp:145, :244), which copied values into a dense tensor.  Here a
// gradient is copied only where that copy is observable or needed: a leaf
// keeps a dense, contiguous gradient of its own (a gradient that is a view,
// or a tensor another handle still sees, is copied first), and a held
// gradient that is a view or whose storage another handle still sees is
// added out of place (same operands, same order) instead of in place, as is
// an incoming view.  The view rules return dense gradients themselves
// (transpose's is made contiguous); the reductions return their gradient as
// a stride-0 broadcast view, which the rules that follow read in place.
#include <algorithm>
#include <atomic>
#include <unordered_map>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"
#include "spar/tensor.hpp"

namespace spar::detail {
namespace {

// Process-wide tallies of what backward() did with gradients.
std::atomic<std::uint64_t> g_backward_calls{0};
std::atomic<std::uint64_t> g_leaf_copies{0};
std::atomic<std::uint64_t> g_in_place_adds{0};
std::atomic<std::uint64_t> g_out_of_place_adds{0};
std::atomic<std::uint64_t> g_window_fusions{0};
std::atomic<std::uint64_t> g_placed_gradients{0};
std::atomic<std::uint64_t> g_scaled_gradients{0};
// Whether backward() may take the hand-overs of contract points 5 and 6
// (narrow chains, placed gradients, scaled products); without them every
// rule runs in its plain form, which the contract says gives the same bits.
std::atomic<bool> g_hand_overs{true};

GradInput input_of(const Tensor& parent) {
  return GradInput{TensorInternals::grad_state(parent), parent.shape(), parent.dtype(),
                   parent.device()};
}

// Gives `output` a fresh tracked identity produced by `function`.
void attach(Tensor& output, std::shared_ptr<GradFunction> function) {
  auto state{std::make_shared<GradState>()};
  state->tracked = true;
  state->producer = std::move(function);
  TensorInternals::grad_state(output) = std::move(state);
}

}  // namespace

void record_operation(Tensor& output, std::vector<Tensor> requiring_parents,
                      BackwardFunction backward) {
  if (requiring_parents.empty()) {
    throw std::logic_error{"Cannot record an autograd operation without requiring-grad parents"};
  }
  auto function{std::make_shared<GradFunction>()};
  function->inputs.reserve(requiring_parents.size());
  for (const Tensor& parent : requiring_parents) {
    if (!parent.requires_grad()) {
      throw std::logic_error{"Autograd nodes may retain only requiring-grad parents"};
    }
    if (parent.device() != output.device()) {
      throw std::logic_error{"Autograd output and parent Device mismatch"};
    }
    function->inputs.push_back(input_of(parent));
  }
  function->rule = std::move(backward);
  attach(output, std::move(function));
}

void record_operation(Tensor& output, std::vector<Tensor> requiring_parents,
                      BackwardFunction backward, PlacedBackward placed) {
  record_operation(output, std::move(requiring_parents), std::move(backward));
  TensorInternals::grad_state(output)->producer->placed = std::move(placed);
}

void set_scaled_backward(Tensor& output, ScaledBackward scaled) {
  const auto& state{TensorInternals::grad_state(output)};
  if (state == nullptr || state->producer == nullptr) {
    throw std::logic_error{"A scaled backward form needs a recorded operation"};
  }
  state->producer->scaled = std::move(scaled);
}

void set_product_factor(Tensor& output, Tensor factor) {
  const auto& state{TensorInternals::grad_state(output)};
  if (state == nullptr || state->producer == nullptr || state->producer->inputs.size() != 1) {
    throw std::logic_error{"A product factor needs an operation with one tracked input"};
  }
  if (factor.requires_grad()) throw std::logic_error{"A product factor must be detached"};
  state->producer->product_factor = std::move(factor);
}

void record_transfer_operation(Tensor& output, Tensor requiring_parent, BackwardFunction backward) {
  if (!requiring_parent.requires_grad()) {
    throw std::logic_error{"Cannot record a transfer from a non-requiring parent"};
  }
  if (requiring_parent.device() == output.device()) {
    throw std::logic_error{
        "Transfer autograd nodes require different source and destination Devices"};
  }
  auto function{std::make_shared<GradFunction>()};
  function->inputs.push_back(input_of(requiring_parent));
  function->rule = std::move(backward);
  attach(output, std::move(function));
}

AutogradCounters autograd_counters() noexcept {
  return AutogradCounters{g_backward_calls.load(), g_leaf_copies.load(), g_in_place_adds.load(),
                          g_out_of_place_adds.load(), g_window_fusions.load(),
                          g_placed_gradients.load(), g_scaled_gradients.load()};
}

void set_autograd_hand_overs(bool enabled) noexcept {
  g_hand_overs.store(enabled, std::memory_order_relaxed);
}

bool shares_autograd_identity(const Tensor& left, const Tensor& right) noexcept {
  const GradState* identity{TensorInternals::grad_state(left).get()};
  return identity != nullptr && identity == TensorInternals::grad_state(right).get();
}

namespace {

void check_same_layout(const Tensor& held, const Tensor& incoming) {
  if (held.shape() != incoming.shape() || held.dtype() != incoming.dtype() ||
      held.device() != incoming.device()) {
    throw std::logic_error{"Internal gradient accumulation shape, dtype, or Device mismatch"};
  }
  if (!is_floating(held.dtype())) throw std::logic_error{"Integer gradients are not supported"};
}

// held[i] += incoming[i] on the device, into held's own storage.
void add_into(Tensor& held, const Tensor& incoming) {
  require_hip(held, "gradient accumulation");
  const Tensor source{incoming.is_contiguous() ? incoming : incoming.contiguous()};
  hip::check(spar_hip_launch_add_in_place(HipTensorAccess::mutable_data(held),
                                          HipTensorAccess::data(source), held.numel(),
                                          hip::dtype_tag(held.dtype()), held.device().index()),
             "gradient accumulation", held.device());
}

// `gradient` (contiguous, the box's lengths) embedded in zeros of `shape` at
// `box`: one pass on a HIP device, else a zero tensor whose box is assigned.
Tensor embed_box(const Tensor& gradient, const Shape& shape, const std::vector<WindowAxis>& box) {
  if (gradient.device().is_hip() && gradient.is_contiguous() &&
      shape.rank() <= static_cast<std::size_t>(SPAR_HIP_MAX_RANK)) {
    std::uint64_t extents[SPAR_HIP_MAX_RANK];
    std::uint64_t starts[SPAR_HIP_MAX_RANK];
    std::uint64_t lengths[SPAR_HIP_MAX_RANK];
    for (std::size_t k{0}; k < shape.rank(); ++k) {
      extents[k] = static_cast<std::uint64_t>(shape[k]);
      starts[k] = box[k].start;
      lengths[k] = box[k].length;
    }
    Tensor result{shape, gradient.dtype(), gradient.device()};
    const auto status{spar_hip_launch_box_embed(
        HipTensorAccess::mutable_data(result), HipTensorAccess::data(gradient),
        static_cast<int>(shape.rank()), extents, starts, lengths, size_of(gradient.dtype()),
        gradient.device().index())};
    if (status.code == 0) return result;
    // status 1 (more box axes than the one-pass kernel takes, or an empty
    // box) falls through to the assignment
    if (status.code != 1) hip::check(status, "narrow backward", gradient.device());
  }
  Tensor result{zeros(shape, gradient.dtype(), gradient.device())};
  Tensor window{result};
  for (std::size_t k{0}; k < shape.rank(); ++k) {
    window = window.narrow(k, box[k].start, box[k].length);
  }
  copy_tensor_values(window, gradient);
  return result;
}

// Zeros over all of `buffer` except `box`, which a producer writes itself.
void zero_border(Tensor& buffer, const std::vector<WindowAxis>& box) {
  const Shape& shape{buffer.shape()};
  void* data{HipTensorAccess::mutable_data(buffer)};
  if (shape.rank() <= static_cast<std::size_t>(SPAR_HIP_MAX_RANK)) {
    std::uint64_t extents[SPAR_HIP_MAX_RANK];
    std::uint64_t starts[SPAR_HIP_MAX_RANK];
    std::uint64_t lengths[SPAR_HIP_MAX_RANK];
    for (std::size_t k{0}; k < shape.rank(); ++k) {
      extents[k] = static_cast<std::uint64_t>(shape[k]);
      starts[k] = box[k].start;
      lengths[k] = box[k].length;
    }
    const auto status{spar_hip_launch_box_embed(data, nullptr, static_cast<int>(shape.rank()),
                                                extents, starts, lengths,
                                                size_of(buffer.dtype()),
                                                buffer.device().index())};
    if (status.code == 0) return;
    // status 1 (more box axes than the one-pass kernel takes): zero it all
    if (status.code != 1) hip::check(status, "narrow backward", buffer.device());
  }
  hip::check(spar_hip_zero(data, buffer.numel() * size_of(buffer.dtype()),
                           buffer.device().index()),
             "narrow backward", buffer.device());
}

// The sweep state of one backward() call.
class Sweep final {
 public:
  explicit Sweep(GradState* loss)
      : hand_overs_{g_hand_overs.load(std::memory_order_relaxed)} {
    order_from(loss);
  }

  void run(GradState* loss, Tensor seed) {
    pending_[slot_.at(loss)] = std::move(seed);
    for (std::size_t position{order_.size()}; position-- > 0;) {
      GradState& state{*order_[position]};
      std::optional<Tensor>& held{pending_[position]};
      if (!held.has_value()) {
        throw std::logic_error{"Reachable autograd identity did not receive a gradient"};
      }
      Tensor gradient{std::move(*held)};
      held.reset();
      if (state.producer == nullptr) {
        deliver_to_leaf(state, std::move(gradient));
        continue;
      }
      std::vector<WindowAxis> box{std::move(deferred_[position])};
      if (placed_[position].has_value()) {
        hand_placed(position, std::move(gradient));
        continue;
      }
      if (!state.producer->window.empty() && narrow_chain(position, gradient, box)) continue;
      // (with the hand-overs off no box, placed buffer or scale is ever set)
      if (scale_[position].has_value()) {
        Tensor value{std::move(*scale_[position])};
        scale_[position].reset();
        propagate(*state.producer, std::move(gradient), &value);
        continue;
      }
      if (hand_overs_ && state.producer->product_factor.has_value() &&
          hand_scaled(*state.producer, gradient)) {
        continue;
      }
      propagate(*state.producer, std::move(gradient));
    }
  }

 private:
  // Depth-first post-order over tracked identities, inputs in recording
  // order, each identity entered once (contract, point 1).
  void order_from(GradState* loss) {
    struct Frame {
      GradState* state;
      std::size_t next_input;
    };
    std::vector<Frame> stack;
    const auto enter = [this, &stack](GradState* state) {
      if (state == nullptr || !state->tracked) return;
      if (!slot_.emplace(state, kUnplaced).second) return;
      stack.push_back(Frame{state, 0});
    };
    enter(loss);
    while (!stack.empty()) {
      Frame& top{stack.back()};
      const GradFunction* producer{top.state->producer.get()};
      if (producer != nullptr && top.next_input < producer->inputs.size()) {
        enter(producer->inputs[top.next_input++].identity.get());
        continue;
      }
      slot_[top.state] = order_.size();
      order_.push_back(top.state);
      stack.pop_back();
    }
    pending_.resize(order_.size());
    deferred_.resize(order_.size());
    placed_.resize(order_.size());
    scale_.resize(order_.size());
    incoming_.assign(order_.size(), 0);
    for (const GradState* state : order_) {
      if (state->producer == nullptr) continue;
      for (const GradInput& input : state->producer->inputs) {
        const auto found{slot_.find(input.identity.get())};
        if (found != slot_.end()) ++incoming_[found->second];
      }
    }
  }

  // The slot of the identity below the narrow at `position` when a gradient
  // may be handed to it down a chain of narrows: it is a narrowed view itself
  // and this narrow's gradient is the only one it receives (none pending).
  std::optional<std::size_t> chain_parent(std::size_t position) const {
    const GradFunction& function{*order_[position]->producer};
    const auto found{slot_.find(function.inputs.front().identity.get())};
    if (found == slot_.end()) return std::nullopt;
    const std::size_t next{found->second};
    const GradState& parent{*order_[next]};
    if (parent.producer == nullptr || parent.producer->window.empty() || incoming_[next] != 1 ||
        pending_[next].has_value()) {
      return std::nullopt;
    }
    return next;
  }

  // The narrow at `position` (window W of its input v) holding `gradient`,
  // which covers `box` of the narrow's own shape (all of it when `box` is
  // empty).  When v is itself a narrowed view whose only incoming gradient
  // is this one, the gradient is handed on unchanged with the composed box
  // (start W + box start, length box length), to be embedded once, at v's
  // own turn in the sweep, so that every other identity receives its
  // gradients in the same order as without the composition.  Returns false
  // when the node's own rule should run instead (no box to apply).
  bool narrow_chain(std::size_t position, Tensor& gradient, const std::vector<WindowAxis>& box) {
    const GradFunction& function{*order_[position]->producer};
    const GradInput& input{function.inputs.front()};
    std::vector<WindowAxis> composed{function.window};
    for (std::size_t k{0}; k < composed.size() && !box.empty(); ++k) {
      composed[k].start += box[k].start;
      composed[k].length = box[k].length;
    }
    if (slot_.find(input.identity.get()) == slot_.end()) return true;  // no longer tracked
    const auto next{hand_overs_ ? chain_parent(position) : std::nullopt};
    if (next && gradient.device().is_hip() && gradient.is_contiguous()) {
      pending_[*next] = std::move(gradient);
      deferred_[*next] = std::move(composed);
      g_window_fusions.fetch_add(1, std::memory_order_relaxed);
      return true;
    }
    if (box.empty()) return false;
    accumulate(input, embed_box(gradient, input.shape, composed));
    return true;
  }

  // A narrow whose gradient a rule wrote straight into the gradient of its
  // chain's base (placed_[position], whose border is zero): the base's
  // gradient is handed down the same chain narrow_chain composes and
  // delivered at the last narrow's turn, where that chain would embed it,
  // so every identity receives the same values in the same order.
  void hand_placed(std::size_t position, Tensor gradient) {
    Tensor buffer{std::move(*placed_[position])};
    placed_[position].reset();
    if (const auto next{chain_parent(position)}) {
      pending_[*next] = std::move(gradient);
      placed_[*next] = std::move(buffer);
      return;
    }
    gradient = Tensor{Shape{}, buffer.dtype(), Device::cpu()};  // drop the view of buffer
    accumulate(order_[position]->producer->inputs.front(), std::move(buffer));
  }

  // Contract, point 6: the product `function` (one tracked input x, whose
  // gradient is `gradient` times the product factor) hands x's producer the
  // factor and `gradient`'s one value when `gradient` is that value
  // broadcast, the producer has a scaled form, and x receives nothing else.
  // Returns false when the product's own rule should run instead.
  bool hand_scaled(const GradFunction& function, const Tensor& gradient) {
    const GradInput& input{function.inputs.front()};
    const Tensor& factor{*function.product_factor};
    const auto found{slot_.find(input.identity.get())};
    if (found == slot_.end()) return false;
    const std::size_t next{found->second};
    const GradFunction* consumer{order_[next]->producer.get()};
    if (consumer == nullptr || !consumer->scaled || incoming_[next] != 1 ||
        pending_[next].has_value() || placed_[next].has_value() || !deferred_[next].empty() ||
        !consumer->window.empty()) {
      return false;
    }
    if (!gradient.device().is_hip() || gradient.numel() == 0 || gradient.shape() != input.shape ||
        gradient.dtype() != input.dtype || gradient.device() != input.device ||
        factor.shape() != input.shape || factor.dtype() != input.dtype ||
        factor.device() != input.device || !factor.is_contiguous()) {
      return false;
    }
    for (std::size_t k{0}; k < gradient.rank(); ++k) {
      if (gradient.shape()[k] != 1 && gradient.strides()[k] != 0) return false;  // not one value
    }
    Tensor value{gradient.detach()};  // its first element, at the gradient's own offset
    for (std::size_t k{0}; k < value.rank(); ++k) value = value.narrow(k, 0, 1);
    pending_[next] = factor;
    scale_[next] = std::move(value);
    g_scaled_gradients.fetch_add(1, std::memory_order_relaxed);
    return true;
  }

  struct Placement {
    std::size_t slot;    // the first input's identity (the top narrow)
    Tensor buffer;       // the chain base's gradient, border zeroed
    Tensor destination;  // the top narrow's box of it
  };

  // Where a rule with a placed form may write its first input's gradient:
  // that input is a narrow fed by this rule alone, so its gradient would go
  // down the chain narrow_chain composes and be embedded in zeros of the
  // base's shape.  The buffer of that shape is made here, its border zeroed
  // once the rule accepts the box's layout.
  std::optional<Placement> placement(const GradFunction& function) {
    if (!hand_overs_ || !function.placed.rule || !function.placed.accepts ||
        function.inputs.empty()) {
      return std::nullopt;
    }
    const GradInput& input{function.inputs.front()};
    const auto found{slot_.find(input.identity.get())};
    if (found == slot_.end() || !input.device.is_hip()) return std::nullopt;
    std::size_t position{found->second};
    const GradState& top{*order_[position]};
    if (top.producer == nullptr || top.producer->window.empty() || incoming_[position] != 1 ||
        pending_[position].has_value()) {
      return std::nullopt;
    }
    std::vector<WindowAxis> box{top.producer->window};
    while (const auto next{chain_parent(position)}) {
      std::vector<WindowAxis> composed{order_[*next]->producer->window};
      for (std::size_t k{0}; k < composed.size(); ++k) {
        composed[k].start += box[k].start;
        composed[k].length = box[k].length;
      }
      box = std::move(composed);
      position = *next;
    }
    // The box of a contiguous buffer shaped like the chain's base: the box's
    // lengths with the base's contiguous strides.  The rule judges that
    // layout before the buffer is allocated.
    const Shape& base_shape{order_[position]->producer->inputs.front().shape};
    const std::vector<Shape::stride_type> base_strides{base_shape.contiguous_strides()};
    std::vector<Shape::dimension_type> lengths;
    for (const WindowAxis& axis : box) {
      lengths.push_back(static_cast<Shape::dimension_type>(axis.length));
    }
    const Shape box_shape{std::move(lengths)};
    if (box_shape.numel() == 0 ||
        !function.placed.accepts(PlacedLayout{box_shape, base_strides, input.dtype, input.device})) {
      return std::nullopt;
    }
    Tensor buffer{base_shape, input.dtype, input.device};
    Tensor destination{buffer};
    for (std::size_t k{0}; k < box.size(); ++k) {
      destination = destination.narrow(k, box[k].start, box[k].length);
    }
    zero_border(buffer, box);
    return Placement{found->second, std::move(buffer), std::move(destination)};
  }

  // Runs one operation's rule and hands each input its gradient.  With
  // `value`, `gradient` is the factor of a product gradient handed over by
  // hand_scaled and the scaled form runs.
  void propagate(const GradFunction& function, Tensor gradient, const Tensor* value = nullptr) {
    std::optional<Placement> placed{placement(function)};
    std::vector<Tensor> contributions{
        value != nullptr
            ? function.scaled(gradient, *value, placed ? &placed->destination : nullptr)
        : placed ? function.placed.rule(gradient, placed->destination)
                 : function.rule(gradient)};
    if (contributions.size() != function.inputs.size()) {
      throw std::logic_error{"Backward rule returned an incorrect number of gradients"};
    }
    if (placed) {
      // the narrow hands on `buffer` at its turn, so the rule's first
      // contribution must be the destination it wrote, not another tensor
      const Tensor& first{contributions.front()};
      if (TensorInternals::storage(first) != TensorInternals::storage(placed->buffer) ||
          first.storage_offset() != placed->destination.storage_offset() ||
          !std::ranges::equal(first.strides(), placed->destination.strides())) {
        throw std::logic_error{"Placed backward rule did not return its destination"};
      }
      placed_[placed->slot] = std::move(placed->buffer);
      g_placed_gradients.fetch_add(1, std::memory_order_relaxed);
    }
    gradient = Tensor{Shape{}, gradient.dtype(), Device::cpu()};  // free it before the adds
    for (std::size_t k{0}; k < contributions.size(); ++k) {
      const GradInput& input{function.inputs[k]};
      const Tensor& produced{contributions[k]};
      if (produced.shape() != input.shape || produced.dtype() != input.dtype ||
          produced.device() != input.device) {
        throw std::logic_error{
            "Backward rule produced a gradient with incorrect shape, dtype, or Device"};
      }
      if (produced.requires_grad()) {
        throw std::logic_error{"Backward rule produced a higher-order gradient"};
      }
      Tensor incoming{produced.detach()};
      contributions[k] = Tensor{Shape{}, produced.dtype(), Device::cpu()};
      accumulate(input, std::move(incoming));
    }
  }

  // Hands `incoming` to the identity of `input` (contract, point 3).
  void accumulate(const GradInput& input, Tensor incoming) {
    const auto found{slot_.find(input.identity.get())};
    if (found == slot_.end()) return;  // an identity no longer tracked
    std::optional<Tensor>& held{pending_[found->second]};
    if (!held.has_value()) {
      held = std::move(incoming);
      return;
    }
    check_same_layout(*held, incoming);
    // In place when the held gradient is dense and its own, and the
    // incoming one dense too (a broadcast view would first be filled out);
    // otherwise out of place, which reads views as they are.
    if (TensorInternals::sole_owner(*held) && held->is_contiguous() &&
        incoming.is_contiguous()) {
      add_into(*held, incoming);
      g_in_place_adds.fetch_add(1, std::memory_order_relaxed);
    } else {
      held = add(held->detach(), incoming.detach());
      g_out_of_place_adds.fetch_add(1, std::memory_order_relaxed);
    }
  }

  static void deliver_to_leaf(GradState& leaf, Tensor gradient) {
    if (leaf.accumulated.has_value()) {
      check_same_layout(*leaf.accumulated, gradient);
      add_into(*leaf.accumulated, gradient);  // in place: grad() handles see it
      g_in_place_adds.fetch_add(1, std::memory_order_relaxed);
      return;
    }
    if (TensorInternals::sole_owner(gradient) && gradient.is_contiguous()) {
      leaf.accumulated = gradient.detach();
    } else {
      leaf.accumulated = gradient.detach().clone();  // dense and contiguous
      g_leaf_copies.fetch_add(1, std::memory_order_relaxed);
    }
  }

  static constexpr std::size_t kUnplaced = static_cast<std::size_t>(-1);

  bool hand_overs_;
  std::vector<GradState*> order_;
  std::unordered_map<const GradState*, std::size_t> slot_;
  std::vector<std::optional<Tensor>> pending_;
  // per identity: the box its pending gradient covers when a narrow handed
  // it on (empty: all of it), and the number of gradients it will receive
  std::vector<std::vector<WindowAxis>> deferred_;
  std::vector<std::size_t> incoming_;
  // per identity: the gradient of its narrow chain's base, when a rule wrote
  // this identity's gradient into it (the pending gradient is then a view)
  std::vector<std::optional<Tensor>> placed_;
  // per identity: the one value its pending gradient (then a product
  // factor) is to be multiplied by, when a product handed it over scaled
  std::vector<std::optional<Tensor>> scale_;
};

}  // namespace
}  // namespace spar::detail

namespace spar {

using detail::GradState;

void Tensor::initialize_autograd() { grad_state_ = std::make_shared<GradState>(); }

bool Tensor::requires_grad() const noexcept { return grad_state_ != nullptr && grad_state_->tracked; }

bool Tensor::is_leaf() const noexcept {
  return grad_state_ == nullptr || grad_state_->producer == nullptr;
}

bool Tensor::has_grad() const noexcept {
  return grad_state_ != nullptr && grad_state_->accumulated.has_value();
}

void Tensor::set_requires_grad(bool enabled) {
  if (!is_leaf()) throw std::invalid_argument{"requires_grad may only be changed on leaf tensors"};
  if (enabled && !is_floating(dtype_)) {
    throw std::invalid_argument{"Only Float32 and Float64 tensors may require gradients"};
  }
  if (grad_state_ == nullptr) initialize_autograd();
  grad_state_->tracked = enabled;
  if (!enabled) grad_state_->accumulated.reset();
}

Tensor Tensor::grad() const {
  if (!is_leaf()) throw std::invalid_argument{"Gradients are retained for leaf tensors only"};
  if (!has_grad()) throw std::logic_error{"Tensor has no accumulated gradient"};
  return grad_state_->accumulated->detach();
}

void Tensor::zero_grad() {
  if (!is_leaf()) throw std::invalid_argument{"zero_grad is supported for leaf tensors only"};
  if (grad_state_ != nullptr) grad_state_->accumulated.reset();
}

void Tensor::backward() {
  if (!requires_grad()) {
    throw std::invalid_argument{"backward requires a Tensor that tracks gradients"};
  }
  if (numel() != 1) {
    throw std::invalid_argument{
        "backward without an explicit gradient requires a one-element Tensor"};
  }
  if (!is_floating(dtype_)) {
    throw std::invalid_argument{"backward supports Float32 and Float64 losses only"};
  }
  detail::g_backward_calls.fetch_add(1, std::memory_order_relaxed);
  detail::Sweep sweep{grad_state_.get()};
  sweep.run(grad_state_.get(), ones(shape_, dtype_, device()));
}

}  // namespace spar
