// spar::Tensor for the HIP device backend.
//
// Mirrors the reference's spar.tensor module (src/core/tensor.cppm:22-218,
// src/core/tensor.cpp:26-632, src/autograd/autograd.cpp:43-265): a typed,
// shaped, strided view over reference-counted Storage with reverse-mode
// autograd.  Storage is host memory (Device::cpu()) or HBM of an MI355X
// (Device::hip(i)) obtained from the backend's caching allocator.  Every
// arithmetic op runs on the HIP device; CPU tensors are host buffers for
// construction, typed access and transfers.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <initializer_list>
#include <memory>
#include <optional>
#include <span>
#include <stdexcept>
#include <string_view>
#include <vector>

#include "spar/core.hpp"

namespace spar {
class Tensor;
}

namespace spar::detail {

struct GradState;
struct HipTensorAccess;
struct TensorInternals;

/// Ref-counted allocation with the interface of src/core/storage.cppm:10-33:
/// host bytes, or a block of a HIP device's caching allocator.  The block
/// and its device travel together in one owner whose deleter returns the
/// block to where it came from.
class Storage final {
 public:
  Storage(std::size_t nbytes, Device device);
  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  ~Storage() noexcept;

  [[nodiscard]] std::byte* host_data();
  [[nodiscard]] const std::byte* host_data() const;
  [[nodiscard]] void* hip_data();
  [[nodiscard]] const void* hip_data() const;
  [[nodiscard]] Device device() const noexcept;
  [[nodiscard]] std::size_t nbytes() const noexcept;
  void swap_payload(Storage& other) noexcept;

 private:
  struct Release {
    Device device;
    void operator()(void* block) const noexcept;
  };
  [[nodiscard]] void* block_on(DeviceType expected) const;

  std::size_t nbytes_;
  std::unique_ptr<void, Release> block_;
};

}  // namespace spar::detail

namespace spar {

/// A typed, shaped, strided view over reference-counted Storage.
/// Copies and metadata-only views share Storage; `clone()` copies.
class Tensor {
 public:
  /// allocates contiguous row-major storage without initialising it.
  Tensor(Shape shape, DType dtype, Device device = Device::cpu());
  Tensor(const Tensor&) = default;
  Tensor& operator=(const Tensor&) = default;
  Tensor(Tensor&& other) noexcept;
  Tensor& operator=(Tensor&& other) noexcept;
  ~Tensor();

  void swap(Tensor& other) noexcept;

  [[nodiscard]] std::size_t rank() const noexcept;
  [[nodiscard]] const Shape& shape() const noexcept;
  [[nodiscard]] std::span<const Shape::stride_type> strides() const noexcept;
  [[nodiscard]] std::size_t storage_offset() const noexcept;
  [[nodiscard]] std::size_t numel() const noexcept;
  [[nodiscard]] DType dtype() const noexcept;
  [[nodiscard]] Device device() const noexcept;
  /// logical tensor bytes, not the size of the shared allocation.
  [[nodiscard]] std::size_t nbytes() const noexcept;
  [[nodiscard]] bool is_contiguous() const noexcept;

  [[nodiscard]] bool requires_grad() const noexcept;
  [[nodiscard]] bool is_leaf() const noexcept;
  [[nodiscard]] bool has_grad() const noexcept;
  void set_requires_grad(bool enabled = true);
  [[nodiscard]] Tensor grad() const;
  void zero_grad();
  /// first-order reverse-mode differentiation from a one-element loss.
  void backward();
  [[nodiscard]] Tensor detach() const;
  /// transfers logical values; a same-Device transfer preserves identity.
  [[nodiscard]] Tensor to(Device target) const;

  [[nodiscard]] Tensor clone() const;
  [[nodiscard]] Tensor contiguous() const;
  [[nodiscard]] Tensor reshape(Shape new_shape) const;
  [[nodiscard]] Tensor transpose(std::size_t axis_a, std::size_t axis_b) const;
  [[nodiscard]] Tensor permute(std::span<const std::size_t> axes) const;
  [[nodiscard]] Tensor permute(std::initializer_list<std::size_t> axes) const;
  [[nodiscard]] Tensor expand(Shape target_shape) const;
  /// metadata-only view of `length` entries of `axis` starting at `start`
  /// (no reference counterpart; needed for offset sub-block views).
  [[nodiscard]] Tensor narrow(std::size_t axis, std::size_t start, std::size_t length) const;

  template <typename T> [[nodiscard]] std::span<T> span() & {
    if (requires_grad()) {
      throw std::logic_error{
          "Mutable tensor access requires a non-grad Tensor identity; detach explicitly first"};
    }
    validate_access<T>();
    if (numel() == 0) return {};
    return {reinterpret_cast<T*>(mutable_host_data()) + storage_offset_, numel()};
  }

  template <typename T> [[nodiscard]] std::span<const T> span() const& {
    validate_access<T>();
    if (numel() == 0) return {};
    return {reinterpret_cast<const T*>(host_data()) + storage_offset_, numel()};
  }

  template <typename T> std::span<T> span() && = delete;
  template <typename T> std::span<const T> span() const&& = delete;

  template <typename T> void fill(T value) & {
    auto values{span<T>()};
    std::fill(values.begin(), values.end(), value);
  }

 private:
  friend struct detail::TensorInternals;
  friend struct detail::HipTensorAccess;
  friend Tensor zeros(Shape shape, DType dtype, Device device);
  friend Tensor full_value(Shape shape, DType dtype, double value, Device device);

  Tensor(std::shared_ptr<detail::Storage> storage, DType dtype, Shape shape,
         std::vector<Shape::stride_type> strides, std::size_t storage_offset);

  // A view on this tensor's storage with new metadata.  When this tensor is
  // tracked, `rule` maps the view's gradient to this tensor's gradient.
  [[nodiscard]] Tensor make_view(Shape shape, std::vector<Shape::stride_type> strides,
                                 std::size_t storage_offset,
                                 std::function<std::vector<Tensor>(const Tensor&)> rule) const;
  // A view whose axis k is this tensor's axis order[k]; `order` is valid.
  [[nodiscard]] Tensor permuted(const std::vector<std::size_t>& order) const;

  void initialize_autograd();
  void reset_to_empty() noexcept;
  void validate_view_bounds() const;

  [[nodiscard]] static std::size_t checked_nbytes(std::size_t numel, DType dtype);
  [[nodiscard]] std::size_t checked_storage_byte_offset() const;
  [[nodiscard]] Tensor materialize_values(Device target) const;
  [[nodiscard]] Tensor gathered() const;
  [[nodiscard]] std::byte* mutable_host_data();
  [[nodiscard]] const std::byte* host_data() const;

  template <typename T> void validate_access() const {
    if (!device().is_cpu()) throw std::logic_error{"Tensor span requires CPU Storage"};
    if (dtype_of<T>() != dtype_) {
      throw std::invalid_argument{"Typed tensor access does not match the tensor dtype"};
    }
    if (!is_contiguous()) throw std::invalid_argument{"Tensor span requires a contiguous tensor"};
  }

  std::shared_ptr<detail::Storage> storage_;
  DType dtype_;
  Shape shape_;
  std::vector<Shape::stride_type> strides_;
  std::size_t storage_offset_;
  std::size_t nbytes_;
  std::shared_ptr<detail::GradState> grad_state_;
};

void swap(Tensor& left, Tensor& right) noexcept;

/// contiguous tensor of zeros (tensor.cpp:429-450).
[[nodiscard]] Tensor zeros(Shape shape, DType dtype, Device device = Device::cpu());
/// contiguous tensor of ones (tensor.cpp:452-481).
[[nodiscard]] Tensor ones(Shape shape, DType dtype, Device device = Device::cpu());
/// contiguous tensor filled with `value` converted to `dtype`.
[[nodiscard]] Tensor full_value(Shape shape, DType dtype, double value,
                                Device device = Device::cpu());

/// contiguous tensor filled with `value`, dtype inferred from T
/// (tensor.cppm:167-178); device tensors are filled by a device kernel.
template <typename T>
[[nodiscard]] Tensor full(Shape shape, T value, Device device = Device::cpu()) {
  if (device.is_cpu()) {
    Tensor tensor{std::move(shape), dtype_of<T>(), device};
    tensor.template fill<T>(value);
    return tensor;
  }
  return full_value(std::move(shape), dtype_of<T>(), static_cast<double>(value), device);
}

/// copies host values into a new CPU tensor of `shape`.
template <typename T>
[[nodiscard]] Tensor from_values(Shape shape, std::span<const T> values) {
  Tensor tensor{std::move(shape), dtype_of<T>(), Device::cpu()};
  if (values.size() != tensor.numel()) {
    throw std::invalid_argument{"from_values needs exactly one value per element"};
  }
  auto out{tensor.template span<T>()};
  std::copy(values.begin(), values.end(), out.begin());
  return tensor;
}

/// A gradient that reaches a broadcast parent of its own shape is passed on
/// as it is, with no copy (the default).  The reference instead adds it into
/// a zeroed buffer (tensor.cpp:597-632), which turns each -0.0 element into
/// +0.0.  With exact zero signs on, such a gradient is re-added to +0.0 the
/// same way (one scalar-add pass), so gradients carry the reference's bits
/// including the signs of zeros.  The setting is process-wide.
void set_exact_gradient_zero_signs(bool enabled) noexcept;
[[nodiscard]] bool exact_gradient_zero_signs() noexcept;

}  // namespace spar

namespace spar::detail {

/// Raw device pointers of contiguous HIP tensors (tensor.cpp:487-506).
struct HipTensorAccess final {
  [[nodiscard]] static void* mutable_data(Tensor& tensor);
  [[nodiscard]] static const void* data(const Tensor& tensor);
  /// base pointer of the tensor's storage (views index from it).
  [[nodiscard]] static const void* storage_base(const Tensor& tensor);
};

[[nodiscard]] Shape broadcast_shape(const Shape& left, const Shape& right);
void validate_same_device(const Tensor& left, const Tensor& right, std::string_view operation);
/// every arithmetic op of this backend runs on a HIP device.
void require_hip(const Tensor& tensor, std::string_view operation);
void copy_tensor_values(Tensor& destination, const Tensor& source);
void swap_storage_payloads(Tensor& original, Tensor& staged) noexcept;
[[nodiscard]] Tensor reduce_gradient_to_shape(const Tensor& gradient, const Shape& original_shape);

using BackwardFunction = std::function<std::vector<Tensor>(const Tensor&)>;

/// The layout of a destination the engine would offer a placed rule: its
/// shape, element strides, dtype and device, described before any storage
/// for it exists.
struct PlacedLayout final {
  const Shape& shape;
  std::span<const Shape::stride_type> strides;
  DType dtype;
  Device device;
};

/// A second form of a backward rule, for ops that can write their first
/// parent's gradient into storage the engine provides: when that parent is a
/// chain of narrowed views, the engine offers a view of the gradient of the
/// chain's base (its border already zero) instead of embedding the gradient
/// afterwards.  `accepts` says whether `rule` can write into a destination
/// of that layout, before the engine allocates it; `rule` then returns the
/// contributions with the destination, written, in the first parent's place.
struct PlacedBackward final {
  std::function<bool(const PlacedLayout& destination)> accepts;
  std::function<std::vector<Tensor>(const Tensor& gradient, const Tensor& destination)> rule;
};

/// A third form of a backward rule, for ops whose kernels can take their
/// output gradient as a product factor x value, `value` a one-element tensor
/// (the value of a gradient broadcast from one element): the rule forms each
/// value * factor[i] itself, with the one rounding and the operand order of
/// the multiply op, so its results are those of the plain rule on the
/// materialised product.  `destination` is null, or the destination the
/// engine offers as for PlacedBackward (accepted by its `accepts`).
using ScaledBackward = std::function<std::vector<Tensor>(
    const Tensor& factor, const Tensor& value, const Tensor* destination)>;

void record_operation(Tensor& output, std::vector<Tensor> requiring_parents,
                      BackwardFunction backward);
void record_operation(Tensor& output, std::vector<Tensor> requiring_parents,
                      BackwardFunction backward, PlacedBackward placed);
/// Gives the operation recorded for `output` its scaled form.
void set_scaled_backward(Tensor& output, ScaledBackward scaled);
/// Marks the operation recorded for `output` as a product whose one tracked
/// input's gradient is the output gradient times `factor` (the other
/// operand, of the input's shape): when that gradient is one value broadcast
/// and the input's producer has a scaled form, the engine hands that
/// producer (factor, value) instead of running this operation's rule.
void set_product_factor(Tensor& output, Tensor factor);
void record_transfer_operation(Tensor& output, Tensor requiring_parent, BackwardFunction backward);
[[nodiscard]] bool shares_autograd_identity(const Tensor& left, const Tensor& right) noexcept;

/// Process-wide tallies of the autograd engine: backward() calls, leaf
/// gradients copied because their storage was shared, gradient
/// accumulations done in place or out of place, narrows whose gradient was
/// handed to the narrow below them unembedded (a chain of narrows is
/// embedded once), gradients a rule wrote straight into the gradient of
/// a narrow chain's base (no embedding pass at all), and product gradients
/// handed to a scaled rule as factor and value (no product pass).  The
/// engine never copies an intermediate gradient.
struct AutogradCounters final {
  std::uint64_t backward_calls;
  std::uint64_t leaf_copies;
  std::uint64_t in_place_adds;
  std::uint64_t out_of_place_adds;
  std::uint64_t window_fusions;
  std::uint64_t placed_gradients;
  std::uint64_t scaled_gradients;
};
[[nodiscard]] AutogradCounters autograd_counters() noexcept;
/// Process-wide: whether backward() hands gradients down narrow chains,
/// writes them in place into a chain's base and hands products over as
/// factor and value (on by default).  Off, every rule runs in its plain
/// form; the gradients are the same bits either way, which tests check.
void set_autograd_hand_overs(bool enabled) noexcept;

}  // namespace spar::detail
