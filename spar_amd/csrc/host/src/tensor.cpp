// Tensor core of the host library: storage, view metadata, materialisation,
// transfers and factories.
//
// The public behaviour (shapes, strides, offsets, error types and messages)
// is Spar's (src/core/storage.cpp:11-68, src/core/tensor.cpp:26-632).  Every
// view op here is one call of make_view(), which builds the view and records
// the gradient rule; every device transfer and gather goes through the C ABI
// (include/spar_hip.h).
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <new>
#include <utility>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"
#include "spar/tensor.hpp"

namespace spar::detail {

void Storage::Release::operator()(void* block) const noexcept {
  if (block == nullptr) return;
  if (device.is_hip()) {
    static_cast<void>(spar_hip_deallocate(block, device.index()));
  } else {
    std::free(block);
  }
}

Storage::Storage(std::size_t nbytes, Device device) : nbytes_{nbytes}, block_{nullptr, {device}} {
  void* block{nullptr};
  if (device.is_hip()) {
    if (device.index() >= hip_device_count()) {
      throw std::invalid_argument{"HIP device index is unavailable: " + device.to_string()};
    }
    hip::check(spar_hip_allocate(&block, nbytes_, device.index()), "allocate", device);
  } else if (nbytes_ != 0) {
    block = std::malloc(nbytes_);
    if (block == nullptr) throw std::bad_alloc{};
  }
  block_.reset(block);
}

Storage::~Storage() noexcept = default;

void* Storage::block_on(DeviceType expected) const {
  if (device().type() != expected) {
    throw std::logic_error{expected == DeviceType::CPU ? "Storage is not host-accessible"
                                                       : "Storage is not HIP-accessible"};
  }
  return block_.get();
}

std::byte* Storage::host_data() { return static_cast<std::byte*>(block_on(DeviceType::CPU)); }

const std::byte* Storage::host_data() const {
  return static_cast<const std::byte*>(block_on(DeviceType::CPU));
}

void* Storage::hip_data() { return block_on(DeviceType::HIP); }

const void* Storage::hip_data() const { return block_on(DeviceType::HIP); }

Device Storage::device() const noexcept { return block_.get_deleter().device; }

std::size_t Storage::nbytes() const noexcept { return nbytes_; }

void Storage::swap_payload(Storage& other) noexcept {
  std::swap(nbytes_, other.nbytes_);
  block_.swap(other.block_);  // swaps the deleters, hence the devices, too
}

}  // namespace spar::detail

namespace spar {
namespace {

// a * b, or std::nullopt on size_t overflow.
std::optional<std::size_t> product(std::size_t a, std::size_t b) {
  std::size_t result{0};
  if (__builtin_mul_overflow(a, b, &result)) return std::nullopt;
  return result;
}

std::vector<Shape::dimension_type> dimensions_of(const Shape& shape) {
  return {shape.dimensions().begin(), shape.dimensions().end()};
}

// Gradient rule of views that keep every value in place (clone, contiguous).
std::vector<Tensor> pass_through(const Tensor& gradient) { return {gradient}; }

}  // namespace

Tensor::Tensor(Shape shape, DType dtype, Device device)
    : storage_{}, dtype_{dtype}, shape_{std::move(shape)}, strides_{shape_.contiguous_strides()},
      storage_offset_{0}, nbytes_{checked_nbytes(shape_.numel(), dtype_)} {
  storage_ = std::make_shared<detail::Storage>(nbytes_, device);
  initialize_autograd();
  validate_view_bounds();
}

Tensor::Tensor(std::shared_ptr<detail::Storage> storage, DType dtype, Shape shape,
               std::vector<Shape::stride_type> strides, std::size_t storage_offset)
    : storage_{std::move(storage)}, dtype_{dtype}, shape_{std::move(shape)},
      strides_{std::move(strides)}, storage_offset_{storage_offset},
      nbytes_{checked_nbytes(shape_.numel(), dtype_)} {
  initialize_autograd();
  validate_view_bounds();
}

Tensor::Tensor(Tensor&& other) noexcept
    : storage_{std::move(other.storage_)}, dtype_{other.dtype_}, shape_{std::move(other.shape_)},
      strides_{std::move(other.strides_)}, storage_offset_{other.storage_offset_},
      nbytes_{other.nbytes_}, grad_state_{std::move(other.grad_state_)} {
  other.reset_to_empty();
}

Tensor& Tensor::operator=(Tensor&& other) noexcept {
  if (this != &other) {
    Tensor moved{std::move(other)};
    swap(moved);
  }
  return *this;
}

Tensor::~Tensor() = default;

void Tensor::reset_to_empty() noexcept {
  storage_.reset();
  strides_.clear();
  storage_offset_ = 0;
  nbytes_ = 0;
  grad_state_.reset();
}

void Tensor::swap(Tensor& other) noexcept {
  std::swap(storage_, other.storage_);
  std::swap(dtype_, other.dtype_);
  std::swap(shape_, other.shape_);
  std::swap(strides_, other.strides_);
  std::swap(storage_offset_, other.storage_offset_);
  std::swap(nbytes_, other.nbytes_);
  std::swap(grad_state_, other.grad_state_);
}

std::size_t Tensor::rank() const noexcept { return shape_.rank(); }
const Shape& Tensor::shape() const noexcept { return shape_; }
std::span<const Shape::stride_type> Tensor::strides() const noexcept { return strides_; }
std::size_t Tensor::storage_offset() const noexcept { return storage_offset_; }
std::size_t Tensor::numel() const noexcept { return shape_.numel(); }
DType Tensor::dtype() const noexcept { return dtype_; }

Device Tensor::device() const noexcept {
  return storage_ == nullptr ? Device::cpu() : storage_->device();
}

std::size_t Tensor::nbytes() const noexcept { return nbytes_; }

// Row-major contiguity as the reference defines it (tensor.cpp:113-128): an
// axis of extent 1 may carry any stride.  Walking the axes innermost first,
// every axis longer than 1 must step by the number of elements inside it.
bool Tensor::is_contiguous() const noexcept {
  if (numel() == 0) return true;
  std::size_t inner_elements{1};
  for (std::size_t axis{rank()}; axis-- > 0;) {
    const auto extent{static_cast<std::size_t>(shape_[axis])};
    if (extent == 1) continue;
    if (strides_[axis] != inner_elements) return false;
    inner_elements *= extent;
  }
  return true;
}

std::size_t Tensor::checked_storage_byte_offset() const {
  const auto offset{product(storage_offset_, size_of(dtype_))};
  if (!offset) throw std::overflow_error{"Tensor Storage byte offset overflow"};
  if (storage_ == nullptr || *offset > storage_->nbytes() ||
      nbytes_ > storage_->nbytes() - *offset) {
    throw std::logic_error{"Contiguous Tensor region exceeds Storage bounds"};
  }
  return *offset;
}

// A contiguous copy of this (non-contiguous) view on its own device.  On a
// HIP device the strided-copy kernel gathers it; on the host each element is
// copied from its storage position (layout only, no arithmetic).
Tensor Tensor::gathered() const {
  Tensor staging{shape_, dtype_, device()};
  if (numel() == 0) return staging;
  if (device().is_hip()) {
    const auto view{detail::hip::view_of(*this)};
    detail::hip::check(
        spar_hip_launch_strided_copy(staging.storage_->hip_data(), storage_->hip_data(),
                                     view.extents.size(), view.extents.data(),
                                     view.strides.data(), view.offset, numel(), size_of(dtype_),
                                     device().index()),
        "contiguous", device());
    return staging;
  }
  // Odometer over the logical index space: position advances by the stride
  // of the innermost axis and carries into outer axes.
  const std::size_t element{size_of(dtype_)};
  const std::byte* source{storage_->host_data()};
  std::byte* destination{staging.storage_->host_data()};
  std::vector<std::size_t> coordinate(rank(), 0);
  std::size_t position{storage_offset_};
  for (std::size_t logical{0}; logical < numel(); ++logical) {
    std::memcpy(destination + logical * element, source + position * element, element);
    for (std::size_t axis{rank()}; axis-- > 0;) {
      position += strides_[axis];
      if (++coordinate[axis] < static_cast<std::size_t>(shape_[axis])) break;
      position -= coordinate[axis] * strides_[axis];
      coordinate[axis] = 0;
    }
  }
  return staging;
}

// The logical values as a new contiguous tensor on `target`.
Tensor Tensor::materialize_values(Device target) const {
  if (!is_contiguous()) {
    Tensor staging{gathered()};
    return target == device() ? staging : staging.materialize_values(target);
  }
  Tensor output{shape_, dtype_, target};
  if (nbytes_ == 0) return output;
  const Device source_device{device()};
  const std::size_t offset{checked_storage_byte_offset()};
  if (source_device.is_cpu()) {
    const std::byte* source{storage_->host_data() + offset};
    if (target.is_cpu()) {
      std::memcpy(output.storage_->host_data(), source, nbytes_);
    } else {
      detail::hip::check(spar_hip_copy_host_to_device(output.storage_->hip_data(), source,
                                                      nbytes_, target.index()),
                         "copy to device", target);
    }
    return output;
  }
  const auto* source{static_cast<const std::byte*>(storage_->hip_data()) + offset};
  if (target.is_cpu()) {
    detail::hip::check(spar_hip_copy_device_to_host(output.storage_->host_data(), source, nbytes_,
                                                    source_device.index()),
                       "copy to host", source_device);
  } else {
    detail::hip::check(spar_hip_copy_device_to_device(output.storage_->hip_data(), target.index(),
                                                      source, source_device.index(), nbytes_),
                       "copy between devices", target);
  }
  return output;
}

Tensor Tensor::make_view(Shape shape, std::vector<Shape::stride_type> strides,
                         std::size_t storage_offset,
                         std::function<std::vector<Tensor>(const Tensor&)> rule) const {
  Tensor view{storage_, dtype_, std::move(shape), std::move(strides), storage_offset};
  if (requires_grad()) detail::record_operation(view, {*this}, std::move(rule));
  return view;
}

Tensor Tensor::clone() const {
  Tensor copy{materialize_values(device())};
  if (requires_grad()) detail::record_operation(copy, {*this}, pass_through);
  return copy;
}

Tensor Tensor::contiguous() const { return is_contiguous() ? *this : clone(); }

Tensor Tensor::reshape(Shape new_shape) const {
  if (!is_contiguous()) throw std::invalid_argument{"reshape requires a contiguous tensor"};
  if (new_shape.numel() != numel()) {
    throw std::invalid_argument{"reshape requires the same number of elements"};
  }
  auto strides{new_shape.contiguous_strides()};
  return make_view(std::move(new_shape), std::move(strides), storage_offset_,
                   [original = shape_](const Tensor& gradient) {
                     // an incoming view (a reduction's broadcast gradient)
                     // is made contiguous first, as reshape requires
                     return std::vector<Tensor>{gradient.contiguous().reshape(original)};
                   });
}

Tensor Tensor::permuted(const std::vector<std::size_t>& order) const {
  std::vector<Shape::dimension_type> dimensions(order.size());
  std::vector<Shape::stride_type> strides(order.size());
  std::vector<std::size_t> inverse(order.size());
  for (std::size_t axis{0}; axis < order.size(); ++axis) {
    dimensions[axis] = shape_[order[axis]];
    strides[axis] = strides_[order[axis]];
    inverse[order[axis]] = axis;
  }
  // The gradient of a permuted view is the gradient permuted back, made
  // contiguous (a pure copy).
  return make_view(Shape{std::move(dimensions)}, std::move(strides), storage_offset_,
                   [inverse = std::move(inverse)](const Tensor& gradient) {
                     return std::vector<Tensor>{gradient.permuted(inverse).contiguous()};
                   });
}

Tensor Tensor::transpose(std::size_t axis_a, std::size_t axis_b) const {
  if (axis_a >= rank() || axis_b >= rank()) throw std::out_of_range{"transpose axis is out of range"};
  std::vector<std::size_t> order(rank());
  for (std::size_t axis{0}; axis < rank(); ++axis) order[axis] = axis;
  std::swap(order[axis_a], order[axis_b]);
  return permuted(order);
}

Tensor Tensor::permute(std::span<const std::size_t> axes) const {
  if (axes.size() != rank()) {
    throw std::invalid_argument{"permute requires exactly one entry per tensor axis"};
  }
  // Entries are checked in order: an out-of-range entry is reported before a
  // later duplicate and a duplicate before a later out-of-range entry.
  std::vector<char> used(rank(), 0);
  for (const std::size_t axis : axes) {
    if (axis >= rank()) throw std::out_of_range{"permute axis is out of range"};
    if (used[axis] != 0) throw std::invalid_argument{"permute axes must not contain duplicates"};
    used[axis] = 1;
  }
  return permuted(std::vector<std::size_t>{axes.begin(), axes.end()});
}

Tensor Tensor::permute(std::initializer_list<std::size_t> axes) const {
  return permute(std::span<const std::size_t>{axes.begin(), axes.size()});
}

Tensor Tensor::expand(Shape target_shape) const {
  if (target_shape.rank() < rank()) {
    throw std::invalid_argument{"expand target rank must not be smaller than the input rank"};
  }
  // Right-aligned: new leading axes and broadcast (extent-1) axes get
  // stride 0, matching axes keep their stride.
  std::vector<Shape::stride_type> strides(target_shape.rank(), 0);
  const std::size_t shift{target_shape.rank() - rank()};
  for (std::size_t axis{0}; axis < rank(); ++axis) {
    const auto extent{shape_[axis]};
    if (extent == target_shape[shift + axis]) {
      strides[shift + axis] = strides_[axis];
    } else if (extent != 1) {
      throw std::invalid_argument{"expand dimensions are not broadcast-compatible"};
    }
  }
  return make_view(std::move(target_shape), std::move(strides), storage_offset_,
                   [original = shape_](const Tensor& gradient) {
                     return std::vector<Tensor>{
                         detail::reduce_gradient_to_shape(gradient, original)};
                   });
}

Tensor Tensor::narrow(std::size_t axis, std::size_t start, std::size_t length) const {
  if (axis >= rank()) throw std::out_of_range{"narrow axis is out of range"};
  const auto extent{static_cast<std::size_t>(shape_[axis])};
  if (start > extent || length > extent - start) {
    throw std::out_of_range{"narrow range exceeds the axis extent"};
  }
  auto dimensions{dimensions_of(shape_)};
  dimensions[axis] = static_cast<Shape::dimension_type>(length);
  const std::size_t offset{length == 0 ? storage_offset_ : storage_offset_ + start * strides_[axis]};
  // The gradient of a narrowed view is zero outside the window.  On a HIP
  // device a contiguous gradient is embedded in one pass; otherwise the
  // window of a zero tensor is assigned.  The node also records its box, so
  // that the engine can embed the gradient of a chain of narrows at once.
  Tensor view{make_view(Shape{std::move(dimensions)}, strides_, offset,
                   [original = shape_, axis, start, length](const Tensor& gradient) {
                     if (gradient.device().is_hip() && gradient.is_contiguous()) {
                       std::size_t outer{1}, inner{1};
                       for (std::size_t k{0}; k < axis; ++k) {
                         outer *= static_cast<std::size_t>(original[k]);
                       }
                       for (std::size_t k{axis + 1}; k < original.rank(); ++k) {
                         inner *= static_cast<std::size_t>(original[k]);
                       }
                       Tensor result{original, gradient.dtype(), gradient.device()};
                       const auto status{spar_hip_launch_window_embed(
                           detail::HipTensorAccess::mutable_data(result),
                           detail::HipTensorAccess::data(gradient), outer,
                           static_cast<std::size_t>(original[axis]), inner, start, length,
                           size_of(gradient.dtype()), gradient.device().index())};
                       if (status.code == 0) return std::vector<Tensor>{result};
                       // status 1 (a shape the one-pass kernel does not take)
                       // falls through to the two-pass form
                       if (status.code != 1) {
                         detail::hip::check(status, "narrow backward", gradient.device());
                       }
                     }
                     Tensor result{zeros(original, gradient.dtype(), gradient.device())};
                     Tensor window{result.narrow(axis, start, length)};
                     detail::copy_tensor_values(window, gradient);
                     return std::vector<Tensor>{result};
                   })};
  if (view.requires_grad()) {
    std::vector<detail::WindowAxis> box;
    box.reserve(rank());
    for (std::size_t k{0}; k < rank(); ++k) {
      box.push_back(k == axis ? detail::WindowAxis{start, length}
                              : detail::WindowAxis{0, static_cast<std::size_t>(shape_[k])});
    }
    detail::TensorInternals::grad_state(view)->producer->window = std::move(box);
  }
  return view;
}

Tensor Tensor::detach() const { return Tensor{storage_, dtype_, shape_, strides_, storage_offset_}; }

Tensor Tensor::to(Device target) const {
  if (target == device()) return *this;
  Tensor moved{materialize_values(target)};
  if (requires_grad()) {
    detail::record_transfer_operation(moved, *this, [home = device()](const Tensor& gradient) {
      return std::vector<Tensor>{gradient.to(home)};
    });
  }
  return moved;
}

std::size_t Tensor::checked_nbytes(std::size_t numel, DType dtype) {
  const auto bytes{product(numel, size_of(dtype))};
  if (!bytes) throw std::overflow_error{"Tensor byte size overflow"};
  return *bytes;
}

// Every element of the view must lie inside the storage (the reference's
// checks and messages, tensor.cpp:370-403).  The farthest element sits at
// offset + sum over axes of (extent - 1) * stride.
void Tensor::validate_view_bounds() const {
  if (strides_.size() != rank()) throw std::logic_error{"Tensor stride rank does not match shape rank"};
  const std::size_t capacity{storage_ == nullptr ? 0 : storage_->nbytes() / size_of(dtype_)};
  if (numel() == 0) {
    if (storage_offset_ > capacity) {
      throw std::logic_error{"Empty tensor view offset exceeds Storage bounds"};
    }
    return;
  }
  if (storage_ == nullptr) throw std::logic_error{"Non-empty tensor view has no Storage"};
  std::size_t farthest{storage_offset_};
  for (std::size_t axis{0}; axis < rank(); ++axis) {
    const auto span{product(static_cast<std::size_t>(shape_[axis]) - 1, strides_[axis])};
    if (!span || __builtin_add_overflow(farthest, *span, &farthest)) {
      throw std::overflow_error{"Tensor view offset calculation overflow"};
    }
  }
  if (farthest >= capacity) throw std::logic_error{"Tensor view exceeds Storage bounds"};
}

std::byte* Tensor::mutable_host_data() { return storage_ == nullptr ? nullptr : storage_->host_data(); }

const std::byte* Tensor::host_data() const {
  return storage_ == nullptr ? nullptr : storage_->host_data();
}

void swap(Tensor& left, Tensor& right) noexcept { left.swap(right); }

Tensor zeros(Shape shape, DType dtype, Device device) {
  Tensor tensor{std::move(shape), dtype, device};
  if (tensor.nbytes() == 0) return tensor;
  if (device.is_hip()) {
    detail::hip::check(spar_hip_zero(tensor.storage_->hip_data(), tensor.nbytes(), device.index()),
                       "zeros", device);
  } else {
    std::memset(tensor.storage_->host_data(), 0, tensor.nbytes());
  }
  return tensor;
}

Tensor full_value(Shape shape, DType dtype, double value, Device device) {
  Tensor tensor{std::move(shape), dtype, device};
  if (device.is_hip()) {
    detail::hip::check(spar_hip_launch_fill(tensor.storage_->hip_data(), tensor.numel(),
                                            detail::hip::dtype_tag(dtype), value, device.index()),
                       "full", device);
    return tensor;
  }
  switch (dtype) {
    case DType::Float32: tensor.fill<float>(static_cast<float>(value)); break;
    case DType::Float64: tensor.fill<double>(value); break;
    case DType::Int32: tensor.fill<std::int32_t>(static_cast<std::int32_t>(value)); break;
    case DType::Int64: tensor.fill<std::int64_t>(static_cast<std::int64_t>(value)); break;
  }
  return tensor;
}

Tensor ones(Shape shape, DType dtype, Device device) {
  return full_value(std::move(shape), dtype, 1.0, device);
}

namespace {
std::atomic<bool> exact_zero_signs{false};
}  // namespace

void set_exact_gradient_zero_signs(bool enabled) noexcept {
  exact_zero_signs.store(enabled, std::memory_order_relaxed);
}

bool exact_gradient_zero_signs() noexcept { return exact_zero_signs.load(std::memory_order_relaxed); }

}  // namespace spar

namespace spar::detail {

namespace {

// Byte address of a contiguous HIP tensor's first element.
std::byte* hip_first_byte(const std::shared_ptr<Storage>& storage, std::size_t byte_offset) {
  return static_cast<std::byte*>(storage->hip_data()) + byte_offset;
}

}  // namespace

void* HipTensorAccess::mutable_data(Tensor& tensor) {
  if (!tensor.device().is_hip() || !tensor.is_contiguous()) {
    throw std::logic_error{"Internal HIP access requires a contiguous HIP Tensor"};
  }
  if (tensor.nbytes_ == 0) return nullptr;
  return hip_first_byte(tensor.storage_, tensor.checked_storage_byte_offset());
}

const void* HipTensorAccess::data(const Tensor& tensor) {
  if (!tensor.device().is_hip() || !tensor.is_contiguous()) {
    throw std::logic_error{"Internal HIP access requires a contiguous HIP Tensor"};
  }
  if (tensor.nbytes_ == 0) return nullptr;
  return hip_first_byte(tensor.storage_, tensor.checked_storage_byte_offset());
}

const void* HipTensorAccess::storage_base(const Tensor& tensor) {
  if (!tensor.device().is_hip()) throw std::logic_error{"Internal HIP access requires a HIP Tensor"};
  return tensor.storage_->hip_data();
}

void require_hip(const Tensor& tensor, std::string_view operation) {
  if (!tensor.device().is_hip()) {
    throw std::runtime_error{std::string{operation} +
                             " requires a HIP tensor: this backend computes on MI355X devices, "
                             "CPU tensors are host buffers (move them with to(Device::hip()))"};
  }
}

// Copies source's logical values into destination (the reference's
// copy_tensor_values, tensor.cpp:514-537).  A HIP destination may be any
// view: the values are scattered into it by the strided-assign kernel.
void copy_tensor_values(Tensor& destination, const Tensor& source) {
  validate_same_device(destination, source, "Tensor value copy");
  if (destination.shape() != source.shape() || destination.dtype() != source.dtype()) {
    throw std::invalid_argument{"Tensor value copy requires identical shapes and dtypes"};
  }
  if (destination.numel() == 0) return;
  if (destination.device().is_hip()) {
    const Tensor packed{source.is_contiguous() ? source : source.detach().contiguous()};
    const auto view{hip::view_of(destination)};
    hip::check(spar_hip_launch_strided_assign(
                   const_cast<void*>(HipTensorAccess::storage_base(destination)),
                   view.extents.size(), view.extents.data(), view.strides.data(), view.offset,
                   HipTensorAccess::data(packed), size_of(destination.dtype()),
                   destination.device().index()),
               "copy", destination.device());
    return;
  }
  if (!destination.is_contiguous()) {
    throw std::invalid_argument{"Tensor value copy requires a contiguous destination"};
  }
  const Tensor packed{source.detach().contiguous()};
  std::memcpy(TensorInternals::host_bytes(destination), TensorInternals::host_bytes(packed),
              destination.nbytes());
}

void swap_storage_payloads(Tensor& original, Tensor& staged) noexcept {
  TensorInternals::storage(original)->swap_payload(*TensorInternals::storage(staged));
}

void validate_same_device(const Tensor& left, const Tensor& right, std::string_view operation) {
  if (left.device() != right.device()) {
    throw std::invalid_argument{std::string{operation} + " requires tensors on the same Device"};
  }
}

// Right-aligned numpy broadcasting (the reference's rule, tensor.cpp:549-570):
// a missing leading axis counts as extent 1; two extents combine when they
// are equal or one of them is 1.
Shape broadcast_shape(const Shape& left, const Shape& right) {
  const Shape& longer{left.rank() >= right.rank() ? left : right};
  const Shape& shorter{left.rank() >= right.rank() ? right : left};
  auto dimensions{dimensions_of(longer)};
  const std::size_t shift{longer.rank() - shorter.rank()};
  for (std::size_t axis{0}; axis < shorter.rank(); ++axis) {
    auto& extent{dimensions[shift + axis]};
    const auto other{shorter[axis]};
    if (extent == other || other == 1) continue;
    if (extent != 1) throw std::invalid_argument{"Tensor shapes are not broadcast-compatible"};
    extent = other;
  }
  return Shape{std::move(dimensions)};
}

// Sums a gradient over the axes its parent was broadcast along (the role of
// tensor.cpp:572-632).  A gradient that already has the parent's shape is
// returned as is (the reference re-accumulated it into a zeroed buffer), or
// re-added to +0 when exact zero signs are on; otherwise one deterministic
// device reduction reads the gradient in place, contiguous or not (its sums
// start from +0, as the reference's do).
Tensor reduce_gradient_to_shape(const Tensor& gradient, const Shape& original_shape) {
  if (!is_floating(gradient.dtype())) {
    throw std::logic_error{"Broadcast gradient reduction requires a floating dtype"};
  }
  if (gradient.shape() != broadcast_shape(gradient.shape(), original_shape)) {
    throw std::logic_error{
        "Gradient shape cannot be reduced to the requested broadcast parent shape"};
  }
  require_hip(gradient, "reduce_gradient_to_shape");
  if (gradient.shape() == original_shape) {
    if (!exact_gradient_zero_signs()) return gradient.detach();
    // g + (+0), read in place whatever its strides (a sum's gradient is a
    // stride-0 view): -0 + +0 = +0, every other value unchanged.
    return add(gradient.detach(), zeros(Shape{}, gradient.dtype(), gradient.device()));
  }
  Tensor result{original_shape, gradient.dtype(), gradient.device()};
  // Reduced: the leading axes the parent lacks, and its extent-1 axes that
  // the gradient spans.
  const std::size_t shift{gradient.rank() - original_shape.rank()};
  std::uint32_t mask{(std::uint32_t{1} << shift) - 1U};
  for (std::size_t axis{shift}; axis < gradient.rank(); ++axis) {
    if (original_shape[axis - shift] == 1 && gradient.shape()[axis] != 1) mask |= 1U << axis;
  }
  const auto view{hip::view_of(gradient)};
  hip::check(spar_hip_launch_axis_reduction(HipTensorAccess::mutable_data(result),
                                            HipTensorAccess::storage_base(gradient),
                                            view.extents.size(), view.extents.data(),
                                            view.strides.data(), view.offset, mask,
                                            hip::dtype_tag(gradient.dtype()), SPAR_HIP_SUM,
                                            gradient.device().index()),
             "reduce_gradient_to_shape", gradient.device());
  return result;
}

}  // namespace spar::detail
