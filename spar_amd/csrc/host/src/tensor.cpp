// Tensor core: storage, views, materialisation, transfers and factories.
// Follows src/core/storage.cpp:11-68 and src/core/tensor.cpp:26-632; device
// work goes through the C ABI (include/spar_hip.h).
#include <cstring>
#include <limits>
#include <numeric>
#include <utility>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/ops.hpp"
#include "spar/tensor.hpp"

namespace spar::detail {

Storage::Storage(std::size_t nbytes, Device device)
    : nbytes_{nbytes}, device_{device}, host_data_{}, hip_data_{nullptr} {
  if (device_.is_cpu()) {
    if (nbytes_ != 0) host_data_ = std::unique_ptr<std::byte[]>(new std::byte[nbytes_]);
    return;
  }
  const int count = hip_device_count();
  if (device_.index() >= count) {
    throw std::invalid_argument{"HIP device index is unavailable: " + device_.to_string()};
  }
  hip::check(spar_hip_allocate(&hip_data_, nbytes_, device_.index()), "allocate", device_);
}

Storage::~Storage() noexcept {
  if (device_.is_hip() && hip_data_ != nullptr) {
    (void)spar_hip_deallocate(hip_data_, device_.index());
  }
}

std::byte* Storage::host_data() {
  if (!device_.is_cpu()) throw std::logic_error{"Storage is not host-accessible"};
  return host_data_.get();
}

const std::byte* Storage::host_data() const {
  if (!device_.is_cpu()) throw std::logic_error{"Storage is not host-accessible"};
  return host_data_.get();
}

void* Storage::hip_data() {
  if (!device_.is_hip()) throw std::logic_error{"Storage is not HIP-accessible"};
  return hip_data_;
}

const void* Storage::hip_data() const {
  if (!device_.is_hip()) throw std::logic_error{"Storage is not HIP-accessible"};
  return hip_data_;
}

Device Storage::device() const noexcept { return device_; }

std::size_t Storage::nbytes() const noexcept { return nbytes_; }

void Storage::swap_payload(Storage& other) noexcept {
  using std::swap;
  swap(nbytes_, other.nbytes_);
  swap(device_, other.device_);
  swap(host_data_, other.host_data_);
  swap(hip_data_, other.hip_data_);
}

}  // namespace spar::detail

namespace spar {

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
      nbytes_{other.nbytes_}, autograd_{std::move(other.autograd_)} {
  other.reset_to_empty();
}

Tensor& Tensor::operator=(Tensor&& other) noexcept {
  if (this != &other) {
    storage_ = std::move(other.storage_);
    dtype_ = other.dtype_;
    shape_ = std::move(other.shape_);
    strides_ = std::move(other.strides_);
    storage_offset_ = other.storage_offset_;
    nbytes_ = other.nbytes_;
    autograd_ = std::move(other.autograd_);
    other.reset_to_empty();
  }
  return *this;
}

Tensor::~Tensor() = default;

void Tensor::reset_to_empty() noexcept {
  storage_.reset();
  strides_.clear();
  storage_offset_ = 0;
  nbytes_ = 0;
  autograd_.reset();
}

void Tensor::swap(Tensor& other) noexcept {
  using std::swap;
  swap(storage_, other.storage_);
  swap(dtype_, other.dtype_);
  swap(shape_, other.shape_);
  swap(strides_, other.strides_);
  swap(storage_offset_, other.storage_offset_);
  swap(nbytes_, other.nbytes_);
  swap(autograd_, other.autograd_);
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

// tensor.cpp:113-128: strides of extent-1 axes are ignored.
bool Tensor::is_contiguous() const noexcept {
  if (numel() == 0 || rank() == 0) return true;
  std::size_t expected_stride{1};
  for (std::size_t index{rank()}; index > 0; --index) {
    const std::size_t axis{index - 1};
    const auto extent{static_cast<std::size_t>(shape_[axis])};
    if (extent > 1 && strides_[axis] != expected_stride) return false;
    expected_stride *= extent;
  }
  return true;
}

std::size_t Tensor::checked_storage_byte_offset() const {
  const std::size_t element_size{size_of(dtype_)};
  if (storage_offset_ > std::numeric_limits<std::size_t>::max() / element_size) {
    throw std::overflow_error{"Tensor Storage byte offset overflow"};
  }
  const std::size_t offset{storage_offset_ * element_size};
  if (storage_ == nullptr || offset > storage_->nbytes() || nbytes_ > storage_->nbytes() - offset) {
    throw std::logic_error{"Contiguous Tensor region exceeds Storage bounds"};
  }
  return offset;
}

// Materialises the logical values on `target` (tensor.cpp:169-210).  A
// non-contiguous device view is gathered by the strided-copy kernel; a
// non-contiguous host view is gathered element by element on the host
// (layout only, no arithmetic).
Tensor Tensor::materialize_values(Device target) const {
  if (!is_contiguous()) {
    Tensor staging{shape_, dtype_, device()};
    if (device().is_hip()) {
      const auto view{detail::hip::view_of(*this)};
      detail::hip::check(
          spar_hip_launch_strided_copy(staging.storage_->hip_data(), storage_->hip_data(),
                                       view.extents.size(), view.extents.data(),
                                       view.strides.data(), view.offset, numel(), size_of(dtype_),
                                       device().index()),
          "contiguous", device());
    } else {
      const std::size_t element{size_of(dtype_)};
      const std::byte* source{storage_->host_data()};
      std::byte* destination{staging.storage_->host_data()};
      for (std::size_t logical = 0; logical < numel(); ++logical) {
        std::size_t remaining{logical};
        std::size_t index{storage_offset_};
        for (std::size_t axis = rank(); axis > 0; --axis) {
          const auto extent{static_cast<std::size_t>(shape_[axis - 1])};
          index += (remaining % extent) * strides_[axis - 1];
          remaining /= extent;
        }
        std::memcpy(destination + logical * element, source + index * element, element);
      }
    }
    return target == device() ? staging : staging.materialize_values(target);
  }

  Tensor output{shape_, dtype_, target};
  if (nbytes_ == 0) return output;
  const std::size_t source_offset{checked_storage_byte_offset()};
  if (device().is_cpu() && target.is_cpu()) {
    std::memcpy(output.storage_->host_data(), storage_->host_data() + source_offset, nbytes_);
  } else if (device().is_cpu()) {
    detail::hip::check(
        spar_hip_copy_host_to_device(output.storage_->hip_data(),
                                     storage_->host_data() + source_offset, nbytes_, target.index()),
        "copy to device", target);
  } else if (target.is_cpu()) {
    const auto* source{static_cast<const std::byte*>(storage_->hip_data()) + source_offset};
    detail::hip::check(spar_hip_copy_device_to_host(output.storage_->host_data(), source, nbytes_,
                                                    device().index()),
                       "copy to host", device());
  } else {
    const auto* source{static_cast<const std::byte*>(storage_->hip_data()) + source_offset};
    detail::hip::check(spar_hip_copy_device_to_device(output.storage_->hip_data(), target.index(),
                                                      source, device().index(), nbytes_),
                       "copy between devices", target);
  }
  return output;
}

Tensor Tensor::clone() const {
  auto output{materialize_values(device())};
  if (requires_grad()) {
    detail::record_operation(output, {*this},
                             [](const Tensor& gradient) { return std::vector<Tensor>{gradient}; });
  }
  return output;
}

Tensor Tensor::contiguous() const {
  if (is_contiguous()) return *this;
  auto output{materialize_values(device())};
  if (requires_grad()) {
    detail::record_operation(output, {*this},
                             [](const Tensor& gradient) { return std::vector<Tensor>{gradient}; });
  }
  return output;
}

Tensor Tensor::reshape(Shape new_shape) const {
  if (!is_contiguous()) throw std::invalid_argument{"reshape requires a contiguous tensor"};
  if (new_shape.numel() != numel()) {
    throw std::invalid_argument{"reshape requires the same number of elements"};
  }
  auto new_strides{new_shape.contiguous_strides()};
  Tensor output{storage_, dtype_, std::move(new_shape), std::move(new_strides), storage_offset_};
  if (requires_grad()) {
    const Shape original_shape{shape_};
    detail::record_operation(output, {*this}, [original_shape](const Tensor& gradient) {
      return std::vector<Tensor>{gradient.reshape(original_shape)};
    });
  }
  return output;
}

Tensor Tensor::transpose(std::size_t axis_a, std::size_t axis_b) const {
  if (axis_a >= rank() || axis_b >= rank()) throw std::out_of_range{"transpose axis is out of range"};
  std::vector<Shape::dimension_type> dimensions{shape_.dimensions().begin(),
                                                shape_.dimensions().end()};
  auto new_strides{strides_};
  std::swap(dimensions[axis_a], dimensions[axis_b]);
  std::swap(new_strides[axis_a], new_strides[axis_b]);
  Tensor output{storage_, dtype_, Shape{std::move(dimensions)}, std::move(new_strides),
                storage_offset_};
  if (requires_grad()) {
    detail::record_operation(output, {*this}, [axis_a, axis_b](const Tensor& gradient) {
      return std::vector<Tensor>{gradient.transpose(axis_a, axis_b).contiguous()};
    });
  }
  return output;
}

Tensor Tensor::permute(std::span<const std::size_t> axes) const {
  if (axes.size() != rank()) {
    throw std::invalid_argument{"permute requires exactly one entry per tensor axis"};
  }
  std::vector<bool> seen(rank(), false);
  std::vector<Shape::dimension_type> dimensions(rank());
  std::vector<Shape::stride_type> new_strides(rank());
  for (std::size_t result_axis{0}; result_axis < axes.size(); ++result_axis) {
    const std::size_t source_axis{axes[result_axis]};
    if (source_axis >= rank()) throw std::out_of_range{"permute axis is out of range"};
    if (seen[source_axis]) throw std::invalid_argument{"permute axes must not contain duplicates"};
    seen[source_axis] = true;
    dimensions[result_axis] = shape_[source_axis];
    new_strides[result_axis] = strides_[source_axis];
  }
  std::vector<std::size_t> inverse_axes(rank());
  for (std::size_t result_axis{0}; result_axis < axes.size(); ++result_axis) {
    inverse_axes[axes[result_axis]] = result_axis;
  }
  Tensor output{storage_, dtype_, Shape{std::move(dimensions)}, std::move(new_strides),
                storage_offset_};
  if (requires_grad()) {
    detail::record_operation(output, {*this},
                             [inverse_axes = std::move(inverse_axes)](const Tensor& gradient) {
                               return std::vector<Tensor>{
                                   gradient.permute(inverse_axes).contiguous()};
                             });
  }
  return output;
}

Tensor Tensor::permute(std::initializer_list<std::size_t> axes) const {
  return permute(std::span<const std::size_t>{axes.begin(), axes.size()});
}

Tensor Tensor::expand(Shape target_shape) const {
  if (target_shape.rank() < rank()) {
    throw std::invalid_argument{"expand target rank must not be smaller than the input rank"};
  }
  std::vector<Shape::stride_type> expanded_strides(target_shape.rank(), 0);
  const std::size_t leading_axes{target_shape.rank() - rank()};
  for (std::size_t source_axis{0}; source_axis < rank(); ++source_axis) {
    const std::size_t target_axis{leading_axes + source_axis};
    const auto source_extent{shape_[source_axis]};
    const auto target_extent{target_shape[target_axis]};
    if (source_extent == target_extent) {
      expanded_strides[target_axis] = strides_[source_axis];
    } else if (source_extent == 1) {
      expanded_strides[target_axis] = 0;
    } else {
      throw std::invalid_argument{"expand dimensions are not broadcast-compatible"};
    }
  }
  Tensor output{storage_, dtype_, std::move(target_shape), std::move(expanded_strides),
                storage_offset_};
  if (requires_grad()) {
    const Shape original_shape{shape_};
    detail::record_operation(output, {*this}, [original_shape](const Tensor& gradient) {
      return std::vector<Tensor>{detail::reduce_gradient_to_shape(gradient, original_shape)};
    });
  }
  return output;
}

Tensor Tensor::narrow(std::size_t axis, std::size_t start, std::size_t length) const {
  if (axis >= rank()) throw std::out_of_range{"narrow axis is out of range"};
  const auto extent{static_cast<std::size_t>(shape_[axis])};
  if (start > extent || length > extent - start) {
    throw std::out_of_range{"narrow range exceeds the axis extent"};
  }
  std::vector<Shape::dimension_type> dimensions{shape_.dimensions().begin(),
                                                shape_.dimensions().end()};
  dimensions[axis] = static_cast<Shape::dimension_type>(length);
  const std::size_t offset{length == 0 ? storage_offset_ : storage_offset_ + start * strides_[axis]};
  Tensor output{storage_, dtype_, Shape{std::move(dimensions)}, strides_, offset};
  if (requires_grad()) {
    const Shape original_shape{shape_};
    detail::record_operation(
        output, {*this}, [original_shape, axis, start, length](const Tensor& gradient) {
          // The gradient of a narrowed view is zero outside the view.
          Tensor result{zeros(original_shape, gradient.dtype(), gradient.device())};
          Tensor window{result.narrow(axis, start, length)};
          detail::copy_tensor_values(window, gradient);
          return std::vector<Tensor>{result};
        });
  }
  return output;
}

Tensor Tensor::detach() const {
  return Tensor{storage_, dtype_, shape_, strides_, storage_offset_};
}

Tensor Tensor::to(Device target) const {
  if (target == device()) return *this;
  auto output{materialize_values(target)};
  if (requires_grad()) {
    const Device source_device{device()};
    detail::record_transfer_operation(output, *this, [source_device](const Tensor& gradient) {
      return std::vector<Tensor>{gradient.to(source_device)};
    });
  }
  return output;
}

std::size_t Tensor::checked_nbytes(std::size_t numel, DType dtype) {
  const auto element_size{size_of(dtype)};
  if (numel != 0 && element_size > std::numeric_limits<std::size_t>::max() / numel) {
    throw std::overflow_error{"Tensor byte size overflow"};
  }
  return numel * element_size;
}

// tensor.cpp:370-403
void Tensor::validate_view_bounds() const {
  if (strides_.size() != rank()) throw std::logic_error{"Tensor stride rank does not match shape rank"};
  const std::size_t element_size{size_of(dtype_)};
  const std::size_t storage_elements{storage_ == nullptr ? 0 : storage_->nbytes() / element_size};
  if (numel() == 0) {
    if (storage_offset_ > storage_elements) {
      throw std::logic_error{"Empty tensor view offset exceeds Storage bounds"};
    }
    return;
  }
  if (storage_ == nullptr) throw std::logic_error{"Non-empty tensor view has no Storage"};
  std::size_t maximum_offset{storage_offset_};
  for (std::size_t axis{0}; axis < rank(); ++axis) {
    const auto extent{static_cast<std::size_t>(shape_[axis])};
    const std::size_t steps{extent - 1};
    if (steps != 0 && strides_[axis] > std::numeric_limits<std::size_t>::max() / steps) {
      throw std::overflow_error{"Tensor view offset calculation overflow"};
    }
    const std::size_t contribution{steps * strides_[axis]};
    if (maximum_offset > std::numeric_limits<std::size_t>::max() - contribution) {
      throw std::overflow_error{"Tensor view offset calculation overflow"};
    }
    maximum_offset += contribution;
  }
  if (maximum_offset >= storage_elements) throw std::logic_error{"Tensor view exceeds Storage bounds"};
}

std::byte* Tensor::mutable_host_data() { return storage_ == nullptr ? nullptr : storage_->host_data(); }

const std::byte* Tensor::host_data() const {
  return storage_ == nullptr ? nullptr : storage_->host_data();
}

void swap(Tensor& left, Tensor& right) noexcept { left.swap(right); }

Tensor zeros(Shape shape, DType dtype, Device device) {
  Tensor tensor{std::move(shape), dtype, device};
  if (device.is_hip()) {
    detail::hip::check(spar_hip_zero(tensor.storage_->hip_data(), tensor.nbytes(), device.index()),
                       "zeros", device);
    return tensor;
  }
  if (tensor.nbytes() != 0) std::memset(tensor.storage_->host_data(), 0, tensor.nbytes());
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

}  // namespace spar

namespace spar::detail {

void* HipTensorAccess::mutable_data(Tensor& tensor) {
  if (!tensor.device().is_hip() || !tensor.is_contiguous()) {
    throw std::logic_error{"Internal HIP access requires a contiguous HIP Tensor"};
  }
  if (tensor.nbytes_ == 0) return nullptr;
  return static_cast<std::byte*>(tensor.storage_->hip_data()) + tensor.checked_storage_byte_offset();
}

const void* HipTensorAccess::data(const Tensor& tensor) {
  if (!tensor.device().is_hip() || !tensor.is_contiguous()) {
    throw std::logic_error{"Internal HIP access requires a contiguous HIP Tensor"};
  }
  if (tensor.nbytes_ == 0) return nullptr;
  return static_cast<const std::byte*>(tensor.storage_->hip_data()) +
         tensor.checked_storage_byte_offset();
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

// tensor.cpp:514-537; a device destination may be any view (scatter).
void copy_tensor_values(Tensor& destination, const Tensor& source) {
  validate_same_device(destination, source, "Tensor value copy");
  if (destination.shape() != source.shape() || destination.dtype() != source.dtype()) {
    throw std::invalid_argument{"Tensor value copy requires identical shapes and dtypes"};
  }
  if (destination.numel() == 0) return;
  if (destination.device().is_hip()) {
    const Tensor contiguous_source{source.is_contiguous() ? source : source.detach().contiguous()};
    const auto view{hip::view_of(destination)};
    hip::check(spar_hip_launch_strided_assign(
                   const_cast<void*>(HipTensorAccess::storage_base(destination)),
                   view.extents.size(), view.extents.data(), view.strides.data(), view.offset,
                   HipTensorAccess::data(contiguous_source), size_of(destination.dtype()),
                   destination.device().index()),
               "copy", destination.device());
    return;
  }
  if (!destination.is_contiguous()) {
    throw std::invalid_argument{"Tensor value copy requires a contiguous destination"};
  }
  const Tensor materialized{source.detach().contiguous()};
  std::memcpy(AutogradAccess::host_bytes(destination), AutogradAccess::host_bytes(materialized),
              destination.nbytes());
}

void swap_storage_payloads(Tensor& original, Tensor& staged) noexcept {
  AutogradAccess::storage(original)->swap_payload(*AutogradAccess::storage(staged));
}

void validate_same_device(const Tensor& left, const Tensor& right, std::string_view operation) {
  if (left.device() != right.device()) {
    throw std::invalid_argument{std::string{operation} + " requires tensors on the same Device"};
  }
}

// tensor.cpp:549-570
Shape broadcast_shape(const Shape& left, const Shape& right) {
  const std::size_t result_rank{std::max(left.rank(), right.rank())};
  std::vector<Shape::dimension_type> dimensions(result_rank, 1);
  for (std::size_t offset{0}; offset < result_rank; ++offset) {
    const auto left_extent{offset < left.rank() ? left[left.rank() - 1 - offset]
                                                : Shape::dimension_type{1}};
    const auto right_extent{offset < right.rank() ? right[right.rank() - 1 - offset]
                                                  : Shape::dimension_type{1}};
    Shape::dimension_type result_extent{0};
    if (left_extent == right_extent) {
      result_extent = left_extent;
    } else if (left_extent == 1) {
      result_extent = right_extent;
    } else if (right_extent == 1) {
      result_extent = left_extent;
    } else {
      throw std::invalid_argument{"Tensor shapes are not broadcast-compatible"};
    }
    dimensions[result_rank - 1 - offset] = result_extent;
  }
  return Shape{std::move(dimensions)};
}

// tensor.cpp:597-632.  A gradient that already has the original shape is
// returned as is (the reference re-accumulated it into a zeroed buffer);
// otherwise the broadcast axes are summed by a deterministic device
// reduction that reads the gradient in place, contiguous or not.
Tensor reduce_gradient_to_shape(const Tensor& gradient, const Shape& original_shape) {
  if (!is_floating(gradient.dtype())) {
    throw std::logic_error{"Broadcast gradient reduction requires a floating dtype"};
  }
  if (gradient.shape() != broadcast_shape(gradient.shape(), original_shape)) {
    throw std::logic_error{"Gradient shape cannot be reduced to the requested broadcast parent shape"};
  }
  require_hip(gradient, "reduce_gradient_to_shape");
  if (gradient.shape() == original_shape) return gradient.detach();
  Tensor result{original_shape, gradient.dtype(), gradient.device()};
  // Reduced axes: leading axes, and axes where the original extent is 1.
  const std::size_t leading{gradient.rank() - original_shape.rank()};
  std::uint32_t mask{0};
  for (std::size_t axis = 0; axis < gradient.rank(); ++axis) {
    if (axis < leading) {
      mask |= 1U << axis;
    } else if (original_shape[axis - leading] == 1 && gradient.shape()[axis] != 1) {
      mask |= 1U << axis;
    }
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
