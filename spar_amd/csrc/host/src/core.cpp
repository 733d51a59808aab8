// Shape (src/core/shape.cpp:9-98), Device (src/core/device.cpp:7-12) and the
// C-ABI bridge helpers.
#include <limits>
#include <string>
#include <utility>

#include "bridge.hpp"
#include "spar/core.hpp"

namespace spar {

Shape::Shape() = default;

Shape::Shape(std::initializer_list<dimension_type> dimensions)
    : Shape{std::vector<dimension_type>{dimensions}} {}

Shape::Shape(std::vector<dimension_type> dimensions)
    : dimensions_{std::move(dimensions)}, numel_{compute_numel(dimensions_)} {}

Shape::Shape(Shape&& other) noexcept
    : dimensions_{std::move(other.dimensions_)}, numel_{other.numel_} {
  other.dimensions_.clear();
  other.numel_ = 0;
}

Shape& Shape::operator=(Shape&& other) noexcept {
  if (this != &other) {
    dimensions_ = std::move(other.dimensions_);
    numel_ = other.numel_;
    other.dimensions_.clear();
    other.numel_ = 0;
  }
  return *this;
}

std::size_t Shape::rank() const noexcept { return dimensions_.size(); }

Shape::dimension_type Shape::operator[](std::size_t index) const { return dimensions_.at(index); }

std::span<const Shape::dimension_type> Shape::dimensions() const noexcept { return dimensions_; }

std::size_t Shape::numel() const noexcept { return numel_; }

std::string Shape::to_string() const {
  std::string text{"["};
  for (std::size_t i = 0; i < dimensions_.size(); ++i) {
    if (i != 0) text += ", ";
    text += std::to_string(dimensions_[i]);
  }
  return text + "]";
}

Shape::stride_type Shape::checked_extent(dimension_type dimension) {
  if (dimension < 0) throw std::invalid_argument{"Shape dimensions cannot be negative"};
  return static_cast<stride_type>(dimension);
}

// Row-major strides: each axis steps over the elements of the axes inside it.
// The running product is formed over every axis, the outermost included, and
// reports overflow as the reference does (shape.cpp:61-75).
std::vector<Shape::stride_type> Shape::contiguous_strides() const {
  std::vector<stride_type> strides(rank());
  stride_type inside{1};
  for (std::size_t axis{rank()}; axis-- > 0;) {
    strides[axis] = inside;
    if (__builtin_mul_overflow(inside, checked_extent(dimensions_[axis]), &inside)) {
      throw std::overflow_error{"Shape stride calculation overflow"};
    }
  }
  return strides;
}

// Number of elements.  Every extent is validated first (a negative one is an
// invalid_argument wherever it appears); a zero extent makes the shape empty
// whatever the other extents are; only a non-empty product can overflow.
std::size_t Shape::compute_numel(const std::vector<dimension_type>& dimensions) {
  std::size_t count{1};
  bool overflowed{false};
  bool empty{false};
  for (const auto dimension : dimensions) {
    const stride_type extent{checked_extent(dimension)};
    empty = empty || extent == 0;
    overflowed = overflowed || (!empty && __builtin_mul_overflow(count, extent, &count));
  }
  if (empty) return 0;
  if (overflowed) throw std::overflow_error{"Shape element count overflow"};
  return count;
}

Device Device::hip(std::int32_t index) {
  if (index < 0) throw std::invalid_argument{"HIP device index must be nonnegative"};
  return Device{DeviceType::HIP, index};
}

std::string Device::to_string() const {
  return is_cpu() ? std::string{"cpu"} : "hip:" + std::to_string(index_);
}

int hip_device_count() {
  int count = 0;
  const SparHipStatus status = spar_hip_device_count(&count);
  return status.code == 0 ? count : 0;
}

void synchronize(Device device) {
  if (device.is_hip()) {
    detail::hip::check(spar_hip_synchronize(device.index()), "synchronize", device);
  }
}

}  // namespace spar

namespace spar::detail::hip {

void check(SparHipStatus status, std::string_view operation, int device) {
  if (status.code == 0) return;
  const char* message = spar_hip_error_string(status.hip_error);
  throw std::runtime_error{std::string{operation} + " failed on hip:" + std::to_string(device) +
                           ": " + (message == nullptr ? "unknown HIP error" : message) +
                           " (code " + std::to_string(status.code) + ", hip error " +
                           std::to_string(status.hip_error) + ")"};
}

void check(SparHipStatus status, std::string_view operation, Device device) {
  check(status, operation, device.index());
}

int dtype_tag(DType dtype) {
  switch (dtype) {
    case DType::Float32: return SPAR_HIP_FLOAT32;
    case DType::Float64: return SPAR_HIP_FLOAT64;
    case DType::Int32: return SPAR_HIP_INT32;
    case DType::Int64: return SPAR_HIP_INT64;
  }
  throw std::logic_error{"unknown dtype"};
}

std::vector<std::uint64_t> extents_of(const Shape& shape) {
  std::vector<std::uint64_t> extents(shape.rank());
  for (std::size_t axis = 0; axis < shape.rank(); ++axis) {
    extents[axis] = static_cast<std::uint64_t>(shape[axis]);
  }
  return extents;
}

View view_of(const Tensor& tensor) {
  View view;
  view.extents = extents_of(tensor.shape());
  view.strides.assign(tensor.strides().begin(), tensor.strides().end());
  view.offset = tensor.storage_offset();
  return view;
}

View expanded_view(const Tensor& tensor, const Shape& shape) {
  // core/tensor.cpp:313-342 (expand) without creating a Tensor
  View view;
  view.extents = extents_of(shape);
  view.strides.assign(shape.rank(), 0);
  view.offset = tensor.storage_offset();
  const std::size_t leading = shape.rank() - tensor.rank();
  for (std::size_t axis = 0; axis < tensor.rank(); ++axis) {
    if (tensor.shape()[axis] == shape[leading + axis]) {
      view.strides[leading + axis] = tensor.strides()[axis];
    } else if (tensor.shape()[axis] != 1) {
      throw std::invalid_argument{"expand dimensions are not broadcast-compatible"};
    }
  }
  return view;
}

}  // namespace spar::detail::hip
