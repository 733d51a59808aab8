// Spar core types for the HIP device backend: DType, Shape, Device.
//
// Same names, values and error behaviour as the reference's modules
// spar.dtype (src/core/dtype.cppm:8-59), spar.shape (src/core/shape.cppm:10-52,
// src/core/shape.cpp:9-98) and spar.device (src/core/device.cppm:7-44), with
// the device tag HIP in place of CUDA.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <type_traits>
#include <vector>

namespace spar {

/// runtime element types supported by Spar tensors (dtype.cppm:8-13).
enum class DType : std::uint8_t {
  Float32,
  Float64,
  Int32,
  Int64,
};

/// storage bytes of one value of `dtype` (dtype.cppm:16-29).
[[nodiscard]] constexpr std::size_t size_of(DType dtype) {
  switch (dtype) {
    case DType::Float32: return sizeof(float);
    case DType::Float64: return sizeof(double);
    case DType::Int32: return sizeof(std::int32_t);
    case DType::Int64: return sizeof(std::int64_t);
  }
  throw std::invalid_argument{"Unknown Spar dtype"};
}

/// stable lowercase name (dtype.cppm:31-44).
[[nodiscard]] constexpr std::string_view name_of(DType dtype) {
  switch (dtype) {
    case DType::Float32: return "float32";
    case DType::Float64: return "float64";
    case DType::Int32: return "int32";
    case DType::Int64: return "int64";
  }
  throw std::invalid_argument{"Unknown Spar dtype"};
}

template <typename T> struct dtype_tag;
template <> struct dtype_tag<float> { static constexpr DType value = DType::Float32; };
template <> struct dtype_tag<double> { static constexpr DType value = DType::Float64; };
template <> struct dtype_tag<std::int32_t> { static constexpr DType value = DType::Int32; };
template <> struct dtype_tag<std::int64_t> { static constexpr DType value = DType::Int64; };

/// maps a C++ scalar type to its dtype (dtype.cppm:46-59).
template <typename T> [[nodiscard]] consteval DType dtype_of() {
  return dtype_tag<std::remove_cv_t<T>>::value;
}

[[nodiscard]] constexpr bool is_floating(DType dtype) {
  return dtype == DType::Float32 || dtype == DType::Float64;
}

/// a validated dense-tensor shape; `Shape{}` is the rank-zero scalar.
class Shape {
 public:
  using dimension_type = std::int64_t;
  using stride_type = std::size_t;

  Shape();
  Shape(std::initializer_list<dimension_type> dimensions);
  explicit Shape(std::vector<dimension_type> dimensions);
  Shape(const Shape&) = default;
  Shape& operator=(const Shape&) = default;
  Shape(Shape&& other) noexcept;
  Shape& operator=(Shape&& other) noexcept;

  [[nodiscard]] std::size_t rank() const noexcept;
  /// throws std::out_of_range for an invalid index.
  [[nodiscard]] dimension_type operator[](std::size_t index) const;
  [[nodiscard]] std::span<const dimension_type> dimensions() const noexcept;
  [[nodiscard]] std::size_t numel() const noexcept;
  [[nodiscard]] std::vector<stride_type> contiguous_strides() const;
  [[nodiscard]] std::string to_string() const;

  friend bool operator==(const Shape&, const Shape&) = default;

 private:
  [[nodiscard]] static stride_type checked_extent(dimension_type dimension);
  [[nodiscard]] static std::size_t compute_numel(const std::vector<dimension_type>& dimensions);

  std::vector<dimension_type> dimensions_;
  std::size_t numel_{1};
};

enum class DeviceType : std::uint8_t {
  CPU,
  HIP,
};

/// Runtime tensor placement.  HIP tensors live in MI355X HBM and are computed
/// by this backend; CPU tensors are host buffers (construction, fill, typed
/// access, layout copies and transfers).
class Device final {
 public:
  [[nodiscard]] static constexpr Device cpu() noexcept { return Device{DeviceType::CPU, 0}; }
  /// throws std::invalid_argument for a negative index (device.cpp:7-12).
  [[nodiscard]] static Device hip(std::int32_t index = 0);

  [[nodiscard]] constexpr DeviceType type() const noexcept { return type_; }
  [[nodiscard]] constexpr std::int32_t index() const noexcept { return index_; }
  [[nodiscard]] constexpr bool is_cpu() const noexcept { return type_ == DeviceType::CPU; }
  [[nodiscard]] constexpr bool is_hip() const noexcept { return type_ == DeviceType::HIP; }
  [[nodiscard]] std::string to_string() const;

  friend constexpr bool operator==(const Device&, const Device&) noexcept = default;

 private:
  constexpr Device(DeviceType type, std::int32_t index) noexcept : type_{type}, index_{index} {}

  DeviceType type_;
  std::int32_t index_;
};

/// number of visible HIP devices (0 without a GPU).
[[nodiscard]] int hip_device_count();
/// waits for all queued work on a HIP device.
void synchronize(Device device);

}  // namespace spar
