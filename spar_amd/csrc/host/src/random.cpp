// SplitMix64 generator (src/core/random.cpp:12-80) with device-side
// generation of the same streams.
#include "spar/random.hpp"

#include <cmath>

#include "autograd_internal.hpp"
#include "bridge.hpp"

namespace spar {

Random::Random(std::uint64_t seed) noexcept : state_{seed} {}

std::uint64_t Random::state() const noexcept { return state_; }

void Random::set_state(std::uint64_t state) noexcept { state_ = state; }

std::uint64_t Random::next_u64() noexcept {
  state_ += 0x9E3779B97F4A7C15ULL;
  auto value{state_};
  value = (value ^ (value >> 30U)) * 0xBF58476D1CE4E5B9ULL;
  value = (value ^ (value >> 27U)) * 0x94D049BB133111EBULL;
  return value ^ (value >> 31U);
}

float Random::uniform_float() noexcept {
  constexpr float denominator{16'777'216.0F};
  return static_cast<float>(next_u64() >> 40U) / denominator;
}

double Random::uniform_double() noexcept {
  constexpr double denominator{9'007'199'254'740'992.0};
  return static_cast<double>(next_u64() >> 11U) / denominator;
}

void Random::skip(std::uint64_t draws) noexcept { state_ += draws * 0x9E3779B97F4A7C15ULL; }

namespace {

void validate_float(DType dtype, const char* name) {
  switch (dtype) {
    case DType::Float32:
    case DType::Float64: return;
    case DType::Int32:
    case DType::Int64:
      throw std::invalid_argument{std::string{name} + " currently supports floating-point dtypes only"};
  }
  throw std::invalid_argument{std::string{name} + " received an unknown dtype"};
}

}  // namespace

Tensor random_uniform(Shape shape, DType dtype, Random& random, double low, double high,
                      Device device) {
  if (!(low < high)) throw std::invalid_argument{"random_uniform requires low < high"};
  validate_float(dtype, "random_uniform");
  if (device.is_hip()) {
    Tensor tensor{std::move(shape), dtype, device};
    if (tensor.numel() != 0) {
      detail::hip::check(spar_hip_random_uniform(detail::HipTensorAccess::mutable_data(tensor),
                                                 tensor.numel(), detail::hip::dtype_tag(dtype),
                                                 random.state(), low, high, device.index()),
                         "random_uniform", device);
    }
    random.skip(tensor.numel());
    return tensor;
  }
  Tensor tensor{std::move(shape), dtype};
  if (dtype == DType::Float32) {
    const auto low_value{static_cast<float>(low)};
    const auto width{static_cast<float>(high - low)};
    for (auto& value : tensor.span<float>()) value = low_value + width * random.uniform_float();
  } else {
    const auto width{high - low};
    for (auto& value : tensor.span<double>()) value = low + width * random.uniform_double();
  }
  return tensor;
}

Tensor random_normal(Shape shape, DType dtype, Random& random, double mean, double stddev,
                     Device device) {
  if (!(stddev >= 0.0)) throw std::invalid_argument{"random_normal requires stddev >= 0"};
  validate_float(dtype, "random_normal");
  if (device.is_hip()) {
    Tensor tensor{std::move(shape), dtype, device};
    const std::uint64_t pairs{(tensor.numel() + 1) / 2};
    if (tensor.numel() != 0) {
      detail::hip::check(spar_hip_random_normal(detail::HipTensorAccess::mutable_data(tensor),
                                                tensor.numel(), detail::hip::dtype_tag(dtype),
                                                random.state(), mean, stddev, device.index()),
                         "random_normal", device);
    }
    random.skip(2 * pairs);
    return tensor;
  }
  Tensor tensor{std::move(shape), dtype};
  const std::size_t count{tensor.numel()};
  constexpr double two_pi{6.283185307179586476925286766559};
  auto write = [&](auto values) {
    for (std::size_t k = 0; 2 * k < count; ++k) {
      const double u0{random.uniform_double()};
      const double u1{random.uniform_double()};
      const double radius{std::sqrt(-2.0 * std::log(1.0 - u0))};
      const double angle{two_pi * u1};
      using T = typename decltype(values)::element_type;
      values[2 * k] = static_cast<T>(mean + stddev * (radius * std::cos(angle)));
      if (2 * k + 1 < count) values[2 * k + 1] = static_cast<T>(mean + stddev * (radius * std::sin(angle)));
    }
  };
  if (dtype == DType::Float32) {
    write(tensor.span<float>());
  } else {
    write(tensor.span<double>());
  }
  return tensor;
}

}  // namespace spar
