// Spar's deterministic generator (src/core/random.cppm:8-34) plus a normal
// sampler and device-side generation of the same streams.
#pragma once

#include <cstdint>

#include "spar/tensor.hpp"

namespace spar {

/// explicit SplitMix64 generator state (random.cpp:12-38).
class Random {
 public:
  explicit Random(std::uint64_t seed) noexcept;

  [[nodiscard]] std::uint64_t state() const noexcept;
  void set_state(std::uint64_t state) noexcept;

  [[nodiscard]] std::uint64_t next_u64() noexcept;
  /// float in [0, 1) from the top 24 bits.
  [[nodiscard]] float uniform_float() noexcept;
  /// double in [0, 1) from the top 53 bits.
  [[nodiscard]] double uniform_double() noexcept;
  /// advances the state past `draws` draws.
  void skip(std::uint64_t draws) noexcept;

 private:
  std::uint64_t state_;
};

/// uniform samples in [low, high) (random.cpp:40-80).  On a HIP device the
/// kernel produces the same bits as the host loop and `random` advances by
/// the same number of draws.
[[nodiscard]] Tensor random_uniform(Shape shape, DType dtype, Random& random, double low = 0.0,
                                    double high = 1.0, Device device = Device::cpu());

/// addition: normal samples by Box-Muller on pairs of uniform_double draws
/// (element 2k from cos, 2k+1 from sin), computed in double.
[[nodiscard]] Tensor random_normal(Shape shape, DType dtype, Random& random, double mean = 0.0,
                                   double stddev = 1.0, Device device = Device::cpu());

}  // namespace spar
