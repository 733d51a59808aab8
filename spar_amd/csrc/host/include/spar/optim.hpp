// Trainable parameters, the AdamW optimizer and the global gradient norm on
// HIP tensors, with the reference's names, argument meaning and exceptions:
// spar.nn.parameter (src/nn/parameter.cppm:8-31), spar.optim.adamw
// (src/optim/adamw.cppm:8-62) and spar.training.gradients
// (src/training/gradients.cppm:6-26).  The per-element work runs in the
// backend's AdamW, norm-summary and scaling kernels.  Parameters and
// optimizer state migrate between the host and HIP devices with
// nn::move_to and AdamW::move_to (src/nn/parameter.cpp:54-87,
// src/optim/adamw.cpp:172-190).
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <span>
#include <vector>

#include "spar/tensor.hpp"

namespace spar::nn {

/// A trainable floating-point leaf Tensor.  Copies share value/gradient
/// identity; clone() creates an independent leaf (parameter.cpp:11-49).
class Parameter {
 public:
  /// detaches and clones `initial_value`, which must be Float32 or Float64,
  /// and enables gradient tracking.
  explicit Parameter(Tensor initial_value);

  [[nodiscard]] const Tensor& tensor() const noexcept;
  [[nodiscard]] bool requires_grad() const noexcept;
  [[nodiscard]] bool shares_identity_with(const Parameter& other) const noexcept;
  void set_requires_grad(bool enabled);
  [[nodiscard]] bool has_grad() const noexcept;
  [[nodiscard]] Tensor grad() const;
  void zero_grad();
  /// an independent trainable leaf with copied values and no gradient.
  [[nodiscard]] Parameter clone() const;

 private:
  friend void move_to(Parameter& parameter, Device target);
  friend void move_to(std::span<Parameter> parameters, Device target);
  Tensor tensor_;
};

/// Moves a Parameter's values to `target` in place: its Tensor, autograd
/// and Storage identities are kept (parameter.cppm:33-39).  Refused with
/// std::logic_error while the Parameter holds a gradient.
void move_to(Parameter& parameter, Device target);

/// Moves every distinct Parameter (aliases once) to `target`.  All copies
/// are made before any Parameter changes, so a failure changes nothing.
void move_to(std::span<Parameter> parameters, Device target);

}  // namespace spar::nn

namespace spar::training {

/// The stable global L2 norm over unique active Parameters (those that
/// require gradients and hold one), gradients.cpp:105-137.
[[nodiscard]] double global_grad_norm(std::span<nn::Parameter> parameters);

/// Scales each unique active Parameter's gradient storage once, in place:
/// g = (T)((double)g * factor); factor must be finite (gradients.cpp:139-174).
void scale_gradients(std::span<nn::Parameter> parameters, double factor);

struct ClipGradNormResult final {
  double total_norm;
  double scale;
  bool clipped;
};

/// Computes the global norm, then scales by max_norm / norm only when the
/// norm exceeds max_norm.  A nonfinite norm throws before any gradient is
/// modified (gradients.cpp:176-190).
[[nodiscard]] ClipGradNormResult clip_grad_norm(std::span<nn::Parameter> parameters,
                                                double max_norm);

}  // namespace spar::training

namespace spar::optim {

struct AdamWParameterState final {
  Tensor first_moment;
  Tensor second_moment;
  std::uint64_t step;
};

/// Decoupled-weight-decay Adam (adamw.cppm:14-62, adamw.cpp:67-272): per
/// Parameter moments and step counter, updated by one fused kernel per
/// Parameter whose double-precision arithmetic matches the CPU loop's bits.
class AdamW {
 public:
  explicit AdamW(std::vector<nn::Parameter> parameters = {}, double learning_rate = 1.0e-3,
                 double beta1 = 0.9, double beta2 = 0.999, double epsilon = 1.0e-8,
                 double weight_decay = 0.01);

  AdamW(const AdamW&) = delete;
  AdamW& operator=(const AdamW&) = delete;
  AdamW(AdamW&&) noexcept = default;
  AdamW& operator=(AdamW&&) noexcept = default;

  void step();
  void zero_grad();
  /// Moves the optimizer moments and every tracked Parameter to `target`;
  /// the moments are copied before any Parameter moves, and committed only
  /// after all of them have (adamw.cppm:25-26).
  void move_to(Device target);

  [[nodiscard]] std::size_t parameter_count() const noexcept;
  [[nodiscard]] double learning_rate() const noexcept;
  void set_learning_rate(double learning_rate);
  [[nodiscard]] double beta1() const noexcept;
  [[nodiscard]] double beta2() const noexcept;
  [[nodiscard]] double epsilon() const noexcept;
  [[nodiscard]] double weight_decay() const noexcept;

  [[nodiscard]] bool tracks(const nn::Parameter& parameter) const noexcept;
  [[nodiscard]] std::optional<AdamWParameterState> parameter_state(
      const nn::Parameter& parameter) const;
  void set_parameter_state(const nn::Parameter& parameter,
                           std::optional<AdamWParameterState> state);

 private:
  struct State final {
    Tensor first_moment;
    Tensor second_moment;
    std::uint64_t step;
  };

  struct Entry final {
    nn::Parameter parameter;
    std::optional<State> state;
  };

  // The entry tracking `parameter` (same identity), or null.
  [[nodiscard]] const Entry* entry_of(const nn::Parameter& parameter) const noexcept;
  // Whether `entry` takes part in a step; throws if it cannot.
  [[nodiscard]] static bool steps(const Entry& entry);
  // One fused update of `entry`'s Parameter and moments.
  void update(Entry& entry) const;

  std::vector<Entry> entries_;
  double learning_rate_;
  double beta1_;
  double beta2_;
  double epsilon_;
  double weight_decay_;
};

}  // namespace spar::optim
