// Parameters, AdamW and the global gradient norm: the host logic of
// src/nn/parameter.cpp, src/optim/adamw.cpp and src/training/gradients.cpp
// with their validation order and messages.  Per-element work runs on the
// device: spar_hip_launch_adamw, spar_hip_launch_gradient_norm_summary and
// spar_hip_launch_scale_in_place.  The norm launches every gradient's summary
// before reading them all back with one copy per device, where the reference
// synchronises once per gradient (gradients.cpp:119).
#include "spar/optim.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>

#include "bridge.hpp"

namespace spar {

namespace nn {

// parameter.cpp:11-16
Parameter::Parameter(Tensor initial_value) : tensor_{initial_value.detach().clone()} {
  if (!is_floating(tensor_.dtype())) {
    throw std::invalid_argument{"Parameter requires a floating-point Tensor"};
  }
  tensor_.set_requires_grad();
}

const Tensor& Parameter::tensor() const noexcept { return tensor_; }

bool Parameter::requires_grad() const noexcept { return tensor_.requires_grad(); }

bool Parameter::shares_identity_with(const Parameter& other) const noexcept {
  return detail::shares_autograd_identity(tensor_, other.tensor_);
}

void Parameter::set_requires_grad(bool enabled) { tensor_.set_requires_grad(enabled); }

bool Parameter::has_grad() const noexcept { return tensor_.has_grad(); }

Tensor Parameter::grad() const { return tensor_.grad(); }

void Parameter::zero_grad() { tensor_.zero_grad(); }

Parameter Parameter::clone() const { return Parameter{tensor_}; }

}  // namespace nn

namespace training {
namespace {

namespace hip = detail::hip;
using detail::HipTensorAccess;

// gradients.cpp:14-26
std::vector<nn::Parameter*> unique_active_parameters(std::span<nn::Parameter> parameters) {
  std::vector<nn::Parameter*> unique;
  unique.reserve(parameters.size());
  for (nn::Parameter& parameter : parameters) {
    const bool duplicate{std::any_of(unique.begin(), unique.end(),
                                     [&parameter](const nn::Parameter* existing) {
                                       return existing->shares_identity_with(parameter);
                                     })};
    if (!duplicate && parameter.requires_grad() && parameter.has_grad()) {
      unique.push_back(&parameter);
    }
  }
  return unique;
}

// The combining half of StableSumSquares (gradients.cpp:57-88); the element
// half runs on the device and arrives as summaries.
struct SumSquares final {
  double scale{0.0};
  double scaled_sum_squares{1.0};
  bool has_infinity{false};
  bool has_nan{false};

  void combine(const SparHipNormSummary& other) noexcept {
    has_nan = has_nan || other.has_nan != 0;
    has_infinity = has_infinity || other.has_infinity != 0;
    if (other.scale == 0.0) return;
    if (scale == 0.0) {
      scale = other.scale;
      scaled_sum_squares = other.scaled_sum_squares;
      return;
    }
    if (scale < other.scale) {
      const double ratio{scale / other.scale};
      scaled_sum_squares = other.scaled_sum_squares + scaled_sum_squares * ratio * ratio;
      scale = other.scale;
    } else {
      const double ratio{other.scale / scale};
      scaled_sum_squares += other.scaled_sum_squares * ratio * ratio;
    }
  }

  [[nodiscard]] double norm() const noexcept {
    if (has_nan) return std::numeric_limits<double>::quiet_NaN();
    if (has_infinity) return std::numeric_limits<double>::infinity();
    return scale == 0.0 ? 0.0 : scale * std::sqrt(scaled_sum_squares);
  }
};

// gradients.cpp:108-118 and :145-155: the checks on an active gradient.
Tensor checked_gradient(const nn::Parameter& parameter, const char* operation) {
  Tensor gradient{parameter.grad()};
  if (gradient.device() != parameter.tensor().device()) {
    throw std::logic_error{"Active Parameter gradient Device mismatch"};
  }
  if (!is_floating(gradient.dtype())) {
    throw std::logic_error{"Active Parameter gradient must be floating point"};
  }
  detail::require_hip(gradient, operation);
  if (!gradient.is_contiguous()) {
    throw std::logic_error{"Active HIP Parameter gradient must be contiguous"};
  }
  return gradient;
}

// Device buffer of `count` summaries, returned to the allocator on exit.
class SummaryBuffer final {
 public:
  SummaryBuffer(std::size_t count, int device) : device_{device} {
    hip::check(spar_hip_allocate(&pointer_, count * sizeof(SparHipNormSummary), device),
               "global gradient norm", device);
  }
  SummaryBuffer(const SummaryBuffer&) = delete;
  SummaryBuffer& operator=(const SummaryBuffer&) = delete;
  ~SummaryBuffer() { static_cast<void>(spar_hip_deallocate(pointer_, device_)); }

  [[nodiscard]] SparHipNormSummary* data() const {
    return static_cast<SparHipNormSummary*>(pointer_);
  }

 private:
  void* pointer_{nullptr};
  int device_;
};

}  // namespace

double global_grad_norm(std::span<nn::Parameter> parameters) {
  std::vector<Tensor> gradients;
  for (const nn::Parameter* parameter : unique_active_parameters(parameters)) {
    gradients.push_back(checked_gradient(*parameter, "global gradient norm"));
  }
  std::map<int, std::vector<std::size_t>> by_device;
  for (std::size_t index{0}; index < gradients.size(); ++index) {
    by_device[gradients[index].device().index()].push_back(index);
  }
  std::vector<SparHipNormSummary> summaries(gradients.size());
  for (const auto& [device, indices] : by_device) {
    SummaryBuffer buffer{indices.size(), device};
    for (std::size_t slot{0}; slot < indices.size(); ++slot) {
      const Tensor& gradient{gradients[indices[slot]]};
      hip::check(spar_hip_launch_gradient_norm_summary(
                     buffer.data() + slot, HipTensorAccess::data(gradient), gradient.numel(),
                     hip::dtype_tag(gradient.dtype()), device),
                 "global gradient norm", device);
    }
    std::vector<SparHipNormSummary> host(indices.size());
    hip::check(spar_hip_copy_device_to_host(host.data(), buffer.data(),
                                            host.size() * sizeof(SparHipNormSummary), device),
               "global gradient norm", device);
    for (std::size_t slot{0}; slot < indices.size(); ++slot) summaries[indices[slot]] = host[slot];
  }
  SumSquares accumulator;
  for (const SparHipNormSummary& summary : summaries) accumulator.combine(summary);
  return accumulator.norm();
}

void scale_gradients(std::span<nn::Parameter> parameters, double factor) {
  if (!std::isfinite(factor)) throw std::invalid_argument{"Gradient scale factor must be finite"};
  std::vector<Tensor> gradients;
  for (const nn::Parameter* parameter : unique_active_parameters(parameters)) {
    gradients.push_back(checked_gradient(*parameter, "gradient scaling"));
  }
  for (Tensor& gradient : gradients) {
    hip::check(spar_hip_launch_scale_in_place(HipTensorAccess::mutable_data(gradient),
                                              gradient.numel(), hip::dtype_tag(gradient.dtype()),
                                              factor, gradient.device().index()),
               "gradient scaling", gradient.device());
  }
}

// gradients.cpp:176-190
ClipGradNormResult clip_grad_norm(std::span<nn::Parameter> parameters, double max_norm) {
  if (!std::isfinite(max_norm) || max_norm < 0.0) {
    throw std::invalid_argument{"Maximum gradient norm must be finite and nonnegative"};
  }
  const double total_norm{global_grad_norm(parameters)};
  if (!std::isfinite(total_norm)) throw std::runtime_error{"Cannot clip nonfinite gradients"};
  if (total_norm == 0.0 || total_norm <= max_norm) {
    return {.total_norm = total_norm, .scale = 1.0, .clipped = false};
  }
  const double scale{max_norm / total_norm};
  scale_gradients(parameters, scale);
  return {.total_norm = total_norm, .scale = scale, .clipped = true};
}

}  // namespace training

namespace optim {
namespace {

namespace hip = detail::hip;
using detail::HipTensorAccess;

// adamw.cpp:14-35
void validate_learning_rate(double learning_rate) {
  if (!std::isfinite(learning_rate) || learning_rate < 0.0) {
    throw std::invalid_argument{"AdamW learning_rate must be finite and nonnegative"};
  }
}

void validate_hyperparameters(double learning_rate, double beta1, double beta2, double epsilon,
                              double weight_decay) {
  validate_learning_rate(learning_rate);
  if (!std::isfinite(beta1) || beta1 < 0.0 || beta1 >= 1.0) {
    throw std::invalid_argument{"AdamW beta1 must be finite and in [0,1)"};
  }
  if (!std::isfinite(beta2) || beta2 < 0.0 || beta2 >= 1.0) {
    throw std::invalid_argument{"AdamW beta2 must be finite and in [0,1)"};
  }
  if (!std::isfinite(epsilon) || epsilon <= 0.0) {
    throw std::invalid_argument{"AdamW epsilon must be finite and positive"};
  }
  if (!std::isfinite(weight_decay) || weight_decay < 0.0) {
    throw std::invalid_argument{"AdamW weight_decay must be finite and nonnegative"};
  }
}

bool same_layout(const Tensor& tensor, const Tensor& reference) {
  return tensor.shape() == reference.shape() && tensor.dtype() == reference.dtype() &&
         tensor.device() == reference.device();
}

}  // namespace

AdamW::AdamW(std::vector<nn::Parameter> parameters, double learning_rate, double beta1,
             double beta2, double epsilon, double weight_decay)
    : learning_rate_{learning_rate},
      beta1_{beta1},
      beta2_{beta2},
      epsilon_{epsilon},
      weight_decay_{weight_decay} {
  validate_hyperparameters(learning_rate, beta1, beta2, epsilon, weight_decay);
  entries_.reserve(parameters.size());
  for (auto& parameter : parameters) {
    const bool duplicate{std::any_of(entries_.begin(), entries_.end(),
                                     [&parameter](const Entry& entry) {
                                       return entry.parameter.shares_identity_with(parameter);
                                     })};
    if (!duplicate) entries_.push_back(Entry{std::move(parameter), std::nullopt});
  }
}

// adamw.cpp:83-170: validate every active entry, stage new states, then
// update each Parameter with one kernel.
void AdamW::step() {
  std::vector<std::size_t> active;
  active.reserve(entries_.size());
  for (std::size_t index{0}; index < entries_.size(); ++index) {
    const Entry& entry{entries_[index]};
    const nn::Parameter& parameter{entry.parameter};
    if (!parameter.requires_grad() || !parameter.has_grad()) continue;
    const Tensor gradient{parameter.grad()};
    if (!same_layout(gradient, parameter.tensor())) {
      throw std::logic_error{"AdamW gradient shape, dtype, or Device does not match its Parameter"};
    }
    if (!is_floating(parameter.tensor().dtype())) {
      throw std::logic_error{"AdamW encountered a non-floating Parameter"};
    }
    if (!parameter.tensor().is_contiguous() || !gradient.is_contiguous()) {
      throw std::logic_error{"AdamW requires contiguous Parameters and gradients"};
    }
    if (entry.state) {
      const State& state{*entry.state};
      for (const Tensor* moment : {&state.first_moment, &state.second_moment}) {
        if (!same_layout(*moment, parameter.tensor()) || !moment->is_contiguous()) {
          throw std::logic_error{"AdamW state shape, dtype, or Device does not match its Parameter"};
        }
      }
      if (state.step == 0) throw std::logic_error{"AdamW initialized state has an invalid zero step"};
      if (state.step == std::numeric_limits<std::uint64_t>::max()) {
        throw std::overflow_error{"AdamW per-Parameter step counter overflow"};
      }
    }
    detail::require_hip(parameter.tensor(), "AdamW update");
    active.push_back(index);
  }

  std::vector<std::optional<std::pair<Tensor, Tensor>>> staged(entries_.size());
  for (const std::size_t index : active) {
    const Tensor& value{entries_[index].parameter.tensor()};
    if (!entries_[index].state) {
      staged[index].emplace(zeros(value.shape(), value.dtype(), value.device()),
                            zeros(value.shape(), value.dtype(), value.device()));
    }
  }
  for (const std::size_t index : active) {
    if (staged[index]) {
      entries_[index].state.emplace(State{std::move(staged[index]->first),
                                          std::move(staged[index]->second), 0});
    }
  }

  for (const std::size_t index : active) {
    Entry& entry{entries_[index]};
    const Tensor gradient{entry.parameter.grad()};
    State& state{*entry.state};
    ++state.step;
    Tensor values{entry.parameter.tensor().detach()};
    // cuda_ops.cppm:675-676: bias corrections on the host.
    const double first_correction{1.0 - std::pow(beta1_, static_cast<double>(state.step))};
    const double second_correction{1.0 - std::pow(beta2_, static_cast<double>(state.step))};
    hip::check(spar_hip_launch_adamw(HipTensorAccess::mutable_data(values),
                                     HipTensorAccess::data(gradient),
                                     HipTensorAccess::mutable_data(state.first_moment),
                                     HipTensorAccess::mutable_data(state.second_moment),
                                     values.numel(), hip::dtype_tag(values.dtype()),
                                     learning_rate_, beta1_, beta2_, epsilon_, weight_decay_,
                                     first_correction, second_correction,
                                     values.device().index()),
               "AdamW update", values.device());
  }
}

void AdamW::zero_grad() {
  for (Entry& entry : entries_) entry.parameter.zero_grad();
}

std::size_t AdamW::parameter_count() const noexcept { return entries_.size(); }
double AdamW::learning_rate() const noexcept { return learning_rate_; }

void AdamW::set_learning_rate(double learning_rate) {
  validate_learning_rate(learning_rate);
  learning_rate_ = learning_rate;
}

double AdamW::beta1() const noexcept { return beta1_; }
double AdamW::beta2() const noexcept { return beta2_; }
double AdamW::epsilon() const noexcept { return epsilon_; }
double AdamW::weight_decay() const noexcept { return weight_decay_; }

bool AdamW::tracks(const nn::Parameter& parameter) const noexcept {
  return std::any_of(entries_.begin(), entries_.end(), [&parameter](const Entry& entry) {
    return entry.parameter.shares_identity_with(parameter);
  });
}

// adamw.cpp:230-243
std::optional<AdamWParameterState> AdamW::parameter_state(const nn::Parameter& parameter) const {
  const auto iterator{std::find_if(entries_.begin(), entries_.end(), [&parameter](const Entry& entry) {
    return entry.parameter.shares_identity_with(parameter);
  })};
  if (iterator == entries_.end()) {
    throw std::invalid_argument{"AdamW does not track the requested Parameter"};
  }
  if (!iterator->state) return std::nullopt;
  return AdamWParameterState{iterator->state->first_moment.detach().clone(),
                             iterator->state->second_moment.detach().clone(),
                             iterator->state->step};
}

// adamw.cpp:245-272
void AdamW::set_parameter_state(const nn::Parameter& parameter,
                                std::optional<AdamWParameterState> state) {
  const auto iterator{std::find_if(entries_.begin(), entries_.end(), [&parameter](const Entry& entry) {
    return entry.parameter.shares_identity_with(parameter);
  })};
  if (iterator == entries_.end()) {
    throw std::invalid_argument{"AdamW does not track the requested Parameter"};
  }
  if (!state) {
    iterator->state.reset();
    return;
  }
  if (state->step == 0) throw std::invalid_argument{"AdamW restored state step must be at least one"};
  for (const Tensor* moment : {&state->first_moment, &state->second_moment}) {
    if (!same_layout(*moment, parameter.tensor())) {
      throw std::invalid_argument{"AdamW restored moment shape, dtype, or Device mismatch"};
    }
    if (!is_floating(moment->dtype())) {
      throw std::invalid_argument{"AdamW restored moments must be floating point"};
    }
  }
  iterator->state.emplace(State{state->first_moment.detach().clone(),
                                state->second_moment.detach().clone(), state->step});
}

}  // namespace optim
}  // namespace spar
