// Parameters, AdamW, the global gradient norm and gradient scaling on HIP
// tensors.  Names, validation order, messages and exception types are
// Spar's (src/nn/parameter.cpp, src/optim/adamw.cpp,
// src/training/gradients.cpp); the per-element work runs in the backend's
// kernels (spar_hip_launch_adamw, spar_hip_launch_gradient_norm_summary,
// spar_hip_launch_scale_in_place).  The norm enqueues every gradient's
// summary before one read-back per device, where the reference synchronises
// once per gradient (gradients.cpp:119).
#include "spar/optim.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <map>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <utility>

#include "autograd_internal.hpp"
#include "bridge.hpp"

namespace spar {
namespace {

namespace hip = detail::hip;
using detail::HipTensorAccess;

// The autograd identity a Parameter and all its copies share.
const void* identity_of(const nn::Parameter& parameter) {
  return detail::TensorInternals::grad_state(parameter.tensor()).get();
}

// Parameters in first-occurrence order, each identity once, filtered by
// `keep`.  A hash set of identities replaces the pairwise identity scan.
template <typename Keep>
std::vector<nn::Parameter*> distinct(std::span<nn::Parameter> parameters, Keep keep) {
  std::vector<nn::Parameter*> result;
  std::unordered_set<const void*> seen;
  for (nn::Parameter& parameter : parameters) {
    if (keep(parameter) && seen.insert(identity_of(parameter)).second) {
      result.push_back(&parameter);
    }
  }
  return result;
}

bool active(const nn::Parameter& parameter) {
  return parameter.requires_grad() && parameter.has_grad();
}

bool matches(const Tensor& tensor, const Tensor& model) {
  return tensor.shape() == model.shape() && tensor.dtype() == model.dtype() &&
         tensor.device() == model.device();
}

}  // namespace

namespace nn {

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

void move_to(Parameter& parameter, Device target) {
  move_to(std::span<Parameter>{&parameter, 1}, target);
}

// Two phases: every copy is made first (a failure leaves all Parameters as
// they were), then each Parameter's Storage takes the copy's payload, which
// cannot fail.  Tensor, autograd and Storage objects keep their identity.
void move_to(std::span<Parameter> parameters, Device target) {
  const auto movers{distinct(parameters, [target](const Parameter& parameter) {
    return parameter.tensor_.device() != target;
  })};
  for (const Parameter* parameter : movers) {
    if (parameter->has_grad()) {
      throw std::logic_error{"Parameter Device migration requires clearing its live gradient first"};
    }
  }
  std::vector<Tensor> copies;
  copies.reserve(movers.size());
  for (const Parameter* parameter : movers) copies.push_back(parameter->tensor_.detach().to(target));
  for (std::size_t k{0}; k < movers.size(); ++k) {
    detail::swap_storage_payloads(movers[k]->tensor_, copies[k]);
  }
}

}  // namespace nn

namespace training {
namespace {

// The running value of Spar's StableSumSquares (gradients.cpp:28-88) over
// whole gradients: every element arrives from the device already folded
// into a per-gradient summary, and summaries merge in Parameter order.
struct NormTotal final {
  double scale{0.0};
  double scaled_sum_squares{1.0};
  bool has_infinity{false};
  bool has_nan{false};
};

// Merges a summary into the total.  The summary with the larger scale (the
// total on a tie) keeps its sum; the other's sum is rescaled by the square
// of the ratio of scales before the addition: big + (small * r) * r.
void merge(NormTotal& total, const SparHipNormSummary& summary) {
  total.has_nan = total.has_nan || summary.has_nan != 0;
  total.has_infinity = total.has_infinity || summary.has_infinity != 0;
  if (summary.scale == 0.0) return;
  if (total.scale == 0.0) {
    total.scale = summary.scale;
    total.scaled_sum_squares = summary.scaled_sum_squares;
    return;
  }
  const bool summary_larger{total.scale < summary.scale};
  const double big_scale{summary_larger ? summary.scale : total.scale};
  const double big_sum{summary_larger ? summary.scaled_sum_squares : total.scaled_sum_squares};
  const double small_scale{summary_larger ? total.scale : summary.scale};
  const double small_sum{summary_larger ? total.scaled_sum_squares : summary.scaled_sum_squares};
  const double ratio{small_scale / big_scale};
  total.scale = big_scale;
  total.scaled_sum_squares = big_sum + small_sum * ratio * ratio;
}

double norm_of(const NormTotal& total) {
  if (total.has_nan) return std::numeric_limits<double>::quiet_NaN();
  if (total.has_infinity) return std::numeric_limits<double>::infinity();
  if (total.scale == 0.0) return 0.0;
  return total.scale * std::sqrt(total.scaled_sum_squares);
}

// An active Parameter's gradient after the reference's checks
// (gradients.cpp:108-118, :145-155).
Tensor checked_gradient(const nn::Parameter& parameter, std::string_view operation) {
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

std::vector<Tensor> checked_gradients(std::span<nn::Parameter> parameters,
                                      std::string_view operation) {
  std::vector<Tensor> gradients;
  for (const nn::Parameter* parameter : distinct(parameters, active)) {
    gradients.push_back(checked_gradient(*parameter, operation));
  }
  return gradients;
}

// Device memory for the summaries, returned to the allocator on scope exit.
class SummarySlots final {
 public:
  SummarySlots(std::size_t count, int device) : device_{device} {
    hip::check(spar_hip_allocate(&block_, count * sizeof(SparHipNormSummary), device),
               "global gradient norm", device);
  }
  SummarySlots(const SummarySlots&) = delete;
  SummarySlots& operator=(const SummarySlots&) = delete;
  ~SummarySlots() { static_cast<void>(spar_hip_deallocate(block_, device_)); }
  [[nodiscard]] SparHipNormSummary* at(std::size_t k) const {
    return static_cast<SparHipNormSummary*>(block_) + k;
  }

 private:
  void* block_{nullptr};
  int device_;
};

// Summaries of the given gradients (all on `device`), computed into one
// device array and read back with one copy.
std::vector<SparHipNormSummary> device_summaries(const std::vector<const Tensor*>& gradients,
                                                 int device) {
  const SummarySlots slots{gradients.size(), device};
  for (std::size_t k{0}; k < gradients.size(); ++k) {
    const Tensor& gradient{*gradients[k]};
    hip::check(spar_hip_launch_gradient_norm_summary(slots.at(k), HipTensorAccess::data(gradient),
                                                     gradient.numel(),
                                                     hip::dtype_tag(gradient.dtype()), device),
               "global gradient norm", device);
  }
  std::vector<SparHipNormSummary> host(gradients.size());
  hip::check(spar_hip_copy_device_to_host(host.data(), slots.at(0),
                                          host.size() * sizeof(SparHipNormSummary), device),
             "global gradient norm", device);
  return host;
}

}  // namespace

double global_grad_norm(std::span<nn::Parameter> parameters) {
  const std::vector<Tensor> gradients{checked_gradients(parameters, "global gradient norm")};
  std::map<int, std::vector<std::size_t>> by_device;
  for (std::size_t k{0}; k < gradients.size(); ++k) {
    by_device[gradients[k].device().index()].push_back(k);
  }
  std::vector<SparHipNormSummary> summaries(gradients.size());
  for (const auto& [device, members] : by_device) {
    std::vector<const Tensor*> group;
    for (const std::size_t k : members) group.push_back(&gradients[k]);
    const auto results{device_summaries(group, device)};
    for (std::size_t j{0}; j < members.size(); ++j) summaries[members[j]] = results[j];
  }
  NormTotal total;
  for (const SparHipNormSummary& summary : summaries) merge(total, summary);
  return norm_of(total);
}

void scale_gradients(std::span<nn::Parameter> parameters, double factor) {
  if (!std::isfinite(factor)) throw std::invalid_argument{"Gradient scale factor must be finite"};
  std::vector<Tensor> gradients{checked_gradients(parameters, "gradient scaling")};
  for (Tensor& gradient : gradients) {
    hip::check(spar_hip_launch_scale_in_place(HipTensorAccess::mutable_data(gradient),
                                              gradient.numel(), hip::dtype_tag(gradient.dtype()),
                                              factor, gradient.device().index()),
               "gradient scaling", gradient.device());
  }
}

ClipGradNormResult clip_grad_norm(std::span<nn::Parameter> parameters, double max_norm) {
  if (!std::isfinite(max_norm) || max_norm < 0.0) {
    throw std::invalid_argument{"Maximum gradient norm must be finite and nonnegative"};
  }
  ClipGradNormResult result{global_grad_norm(parameters), 1.0, false};
  if (!std::isfinite(result.total_norm)) {
    throw std::runtime_error{"Cannot clip nonfinite gradients"};
  }
  if (result.total_norm > max_norm) {  // a zero norm never exceeds max_norm >= 0
    result.scale = max_norm / result.total_norm;
    result.clipped = true;
    scale_gradients(parameters, result.scale);
  }
  return result;
}

}  // namespace training

namespace optim {
namespace {

void check_learning_rate(double value) {
  if (!std::isfinite(value) || value < 0.0) {
    throw std::invalid_argument{"AdamW learning_rate must be finite and nonnegative"};
  }
}

// The hyperparameter rules of adamw.cpp:14-35, in their order.
void check_hyperparameters(double learning_rate, double beta1, double beta2, double epsilon,
                           double weight_decay) {
  check_learning_rate(learning_rate);
  const auto unit_interval = [](double beta) {
    return std::isfinite(beta) && beta >= 0.0 && beta < 1.0;
  };
  if (!unit_interval(beta1)) throw std::invalid_argument{"AdamW beta1 must be finite and in [0,1)"};
  if (!unit_interval(beta2)) throw std::invalid_argument{"AdamW beta2 must be finite and in [0,1)"};
  if (!std::isfinite(epsilon) || epsilon <= 0.0) {
    throw std::invalid_argument{"AdamW epsilon must be finite and positive"};
  }
  if (!std::isfinite(weight_decay) || weight_decay < 0.0) {
    throw std::invalid_argument{"AdamW weight_decay must be finite and nonnegative"};
  }
}

}  // namespace

AdamW::AdamW(std::vector<nn::Parameter> parameters, double learning_rate, double beta1,
             double beta2, double epsilon, double weight_decay)
    : learning_rate_{learning_rate}, beta1_{beta1}, beta2_{beta2}, epsilon_{epsilon},
      weight_decay_{weight_decay} {
  check_hyperparameters(learning_rate, beta1, beta2, epsilon, weight_decay);
  for (nn::Parameter* parameter :
       distinct(std::span<nn::Parameter>{parameters}, [](const nn::Parameter&) { return true; })) {
    entries_.push_back(Entry{std::move(*parameter), std::nullopt});
  }
}

const AdamW::Entry* AdamW::entry_of(const nn::Parameter& parameter) const noexcept {
  const void* identity{identity_of(parameter)};
  if (identity == nullptr) return nullptr;
  const auto found{std::find_if(entries_.begin(), entries_.end(), [identity](const Entry& entry) {
    return identity_of(entry.parameter) == identity;
  })};
  return found == entries_.end() ? nullptr : &*found;
}

// adamw.cpp:85-124: an entry steps when its Parameter requires a gradient
// and holds one; its gradient, state and placement are checked first.
bool AdamW::steps(const Entry& entry) {
  const nn::Parameter& parameter{entry.parameter};
  if (!active(parameter)) return false;
  const Tensor& value{parameter.tensor()};
  const Tensor gradient{parameter.grad()};
  if (!matches(gradient, value)) {
    throw std::logic_error{"AdamW gradient shape, dtype, or Device does not match its Parameter"};
  }
  if (!is_floating(value.dtype())) {
    throw std::logic_error{"AdamW encountered a non-floating Parameter"};
  }
  if (!value.is_contiguous() || !gradient.is_contiguous()) {
    throw std::logic_error{"AdamW requires contiguous Parameters and gradients"};
  }
  if (const auto& state{entry.state}) {
    for (const Tensor* moment : {&state->first_moment, &state->second_moment}) {
      if (!matches(*moment, value) || !moment->is_contiguous()) {
        throw std::logic_error{"AdamW state shape, dtype, or Device does not match its Parameter"};
      }
    }
    if (state->step == 0) throw std::logic_error{"AdamW initialized state has an invalid zero step"};
    if (state->step == std::numeric_limits<std::uint64_t>::max()) {
      throw std::overflow_error{"AdamW per-Parameter step counter overflow"};
    }
  }
  detail::require_hip(value, "AdamW update");
  return true;
}

void AdamW::update(Entry& entry) const {
  State& state{*entry.state};
  ++state.step;
  Tensor value{entry.parameter.tensor().detach()};
  const Tensor gradient{entry.parameter.grad()};
  // Bias corrections computed on the host, as the reference's device path
  // does (cuda_ops.cppm:675-676).
  const auto correction = [step = static_cast<double>(state.step)](double beta) {
    return 1.0 - std::pow(beta, step);
  };
  hip::check(spar_hip_launch_adamw(HipTensorAccess::mutable_data(value),
                                   HipTensorAccess::data(gradient),
                                   HipTensorAccess::mutable_data(state.first_moment),
                                   HipTensorAccess::mutable_data(state.second_moment),
                                   value.numel(), hip::dtype_tag(value.dtype()), learning_rate_,
                                   beta1_, beta2_, epsilon_, weight_decay_, correction(beta1_),
                                   correction(beta2_), value.device().index()),
             "AdamW update", value.device());
}

// Every stepping entry is validated before anything changes, and the zero
// moments of first steps are all allocated before any is installed.
void AdamW::step() {
  std::vector<Entry*> stepping;
  for (Entry& entry : entries_) {
    if (steps(entry)) stepping.push_back(&entry);
  }
  std::vector<std::pair<Entry*, State>> first_states;
  for (Entry* entry : stepping) {
    if (entry->state) continue;
    const Tensor& value{entry->parameter.tensor()};
    first_states.emplace_back(entry, State{zeros(value.shape(), value.dtype(), value.device()),
                                           zeros(value.shape(), value.dtype(), value.device()),
                                           0});
  }
  for (auto& [entry, state] : first_states) entry->state.emplace(std::move(state));
  for (Entry* entry : stepping) update(*entry);
}

void AdamW::move_to(Device target) {
  std::vector<std::optional<std::pair<Tensor, Tensor>>> moved(entries_.size());
  for (std::size_t k{0}; k < entries_.size(); ++k) {
    if (const auto& state{entries_[k].state}) {
      moved[k].emplace(state->first_moment.to(target), state->second_moment.to(target));
    }
  }
  std::vector<nn::Parameter> tracked;
  tracked.reserve(entries_.size());
  for (const Entry& entry : entries_) tracked.push_back(entry.parameter);
  nn::move_to(std::span<nn::Parameter>{tracked}, target);
  for (std::size_t k{0}; k < entries_.size(); ++k) {
    if (moved[k]) {
      entries_[k].state->first_moment = std::move(moved[k]->first);
      entries_[k].state->second_moment = std::move(moved[k]->second);
    }
  }
}

void AdamW::zero_grad() {
  for (Entry& entry : entries_) entry.parameter.zero_grad();
}

std::size_t AdamW::parameter_count() const noexcept { return entries_.size(); }
double AdamW::learning_rate() const noexcept { return learning_rate_; }

void AdamW::set_learning_rate(double learning_rate) {
  check_learning_rate(learning_rate);
  learning_rate_ = learning_rate;
}

double AdamW::beta1() const noexcept { return beta1_; }
double AdamW::beta2() const noexcept { return beta2_; }
double AdamW::epsilon() const noexcept { return epsilon_; }
double AdamW::weight_decay() const noexcept { return weight_decay_; }

bool AdamW::tracks(const nn::Parameter& parameter) const noexcept {
  return entry_of(parameter) != nullptr;
}

std::optional<AdamWParameterState> AdamW::parameter_state(const nn::Parameter& parameter) const {
  const Entry* entry{entry_of(parameter)};
  if (entry == nullptr) throw std::invalid_argument{"AdamW does not track the requested Parameter"};
  if (!entry->state) return std::nullopt;
  const State& state{*entry->state};
  return AdamWParameterState{state.first_moment.detach().clone(),
                             state.second_moment.detach().clone(), state.step};
}

void AdamW::set_parameter_state(const nn::Parameter& parameter,
                                std::optional<AdamWParameterState> state) {
  Entry* entry{const_cast<Entry*>(entry_of(parameter))};
  if (entry == nullptr) throw std::invalid_argument{"AdamW does not track the requested Parameter"};
  if (!state) {
    entry->state.reset();
    return;
  }
  if (state->step == 0) throw std::invalid_argument{"AdamW restored state step must be at least one"};
  for (const Tensor* moment : {&state->first_moment, &state->second_moment}) {
    if (!matches(*moment, parameter.tensor())) {
      throw std::invalid_argument{"AdamW restored moment shape, dtype, or Device mismatch"};
    }
    if (!is_floating(moment->dtype())) {
      throw std::invalid_argument{"AdamW restored moments must be floating point"};
    }
  }
  entry->state.emplace(State{state->first_moment.detach().clone(),
                             state->second_moment.detach().clone(), state->step});
}

}  // namespace optim
}  // namespace spar
