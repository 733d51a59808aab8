// A consumer of the spar.hip_ops module: imports it, calls every wrapper and
// reports what came back.  Needs no GPU: a zero-element launch returns
// success before touching a device, a bad element type (or a request the
// host can refuse, such as a mean of nothing) is rejected with
// SPAR_HIP_STATUS 1, which the module turns into std::invalid_argument, and
// the module's own checks (AdamW step 0, no classes) throw std::logic_error
// before any launch.
#include <cstdint>
#include <cstdio>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

import spar.hip_ops;

namespace ops = spar::detail::hip_ops;

namespace {

enum class Expect { Success, InvalidArgument, LogicError };

struct Case {
  std::string name;
  Expect expect;
  std::function<void()> call;
};

const char* outcome(const std::function<void()>& call, Expect& got) {
  try {
    call();
    got = Expect::Success;
    return "success";
  } catch (const std::invalid_argument&) {
    got = Expect::InvalidArgument;
    return "std::invalid_argument";
  } catch (const std::logic_error&) {
    got = Expect::LogicError;
    return "std::logic_error";
  } catch (const std::exception& error) {
    std::printf("  unexpected exception: %s\n", error.what());
    return "other exception";
  }
}

}  // namespace

int main() {
  const auto f32 = ops::ElementType::Float32;
  const auto bad = static_cast<ops::ElementType>(7);
  const auto i64 = ops::IndexType::Int64;
  std::int32_t flags[1] = {0};
  const std::vector<Case> cases{
      {"binary, empty", Expect::Success,
       [&] { ops::binary(nullptr, nullptr, nullptr, 0, f32, ops::BinaryOperation::Add, 0); }},
      {"binary, invalid dtype", Expect::InvalidArgument,
       [&] { ops::binary(nullptr, nullptr, nullptr, 4, bad, ops::BinaryOperation::Add, 0); }},
      {"scalar, empty", Expect::Success,
       [&] { ops::scalar(nullptr, nullptr, 0, f32, 2.0, ops::BinaryOperation::Multiply, 0); }},
      {"scalar, invalid dtype", Expect::InvalidArgument,
       [&] { ops::scalar(nullptr, nullptr, 4, bad, 2.0, ops::BinaryOperation::Multiply, 0); }},
      {"unary, empty", Expect::Success,
       [&] { ops::unary(nullptr, nullptr, 0, f32, ops::UnaryOperation::Exp, 0); }},
      {"unary, invalid dtype", Expect::InvalidArgument,
       [&] { ops::unary(nullptr, nullptr, 4, bad, ops::UnaryOperation::Exp, 0); }},
      {"reduction, mean of nothing", Expect::InvalidArgument,
       [&] { ops::reduction(flags, nullptr, 0, f32, ops::ReductionOperation::Mean, 0); }},
      {"reduction, invalid dtype", Expect::InvalidArgument,
       [&] { ops::reduction(flags, nullptr, 4, bad, ops::ReductionOperation::Sum, 0); }},
      {"row_reduction, no rows", Expect::Success,
       [&] { ops::row_reduction(nullptr, nullptr, 0, 8, f32, ops::ReductionOperation::Sum, 0); }},
      {"row_reduction, invalid dtype", Expect::InvalidArgument,
       [&] { ops::row_reduction(nullptr, nullptr, 4, 8, bad, ops::ReductionOperation::Max, 0); }},
      {"probability_forward, invalid dtype", Expect::InvalidArgument,
       [&] { ops::probability_forward(flags, flags, flags, 1, 4, 1, bad, false, 0); }},
      {"probability_backward, invalid dtype", Expect::InvalidArgument,
       [&] { ops::probability_backward(flags, flags, flags, flags, 1, 4, 1, bad, true, 0); }},
      {"fill_from_device_scalar, no scalar", Expect::InvalidArgument,
       [&] { ops::fill_from_device_scalar(nullptr, 4, nullptr, f32, 1.0, 0); }},
      {"validate_targets, empty", Expect::Success,
       [&] { ops::validate_targets(nullptr, 0, i64, 10, 0); }},
      {"validate_targets, no classes", Expect::LogicError,
       [&] { ops::validate_targets(nullptr, 4, i64, 0, 0); }},
      {"nll_forward, empty", Expect::Success,
       [&] { ops::nll_forward(nullptr, nullptr, nullptr, 0, 10, f32, i64, 0, 0); }},
      {"nll_forward, invalid dtype", Expect::InvalidArgument,
       [&] { ops::nll_forward(flags, flags, flags, 4, 10, bad, i64, 0, 0); }},
      {"nll_backward, empty", Expect::Success,
       [&] { ops::nll_backward(nullptr, nullptr, nullptr, 0, 10, f32, i64, 8, 0); }},
      {"nll_backward, invalid dtype", Expect::InvalidArgument,
       [&] { ops::nll_backward(flags, flags, flags, 4, 10, bad, i64, 8, 0); }},
      {"gradient_norm_summary, empty", Expect::Success,
       [&] {
         const auto summary = ops::gradient_norm_summary(nullptr, 0, f32, 0);
         if (summary.scale != 0.0 || summary.has_nan || summary.has_infinity) {
           throw std::runtime_error{"empty summary is not zero"};
         }
       }},
      {"gradient_norm_summary, invalid dtype", Expect::InvalidArgument,
       [&] { static_cast<void>(ops::gradient_norm_summary(flags, 4, bad, 0)); }},
      {"scale_in_place, empty", Expect::Success,
       [&] { ops::scale_in_place(nullptr, 0, f32, 0.5, 0); }},
      {"scale_in_place, invalid dtype", Expect::InvalidArgument,
       [&] { ops::scale_in_place(flags, 4, bad, 0.5, 0); }},
      {"adamw_update, empty", Expect::Success,
       [&] {
         ops::adamw_update(nullptr, nullptr, nullptr, nullptr, 0, f32, 1, 1e-3, 0.9, 0.999, 1e-8,
                           0.01, 0);
       }},
      {"adamw_update, step 0", Expect::LogicError,
       [&] {
         ops::adamw_update(flags, flags, flags, flags, 4, f32, 0, 1e-3, 0.9, 0.999, 1e-8, 0.01,
                           0);
       }},
      {"adamw_update, invalid dtype", Expect::InvalidArgument,
       [&] {
         ops::adamw_update(flags, flags, flags, flags, 4, bad, 1, 1e-3, 0.9, 0.999, 1e-8, 0.01,
                           0);
       }},
  };
  int failures = 0;
  for (const Case& c : cases) {
    Expect got{};
    const char* text = outcome(c.call, got);
    const bool ok = got == c.expect;
    failures += ok ? 0 : 1;
    std::printf("%s %s: %s\n", ok ? "ok  " : "FAIL", c.name.c_str(), text);
  }
  std::printf("spar.hip_ops: %zu wrappers checked, %d failed; empty launch ok, invalid dtype "
              "rejected; %d HIP device(s)\n",
              cases.size(), failures, ops::device_count());
  return failures == 0 ? 0 : 1;
}
