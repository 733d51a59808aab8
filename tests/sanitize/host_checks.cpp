// Host-side checks of the C++ host library and the oracle's C loops, built
// with AddressSanitizer and UndefinedBehaviorSanitizer (tests/sanitize/Makefile)
// and run on the CPU: shapes and their overflow checks, views and their
// bounds, host gathers of every view kind, broadcast rules, the autograd
// engine over view-only graphs (whose backward needs no device), the
// optimizer's host logic and its errors, and the oracle's strided loops.
// Anything that needs a HIP device must fail with an exception, not touch
// memory.  Exit status 0 means every check held and the sanitizers stayed
// silent (they abort on the first report).
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "spar/optim.hpp"
#include "spar/spar.hpp"

extern "C" {
#include "spar_oracle.h"
}

namespace {

int failures = 0;

void expect(bool condition, const char* what) {
  if (!condition) {
    std::fprintf(stderr, "FAILED: %s\n", what);
    ++failures;
  }
}

template <typename E, typename F>
void expect_throw(F&& body, const char* what) {
  try {
    body();
  } catch (const E&) {
    return;
  } catch (...) {
    std::fprintf(stderr, "FAILED (wrong exception): %s\n", what);
    ++failures;
    return;
  }
  std::fprintf(stderr, "FAILED (no exception): %s\n", what);
  ++failures;
}

spar::Tensor iota(std::vector<std::int64_t> dims) {
  spar::Tensor t{spar::Shape{std::move(dims)}, spar::DType::Float32};
  auto values = t.span<float>();
  for (std::size_t i = 0; i < values.size(); ++i) values[i] = static_cast<float>(i);
  return t;
}

// Logical element (coordinates) of a CPU view, read through its strides.
float at(const spar::Tensor& view, std::vector<std::size_t> coordinate) {
  const spar::Tensor packed = view.contiguous();
  std::size_t flat = 0;
  for (std::size_t axis = 0; axis < coordinate.size(); ++axis) {
    flat = flat * static_cast<std::size_t>(view.shape()[axis]) + coordinate[axis];
  }
  return packed.span<float>()[flat];
}

void shapes() {
  using spar::Shape;
  expect(Shape{}.numel() == 1, "scalar shape");
  expect(Shape{3, 0, 5}.numel() == 0, "empty shape");
  expect((Shape{2, 3, 4}.contiguous_strides() == std::vector<std::size_t>{12, 4, 1}),
         "contiguous strides");
  expect_throw<std::invalid_argument>([] { Shape s{2, -1}; }, "negative extent");
  const auto big = std::numeric_limits<std::int64_t>::max() / 2;
  expect_throw<std::overflow_error>([&] { Shape s{big, big}; }, "numel overflow");
  expect(Shape{big, big, 0}.numel() == 0, "zero extent wins over overflow");
  expect_throw<std::invalid_argument>([&] { Shape s{big, big, -1}; }, "negative after overflow");
}

void views() {
  const spar::Tensor x = iota({3, 4, 5});
  const spar::Tensor t = x.transpose(0, 2);
  expect(t.shape() == spar::Shape{5, 4, 3} && !t.is_contiguous(), "transpose metadata");
  expect(at(t, {4, 1, 2}) == 2 * 20 + 1 * 5 + 4, "transpose values");
  const spar::Tensor p = x.permute({1, 2, 0});
  expect(at(p, {3, 1, 2}) == 2 * 20 + 3 * 5 + 1, "permute values");
  const spar::Tensor n = x.narrow(1, 1, 2).narrow(2, 3, 2);
  expect(n.storage_offset() == 8 && at(n, {2, 1, 1}) == 2 * 20 + 2 * 5 + 4, "narrow values");
  const spar::Tensor e = iota({1, 5}).expand(spar::Shape{4, 5});
  expect(e.strides()[0] == 0 && at(e, {3, 2}) == 2, "expand values");
  const spar::Tensor r = x.reshape(spar::Shape{12, 5});
  expect(at(r, {7, 3}) == 38, "reshape values");
  const spar::Tensor empty = iota({0, 3}).transpose(0, 1);
  expect(empty.contiguous().numel() == 0, "empty gather");
  expect_throw<std::out_of_range>([&] { (void)x.transpose(0, 3); }, "transpose axis");
  expect_throw<std::out_of_range>([&] { (void)x.permute({0, 1, 7}); }, "permute range");
  expect_throw<std::invalid_argument>([&] { (void)x.permute({0, 0, 7}); },
                                      "permute duplicate reported first");
  expect_throw<std::invalid_argument>([&] { (void)x.permute({0, 1}); }, "permute rank");
  expect_throw<std::out_of_range>([&] { (void)x.narrow(2, 4, 2); }, "narrow range");
  expect_throw<std::invalid_argument>([&] { (void)x.expand(spar::Shape{3, 4, 6}); },
                                      "expand incompatible");
  expect_throw<std::invalid_argument>([&] { (void)t.reshape(spar::Shape{60}); },
                                      "reshape of a non-contiguous view");
  const spar::Tensor c = t.clone();
  expect(c.is_contiguous() && at(c, {4, 3, 2}) == at(t, {4, 3, 2}), "clone of a view");
  const spar::Tensor moved = t.to(spar::Device::cpu());
  expect(moved.shape() == t.shape(), "same-device to");
}

void broadcasting() {
  using spar::Shape;
  expect(spar::detail::broadcast_shape(Shape{3, 1, 5}, Shape{4, 5}) == Shape{3, 4, 5},
         "broadcast");
  expect(spar::detail::broadcast_shape(Shape{}, Shape{2}) == Shape{2}, "broadcast scalar");
  expect_throw<std::invalid_argument>(
      [] { (void)spar::detail::broadcast_shape(Shape{3}, Shape{4}); }, "broadcast mismatch");
}

void autograd_on_views() {
  // View-only graphs: their gradients are layout copies (permute + gather,
  // narrow's zero fill and window copy, reshape), so backward runs on the
  // host.  z picks element 4 of leaf^T flattened, i.e. leaf[0][2].
  spar::Tensor leaf = iota({2, 3});
  leaf.set_requires_grad(true);
  spar::Tensor z = leaf.transpose(0, 1)
                             .contiguous()
                             .reshape(spar::Shape{6})
                             .narrow(0, 4, 1)
                             .reshape(spar::Shape{});
  expect(z.requires_grad() && !z.is_leaf(), "graph recorded");
  z.backward();
  const spar::Tensor gradient = leaf.grad();
  const auto grad = gradient.span<float>();
  expect(grad.size() == 6, "gradient shape");
  for (std::size_t i = 0; i < grad.size(); ++i) {
    expect(grad[i] == (i == 2 ? 1.0F : 0.0F), "one-hot gradient through views");
  }
  // a second backward adds into the leaf gradient in place: device work
  expect_throw<std::runtime_error>([&] { z.backward(); }, "accumulation needs a device");
  leaf.zero_grad();
  expect(!leaf.has_grad(), "zero_grad");
  spar::Tensor other = iota({1});
  other.set_requires_grad(true);
  spar::Tensor w = other.reshape(spar::Shape{1, 1}).transpose(0, 1).reshape(spar::Shape{});
  w.backward();
  const spar::Tensor other_grad = other.grad();
  expect(other.has_grad() && other_grad.span<float>()[0] == 1.0F, "view chain backward");
  expect_throw<std::invalid_argument>([&] { (void)z.grad(); }, "grad of a non-leaf");
  expect_throw<std::invalid_argument>([&] { leaf.backward(); }, "backward of non-scalar");
  spar::Tensor ints{spar::Shape{2}, spar::DType::Int32};
  expect_throw<std::invalid_argument>([&] { ints.set_requires_grad(true); }, "integer leaf");
  // expand's backward sums over the broadcast axis: device work
  spar::Tensor row = iota({1, 3});
  row.set_requires_grad(true);
  spar::Tensor picked =
      row.expand(spar::Shape{2, 3}).contiguous().reshape(spar::Shape{6}).narrow(0, 0, 1)
          .reshape(spar::Shape{});
  expect_throw<std::runtime_error>([&] { picked.backward(); }, "broadcast sum needs a device");
}

void optimizer_host_logic() {
  spar::nn::Parameter p{iota({4})};
  spar::nn::Parameter alias = p;
  expect(p.shares_identity_with(alias) && !p.shares_identity_with(p.clone()), "identity");
  expect_throw<std::invalid_argument>([] { spar::optim::AdamW opt{{}, -1.0}; }, "lr check");
  expect_throw<std::invalid_argument>([] { spar::optim::AdamW opt{{}, 1e-3, 1.0}; },
                                      "beta1 check");
  spar::optim::AdamW opt{{p, alias}};
  expect(opt.parameter_count() == 1 && opt.tracks(alias), "dedupe");
  expect(!opt.parameter_state(p).has_value(), "no state yet");
  opt.set_parameter_state(p, spar::optim::AdamWParameterState{iota({4}), iota({4}), 3});
  expect(opt.parameter_state(p)->step == 3, "restored state");
  expect_throw<std::invalid_argument>(
      [&] { opt.set_parameter_state(p, spar::optim::AdamWParameterState{iota({5}), iota({4}), 1}); },
      "restored moment shape");
  opt.step();  // no gradient: nothing steps
  std::vector<spar::nn::Parameter> list{p};
  spar::nn::move_to(list, spar::Device::cpu());
  opt.move_to(spar::Device::cpu());
  expect(spar::training::global_grad_norm(list) == 0.0, "norm without gradients");
  expect_throw<std::invalid_argument>([&] { spar::training::scale_gradients(list, NAN); },
                                      "nonfinite scale");
}

void device_paths_fail_cleanly() {
  const spar::Tensor x = iota({4});
  expect_throw<std::runtime_error>([&] { (void)spar::add(x, x); }, "arithmetic needs HIP");
  expect_throw<std::runtime_error>([&] { (void)spar::sum(x); }, "reduction needs HIP");
  if (spar::hip_device_count() == 0) {
    expect_throw<std::invalid_argument>([] { spar::Tensor t{spar::Shape{2}, spar::DType::Float32,
                                                          spar::Device::hip(0)}; },
                                        "no HIP device");
  }
}

void oracle_loops() {
  // A transposed view and a broadcast operand through the oracle's strided
  // binary loop and axis sum (float32).
  std::vector<float> a(12), b(4), out(12), sums(3);
  for (int i = 0; i < 12; ++i) a[i] = static_cast<float>(i) * 0.5F;
  for (int i = 0; i < 4; ++i) b[i] = static_cast<float>(i);
  const std::uint64_t extents[2] = {3, 4};
  const std::uint64_t a_strides[2] = {1, 3};   // [4, 3] viewed transposed as [3, 4]
  const std::uint64_t b_strides[2] = {0, 1};   // [4] broadcast over rows
  spar_oracle_binary_f32(out.data(), a.data(), a_strides, 0, b.data(), b_strides, 0, 2, extents, 0);
  expect(out[1 * 4 + 2] == a[2 * 3 + 1] + b[2], "oracle strided binary");
  spar_oracle_axis_sum_f32(sums.data(), 3, out.data(), 2, extents,
                           std::vector<std::uint64_t>{4, 1}.data(), 0, 2U);
  expect(sums[1] == out[4] + out[5] + out[6] + out[7], "oracle axis sum order");
}

}  // namespace

int main() {
  shapes();
  views();
  broadcasting();
  autograd_on_views();
  optimizer_host_logic();
  device_paths_fail_cleanly();
  oracle_loops();
  std::printf("host checks: %d failure(s)\n", failures);
  return failures == 0 ? 0 : 1;
}
