// cross_entropy and language_model_cross_entropy (src/loss/cross_entropy.cpp:
// 107-214) over the fused log-softmax -> NLL kernels.  The reference computes
// log_softmax over the whole logits tensor, selects the target entries
// (select_nll, :83-105) and reduces; here one forward kernel yields the
// selected losses and the per-row statistics, and one backward kernel the
// logits gradient, with the same values and the same autograd interface:
// the node takes the upstream gradient of the unreduced losses.
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "autograd_internal.hpp"
#include "bridge.hpp"
#include "spar/loss.hpp"
#include "spar/ops.hpp"

namespace spar::loss {
namespace {

using detail::HipTensorAccess;
namespace hip = detail::hip;

// cross_entropy.cpp:48-55
void validate_target_metadata(const Tensor& targets) {
  if (targets.dtype() != DType::Int32 && targets.dtype() != DType::Int64) {
    throw std::invalid_argument{"cross_entropy targets must have Int32 or Int64 dtype"};
  }
  if (targets.requires_grad()) {
    throw std::invalid_argument{"cross_entropy targets must not require gradients"};
  }
}

// cross_entropy.cpp:119-129
void validate_logits(const Tensor& logits) {
  if (logits.dtype() != DType::Float32 && logits.dtype() != DType::Float64) {
    throw std::invalid_argument{"cross_entropy logits must have Float32 or Float64 dtype"};
  }
  if (logits.rank() == 0) {
    throw std::invalid_argument{"cross_entropy logits must have a class dimension"};
  }
  if (logits.shape()[logits.rank() - 1] <= 0) {
    throw std::invalid_argument{"cross_entropy class dimension must be positive"};
  }
}

// cross_entropy.cpp:107-117
Tensor reduce_loss(const Tensor& losses, Reduction reduction) {
  switch (reduction) {
    case Reduction::None:
      return losses;
    case Reduction::Sum:
      return sum(losses);
    case Reduction::Mean:
      return mean(losses);
  }
  throw std::invalid_argument{"cross_entropy received an unknown Reduction"};
}

// The fused log_softmax -> select_nll node.  `sequence_length` is 0 for plain
// cross entropy and T for the language-model form.
Tensor fused_nll(const Tensor& logits, const Tensor& targets, Shape output_shape,
                 std::size_t sequence_length) {
  detail::require_hip(logits, "cross_entropy");
  const std::size_t classes{static_cast<std::size_t>(logits.shape()[logits.rank() - 1])};
  const std::size_t rows{logits.numel() / classes};
  const Tensor x{logits.is_contiguous() ? logits : logits.contiguous()};
  // A snapshot, as the reference keeps (cross_entropy.cpp:140, :185).
  const Tensor snapshot{targets.detach().clone()};
  const Device device{logits.device()};
  const Shape row_shape{static_cast<Shape::dimension_type>(rows)};
  Tensor losses{std::move(output_shape), logits.dtype(), device};
  Tensor row_max{row_shape, logits.dtype(), device};
  Tensor row_log_sum{row_shape, logits.dtype(), device};
  Tensor undefined{row_shape, DType::Int32, device};
  Tensor invalid{Shape{1}, DType::Int32, device};
  const int dtype{hip::dtype_tag(logits.dtype())};
  const int target_dtype{hip::dtype_tag(snapshot.dtype())};
  const int language_model{sequence_length == 0 ? 0 : 1};
  hip::check(spar_hip_launch_cross_entropy_forward(
                 HipTensorAccess::mutable_data(losses), HipTensorAccess::mutable_data(row_max),
                 HipTensorAccess::mutable_data(row_log_sum),
                 static_cast<std::int32_t*>(HipTensorAccess::mutable_data(undefined)),
                 static_cast<std::int32_t*>(HipTensorAccess::mutable_data(invalid)),
                 HipTensorAccess::data(x), HipTensorAccess::data(snapshot), rows, classes,
                 sequence_length, dtype, target_dtype, language_model, device.index()),
             "cross_entropy forward", device);
  // Target validation (cross_entropy.cpp:141, cuda_ops.cppm:550-566) reads
  // the device flag back, which synchronises, as the reference's does.
  std::int32_t invalid_target{0};
  hip::check(spar_hip_copy_device_to_host(&invalid_target, HipTensorAccess::data(invalid),
                                          sizeof(invalid_target), device.index()),
             "cross_entropy target validation", device);
  if (invalid_target != 0) {
    throw std::out_of_range{"cross_entropy target is outside the class range"};
  }
  if (x.requires_grad()) {
    const Tensor saved_logits{x.detach()};
    detail::record_operation(
        losses, {x},
        [saved_logits, snapshot, row_max, row_log_sum, undefined, rows, classes, sequence_length,
         dtype, target_dtype, language_model](const Tensor& gradient) {
          const Tensor upstream{gradient.is_contiguous() ? gradient.detach()
                                                         : gradient.detach().contiguous()};
          Tensor contribution{saved_logits.shape(), saved_logits.dtype(), saved_logits.device()};
          hip::check(spar_hip_launch_cross_entropy_backward(
                         HipTensorAccess::mutable_data(contribution), HipTensorAccess::data(upstream),
                         HipTensorAccess::data(saved_logits), HipTensorAccess::data(row_max),
                         HipTensorAccess::data(row_log_sum),
                         static_cast<const std::int32_t*>(HipTensorAccess::data(undefined)),
                         HipTensorAccess::data(snapshot), rows, classes, sequence_length, dtype,
                         target_dtype, language_model, saved_logits.device().index()),
                     "cross_entropy backward", saved_logits.device());
          return std::vector<Tensor>{contribution};
        });
  }
  return losses;
}

}  // namespace

// cross_entropy.cpp:131-160
Tensor cross_entropy(const Tensor& logits, const Tensor& targets, Reduction reduction) {
  detail::validate_same_device(logits, targets, "cross_entropy");
  validate_logits(logits);
  if (targets.numel() == 0) {
    throw std::invalid_argument{"cross_entropy requires at least one target"};
  }
  std::vector<Shape::dimension_type> expected_dimensions{logits.shape().dimensions().begin(),
                                                         logits.shape().dimensions().end() - 1};
  if (targets.shape() != Shape{expected_dimensions}) {
    throw std::invalid_argument{"cross_entropy target shape does not match logits"};
  }
  validate_target_metadata(targets);
  return reduce_loss(fused_nll(logits, targets, targets.shape(), 0), reduction);
}

// cross_entropy.cpp:162-212
Tensor language_model_cross_entropy(const Tensor& logits, const Tensor& token_ids,
                                    Reduction reduction) {
  detail::validate_same_device(logits, token_ids, "language_model_cross_entropy");
  validate_logits(logits);
  if (logits.rank() != 3 || token_ids.rank() != 2) {
    throw std::invalid_argument{
        "language_model_cross_entropy requires logits [B,T,V] and IDs [B,T]"};
  }
  if (logits.shape()[0] <= 0 || logits.shape()[1] < 2 ||
      token_ids.shape()[0] != logits.shape()[0] || token_ids.shape()[1] != logits.shape()[1]) {
    throw std::invalid_argument{"language_model_cross_entropy received incompatible shapes"};
  }
  validate_target_metadata(token_ids);
  const auto batch{logits.shape()[0]};
  const auto sequence{logits.shape()[1]};
  return reduce_loss(fused_nll(logits, token_ids, Shape{batch, sequence - 1},
                               static_cast<std::size_t>(sequence)),
                     reduction);
}

}  // namespace spar::loss
