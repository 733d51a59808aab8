// Spar's cross-entropy losses on HIP tensors (src/loss/cross_entropy.cppm:8-17):
// the same Reduction, functions, argument meaning and exceptions.  The
// log-softmax and the target selection run as one fused kernel each way.
#pragma once

#include "spar/tensor.hpp"

namespace spar::loss {

enum class Reduction { None, Sum, Mean };

/// logits [..., C] (Float32/Float64), targets [...] (Int32/Int64) class
/// indices; loss = -log_softmax(logits, last axis)[target], reduced.
[[nodiscard]] Tensor cross_entropy(const Tensor& logits, const Tensor& targets,
                                   Reduction reduction = Reduction::Mean);

/// logits [B, T, V], token_ids [B, T]: position t predicts token t + 1; the
/// unreduced loss is [B, T - 1].
[[nodiscard]] Tensor language_model_cross_entropy(const Tensor& logits, const Tensor& token_ids,
                                                  Reduction reduction = Reduction::Mean);

}  // namespace spar::loss
