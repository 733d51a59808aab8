// Internal bridge from spar::Tensor to the C ABI (include/spar_hip.h):
// status checking and view geometry.  Plays the role of the reference's
// spar.cuda_ops / spar.cuda_runtime modules (src/backend/cuda_ops.cppm:194-223,
// src/backend/cuda_runtime.cppm:45-64).
#pragma once

#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

#include "spar/tensor.hpp"
#include "spar_hip.h"

namespace spar::detail::hip {

/// throws std::runtime_error("<operation> failed on hip:N: <message> (code X)")
/// for a non-zero status (cuda_ops.cppm:194-206).
void check(SparHipStatus status, std::string_view operation, Device device);
void check(SparHipStatus status, std::string_view operation, int device);

[[nodiscard]] int dtype_tag(DType dtype);

/// Extents, element strides and storage offset of a tensor view, as the
/// C ABI takes them.
struct View {
  std::vector<std::uint64_t> extents;
  std::vector<std::uint64_t> strides;
  std::uint64_t offset = 0;
};

[[nodiscard]] View view_of(const Tensor& tensor);
/// the view of `tensor` expanded (right-aligned, zero strides) to `shape`.
[[nodiscard]] View expanded_view(const Tensor& tensor, const Shape& shape);

[[nodiscard]] std::vector<std::uint64_t> extents_of(const Shape& shape);

}  // namespace spar::detail::hip
