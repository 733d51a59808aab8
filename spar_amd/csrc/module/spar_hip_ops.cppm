// spar.hip_ops: the C ABI of include/spar_hip.h as a C++23 named module, the
// way Spar's backend modules bind its CUDA launcher header
// (src/backend/cuda_ops.cppm:1-15: the header in the global module
// fragment, checked wrappers in an exported namespace).  Spar's own modules
// also `import std;`, which this toolchain lacks, so the standard headers go
// into the global module fragment as well.
module;

#include <cstdint>
#include <stdexcept>
#include <string>
#include <string_view>

#include "spar_hip.h"

export module spar.hip_ops;

export namespace spar::detail::hip_ops {

enum class BinaryOperation : int {
  Add = SPAR_HIP_ADD,
  Subtract = SPAR_HIP_SUBTRACT,
  Multiply = SPAR_HIP_MULTIPLY,
  Divide = SPAR_HIP_DIVIDE,
};

enum class ElementType : int { Float32 = SPAR_HIP_FLOAT32, Float64 = SPAR_HIP_FLOAT64 };

// Status -> exception, with the reference's conventions: an invalid
// argument is std::invalid_argument, a HIP failure std::runtime_error naming
// the operation and the device (cuda_ops.cppm:194-206).
void check(SparHipStatus status, std::string_view operation, int device) {
  if (status.code == 0) return;
  const char* text = spar_hip_error_string(status.hip_error);
  const std::string message = std::string{operation} + " failed on hip:" + std::to_string(device) +
                              ": " + (text == nullptr ? "unknown HIP error" : text);
  if (status.code == 1) throw std::invalid_argument{message};
  throw std::runtime_error{message};
}

// output[i] = left[i] op right[i] over `count` elements on `device`.
void binary(void* output, const void* left, const void* right, std::uint64_t count,
            ElementType type, BinaryOperation operation, int device) {
  check(spar_hip_launch_binary(output, left, right, count, static_cast<int>(type),
                               static_cast<int>(operation), device),
        "binary", device);
}

// output[0] = sum of `count` elements (reduction.cpp:21-30 for count 0).
void sum(void* output, const void* input, std::uint64_t count, ElementType type, int device) {
  check(spar_hip_launch_reduction(output, input, count, static_cast<int>(type), SPAR_HIP_SUM,
                                  device),
        "sum", device);
}

[[nodiscard]] int device_count() {
  int count = 0;
  return spar_hip_device_count(&count).code == 0 ? count : 0;
}

}  // namespace spar::detail::hip_ops
