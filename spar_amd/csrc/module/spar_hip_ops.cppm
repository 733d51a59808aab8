// spar.hip_ops: the C ABI of include/spar_hip.h as a C++23 named module, the
// way Spar's backend modules bind its CUDA launcher header
// (src/backend/cuda_ops.cppm:1-15: the header in the global module
// fragment, checked wrappers in an exported namespace).  Spar's own modules
// also `import std;`, which this toolchain lacks, so the standard headers go
// into the global module fragment as well.
//
// The wrappers carry the names, enums and error conventions of the
// reference's spar.cuda_ops (cuda_ops.cppm:15-65, :227-699) over device
// pointers and element counts: the buffers a Tensor-level caller passes
// after its own shape and device checks (the Tensor layer of this backend,
// spar_amd/csrc/host, calls the C ABI the same way).
module;

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <string_view>

#include "spar_hip.h"

export module spar.hip_ops;

export namespace spar::detail::hip_ops {

enum class ElementType : int { Float32 = SPAR_HIP_FLOAT32, Float64 = SPAR_HIP_FLOAT64 };
enum class IndexType : int { Int32 = SPAR_HIP_INT32, Int64 = SPAR_HIP_INT64 };

// cuda_ops.cppm:17-19; Argmax is this backend's addition.
enum class BinaryOperation : int {
  Add = SPAR_HIP_ADD,
  Subtract = SPAR_HIP_SUBTRACT,
  Multiply = SPAR_HIP_MULTIPLY,
  Divide = SPAR_HIP_DIVIDE,
};
enum class UnaryOperation : int {
  Negate = SPAR_HIP_NEGATE,
  Square = SPAR_HIP_SQUARE,
  Reciprocal = SPAR_HIP_RECIPROCAL,
  Exp = SPAR_HIP_EXP,
  Log = SPAR_HIP_LOG,
  Sqrt = SPAR_HIP_SQRT,
  Sigmoid = SPAR_HIP_SIGMOID,
  Silu = SPAR_HIP_SILU,
};
enum class ReductionOperation : int {
  Sum = SPAR_HIP_SUM,
  Mean = SPAR_HIP_MEAN,
  Max = SPAR_HIP_MAX,
  Argmax = SPAR_HIP_ARGMAX,
};

// cuda_ops.cppm:26-31.
struct GradientNormSummary final {
  double scale;
  double scaled_sum_squares;
  bool has_infinity;
  bool has_nan;
};

// Status -> exception, with the reference's conventions: an invalid
// argument is std::invalid_argument, a HIP failure std::runtime_error naming
// the operation, the device and the code (cuda_ops.cppm:194-206).
void check(SparHipStatus status, std::string_view operation, int device) {
  if (status.code == 0) return;
  const char* text = spar_hip_error_string(status.hip_error);
  const std::string message = std::string{operation} + " failed on hip:" + std::to_string(device) +
                              ": " + (text == nullptr ? "unknown HIP error" : text) + " (code " +
                              std::to_string(status.hip_error) + ")";
  if (status.code == 1) throw std::invalid_argument{message};
  throw std::runtime_error{message};
}

// output[i] = left[i] op right[i] (cuda_ops.cppm:227-247).
void binary(void* output, const void* left, const void* right, std::uint64_t count,
            ElementType type, BinaryOperation operation, int device) {
  check(spar_hip_launch_binary(output, left, right, count, static_cast<int>(type),
                               static_cast<int>(operation), device),
        "binary", device);
}

// output[i] = input[i] op (T)value (cuda_ops.cppm:249-267).
void scalar(void* output, const void* input, std::uint64_t count, ElementType type, double value,
            BinaryOperation operation, int device) {
  check(spar_hip_launch_scalar(output, input, count, static_cast<int>(type),
                               static_cast<int>(operation), value, device),
        "scalar", device);
}

// output[i] = op(input[i]) (cuda_ops.cppm:269-286).
void unary(void* output, const void* input, std::uint64_t count, ElementType type,
           UnaryOperation operation, int device) {
  check(spar_hip_launch_unary(output, input, count, static_cast<int>(type),
                              static_cast<int>(operation), device),
        "unary", device);
}

// output[0] = op over `count` elements (cuda_ops.cppm:288-305).
void reduction(void* output, const void* input, std::uint64_t count, ElementType type,
               ReductionOperation operation, int device) {
  check(spar_hip_launch_reduction(output, input, count, static_cast<int>(type),
                                  static_cast<int>(operation), device),
        "reduction", device);
}

// One result per contiguous row (cuda_ops.cppm:307-335).
void row_reduction(void* output, const void* input, std::uint64_t row_count,
                   std::uint64_t reduction_count, ElementType type, ReductionOperation operation,
                   int device) {
  check(spar_hip_launch_row_reduction(output, input, row_count, reduction_count,
                                      static_cast<int>(type), static_cast<int>(operation), device),
        "row reduction", device);
}

// Softmax / log-softmax forward over (outer, axis, inner) slices; the
// undefined flags are int32 per slice (cuda_ops.cppm:337-370).
void probability_forward(void* output, std::int32_t* undefined_slices, const void* input,
                         std::uint64_t outer, std::uint64_t axis_extent, std::uint64_t inner,
                         ElementType type, bool logarithmic, int device) {
  check(spar_hip_launch_probability_forward(output, undefined_slices, input, outer, axis_extent,
                                            inner, static_cast<int>(type), logarithmic ? 1 : 0,
                                            device),
        logarithmic ? "log_softmax" : "softmax", device);
}

// Its backward (cuda_ops.cppm:372-409).
void probability_backward(void* output, const void* gradient, const void* saved_output,
                          const std::int32_t* undefined_slices, std::uint64_t outer,
                          std::uint64_t axis_extent, std::uint64_t inner, ElementType type,
                          bool logarithmic, int device) {
  check(spar_hip_launch_probability_backward(output, gradient, saved_output, undefined_slices,
                                             outer, axis_extent, inner, static_cast<int>(type),
                                             logarithmic ? 1 : 0, device),
        logarithmic ? "log_softmax backward" : "softmax backward", device);
}

// output[i] = scalar[0] * (T)scale (cuda_ops.cppm:530-548).
void fill_from_device_scalar(void* output, std::uint64_t count, const void* scalar,
                             ElementType type, double scale, int device) {
  check(spar_hip_launch_fill_from_scalar(output, scalar, count, static_cast<int>(type), scale,
                                         device),
        "fill from device scalar", device);
}

// Throws std::out_of_range when a class index is outside [0, classes)
// (cuda_ops.cppm:550-569).
void validate_targets(const void* targets, std::uint64_t count, IndexType type,
                      std::uint64_t classes, int device) {
  if (classes == 0) {
    throw std::logic_error{"Internal HIP target validation received no classes"};
  }
  std::int32_t invalid_target{0};
  check(spar_hip_validate_targets(&invalid_target, targets, count, classes,
                                  static_cast<int>(type), device),
        "cross_entropy target validation", device);
  if (invalid_target != 0) {
    throw std::out_of_range{"cross_entropy target is outside the class range"};
  }
}

// -log_probabilities at each target; sequence_length > 0 selects the
// language-model form (cuda_ops.cppm:571-597).
void nll_forward(void* output, const void* log_probabilities, const void* targets,
                 std::uint64_t output_count, std::uint64_t classes, ElementType type,
                 IndexType target_type, std::uint64_t sequence_length, int device) {
  check(spar_hip_launch_nll_forward(output, log_probabilities, targets, output_count, classes,
                                    sequence_length, static_cast<int>(type),
                                    static_cast<int>(target_type), sequence_length > 0 ? 1 : 0,
                                    device),
        "nll forward", device);
}

// Its scatter into a zeroed [rows, classes] output (cuda_ops.cppm:599-624).
void nll_backward(void* output, const void* gradient, const void* targets,
                  std::uint64_t output_count, std::uint64_t classes, ElementType type,
                  IndexType target_type, std::uint64_t sequence_length, int device) {
  check(spar_hip_launch_nll_backward(output, gradient, targets, output_count, classes,
                                     sequence_length, static_cast<int>(type),
                                     static_cast<int>(target_type), sequence_length > 0 ? 1 : 0,
                                     device),
        "nll backward", device);
}

// StableSumSquares summary of one gradient (cuda_ops.cppm:626-644).
[[nodiscard]] GradientNormSummary gradient_norm_summary(const void* gradient,
                                                        std::uint64_t count, ElementType type,
                                                        int device) {
  SparHipNormSummary summary{};
  check(spar_hip_gradient_norm_summary(&summary, gradient, count, static_cast<int>(type), device),
        "global gradient norm", device);
  return {.scale = summary.scale,
          .scaled_sum_squares = summary.scaled_sum_squares,
          .has_infinity = summary.has_infinity != 0,
          .has_nan = summary.has_nan != 0};
}

// values[i] = (T)((double)values[i] * factor) (cuda_ops.cppm:646-660).
void scale_in_place(void* values, std::uint64_t count, ElementType type, double factor,
                    int device) {
  check(spar_hip_launch_scale_in_place(values, count, static_cast<int>(type), factor, device),
        "gradient scaling", device);
}

// One AdamW step; the bias corrections 1 - beta^step are formed here with
// the C library's pow, as the reference's wrapper forms them
// (cuda_ops.cppm:662-699).
void adamw_update(void* parameter, const void* gradient, void* first_moment, void* second_moment,
                  std::uint64_t count, ElementType type, std::uint64_t step, double learning_rate,
                  double beta1, double beta2, double epsilon, double weight_decay, int device) {
  if (step == 0) throw std::logic_error{"Internal HIP AdamW update received step 0"};
  const double first_correction{1.0 - std::pow(beta1, static_cast<double>(step))};
  const double second_correction{1.0 - std::pow(beta2, static_cast<double>(step))};
  check(spar_hip_launch_adamw(parameter, gradient, first_moment, second_moment, count,
                              static_cast<int>(type), learning_rate, beta1, beta2, epsilon,
                              weight_decay, first_correction, second_correction, device),
        "AdamW update", device);
}

// output[0] = sum of `count` elements (reduction.cpp:21-30 for count 0).
void sum(void* output, const void* input, std::uint64_t count, ElementType type, int device) {
  reduction(output, input, count, type, ReductionOperation::Sum, device);
}

[[nodiscard]] int device_count() {
  int count = 0;
  return spar_hip_device_count(&count).code == 0 ? count : 0;
}

}  // namespace spar::detail::hip_ops
