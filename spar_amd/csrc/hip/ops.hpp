// Elementwise operation functors shared by the contiguous and strided kernels.
//
// Arithmetic follows the CPU path element for element (one IEEE operation per
// output, src/ops/elementwise.cpp:50-220, src/ops/unary.cpp:55-164); the
// backend is compiled with -ffp-contract=off so no multiply-add is fused.
// Transcendentals call the ROCm device math library (ocml).
#pragma once

#include <hip/hip_runtime.h>

#include "spar_hip.h"

namespace spar_hip {

struct AddOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct SubtractOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a - b; }
};
struct MultiplyOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a * b; }
};
struct DivideOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a / b; }
};
struct EqualOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const {
    return a == b ? T(1) : T(0);
  }
};
struct NotEqualOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const {
    return a != b ? T(1) : T(0);
  }
};
struct LessOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const {
    return a < b ? T(1) : T(0);
  }
};
struct LessEqualOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const {
    return a <= b ? T(1) : T(0);
  }
};
struct GreaterOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const {
    return a > b ? T(1) : T(0);
  }
};
struct GreaterEqualOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const {
    return a >= b ? T(1) : T(0);
  }
};

// Calls `body(Op{})` for the binary operation tag; returns false for an
// unknown tag.
template <typename Body>
inline bool dispatch_binary(int operation, Body&& body) {
  switch (operation) {
    case SPAR_HIP_ADD: body(AddOp{}); return true;
    case SPAR_HIP_SUBTRACT: body(SubtractOp{}); return true;
    case SPAR_HIP_MULTIPLY: body(MultiplyOp{}); return true;
    case SPAR_HIP_DIVIDE: body(DivideOp{}); return true;
    case SPAR_HIP_EQUAL: body(EqualOp{}); return true;
    case SPAR_HIP_NOT_EQUAL: body(NotEqualOp{}); return true;
    case SPAR_HIP_LESS: body(LessOp{}); return true;
    case SPAR_HIP_LESS_EQUAL: body(LessEqualOp{}); return true;
    case SPAR_HIP_GREATER: body(GreaterOp{}); return true;
    case SPAR_HIP_GREATER_EQUAL: body(GreaterEqualOp{}); return true;
    default: return false;
  }
}

// ---------------------------------------------------------------- unary

__device__ __forceinline__ float math_exp(float x) { return expf(x); }
__device__ __forceinline__ double math_exp(double x) { return exp(x); }
__device__ __forceinline__ float math_log(float x) { return logf(x); }
__device__ __forceinline__ double math_log(double x) { return log(x); }
__device__ __forceinline__ float math_sqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ double math_sqrt(double x) { return sqrt(x); }
__device__ __forceinline__ float math_tanh(float x) { return tanhf(x); }
__device__ __forceinline__ double math_tanh(double x) { return tanh(x); }

// exp rounded once from double precision: (float)exp((double)x) is the
// correctly rounded float32 exponential except when exp(x) lies within about
// 2^-52 (relative) of a float32 rounding boundary.  glibc's expf, which the
// CPU path calls, is correctly rounded in the same sense, so composite ops
// built on it (sigmoid, silu) reproduce the CPU's float operations.
__device__ __forceinline__ float rounded_exp(float x) {
  return static_cast<float>(exp(static_cast<double>(x)));
}
__device__ __forceinline__ double rounded_exp(double x) { return exp(x); }

// The two-branch sigmoid of src/ops/unary.cpp:55-61.
template <typename T>
__device__ __forceinline__ T stable_sigmoid(T x) {
  if (x >= T(0)) return T(1) / (T(1) + rounded_exp(-x));
  const T e = rounded_exp(x);
  return e / (T(1) + e);
}

struct NegateOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return -x; }
};
struct SquareOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return x * x; }
};
struct ReciprocalOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return T(1) / x; }
};
struct ExpOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return math_exp(x); }
};
struct LogOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return math_log(x); }
};
struct SqrtOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return math_sqrt(x); }
};
struct SigmoidOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const {
    return stable_sigmoid(x);
  }
};
struct SiluOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const {
    return x * stable_sigmoid(x);
  }
};
struct TanhOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return math_tanh(x); }
};
// gelu(x) = (0.5 * x) * erfc(-x / sqrt(2)), evaluated in double precision
// and rounded once to T.  The erfc form avoids the cancellation of
// 0.5 * x * (1 + erf(x / sqrt(2))) for x << 0; double evaluation makes the
// float32 result the correctly rounded value in all but near-halfway cases
// (float32 erfcf implementations differ by several ulp in the tail).
__device__ __forceinline__ double gelu_double(double x) {
  const double t = -x * 0.70710678118654752440;
  return (0.5 * x) * erfc(t);
}
struct GeluOp {
  __device__ __forceinline__ float operator()(float x) const {
    return static_cast<float>(gelu_double(static_cast<double>(x)));
  }
  __device__ __forceinline__ double operator()(double x) const { return gelu_double(x); }
};

// gelu'(x) = Phi(x) + x phi(x) = 0.5 erfc(-x/sqrt 2) + x exp(-x^2/2)/sqrt(2 pi),
// in double precision, rounded once.
__device__ __forceinline__ double gelu_derivative_double(double x) {
  const double cdf = 0.5 * erfc(-x * 0.70710678118654752440);
  const double pdf = exp(-0.5 * (x * x)) * 0.39894228040143267794;
  return cdf + x * pdf;
}
struct GeluDerivativeOp {
  __device__ __forceinline__ float operator()(float x) const {
    return static_cast<float>(gelu_derivative_double(static_cast<double>(x)));
  }
  __device__ __forceinline__ double operator()(double x) const {
    return gelu_derivative_double(x);
  }
};

template <typename Body>
inline bool dispatch_unary(int operation, Body&& body) {
  switch (operation) {
    case SPAR_HIP_NEGATE: body(NegateOp{}); return true;
    case SPAR_HIP_SQUARE: body(SquareOp{}); return true;
    case SPAR_HIP_RECIPROCAL: body(ReciprocalOp{}); return true;
    case SPAR_HIP_EXP: body(ExpOp{}); return true;
    case SPAR_HIP_LOG: body(LogOp{}); return true;
    case SPAR_HIP_SQRT: body(SqrtOp{}); return true;
    case SPAR_HIP_SIGMOID: body(SigmoidOp{}); return true;
    case SPAR_HIP_SILU: body(SiluOp{}); return true;
    case SPAR_HIP_TANH: body(TanhOp{}); return true;
    case SPAR_HIP_GELU: body(GeluOp{}); return true;
    case SPAR_HIP_GELU_DERIVATIVE: body(GeluDerivativeOp{}); return true;
    default: return false;
  }
}

// A binary functor with its right operand fixed (scalar ops).
template <typename Op, typename T>
struct BindRight {
  Op op;
  T scalar;
  __device__ __forceinline__ T operator()(T x) const { return op(x, scalar); }
};

}  // namespace spar_hip
