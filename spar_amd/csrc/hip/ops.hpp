// Elementwise operation functors shared by the contiguous and strided kernels.
//
// Arithmetic follows the CPU path element for element (one IEEE operation per
// output, src/ops/elementwise.cpp:50-220, src/ops/unary.cpp:55-164); the
// backend is compiled with -ffp-contract=off so no multiply-add is fused.
// Transcendentals call the ROCm device math library (ocml).
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"
#include "gelu_table.hpp"
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
// gelu(x) = (0.5 * x) * erfc(-x / sqrt(2)), defined as its double-precision
// value rounded once to T.  The erfc form avoids the cancellation of
// 0.5 * x * (1 + erf(x / sqrt(2))) for x << 0.  fp64 inputs use the device
// library's erfc.
__device__ __forceinline__ double gelu_double(double x) {
  const double t = -x * 0.70710678118654752440;
  return (0.5 * x) * erfc(t);
}

// gelu'(x) = Phi(x) + x phi(x) = 0.5 erfc(-x/sqrt 2) + x exp(-x^2/2)/sqrt(2 pi),
// in double precision, rounded once.
__device__ __forceinline__ double gelu_derivative_double(double x) {
  const double cdf = 0.5 * erfc(-x * 0.70710678118654752440);
  const double pdf = exp(-0.5 * (x * x)) * 0.39894228040143267794;
  return cdf + x * pdf;
}

// fp32 inputs need the double value of the definition only to within 2^-25
// relative for the rounded float32 result to stay within 1 ulp of the
// correctly rounded one, which short dedicated evaluations give at a
// fraction of a full double erfc's cost (the library erfc made GELU
// compute-bound at 29% of HBM bandwidth).
//
// GELU reads Q(a) = 0.5 erfc(a / sqrt 2), 0 <= a <= 15, from a table of
// piecewise polynomials (gelu_table.hpp, fit_gelu_table.py): the piece is
// i = floor(g) for g = 4 (2a + a^2/2), and with t = fract(g),
// Q = scale (1 + t (c1 + t (d2 + t (d3 + t d4)))) to 9.9e-9 relative, the
// d terms in float32 and the rest in double: about 21 VALU instructions and
// 32 bytes of table per element.  The contiguous kernel holds the table in
// LDS; other layouts read it from global memory.
//
// The derivative needs the density exp(-a^2/2) as well, and keeps the
// direct evaluation: the normal upper tail Q(a) is exp(-a^2/2) * M(a) with
// M(a) = 0.5 erfcx(a / sqrt 2) a degree-10 polynomial in t = s - mid,
// s = 1 / (1 + a / 3.5), relative error 2.0e-9 (coefficients from
// fit_normal_tail.py).  a^2 / 2 is exact in double for a float a; its exp
// uses a Cody-Waite reduction by ln 2 and a degree-8 Taylor polynomial on
// |r| <= ln(2)/2 (error 2.0e-10).  The reciprocal is v_rcp_f64 (measured
// 2^-24.4) with one Newton step.  Checked on every float32 input against
// the double definition: the derivative within 1 ulp except for x in
// [-0.7576, -0.7473], where Phi(x) + x phi(x) cancels near its root and the
// error stays below 2.4e-10 absolute.
constexpr double kTailInvKappa = 0x1.2492492492492p-2;
constexpr double kTailMid = 0x1.306eb3e45306fp-1;
constexpr double kTailCoefficient[11] = {
    0x1.2c6f5bb4f12e0p-3,  0x1.ef6b2713cfd1fp-2,  0x1.51f19eed9c16dp-1,
    0x1.3908154c15e3dp-1,  0x1.431e8a1b994a1p-2,  -0x1.fbad36cff239fp-8,
    -0x1.c7e02fce56efcp-4, -0x1.202d9626843f4p-6, 0x1.8884025989592p-5,
    0x1.a5cb80b2edea0p-8,  -0x1.4bebcb7e53f99p-6,
};

// A wave-uniform constant placed in a scalar register at its use, so that
// the fma reads it from there instead of from a vector register copied for
// each step (what the compiler otherwise does when the constants are hoisted
// out of a kernel's loop).
__device__ __forceinline__ double scalar_constant(double c) {
  asm volatile("" : "+s"(c));
  return c;
}

// exp(y) for -113 <= y <= 0.
__device__ __forceinline__ double exp_nonpositive(double y) {
  constexpr double kLog2e = 0x1.71547652b82fep0;
  constexpr double kLn2High = 0x1.62e42fefa39efp-1;
  constexpr double kLn2Low = 0x1.abc9e3b39803fp-56;
  const double k = __builtin_rint(y * kLog2e);
  double r = __builtin_fma(-k, kLn2High, y);
  r = __builtin_fma(-k, kLn2Low, r);
  double p = 1.0 / 40320.0;
  p = __builtin_fma(p, r, scalar_constant(1.0 / 5040.0));
  p = __builtin_fma(p, r, scalar_constant(1.0 / 720.0));
  p = __builtin_fma(p, r, scalar_constant(1.0 / 120.0));
  p = __builtin_fma(p, r, scalar_constant(1.0 / 24.0));
  p = __builtin_fma(p, r, scalar_constant(1.0 / 6.0));
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  return __builtin_ldexp(p, static_cast<int>(k));
}

struct NormalTail {
  double density;  // exp(-a^2 / 2)
  double upper;    // Q(a) = 0.5 erfc(a / sqrt 2)
};

// 0 <= a <= 15.
__device__ __forceinline__ NormalTail normal_tail(double a) {
  const double d = __builtin_fma(a, kTailInvKappa, 1.0);
  double s = __builtin_amdgcn_rcp(d);
  s = __builtin_fma(s, __builtin_fma(-d, s, 1.0), s);
  const double t = s - kTailMid;
  double m = kTailCoefficient[10];
#pragma unroll
  for (int i = 9; i >= 0; --i) m = __builtin_fma(m, t, scalar_constant(kTailCoefficient[i]));
  const double density = exp_nonpositive((a * a) * -0.5);
  return NormalTail{density, density * m};
}

// GELU of a float32 from the tail table at `table` (global memory or an LDS
// copy: the same values, so the same bits), pieces STRIDE 16-byte units
// apart: unit 0 holds (scale, c1) as doubles, unit 1 (d2, d3, d4, pad) as
// floats.  With a = |x| clamped to 15 and q = Q(a), GELU is x - a q for
// x >= 0 and -a q (that is x Q(|x|)) below 0: one fused multiply-add,
// -a q + base, with base = x above 0 and x - x below (0 for a finite x, NaN
// for -inf, as (0.5 x) erfc(-x / sqrt 2) is).  The clamp (exact at +-15) and
// base are formed in float32, as is the polynomial's d part; the table
// lookup, the last two Horner steps, the scaling and that multiply-add run in
// double.  No branches and no patched results: Q(15) = 3.7e-51 already makes
// GELU round to -0 below -15 and to x above 15, +inf stays +inf
// (inf - 15 Q(15)), NaN propagates through base, and -0 gives -0.  Simulated
// on the CPU over all 2^32 float32 inputs (fmaf, fma and conversions as the
// GPU rounds them), every result is within 1 ulp of the double definition.
static_assert(sizeof(GeluPiece) == 32, "a GELU piece is two 16-byte units");

template <int STRIDE = 2>
__device__ __forceinline__ float gelu_float(float value, const f64x2* table) {
  constexpr float kLimit = static_cast<float>(kGeluTailLimit);
  // median of three: a NaN gives NaN or a bound, either of which indexes a
  // piece in range (v_cvt_i32_f64 maps NaN to 0), and base carries the NaN
  const double a = __builtin_fabs(static_cast<double>(__builtin_amdgcn_fmed3f(value, -kLimit, kLimit)));
  const double g = a * __builtin_fma(kGeluBeta, a, kGeluAlpha);  // 0 <= g <= 570
  // piece index < 2^24: a full-rate 24-bit multiply, not the quarter-rate 32-bit one
  const f64x2* piece = table + __umul24(static_cast<uint32_t>(static_cast<int>(g)), STRIDE);
  const f64x2 high = piece[0];
  const f32x4 low = *reinterpret_cast<const f32x4*>(piece + 1);
  const double t = __builtin_amdgcn_fract(g);
  const float tf = static_cast<float>(t);
  const float p = __builtin_fmaf(__builtin_fmaf(low[2], tf, low[1]), tf, low[0]);
  const double q =
      high[0] * __builtin_fma(__builtin_fma(static_cast<double>(p), t, high[1]), t, 1.0);
  const float base = value < 0.0f ? value - value : value;
  return static_cast<float>(__builtin_fma(-a, q, static_cast<double>(base)));
}

// gelu_float of four values with their piece reads issued together, so the
// LDS latency is paid once per group rather than per element.  The same
// operations on each value, so the same bits.
template <int STRIDE = 2>
__device__ __forceinline__ f32x4 gelu_float4(f32x4 value, const f64x2* table) {
  constexpr float kLimit = static_cast<float>(kGeluTailLimit);
  double a[4];
  double g[4];
  const f64x2* piece[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a[k] = __builtin_fabs(static_cast<double>(__builtin_amdgcn_fmed3f(value[k], -kLimit, kLimit)));
    g[k] = a[k] * __builtin_fma(kGeluBeta, a[k], kGeluAlpha);
    piece[k] = table + __umul24(static_cast<uint32_t>(static_cast<int>(g[k])), STRIDE);
  }
  f64x2 high[4];
  f32x4 low[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    high[k] = piece[k][0];
    low[k] = *reinterpret_cast<const f32x4*>(piece[k] + 1);
  }
  f32x4 out;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const double t = __builtin_amdgcn_fract(g[k]);
    const float tf = static_cast<float>(t);
    const float p = __builtin_fmaf(__builtin_fmaf(low[k][2], tf, low[k][1]), tf, low[k][0]);
    const double q =
        high[k][0] * __builtin_fma(__builtin_fma(static_cast<double>(p), t, high[k][1]), t, 1.0);
    const float base = value[k] < 0.0f ? value[k] - value[k] : value[k];
    out[k] = static_cast<float>(__builtin_fma(-a[k], q, static_cast<double>(base)));
  }
  return out;
}

// The derivative: |x| is clamped to 15 and the results outside [-15, 15]
// are patched.  There the exact derivative rounds to -0 in float32 below
// -15 and to 1 above 15, which the clamped evaluation already gives for
// finite x; both infinities give NaN (x exp(-x^2/2) = inf * 0).  NaN inputs
// propagate through the arithmetic.
__device__ __forceinline__ float gelu_derivative_float(float value) {
  const double x = value;
  const NormalTail tail = normal_tail(fmin(__builtin_fabs(x), 15.0));
  const double cdf = x < 0.0 ? tail.upper : 1.0 - tail.upper;
  float out = static_cast<float>(cdf + x * (tail.density * 0.39894228040143267794));
  out = value < -15.0f ? -0.0f : out;
  out = __builtin_isinf(value) ? __builtin_nanf("") : out;
  return out;
}

// Ops with tens of fp64 operations per element take two vectors per lane
// in the contiguous kernels, for more independent work per wave.
template <typename F> struct VectorsPerLane { static constexpr int value = 1; };

struct GeluOp {
  __device__ __forceinline__ float operator()(float x) const {
    return gelu_float(x, reinterpret_cast<const f64x2*>(kGeluTable));
  }
  __device__ __forceinline__ double operator()(double x) const { return gelu_double(x); }
};

struct GeluDerivativeOp {
  __device__ __forceinline__ float operator()(float x) const { return gelu_derivative_float(x); }
  __device__ __forceinline__ double operator()(double x) const {
    return gelu_derivative_double(x);
  }
};

template <> struct VectorsPerLane<GeluOp> { static constexpr int value = 2; };
template <> struct VectorsPerLane<GeluDerivativeOp> { static constexpr int value = 2; };

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
