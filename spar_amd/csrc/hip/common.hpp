// Shared device-side and launcher-side helpers for the gfx950 backend.
//
// Every .hip translation unit of the backend includes this header.  It holds
// the status convention (mirrors src/backend/cuda_kernels.cu:12-22), the
// per-device stream/launch bookkeeping, geometry structs passed to kernels by
// value, fast 32-bit division by invariant integers, and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "spar_hip.h"

namespace spar_hip {

constexpr int kMaxRank = SPAR_HIP_MAX_RANK;
constexpr int kWave = 64;

// ------------------------------------------------------------------ status

inline SparHipStatus ok() { return {0, static_cast<int>(hipSuccess)}; }
inline SparHipStatus invalid() { return {1, static_cast<int>(hipErrorInvalidValue)}; }
inline SparHipStatus runtime(hipError_t error) { return {2, static_cast<int>(error)}; }

inline bool valid_float_dtype(int dtype) {
  return dtype == SPAR_HIP_FLOAT32 || dtype == SPAR_HIP_FLOAT64;
}

// --------------------------------------------------------- device context

// Per-device state owned by the runtime TU (runtime.hip).  Launchers call
// `enter(device)` which makes `device` current for the calling thread,
// creates its stream on first use, and restores the previous device when the
// returned guard goes out of scope.
struct DeviceGuard {
  int previous = -1;
  bool changed = false;
  hipStream_t stream = nullptr;
  hipError_t error = hipSuccess;
  int multiprocessors = 256;
  ~DeviceGuard();
};

// Fills `guard`; returns hipSuccess or the failing HIP error.  It also
// clears the calling thread's last-error slot, so that finish() reports only
// errors raised by the launches of the current call.
hipError_t enter(int device, DeviceGuard& guard);

// Workgroups of `kernel` resident on the device at once (at least one per
// CU), or 0 when the runtime cannot say.  A failed query's error is consumed
// here: callers fall back to a launch shape that does not need the answer,
// and the error must not surface later as the status of that launch.
template <typename K>
uint64_t resident_blocks(K kernel, int threads, const DeviceGuard& guard) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess) {
    static_cast<void>(hipGetLastError());
    return 0;
  }
  if (per_cu < 1) per_cu = 1;
  return static_cast<uint64_t>(per_cu) * static_cast<uint64_t>(guard.multiprocessors);
}

// Checks hipGetLastError after a launch and converts it to a status.
SparHipStatus finish(const DeviceGuard& guard);

// Temporary device memory from the caching allocator, for kernel scratch.
// Freed blocks return to the free list immediately; since every launch is on
// the same stream, a later reuse is ordered after the kernel that used it.
hipError_t scratch_allocate(void** pointer, uint64_t bytes, int device);
void scratch_release(void* pointer, int device);

// ------------------------------------------------------------- geometry

// Fast unsigned division by an invariant divisor, following Granlund &
// Montgomery, "Division by Invariant Integers using Multiplication" (PLDI
// 1994): with s = ceil(log2 d) and magic = floor(2^32 (2^s - d) / d) + 1,
// q = (mulhi(n, magic) + n) >> s for 1 <= d <= 2^31 - 1 and n < 2^31.
// Launchers use it only when every dividend is below 2^31.
struct FastDiv {
  uint32_t divisor;
  uint32_t magic;
  uint32_t shift;

  __host__ __device__ void init(uint32_t d) {
    divisor = d;
    uint32_t s = 0;
    while (s < 32 && (uint64_t{1} << s) < d) ++s;
    shift = s;
    const uint64_t numerator = (uint64_t{1} << 32) * ((uint64_t{1} << s) - d);
    magic = static_cast<uint32_t>(numerator / d + 1);
  }

  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint64_t hi = __umulhi(n, magic);
    return static_cast<uint32_t>((hi + n) >> shift);
  }
};

// Largest element count for which 32-bit index arithmetic is used.
constexpr uint64_t kIndex32Limit = (uint64_t{1} << 31) - 1;

// A strided operand of up to kMaxRank coalesced dimensions, passed by value.
struct StridedGeometry {
  int rank;
  uint64_t extents[kMaxRank];
  uint64_t strides[kMaxRank];
  uint64_t offset;
};

// --------------------------------------------------------- wave reductions

template <typename T>
__device__ __forceinline__ T wave_sum(T value) {
#pragma unroll
  for (int lane_mask = kWave / 2; lane_mask > 0; lane_mask >>= 1) {
    value += __shfl_xor(value, lane_mask, kWave);
  }
  return value;
}

// (value, index) pair under Spar's max rule: NaN beats everything (smaller
// index first among NaNs), otherwise the larger value wins and equal values
// keep the smaller index, so the result is the first occurrence of the
// maximum in logical order.
template <typename T>
struct ArgMax {
  T value;
  int64_t index;
};

template <typename T>
__device__ __forceinline__ bool argmax_better(T value, int64_t index, T best, int64_t best_index) {
  const bool nan_v = value != value;
  const bool nan_b = best != best;
  if (nan_v || nan_b) {
    if (nan_v && nan_b) return index < best_index;
    return nan_v;
  }
  if (value > best) return true;
  if (value == best) return index < best_index;
  return false;
}

template <typename T>
__device__ __forceinline__ void argmax_update(ArgMax<T>& best, T value, int64_t index) {
  if (argmax_better(value, index, best.value, best.index)) {
    best.value = value;
    best.index = index;
  }
}

template <typename T>
__device__ __forceinline__ ArgMax<T> wave_argmax(ArgMax<T> best) {
#pragma unroll
  for (int lane_mask = kWave / 2; lane_mask > 0; lane_mask >>= 1) {
    const T other_value = __shfl_xor(best.value, lane_mask, kWave);
    const int64_t other_index = __shfl_xor(best.index, lane_mask, kWave);
    argmax_update(best, other_value, other_index);
  }
  return best;
}

// Identity element for the argmax reduction: loses to every real element.
template <typename T>
__device__ __forceinline__ ArgMax<T> argmax_identity() {
  return ArgMax<T>{-__builtin_huge_valf(), INT64_MAX};
}

template <>
__device__ __forceinline__ ArgMax<double> argmax_identity<double>() {
  return ArgMax<double>{-__builtin_huge_val(), INT64_MAX};
}

// --------------------------------------------------------------- vectors

// 16-byte vectors as clang extended vectors (one global_load/store_dwordx4).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int64_t i64x2 __attribute__((ext_vector_type(2)));

template <typename T> struct Vec16;
template <> struct Vec16<float> { using type = f32x4; static constexpr int width = 4; };
template <> struct Vec16<double> { using type = f64x2; static constexpr int width = 2; };
template <> struct Vec16<int32_t> { using type = i32x4; static constexpr int width = 4; };
template <> struct Vec16<int64_t> { using type = i64x2; static constexpr int width = 2; };

template <typename T>
__device__ __forceinline__ T vec_get(const typename Vec16<T>::type& v, int i) {
  return v[i];
}

template <typename T>
__device__ __forceinline__ void vec_set(typename Vec16<T>::type& v, int i, T x) {
  v[i] = x;
}

// Streaming read: a non-temporal load, which on gfx950 keeps data that is
// read once from displacing cache lines.
template <typename V>
__device__ __forceinline__ V stream_load(const V* pointer) {
  return __builtin_nontemporal_load(pointer);
}

constexpr uint64_t kStreamStoreBytes = uint64_t{64} << 20;

inline bool stream_output(uint64_t bytes) { return bytes >= kStreamStoreBytes; }

// Streaming write: NT selects a non-temporal store.  Measured on MI355X over
// runs of back-to-back launches (512 MiB operands, random data), a fp32 add
// reaches ~6.45 TB/s with non-temporal stores and ~6.25 TB/s with ordinary
// ones: an ordinary store leaves up to 256 MB of dirty lines in the Infinity
// Cache whose write-back then competes with the next kernel's traffic.
// Outputs smaller than kStreamStoreBytes keep ordinary stores so that the
// consumer of a small result can still find it in cache.
//
// The policy is fixed at compile time.  A run-time choice such as
// `if (flag) nontemporal_store(p, v); else *p = v;` does not survive
// optimisation: the compiler sinks both stores into one ordinary store and
// drops the non-temporal hint (checked in the gfx950 assembly), so every
// kernel takes the policy as a template parameter and launchers select the
// instantiation with `with_policy`.
template <bool NT, typename V>
__device__ __forceinline__ void store_vector(V* pointer, V value) {
  if constexpr (NT) {
    __builtin_nontemporal_store(value, pointer);
  } else {
    *pointer = value;
  }
}

template <bool NT, typename V>
__device__ __forceinline__ V load_vector_policy(const V* pointer) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(pointer);
  } else {
    return *pointer;
  }
}

template <bool B>
struct Policy {
  static constexpr bool value = B;
};

// Calls body(Policy<true>{}) or body(Policy<false>{}).
template <typename Body>
inline void with_policy(bool flag, Body&& body) {
  if (flag) {
    body(Policy<true>{});
  } else {
    body(Policy<false>{});
  }
}

inline bool aligned16(const void* pointer) {
  return (reinterpret_cast<uintptr_t>(pointer) & 15U) == 0;
}

inline uint32_t ceil_div_u32(uint64_t a, uint64_t b) {
  return static_cast<uint32_t>((a + b - 1) / b);
}

}  // namespace spar_hip
