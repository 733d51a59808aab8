// Softmax and log-softmax over slices (outer, axis, inner), forward and
// backward, with the reference's special cases for NaN and infinities.
//
// Replaces K7/K8 (src/backend/cuda_kernels.cu:482-617), which launched
// ceil(rows/256) blocks (32 for 8192 rows) and read each row three times.
// Semantics follow the CPU path (src/ops/softmax.cpp:42-150, :342-444).
//
// CDNA4 design for the last axis (inner == 1), the common case: one
// workgroup per row holds the whole row in VGPRs (up to 32768 float32 with
// 1024 lanes x 8 float4), so the row is read from HBM once and written once:
//   pass over registers 1: first-occurrence max;
//   workgroup combine through wave64 shuffles and a 16-entry LDS exchange;
//   pass 2: e = exp(x - max), sum; pass 3: p = e / sum (log: (x-max) - log sum).
// A row's workgroup stays under 64 VGPRs per lane, so two or more rows share
// a CU and one row's loads overlap another's reductions and stores.
// Backward keeps g and y (or log p) in registers the same way.  Rows longer
// than the register budget take a three-read loop, and a non-last axis
// (inner > 1) a lane-per-slice kernel that is coalesced across `inner`.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "ops.hpp"

namespace spar_hip {
namespace {

constexpr uint64_t kMaxGrid = uint64_t{1} << 20;

// Statistics of a slice: first-occurrence maximum (value and 32-bit column;
// rows are far shorter than 2^31), NaN flag, +inf count.
template <typename T>
struct SliceStats {
  T value;
  int32_t index;
  unsigned nan;
  unsigned positive_infinities;
};

// Barrier for the reductions' LDS exchanges: waits for this wave's LDS
// accesses (lgkmcnt(0)) and meets the other waves at s_barrier.  Unlike
// __syncthreads() it is not a release fence, so global stores in flight keep
// draining across it.  The signal fences stop the compiler from moving memory
// accesses across the barrier; they emit no instructions.
__device__ __forceinline__ void exchange_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt and expcnt unchanged, lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename T>
__device__ __forceinline__ void stats_init(SliceStats<T>& s) {
  s.value = -static_cast<T>(__builtin_huge_val());
  s.index = INT32_MAX;
  s.nan = 0;
  s.positive_infinities = 0;
}

// NaN never becomes the maximum here: a slice with a NaN is undefined and
// its maximum is not used.  Larger value wins; ties keep the smaller column.
template <typename T>
__device__ __forceinline__ void stats_max(SliceStats<T>& s, T x, int32_t index) {
  if (x > s.value || (x == s.value && index < s.index)) {
    s.value = x;
    s.index = index;
  }
}

template <typename T>
__device__ __forceinline__ void stats_add(SliceStats<T>& s, T x, int64_t index) {
  s.nan |= (x != x) ? 1U : 0U;
  s.positive_infinities += (x == static_cast<T>(__builtin_huge_val())) ? 1U : 0U;
  stats_max(s, x, static_cast<int32_t>(index));
}

template <typename T>
__device__ __forceinline__ void stats_merge(SliceStats<T>& s, const SliceStats<T>& o) {
  s.nan |= o.nan;
  s.positive_infinities += o.positive_infinities;
  stats_max(s, o.value, o.index);
}

template <typename T>
__device__ __forceinline__ SliceStats<T> wave_stats(SliceStats<T> s) {
#pragma unroll
  for (int mask = kWave / 2; mask > 0; mask >>= 1) {
    SliceStats<T> o;
    o.value = __shfl_xor(s.value, mask, kWave);
    o.index = __shfl_xor(s.index, mask, kWave);
    o.nan = __shfl_xor(s.nan, mask, kWave);
    o.positive_infinities = __shfl_xor(s.positive_infinities, mask, kWave);
    stats_merge(s, o);
  }
  return s;
}

// GUARD: wait before writing the LDS slots, which a previous call of the
// same kernel may still be reading; a kernel that calls it once skips it.
template <typename T, int THREADS, bool GUARD = true>
__device__ __forceinline__ SliceStats<T> block_stats(SliceStats<T> s) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ SliceStats<T> lds[kWavesPerBlock];
  s = wave_stats(s);
  if constexpr (GUARD) exchange_barrier();
  if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = s;
  exchange_barrier();
  SliceStats<T> total = lds[0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) stats_merge(total, lds[w]);
  return total;
}

template <typename T, int THREADS, bool GUARD = true>
__device__ __forceinline__ T block_sum(T value) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ T lds[kWavesPerBlock];
  value = wave_sum(value);
  if constexpr (GUARD) exchange_barrier();
  if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = value;
  exchange_barrier();
  T total = lds[0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) total += lds[w];
  return total;
}

template <typename T> __device__ __forceinline__ T positive_infinity() {
  return static_cast<T>(__builtin_huge_val());
}
template <typename T> __device__ __forceinline__ T quiet_nan() {
  return static_cast<T>(__builtin_nan(""));
}

// Value written at element x of an undefined slice (forward).
template <typename T, bool LOG>
__device__ __forceinline__ T undefined_value(const SliceStats<T>& s, T x) {
  if (s.nan != 0 || s.value == -positive_infinity<T>()) return quiet_nan<T>();
  // k > 0 entries of +inf share the mass (softmax.cpp:82-91, :381-390)
  if constexpr (LOG) {
    const T at_infinity = -math_log(static_cast<T>(s.positive_infinities));
    return x == positive_infinity<T>() ? at_infinity : -positive_infinity<T>();
  } else {
    const T probability = T(1) / static_cast<T>(s.positive_infinities);
    return x == positive_infinity<T>() ? probability : T(0);
  }
}

// e / total for many e and one total: q0 = e * (1 / total) corrected by one
// residual step, q = q0 + (e - q0 * total) / total, with the residual exact
// through a fused multiply-add (Markstein's correction).  The result is
// within one ulp of the correctly rounded quotient (equal to it in almost
// all cases) at three instructions instead of a full IEEE division.
template <typename T>
struct RowDivisor {
  T total;
  T reciprocal;
  __device__ __forceinline__ explicit RowDivisor(T t) : total(t), reciprocal(T(1) / t) {}
  __device__ __forceinline__ T operator()(T e) const {
    const T q0 = e * reciprocal;
    const T residual = __builtin_fma(-q0, total, e);
    return __builtin_fma(residual, reciprocal, q0);
  }
};

template <>
__device__ __forceinline__ float RowDivisor<float>::operator()(float e) const {
  const float q0 = e * reciprocal;
  const float residual = __builtin_fmaf(-q0, total, e);
  return __builtin_fmaf(residual, reciprocal, q0);
}

template <typename T>
__device__ __forceinline__ bool slice_undefined(const SliceStats<T>& s) {
  return s.nan != 0 || s.value == -positive_infinity<T>() || s.positive_infinities != 0;
}

// Element j of a thread's register array maps to column col(t, j):
// VEC: 16-byte groups interleaved across lanes; scalar: lanes interleaved.
// Register rows hold at most 32768 elements, so columns are 32-bit and a
// row access is a uniform row base plus a 32-bit lane offset.
template <typename T, int THREADS, bool VEC>
__device__ __forceinline__ uint32_t column_of(int j) {
  if constexpr (VEC) {
    constexpr int W = Vec16<T>::width;
    return (static_cast<uint32_t>(j / W) * THREADS + threadIdx.x) * W + (j % W);
  } else {
    return static_cast<uint32_t>(j) * THREADS + threadIdx.x;
  }
}

// Columns grow with the register slot j, so the slots of a lane that hold
// columns < n are a prefix j < live_slots(n) (whole 16-byte groups for VEC,
// where n is a multiple of the vector width).  One 32-bit bound per lane
// replaces a 64-bit column compare per slot.
template <typename T, int THREADS, int E, bool VEC>
__device__ __forceinline__ int live_slots(uint64_t n) {
  constexpr int W = VEC ? Vec16<T>::width : 1;
  const int units = static_cast<int>(n / W);  // n <= THREADS * E
  const int lane = static_cast<int>(threadIdx.x);
  return units > lane ? ((units - lane + THREADS - 1) / THREADS) * W : 0;
}

// Loads a row into registers; slots past the row hold `pad`.
template <typename T, int THREADS, int E, bool VEC, bool FULL>
__device__ __forceinline__ void load_row(T (&x)[E], const T* row, int live, T pad) {
  if constexpr (VEC) {
    using V = typename Vec16<T>::type;
    constexpr int W = Vec16<T>::width;
#pragma unroll
    for (int v = 0; v < E / W; ++v) {
      if (FULL || v * W < live) {
        const V value = stream_load(reinterpret_cast<const V*>(row + column_of<T, THREADS, true>(v * W)));
#pragma unroll
        for (int k = 0; k < W; ++k) x[v * W + k] = vec_get<T>(value, k);
      } else {
#pragma unroll
        for (int k = 0; k < W; ++k) x[v * W + k] = pad;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = FULL || j < live ? row[column_of<T, THREADS, false>(j)] : pad;
  }
}

// NT: non-temporal stores (outputs of 64 MiB or more).
template <typename T, int THREADS, int E, bool VEC, bool FULL, bool NT>
__device__ __forceinline__ void store_row(T* row, const T (&y)[E], int live) {
  if constexpr (VEC) {
    using V = typename Vec16<T>::type;
    constexpr int W = Vec16<T>::width;
#pragma unroll
    for (int v = 0; v < E / W; ++v) {
      if (FULL || v * W < live) {
        const uint32_t col = column_of<T, THREADS, true>(v * W);
        V value;
#pragma unroll
        for (int k = 0; k < W; ++k) vec_set<T>(value, k, y[v * W + k]);
        store_vector<NT>(reinterpret_cast<V*>(row + col), value);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if (FULL || j < live) row[column_of<T, THREADS, false>(j)] = y[j];
    }
  }
}

// ----------------------------------------------------- register-row kernels

// Block-wide first-occurrence maximum of (value, column) pairs: the larger
// value wins, equal values (including -0 and +0) keep the smaller column.
// NaN never enters (a lane only takes an element that compares larger).
template <typename T, int THREADS, bool GUARD = true>
__device__ __forceinline__ T block_max_first(T value, int32_t index) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ T lds_value[kWavesPerBlock];
  __shared__ int32_t lds_index[kWavesPerBlock];
#pragma unroll
  for (int mask = kWave / 2; mask > 0; mask >>= 1) {
    const T other = __shfl_xor(value, mask, kWave);
    const int32_t other_index = __shfl_xor(index, mask, kWave);
    const bool take = other > value || (other == value && other_index < index);
    value = take ? other : value;
    index = take ? other_index : index;
  }
  if constexpr (GUARD) exchange_barrier();
  if (threadIdx.x % kWave == 0) {
    lds_value[threadIdx.x / kWave] = value;
    lds_index[threadIdx.x / kWave] = index;
  }
  exchange_barrier();
  T best = lds_value[0];
  int32_t best_index = lds_index[0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) {
    const T other = lds_value[w];
    const int32_t other_index = lds_index[w];
    const bool take = other > best || (other == best && other_index < best_index);
    best = take ? other : best;
    best_index = take ? other_index : best_index;
  }
  return best;
}

template <typename T>
__device__ __forceinline__ T value_max(T a, T b) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_fmaxf(a, b);
  } else {
    return __builtin_fmax(a, b);
  }
}

// Block-wide maximum by value (maxNum: NaN operands are skipped), for a
// reduction that runs once per kernel (no guard barrier).
template <typename T, int THREADS>
__device__ __forceinline__ T block_max_value(T value) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ T lds_value[kWavesPerBlock];
#pragma unroll
  for (int mask = kWave / 2; mask > 0; mask >>= 1) {
    value = value_max(value, __shfl_xor(value, mask, kWave));
  }
  if (threadIdx.x % kWave == 0) lds_value[threadIdx.x / kWave] = value;
  exchange_barrier();
  T best = lds_value[0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) best = value_max(best, lds_value[w]);
  return best;
}

// Forward over rows held in registers, one row per workgroup (the launcher
// splits the rows into grids of at most kMaxGrid workgroups).  With no row
// loop nothing is hoisted across rows, so a lane needs E + ~30 VGPRs and
// several workgroups share a CU: while one reduces or stores, the others'
// loads are in flight.
//
// The fast path keeps no NaN or infinity bookkeeping: with m the maximum
// over the non-NaN elements, S = sum exp(x - m) is
// NaN exactly when the slice is undefined (a NaN element gives NaN - m; a +inf
// maximum gives inf - inf; an all -inf slice gives -inf - -inf), and is
// otherwise finite (1 <= S <= n).  Undefined rows, which are rare, reload the
// row and apply the reference's special cases from full slice statistics.
//
// Waves per SIMD the register budget must allow: a row of up to 128 bytes
// per lane fits in 64 VGPRs (8 waves, two 1024-lane workgroups per CU);
// longer rows get 128 (4 waves).
template <typename T, int E>
constexpr int row_waves() {
  return sizeof(T) * E <= 128 ? 8 : 4;
}

template <typename T, int THREADS, int E, bool LOG, bool VEC, bool FULL, bool NT>
__global__ void __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(row_waves<T, E>())))
    forward_row_kernel(T* out, int32_t* undefined, const T* in, uint64_t n) {
  const uint64_t r = blockIdx.x;
  const int live = FULL ? E : live_slots<T, THREADS, E, VEC>(n);
  // Slots past the row hold -inf: never a strict maximum, and exp(-inf - m)
  // adds an exact +0 to the sum for every m that leaves the row defined.
  T x[E];
  load_row<T, THREADS, E, VEC, FULL>(x, in + r * n, live, -positive_infinity<T>());
  // The row maximum over the non-NaN elements, by value only (IEEE maxNum,
  // one v_max per element, which skips NaNs as the CPU's strict `>` scan
  // does).  Which element is the first maximum does not matter here: the
  // value is the same, and when it is a zero of either sign the results are
  // too (x - m is the same nonzero value for x != 0 and a zero for x = +-0,
  // whose exp is 1; for log-softmax a zero x - m meets log S = 0 only when
  // S = 1, that is when the maximum is the row's only zero, and then m is
  // that element).
  T lane_max = -positive_infinity<T>();
#pragma unroll
  for (int j = 0; j < E; ++j) lane_max = value_max(lane_max, x[j]);
  // Each block reduction below runs once per kernel: no guard barriers.
  const T maximum = block_max_value<T, THREADS>(lane_max);
  // The results overwrite x in place so one row costs E registers per lane.
  T local = T(0);
#pragma unroll
  for (int j = 0; j < E; ++j) {
    if constexpr (LOG) {
      x[j] = x[j] - maximum;
      local += math_exp(x[j]);
    } else {
      x[j] = math_exp(x[j] - maximum);
      local += x[j];
    }
  }
  const T total = block_sum<T, THREADS, false>(local);
  const bool bad = total != total;
  if (threadIdx.x == 0) undefined[r] = bad ? 1 : 0;
  if (!bad) {
    if constexpr (LOG) {
      const T log_sum = math_log(total);
#pragma unroll
      for (int j = 0; j < E; ++j) x[j] = x[j] - log_sum;
    } else {
      const RowDivisor<T> divide(total);
#pragma unroll
      for (int j = 0; j < E; ++j) x[j] = divide(x[j]);
    }
  } else {
    load_row<T, THREADS, E, VEC, FULL>(x, in + r * n, live, T(0));
    SliceStats<T> s;
    stats_init(s);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if (FULL || j < live) stats_add(s, x[j], static_cast<int64_t>(column_of<T, THREADS, VEC>(j)));
    }
    s = block_stats<T, THREADS, false>(s);
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = undefined_value<T, LOG>(s, x[j]);
  }
  store_row<T, THREADS, E, VEC, FULL, NT>(out + r * n, x, live);
}

template <typename T, int THREADS, int E, bool LOG, bool VEC, bool FULL, bool NT>
__global__ void __launch_bounds__(THREADS)
    backward_row_kernel(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                        uint64_t rows, uint64_t n) {
  const int live = FULL ? E : live_slots<T, THREADS, E, VEC>(n);
  for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    T* out_row = out + r * n;
    T g[E];
    if (undefined[r] != 0) {
#pragma unroll
      for (int j = 0; j < E; ++j) g[j] = quiet_nan<T>();
      store_row<T, THREADS, E, VEC, FULL, NT>(out_row, g, live);
      continue;
    }
    // Slots past the row hold +0 in both, adding an exact +0 to the sum.
    T y[E];
    load_row<T, THREADS, E, VEC, FULL>(g, gradient + r * n, live, T(0));
    load_row<T, THREADS, E, VEC, FULL>(y, saved + r * n, live, T(0));
    T local = T(0);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if constexpr (LOG) {
        local += g[j];
      } else {
        local += g[j] * y[j];
      }
    }
    const T reduced = block_sum<T, THREADS>(local);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if constexpr (LOG) {
        g[j] = g[j] - math_exp(y[j]) * reduced;
      } else {
        g[j] = y[j] * (g[j] - reduced);
      }
    }
    store_row<T, THREADS, E, VEC, FULL, NT>(out_row, g, live);
  }
}

// ------------------------------------------------------ long rows (looped)

constexpr int kLoopThreads = 1024;

template <typename T, bool LOG>
__global__ void __launch_bounds__(kLoopThreads)
    forward_loop_kernel(T* out, int32_t* undefined, const T* in, uint64_t rows, uint64_t n) {
  for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = in + r * n;
    T* out_row = out + r * n;
    SliceStats<T> s;
    stats_init(s);
    for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) stats_add(s, row[c], static_cast<int64_t>(c));
    s = block_stats<T, kLoopThreads>(s);
    const bool bad = slice_undefined(s);
    if (threadIdx.x == 0) undefined[r] = bad ? 1 : 0;
    if (bad) {
      for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) {
        out_row[c] = undefined_value<T, LOG>(s, row[c]);
      }
      continue;
    }
    const T maximum = s.value;
    T local = T(0);
    for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) local += math_exp(row[c] - maximum);
    const T total = block_sum<T, kLoopThreads>(local);
    const T log_sum = LOG ? math_log(total) : T(0);
    const RowDivisor<T> divide(total);
    for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) {
      if constexpr (LOG) {
        out_row[c] = (row[c] - maximum) - log_sum;
      } else {
        out_row[c] = divide(math_exp(row[c] - maximum));
      }
    }
  }
}

template <typename T, bool LOG>
__global__ void __launch_bounds__(kLoopThreads)
    backward_loop_kernel(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                         uint64_t rows, uint64_t n) {
  for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* g = gradient + r * n;
    const T* y = saved + r * n;
    T* o = out + r * n;
    if (undefined[r] != 0) {
      for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) o[c] = quiet_nan<T>();
      continue;
    }
    T local = T(0);
    for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) {
      if constexpr (LOG) {
        local += g[c];
      } else {
        local += g[c] * y[c];
      }
    }
    const T reduced = block_sum<T, kLoopThreads>(local);
    for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) {
      if constexpr (LOG) {
        o[c] = g[c] - math_exp(y[c]) * reduced;
      } else {
        o[c] = y[c] * (g[c] - reduced);
      }
    }
  }
}

// -------------------------------------------- non-last axis (inner > 1)

constexpr int kSliceThreads = 256;

template <typename T, bool LOG>
__global__ void __launch_bounds__(kSliceThreads)
    forward_slice_kernel(T* out, int32_t* undefined, const T* in, uint64_t outer,
                         uint64_t axis_extent, uint64_t inner) {
  const uint64_t slices = outer * inner;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kSliceThreads;
  for (uint64_t slice = static_cast<uint64_t>(blockIdx.x) * kSliceThreads + threadIdx.x;
       slice < slices; slice += stride) {
    const uint64_t o = slice / inner;
    const uint64_t i = slice - o * inner;
    const T* base = in + o * axis_extent * inner + i;
    T* out_base = out + o * axis_extent * inner + i;
    SliceStats<T> s;
    stats_init(s);
    for (uint64_t a = 0; a < axis_extent; ++a) stats_add(s, base[a * inner], static_cast<int64_t>(a));
    const bool bad = slice_undefined(s);
    undefined[slice] = bad ? 1 : 0;
    if (bad) {
      for (uint64_t a = 0; a < axis_extent; ++a) {
        out_base[a * inner] = undefined_value<T, LOG>(s, base[a * inner]);
      }
      continue;
    }
    const T maximum = s.value;
    T total = T(0);
    for (uint64_t a = 0; a < axis_extent; ++a) total += math_exp(base[a * inner] - maximum);
    const T log_sum = LOG ? math_log(total) : T(0);
    const RowDivisor<T> divide(total);
    for (uint64_t a = 0; a < axis_extent; ++a) {
      if constexpr (LOG) {
        out_base[a * inner] = (base[a * inner] - maximum) - log_sum;
      } else {
        out_base[a * inner] = divide(math_exp(base[a * inner] - maximum));
      }
    }
  }
}

template <typename T, bool LOG>
__global__ void __launch_bounds__(kSliceThreads)
    backward_slice_kernel(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                          uint64_t outer, uint64_t axis_extent, uint64_t inner) {
  const uint64_t slices = outer * inner;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kSliceThreads;
  for (uint64_t slice = static_cast<uint64_t>(blockIdx.x) * kSliceThreads + threadIdx.x;
       slice < slices; slice += stride) {
    const uint64_t o = slice / inner;
    const uint64_t i = slice - o * inner;
    const uint64_t base = o * axis_extent * inner + i;
    if (undefined[slice] != 0) {
      for (uint64_t a = 0; a < axis_extent; ++a) out[base + a * inner] = quiet_nan<T>();
      continue;
    }
    T reduced = T(0);
    for (uint64_t a = 0; a < axis_extent; ++a) {
      const uint64_t idx = base + a * inner;
      if constexpr (LOG) {
        reduced += gradient[idx];
      } else {
        reduced += gradient[idx] * saved[idx];
      }
    }
    for (uint64_t a = 0; a < axis_extent; ++a) {
      const uint64_t idx = base + a * inner;
      if constexpr (LOG) {
        out[idx] = gradient[idx] - math_exp(saved[idx]) * reduced;
      } else {
        out[idx] = saved[idx] * (gradient[idx] - reduced);
      }
    }
  }
}

uint32_t grid_for(uint64_t blocks) {
  if (blocks == 0) blocks = 1;
  return static_cast<uint32_t>(blocks > kMaxGrid ? kMaxGrid : blocks);
}

// Register-row configurations (threads, elements per lane), smallest first;
// FULL drops the bounds checks when the row exactly fills the registers.
// One workgroup per row, launched in grids of at most kMaxGrid rows.
template <typename T, int THREADS, int E, bool LOG, bool VEC, bool FULL>
void forward_rows_as(T* out, int32_t* undefined, const T* in, uint64_t rows, uint64_t n,
                     const DeviceGuard& guard) {
  with_policy(stream_output(rows * n * sizeof(T)), [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    for (uint64_t first = 0; first < rows; first += kMaxGrid) {
      const uint64_t count = rows - first < kMaxGrid ? rows - first : kMaxGrid;
      forward_row_kernel<T, THREADS, E, LOG, VEC, FULL, NT>
          <<<static_cast<uint32_t>(count), THREADS, 0, guard.stream>>>(
              out + first * n, undefined + first, in + first * n, n);
    }
  });
}

template <typename T, int THREADS, int E, bool LOG, bool VEC>
void forward_rows(T* out, int32_t* undefined, const T* in, uint64_t rows, uint64_t n,
                  const DeviceGuard& guard) {
  if (n == static_cast<uint64_t>(THREADS) * E) {
    forward_rows_as<T, THREADS, E, LOG, VEC, true>(out, undefined, in, rows, n, guard);
  } else {
    forward_rows_as<T, THREADS, E, LOG, VEC, false>(out, undefined, in, rows, n, guard);
  }
}

template <typename T, int THREADS, int E, bool LOG, bool VEC>
void backward_rows(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                   uint64_t rows, uint64_t n, const DeviceGuard& guard) {
  with_policy(stream_output(rows * n * sizeof(T)), [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    if (n == static_cast<uint64_t>(THREADS) * E) {
      backward_row_kernel<T, THREADS, E, LOG, VEC, true, NT>
          <<<grid_for(rows), THREADS, 0, guard.stream>>>(out, gradient, saved, undefined, rows, n);
    } else {
      backward_row_kernel<T, THREADS, E, LOG, VEC, false, NT>
          <<<grid_for(rows), THREADS, 0, guard.stream>>>(out, gradient, saved, undefined, rows, n);
    }
  });
}

// Row lengths up to 1024 take one wave per row (no cross-wave exchange);
// 8192 takes 256 lanes x 32, which measured faster than 512 x 16.
template <typename T, bool LOG, bool VEC>
bool launch_forward_rows(T* out, int32_t* undefined, const T* in, uint64_t rows, uint64_t n,
                         const DeviceGuard& guard) {
  if (n <= 64 * 4) {
    forward_rows<T, 64, 4, LOG, VEC>(out, undefined, in, rows, n, guard);
  } else if (n <= 64 * 16) {
    forward_rows<T, 64, 16, LOG, VEC>(out, undefined, in, rows, n, guard);
  } else if (n <= 256 * 16) {
    forward_rows<T, 256, 16, LOG, VEC>(out, undefined, in, rows, n, guard);
  } else if (n <= 256 * 32) {
    forward_rows<T, 256, 32, LOG, VEC>(out, undefined, in, rows, n, guard);
  } else if (n <= 1024 * 16) {
    forward_rows<T, 1024, 16, LOG, VEC>(out, undefined, in, rows, n, guard);
  } else if (n <= 1024 * 32) {
    forward_rows<T, 1024, 32, LOG, VEC>(out, undefined, in, rows, n, guard);
  } else {
    return false;
  }
  return true;
}

template <typename T, bool LOG, bool VEC>
bool launch_backward_rows(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                          uint64_t rows, uint64_t n, const DeviceGuard& guard) {
  if (n <= 256 * 4) {
    backward_rows<T, 256, 4, LOG, VEC>(out, gradient, saved, undefined, rows, n, guard);
  } else if (n <= 256 * 16) {
    backward_rows<T, 256, 16, LOG, VEC>(out, gradient, saved, undefined, rows, n, guard);
  } else if (n <= 512 * 16) {
    backward_rows<T, 512, 16, LOG, VEC>(out, gradient, saved, undefined, rows, n, guard);
  } else if (n <= 1024 * 16) {
    backward_rows<T, 1024, 16, LOG, VEC>(out, gradient, saved, undefined, rows, n, guard);
  } else if (n <= 1024 * 32) {
    backward_rows<T, 1024, 32, LOG, VEC>(out, gradient, saved, undefined, rows, n, guard);
  } else {
    return false;
  }
  return true;
}

template <typename T, bool LOG>
void forward(void* output, int32_t* undefined, const void* input, uint64_t outer, uint64_t axis,
             uint64_t inner, const DeviceGuard& guard) {
  T* out = static_cast<T*>(output);
  const T* in = static_cast<const T*>(input);
  if (inner == 1) {
    const bool vec = axis % Vec16<T>::width == 0 && aligned16(out) && aligned16(in);
    const bool done = vec ? launch_forward_rows<T, LOG, true>(out, undefined, in, outer, axis, guard)
                          : launch_forward_rows<T, LOG, false>(out, undefined, in, outer, axis, guard);
    if (!done) {
      forward_loop_kernel<T, LOG><<<grid_for(outer), kLoopThreads, 0, guard.stream>>>(
          out, undefined, in, outer, axis);
    }
    return;
  }
  forward_slice_kernel<T, LOG>
      <<<grid_for((outer * inner + kSliceThreads - 1) / kSliceThreads), kSliceThreads, 0,
         guard.stream>>>(out, undefined, in, outer, axis, inner);
}

template <typename T, bool LOG>
void backward(void* output, const void* gradient, const void* saved, const int32_t* undefined,
              uint64_t outer, uint64_t axis, uint64_t inner, const DeviceGuard& guard) {
  T* out = static_cast<T*>(output);
  const T* g = static_cast<const T*>(gradient);
  const T* y = static_cast<const T*>(saved);
  if (inner == 1) {
    const bool vec = axis % Vec16<T>::width == 0 && aligned16(out) && aligned16(g) && aligned16(y);
    const bool done =
        vec ? launch_backward_rows<T, LOG, true>(out, g, y, undefined, outer, axis, guard)
            : launch_backward_rows<T, LOG, false>(out, g, y, undefined, outer, axis, guard);
    if (!done) {
      backward_loop_kernel<T, LOG><<<grid_for(outer), kLoopThreads, 0, guard.stream>>>(
          out, g, y, undefined, outer, axis);
    }
    return;
  }
  backward_slice_kernel<T, LOG>
      <<<grid_for((outer * inner + kSliceThreads - 1) / kSliceThreads), kSliceThreads, 0,
         guard.stream>>>(out, g, y, undefined, outer, axis, inner);
}

// ------------------------------------------- cross entropy (log-softmax + NLL)

// Target of logits row `row` and the index of its loss, for plain
// cross entropy (one target per row) or the language-model form, where
// position t of a length-T sequence predicts token t + 1 and the last
// position has no target (cross_entropy.cpp:146-214).
struct TargetMap {
  uint64_t sequence_length;  // 0: plain cross entropy
  __device__ __forceinline__ bool lookup(uint64_t row, uint64_t& target_index,
                                         uint64_t& output_index) const {
    if (sequence_length == 0) {
      target_index = row;
      output_index = row;
      return true;
    }
    const uint64_t batch = row / sequence_length;
    const uint64_t time = row - batch * sequence_length;
    if (time + 1 == sequence_length) return false;
    target_index = row + 1;
    output_index = batch * (sequence_length - 1) + time;
    return true;
  }
};

constexpr int kEntropyThreads = 256;

// Row statistics in one streaming pass, branch-free: each lane keeps a
// running maximum m and s = sum exp(x - m); per batch of 8 vectors it takes
// the batch maximum (v_max, which passes over NaN), rescales s once by
// exp(m - m_new) and adds exp(x - m_new) per element, where a -inf element
// adds exactly 0 (as it does to a row with a finite maximum).  A NaN element
// makes s NaN (NaN - m) and a +inf maximum does too (inf - inf); a row of
// nothing above -inf keeps m = -inf.  Only the sign of a zero maximum can
// differ from the first-occurrence rule, which changes no loss or gradient.
template <typename T>
__device__ __forceinline__ T rescaled(T s, T m, T top) {
  return s == T(0) ? T(0) : s * math_exp(m - top);
}

template <typename T>
__device__ __forceinline__ T exp_term(T x, T top) {
  return x == -positive_infinity<T>() ? T(0) : math_exp(x - top);
}

template <typename T> __device__ __forceinline__ T fmax_of(T a, T b);
template <> __device__ __forceinline__ float fmax_of<float>(float a, float b) { return fmaxf(a, b); }
template <> __device__ __forceinline__ double fmax_of<double>(double a, double b) { return fmax(a, b); }

// Block-wide merge of the lanes' (m, s): the maximum M of the lane maxima
// (wave shuffles, then the waves through LDS), then each lane's sum rescaled
// once by exp(m - M) and the rescaled sums added (wave sums, then in wave
// order).
template <typename T, int THREADS>
__device__ __forceinline__ void block_online(T& m, T& s) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ T lds_m[kWavesPerBlock];
  __shared__ T lds_s[kWavesPerBlock];
  T wave_m = m;
#pragma unroll
  for (int mask = kWave / 2; mask > 0; mask >>= 1) {
    wave_m = fmax_of(wave_m, __shfl_xor(wave_m, mask, kWave));
  }
  const T wave_s = wave_sum(rescaled(s, m, wave_m));
  exchange_barrier();
  if (threadIdx.x % kWave == 0) {
    lds_m[threadIdx.x / kWave] = wave_m;
    lds_s[threadIdx.x / kWave] = wave_s;
  }
  exchange_barrier();
  T top = lds_m[0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) top = fmax_of(top, lds_m[w]);
  T total = T(0);
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) total += rescaled(lds_s[w], lds_m[w], top);
  m = top;
  s = total;
}

// Forward: one streaming pass per logits row (non-temporal 16-byte loads,
// batches of eight per lane) gives the row maximum m and S = sum exp(x - m);
// then loss = -((x_t - m) - log S), the log-softmax value at the target
// negated, with log-softmax's operations.  S carries the rescaling roundings
// of the online sum (a few ulp; log-softmax's tolerance covers it).  The
// target and its logit are fetched at the start of the row.  Saves m and
// log S per row for the backward.  A row is undefined when S is NaN or the
// row has no element above -inf (log-softmax's special cases then apply,
// from a second read of that row).  An out-of-range target is never read: it
// sets *invalid.
template <typename T, typename I, bool VEC>
__global__ void __launch_bounds__(kEntropyThreads)
    entropy_forward_kernel(T* losses, T* row_max, T* row_log_sum, int32_t* undefined,
                           int32_t* invalid, const T* logits, const I* targets, uint64_t rows,
                           uint64_t classes, TargetMap map) {
  constexpr int W = VEC ? Vec16<T>::width : 1;
  constexpr int U = 8;
  using V = typename Vec16<T>::type;
  constexpr uint64_t kStep = static_cast<uint64_t>(kEntropyThreads) * W;
  for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = logits + r * classes;
    // lane 0 looks up the target and its logit while the row streams in
    bool has_target = false;
    bool target_ok = false;
    uint64_t output_index = 0;
    T target_logit = T(0);
    if (threadIdx.x == 0) {
      uint64_t target_index;
      has_target = map.lookup(r, target_index, output_index);
      if (has_target) {
        const I target = targets[target_index];
        target_ok = target >= 0 && static_cast<uint64_t>(target) < classes;
        if (target_ok) target_logit = row[static_cast<uint64_t>(target)];
      }
    }
    T m = -positive_infinity<T>();
    T s = T(0);
    // Batch `start` (the same for every lane) covers columns [start, start +
    // kStep * U): lane l reads W columns at start + l * W + u * kStep.  Whole
    // batches load without bounds tests, so their U loads go out back to
    // back (behind a test per load the compiler branched around each load
    // and waited in the middle of the batch); a partial last batch pads
    // with -inf.
    const uint64_t lane_column = static_cast<uint64_t>(threadIdx.x) * W;
    constexpr uint64_t kBatch = kStep * U;
    auto load_whole = [&](T (&x)[U * W], uint64_t start) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint64_t c = start + lane_column + u * kStep;
        if constexpr (VEC) {
          const V v = stream_load(reinterpret_cast<const V*>(row + c));
#pragma unroll
          for (int k = 0; k < W; ++k) x[u * W + k] = vec_get<T>(v, k);
        } else {
          x[u] = row[c];
        }
      }
    };
    auto update = [&](const T (&x)[U * W]) {
      T top = m;
#pragma unroll
      for (int j = 0; j < U * W; ++j) top = fmax_of(top, x[j]);
      // exp(x - top) already gives an exact 0 for x = -inf whenever top is
      // above -inf; only a lane whose elements so far are all -inf (or NaN)
      // needs exp_term's guard against -inf - -inf, so it alone recomputes.
      T batch = T(0);
#pragma unroll
      for (int j = 0; j < U * W; ++j) batch += math_exp(x[j] - top);
      if (top == -positive_infinity<T>()) {
        batch = T(0);
#pragma unroll
        for (int j = 0; j < U * W; ++j) batch += exp_term(x[j], top);
      }
      s = rescaled(s, m, top) + batch;
      m = top;
    };
    // Whole batches through two register sets used in turn: batch k + 1
    // loads while batch k is reduced, with the last one or two peeled so
    // that every load in the loop is unconditional.
    const uint64_t whole = classes / kBatch;
    uint64_t start = 0;
    if (whole > 0) {
      T xa[U * W];
      T xb[U * W];
      load_whole(xa, 0);
      uint64_t k = 0;
      for (; k + 2 < whole; k += 2) {
        load_whole(xb, start + kBatch);
        __builtin_amdgcn_sched_barrier(0);
        update(xa);
        load_whole(xa, start + 2 * kBatch);
        __builtin_amdgcn_sched_barrier(0);
        update(xb);
        start += 2 * kBatch;
      }
      if (k + 1 < whole) {
        load_whole(xb, start + kBatch);
        __builtin_amdgcn_sched_barrier(0);
        update(xa);
        update(xb);
        start += 2 * kBatch;
      } else {
        update(xa);
        start += kBatch;
      }
    }
    // A partial last batch pads with -inf.
    if (start < classes) {
      T x[U * W];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint64_t c = start + lane_column + u * kStep;
        if (c < classes) {
          if constexpr (VEC) {
            const V v = stream_load(reinterpret_cast<const V*>(row + c));
#pragma unroll
            for (int k = 0; k < W; ++k) x[u * W + k] = vec_get<T>(v, k);
          } else {
            x[u] = row[c];
          }
        } else {
#pragma unroll
          for (int k = 0; k < W; ++k) x[u * W + k] = -positive_infinity<T>();
        }
      }
      update(x);
    }
    block_online<T, kEntropyThreads>(m, s);
    const T maximum = m;
    const bool bad = s != s || maximum == -positive_infinity<T>();
    SliceStats<T> stats;
    if (bad) {
      stats_init(stats);
      for (uint64_t c = threadIdx.x; c < classes; c += kEntropyThreads) {
        stats_add(stats, row[c], static_cast<int64_t>(c));
      }
      stats = block_stats<T, kEntropyThreads>(stats);
    }
    if (threadIdx.x == 0) {
      const T log_sum = math_log(s);
      undefined[r] = bad ? 1 : 0;
      row_max[r] = maximum;
      row_log_sum[r] = log_sum;
      if (has_target) {
        if (!target_ok) {
          *invalid = 1;
          losses[output_index] = quiet_nan<T>();
        } else {
          const T lp = bad ? undefined_value<T, true>(stats, target_logit)
                           : (target_logit - maximum) - log_sum;
          losses[output_index] = -lp;
        }
      }
    }
  }
}

// Backward through NLL and log-softmax at once.  The reference's gradient of
// the selected losses is a zero tensor with g_t = 0 - u at each row's target
// (u the upstream loss gradient; cross_entropy.cpp:69-81), and log-softmax's
// backward turns it into dx = g - exp(lp) * s with s = sum of g = g_t
// (softmax.cpp:406-444).  Here lp = (x - m) - log S is recomputed with the
// forward's operations, so dx is that expression without either tensor
// materialised; undefined rows are NaN.  Single-wave workgroups over tiles of
// 64 x W x kEntropyVectors columns of one row (single-wave workgroups stream
// fastest; see elementwise.hip).  A lane issues its kEntropyVectors logit
// loads before the row's statistics loads, so two 16-byte loads per lane are
// in flight while the row's scalars arrive: 15% faster than one load per
// lane on [8192, 32768] (bitwise equal).  Tile counts below 2^31 use
// multiply-shift division.
constexpr int kEntropyTileThreads = 64;
constexpr int kEntropyVectors = 2;

template <typename T, typename I, bool VEC, bool NT>
__global__ void __launch_bounds__(kEntropyTileThreads)
    entropy_backward_kernel(T* dx, const T* loss_gradient, const T* logits, const T* row_max,
                            const T* row_log_sum, const int32_t* undefined, const I* targets,
                            uint64_t rows, uint64_t classes, uint64_t column_tiles,
                            FastDiv tiles_per_row, TargetMap map) {
  constexpr int W = VEC ? Vec16<T>::width : 1;
  constexpr int U = kEntropyVectors;
  constexpr uint64_t kSpan = static_cast<uint64_t>(kEntropyTileThreads) * W;  // columns per load step
  using V = typename Vec16<T>::type;
  const uint64_t tiles = rows * column_tiles;
  const bool small = tiles <= kIndex32Limit;
  for (uint64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const uint64_t r = small ? tiles_per_row.div(static_cast<uint32_t>(tile)) : tile / column_tiles;
    const uint64_t c0 = (tile - r * column_tiles) * kSpan * U + threadIdx.x * W;
    if (c0 >= classes) continue;
    const T* row = logits + r * classes;
    T values[U][W];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t c = c0 + u * kSpan;
      if (c < classes) {
        if constexpr (VEC) {
          const V v = stream_load(reinterpret_cast<const V*>(row + c));
#pragma unroll
          for (int k = 0; k < W; ++k) values[u][k] = vec_get<T>(v, k);
        } else {
          values[u][0] = row[c];
        }
      }
    }
    uint64_t target_index, output_index;
    T g_t = T(0);
    uint64_t t = classes;  // no target column
    if (map.lookup(r, target_index, output_index)) {
      g_t = T(0) - loss_gradient[output_index];
      t = static_cast<uint64_t>(targets[target_index]);
    }
    const bool bad = undefined[r] != 0;
    const T m = row_max[r];
    const T log_sum = row_log_sum[r];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t c = c0 + u * kSpan;
      if (c >= classes) continue;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const T lp = (values[u][k] - m) - log_sum;
        const T g = (c + k == t) ? g_t : T(0);
        values[u][k] = bad ? quiet_nan<T>() : g - math_exp(lp) * g_t;
      }
      if constexpr (VEC) {
        V o;
#pragma unroll
        for (int k = 0; k < W; ++k) vec_set<T>(o, k, values[u][k]);
        store_vector<NT>(reinterpret_cast<V*>(dx + r * classes + c), o);
      } else {
        dx[r * classes + c] = values[u][0];
      }
    }
  }
}

// The reference's separate NLL kernels (cuda_kernels.cu:313-365), for callers
// that keep the composed log_softmax -> NLL path.
template <typename I>
__global__ void __launch_bounds__(256)
    validate_targets_kernel(int32_t* invalid, const I* targets, uint64_t count, uint64_t classes) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
       i += stride) {
    const I target = targets[i];
    if (target < 0 || static_cast<uint64_t>(target) >= classes) *invalid = 1;
  }
}

struct OutputMap {
  uint64_t sequence_length;  // 0: plain
  __device__ __forceinline__ void lookup(uint64_t index, uint64_t& target_index,
                                         uint64_t& source_row) const {
    if (sequence_length == 0) {
      target_index = index;
      source_row = index;
      return;
    }
    const uint64_t prediction = sequence_length - 1;
    const uint64_t batch = index / prediction;
    const uint64_t time = index - batch * prediction;
    target_index = batch * sequence_length + time + 1;
    source_row = batch * sequence_length + time;
  }
};

template <typename T, typename I>
__global__ void __launch_bounds__(256)
    nll_forward_kernel(T* output, const T* log_probabilities, const I* targets, uint64_t count,
                       uint64_t classes, OutputMap map) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
       i += stride) {
    uint64_t target_index, source_row;
    map.lookup(i, target_index, source_row);
    output[i] = -log_probabilities[source_row * classes + static_cast<uint64_t>(targets[target_index])];
  }
}

template <typename T, typename I>
__global__ void __launch_bounds__(256)
    nll_backward_kernel(T* output, const T* gradient, const I* targets, uint64_t count,
                        uint64_t classes, OutputMap map) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
       i += stride) {
    uint64_t target_index, source_row;
    map.lookup(i, target_index, source_row);
    // the CPU path's values[...] -= upstream over a zero tensor (cross_entropy.cpp:78-80)
    output[source_row * classes + static_cast<uint64_t>(targets[target_index])] = T(0) - gradient[i];
  }
}

uint32_t stride_grid(uint64_t count, const DeviceGuard& guard) {
  uint64_t blocks = (count + 255) / 256;
  const uint64_t cap = static_cast<uint64_t>(guard.multiprocessors) * 16;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  return static_cast<uint32_t>(blocks);
}

bool valid_target_dtype(int dtype) { return dtype == SPAR_HIP_INT32 || dtype == SPAR_HIP_INT64; }

bool geometry_ok(uint64_t outer, uint64_t axis_extent, uint64_t inner) {
  if (inner == 0 || outer == 0 || axis_extent == 0) return false;
  if (outer > UINT64_MAX / inner) return false;
  if (outer * inner > UINT64_MAX / axis_extent) return false;
  return true;
}

}  // namespace
}  // namespace spar_hip

using namespace spar_hip;

extern "C" SparHipStatus spar_hip_launch_probability_forward(void* output,
                                                             int32_t* undefined_slices,
                                                             const void* input, uint64_t outer,
                                                             uint64_t axis_extent, uint64_t inner,
                                                             int dtype, int logarithmic,
                                                             int device) {
  if (!geometry_ok(outer, axis_extent, inner) || !valid_float_dtype(dtype) ||
      (logarithmic != 0 && logarithmic != 1) || output == nullptr ||
      undefined_slices == nullptr || input == nullptr) {
    return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (dtype == SPAR_HIP_FLOAT32) {
    if (logarithmic) {
      forward<float, true>(output, undefined_slices, input, outer, axis_extent, inner, guard);
    } else {
      forward<float, false>(output, undefined_slices, input, outer, axis_extent, inner, guard);
    }
  } else {
    if (logarithmic) {
      forward<double, true>(output, undefined_slices, input, outer, axis_extent, inner, guard);
    } else {
      forward<double, false>(output, undefined_slices, input, outer, axis_extent, inner, guard);
    }
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_probability_backward(
    void* output, const void* gradient, const void* saved_output, const int32_t* undefined_slices,
    uint64_t outer, uint64_t axis_extent, uint64_t inner, int dtype, int logarithmic, int device) {
  if (!geometry_ok(outer, axis_extent, inner) || !valid_float_dtype(dtype) ||
      (logarithmic != 0 && logarithmic != 1) || output == nullptr || gradient == nullptr ||
      saved_output == nullptr || undefined_slices == nullptr) {
    return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (dtype == SPAR_HIP_FLOAT32) {
    if (logarithmic) {
      backward<float, true>(output, gradient, saved_output, undefined_slices, outer, axis_extent,
                            inner, guard);
    } else {
      backward<float, false>(output, gradient, saved_output, undefined_slices, outer, axis_extent,
                             inner, guard);
    }
  } else {
    if (logarithmic) {
      backward<double, true>(output, gradient, saved_output, undefined_slices, outer, axis_extent,
                             inner, guard);
    } else {
      backward<double, false>(output, gradient, saved_output, undefined_slices, outer,
                              axis_extent, inner, guard);
    }
  }
  return finish(guard);
}

namespace {

template <typename T, typename I>
void launch_entropy_forward(void* losses, void* row_max, void* row_log_sum,
                            int32_t* undefined_rows, int32_t* invalid, const void* logits,
                            const void* targets, uint64_t rows, uint64_t classes,
                            TargetMap map, const DeviceGuard& guard) {
  const bool vec = classes % Vec16<T>::width == 0 && aligned16(logits);
  auto launch = [&](auto kernel) {
    kernel<<<grid_for(rows), kEntropyThreads, 0, guard.stream>>>(
        static_cast<T*>(losses), static_cast<T*>(row_max), static_cast<T*>(row_log_sum),
        undefined_rows, invalid, static_cast<const T*>(logits), static_cast<const I*>(targets),
        rows, classes, map);
  };
  if (vec) {
    launch(entropy_forward_kernel<T, I, true>);
  } else {
    launch(entropy_forward_kernel<T, I, false>);
  }
}

template <typename T, typename I>
void launch_entropy_backward(void* logits_gradient, const void* loss_gradient,
                             const void* logits, const void* row_max, const void* row_log_sum,
                             const int32_t* undefined_rows, const void* targets, uint64_t rows,
                             uint64_t classes, TargetMap map, const DeviceGuard& guard) {
  const bool vec = classes % Vec16<T>::width == 0 && aligned16(logits) &&
                   aligned16(logits_gradient);
  const uint64_t tile_columns = kEntropyTileThreads * (vec ? Vec16<T>::width : 1) * kEntropyVectors;
  const uint64_t column_tiles = (classes + tile_columns - 1) / tile_columns;
  FastDiv tiles_per_row;
  tiles_per_row.init(column_tiles <= kIndex32Limit ? static_cast<uint32_t>(column_tiles) : 1U);
  auto launch = [&](auto kernel) {
    kernel<<<grid_for(rows * column_tiles), kEntropyTileThreads, 0, guard.stream>>>(
        static_cast<T*>(logits_gradient), static_cast<const T*>(loss_gradient),
        static_cast<const T*>(logits), static_cast<const T*>(row_max),
        static_cast<const T*>(row_log_sum), undefined_rows, static_cast<const I*>(targets), rows,
        classes, column_tiles, tiles_per_row, map);
  };
  if (vec) {
    with_policy(stream_output(rows * classes * sizeof(T)), [&](auto nt) {
      launch(entropy_backward_kernel<T, I, true, decltype(nt)::value>);
    });
  } else {
    launch(entropy_backward_kernel<T, I, false, false>);
  }
}

bool entropy_geometry_ok(uint64_t rows, uint64_t classes, uint64_t sequence_length,
                         int language_model) {
  if (rows == 0 || classes == 0 || classes > kIndex32Limit) return false;
  if (language_model != 0 && language_model != 1) return false;
  if (language_model) return sequence_length >= 2 && rows % sequence_length == 0;
  return rows <= UINT64_MAX / classes;
}

}  // namespace

// Validates class indices: *invalid_target (host memory) becomes 1 if any
// target is negative or >= classes.  Synchronises.
extern "C" SparHipStatus spar_hip_validate_targets(int32_t* invalid_target, const void* targets,
                                                   uint64_t count, uint64_t classes,
                                                   int target_dtype, int device) {
  if (invalid_target == nullptr || !valid_target_dtype(target_dtype) || classes == 0 ||
      (count != 0 && targets == nullptr)) {
    return invalid();
  }
  *invalid_target = 0;
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  void* flag = nullptr;
  hipError_t error = scratch_allocate(&flag, sizeof(int32_t), device);
  if (error != hipSuccess) return runtime(error);
  SparHipStatus status = spar_hip_zero(flag, sizeof(int32_t), device);
  if (status.code == 0) {
    if (target_dtype == SPAR_HIP_INT32) {
      validate_targets_kernel<int32_t><<<stride_grid(count, guard), 256, 0, guard.stream>>>(
          static_cast<int32_t*>(flag), static_cast<const int32_t*>(targets), count, classes);
    } else {
      validate_targets_kernel<int64_t><<<stride_grid(count, guard), 256, 0, guard.stream>>>(
          static_cast<int32_t*>(flag), static_cast<const int64_t*>(targets), count, classes);
    }
    status = finish(guard);
  }
  if (status.code == 0) status = spar_hip_copy_device_to_host(invalid_target, flag, sizeof(int32_t), device);
  scratch_release(flag, device);
  return status;
}

extern "C" SparHipStatus spar_hip_launch_nll_forward(void* output, const void* log_probabilities,
                                                     const void* targets, uint64_t output_count,
                                                     uint64_t classes, uint64_t sequence_length,
                                                     int dtype, int target_dtype,
                                                     int language_model, int device) {
  if (!valid_float_dtype(dtype) || !valid_target_dtype(target_dtype) || classes == 0 ||
      (language_model != 0 && language_model != 1) || (language_model && sequence_length < 2) ||
      (output_count != 0 && (output == nullptr || log_probabilities == nullptr || targets == nullptr))) {
    return invalid();
  }
  if (output_count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const OutputMap map{language_model ? sequence_length : 0};
  const uint32_t grid = stride_grid(output_count, guard);
  if (dtype == SPAR_HIP_FLOAT32) {
    if (target_dtype == SPAR_HIP_INT32) {
      nll_forward_kernel<float, int32_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<float*>(output), static_cast<const float*>(log_probabilities),
          static_cast<const int32_t*>(targets), output_count, classes, map);
    } else {
      nll_forward_kernel<float, int64_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<float*>(output), static_cast<const float*>(log_probabilities),
          static_cast<const int64_t*>(targets), output_count, classes, map);
    }
  } else {
    if (target_dtype == SPAR_HIP_INT32) {
      nll_forward_kernel<double, int32_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<double*>(output), static_cast<const double*>(log_probabilities),
          static_cast<const int32_t*>(targets), output_count, classes, map);
    } else {
      nll_forward_kernel<double, int64_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<double*>(output), static_cast<const double*>(log_probabilities),
          static_cast<const int64_t*>(targets), output_count, classes, map);
    }
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_nll_backward(void* output, const void* gradient,
                                                      const void* targets, uint64_t output_count,
                                                      uint64_t classes, uint64_t sequence_length,
                                                      int dtype, int target_dtype,
                                                      int language_model, int device) {
  if (!valid_float_dtype(dtype) || !valid_target_dtype(target_dtype) || classes == 0 ||
      (language_model != 0 && language_model != 1) || (language_model && sequence_length < 2) ||
      (output_count != 0 && (output == nullptr || gradient == nullptr || targets == nullptr))) {
    return invalid();
  }
  if (output_count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const OutputMap map{language_model ? sequence_length : 0};
  const uint32_t grid = stride_grid(output_count, guard);
  if (dtype == SPAR_HIP_FLOAT32) {
    if (target_dtype == SPAR_HIP_INT32) {
      nll_backward_kernel<float, int32_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<float*>(output), static_cast<const float*>(gradient),
          static_cast<const int32_t*>(targets), output_count, classes, map);
    } else {
      nll_backward_kernel<float, int64_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<float*>(output), static_cast<const float*>(gradient),
          static_cast<const int64_t*>(targets), output_count, classes, map);
    }
  } else {
    if (target_dtype == SPAR_HIP_INT32) {
      nll_backward_kernel<double, int32_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<double*>(output), static_cast<const double*>(gradient),
          static_cast<const int32_t*>(targets), output_count, classes, map);
    } else {
      nll_backward_kernel<double, int64_t><<<grid, 256, 0, guard.stream>>>(
          static_cast<double*>(output), static_cast<const double*>(gradient),
          static_cast<const int64_t*>(targets), output_count, classes, map);
    }
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_cross_entropy_forward(
    void* losses, void* row_max, void* row_log_sum, int32_t* undefined_rows,
    int32_t* invalid_target, const void* logits, const void* targets, uint64_t logits_rows,
    uint64_t classes, uint64_t sequence_length, int dtype, int target_dtype, int language_model,
    int device) {
  if (!valid_float_dtype(dtype) || !valid_target_dtype(target_dtype) ||
      !entropy_geometry_ok(logits_rows, classes, sequence_length, language_model) ||
      losses == nullptr || row_max == nullptr || row_log_sum == nullptr ||
      undefined_rows == nullptr || invalid_target == nullptr || logits == nullptr ||
      targets == nullptr) {
    return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  SparHipStatus status = spar_hip_zero(invalid_target, sizeof(int32_t), device);
  if (status.code != 0) return status;
  const TargetMap map{language_model ? sequence_length : 0};
  if (dtype == SPAR_HIP_FLOAT32) {
    if (target_dtype == SPAR_HIP_INT32) {
      launch_entropy_forward<float, int32_t>(losses, row_max, row_log_sum, undefined_rows,
                                             invalid_target, logits, targets, logits_rows,
                                             classes, map, guard);
    } else {
      launch_entropy_forward<float, int64_t>(losses, row_max, row_log_sum, undefined_rows,
                                             invalid_target, logits, targets, logits_rows,
                                             classes, map, guard);
    }
  } else {
    if (target_dtype == SPAR_HIP_INT32) {
      launch_entropy_forward<double, int32_t>(losses, row_max, row_log_sum, undefined_rows,
                                              invalid_target, logits, targets, logits_rows,
                                              classes, map, guard);
    } else {
      launch_entropy_forward<double, int64_t>(losses, row_max, row_log_sum, undefined_rows,
                                              invalid_target, logits, targets, logits_rows,
                                              classes, map, guard);
    }
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_cross_entropy_backward(
    void* logits_gradient, const void* loss_gradient, const void* logits, const void* row_max,
    const void* row_log_sum, const int32_t* undefined_rows, const void* targets,
    uint64_t logits_rows, uint64_t classes, uint64_t sequence_length, int dtype,
    int target_dtype, int language_model, int device) {
  if (!valid_float_dtype(dtype) || !valid_target_dtype(target_dtype) ||
      !entropy_geometry_ok(logits_rows, classes, sequence_length, language_model) ||
      logits_gradient == nullptr || loss_gradient == nullptr || logits == nullptr ||
      row_max == nullptr || row_log_sum == nullptr || undefined_rows == nullptr ||
      targets == nullptr) {
    return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const TargetMap map{language_model ? sequence_length : 0};
  if (dtype == SPAR_HIP_FLOAT32) {
    if (target_dtype == SPAR_HIP_INT32) {
      launch_entropy_backward<float, int32_t>(logits_gradient, loss_gradient, logits, row_max,
                                              row_log_sum, undefined_rows, targets, logits_rows,
                                              classes, map, guard);
    } else {
      launch_entropy_backward<float, int64_t>(logits_gradient, loss_gradient, logits, row_max,
                                              row_log_sum, undefined_rows, targets, logits_rows,
                                              classes, map, guard);
    }
  } else {
    if (target_dtype == SPAR_HIP_INT32) {
      launch_entropy_backward<double, int32_t>(logits_gradient, loss_gradient, logits, row_max,
                                               row_log_sum, undefined_rows, targets, logits_rows,
                                               classes, map, guard);
    } else {
      launch_entropy_backward<double, int64_t>(logits_gradient, loss_gradient, logits, row_max,
                                               row_log_sum, undefined_rows, targets, logits_rows,
                                               classes, map, guard);
    }
  }
  return finish(guard);
}
