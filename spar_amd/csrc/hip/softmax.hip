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
//   pass over registers 1: max (first occurrence), NaN flag, +inf count;
//   workgroup combine through wave64 shuffles and a 16-entry LDS exchange;
//   pass 2: e = exp(x - max), sum; pass 3: p = e / sum (log: (x-max) - log sum).
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

template <typename T, int THREADS>
__device__ __forceinline__ SliceStats<T> block_stats(SliceStats<T> s) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ SliceStats<T> lds[kWavesPerBlock];
  s = wave_stats(s);
  __syncthreads();
  if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = s;
  __syncthreads();
  SliceStats<T> total = lds[0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) stats_merge(total, lds[w]);
  return total;
}

template <typename T, int THREADS>
__device__ __forceinline__ T block_sum(T value) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ T lds[kWavesPerBlock];
  value = wave_sum(value);
  __syncthreads();
  if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = value;
  __syncthreads();
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

template <typename T>
__device__ __forceinline__ bool slice_undefined(const SliceStats<T>& s) {
  return s.nan != 0 || s.value == -positive_infinity<T>() || s.positive_infinities != 0;
}

// Element j of a thread's register array maps to column col(t, j):
// VEC: 16-byte groups interleaved across lanes; scalar: lanes interleaved.
template <typename T, int THREADS, bool VEC>
__device__ __forceinline__ uint64_t column_of(int j) {
  if constexpr (VEC) {
    constexpr int W = Vec16<T>::width;
    return (static_cast<uint64_t>(j / W) * THREADS + threadIdx.x) * W + (j % W);
  } else {
    return static_cast<uint64_t>(j) * THREADS + threadIdx.x;
  }
}

template <typename T, int THREADS, int E, bool VEC, bool FULL>
__device__ __forceinline__ void load_row(T (&x)[E], const T* row, uint64_t n) {
  if constexpr (VEC) {
    using V = typename Vec16<T>::type;
    constexpr int W = Vec16<T>::width;
#pragma unroll
    for (int v = 0; v < E / W; ++v) {
      const uint64_t col = (static_cast<uint64_t>(v) * THREADS + threadIdx.x) * W;
      if (FULL || col < n) {
        const V value = stream_load(reinterpret_cast<const V*>(row + col));
#pragma unroll
        for (int k = 0; k < W; ++k) x[v * W + k] = vec_get<T>(value, k);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t col = column_of<T, THREADS, false>(j);
      if (FULL || col < n) x[j] = row[col];
    }
  }
}

template <typename T, int THREADS, int E, bool VEC, bool FULL>
__device__ __forceinline__ void store_row(T* row, const T (&y)[E], uint64_t n) {
  if constexpr (VEC) {
    using V = typename Vec16<T>::type;
    constexpr int W = Vec16<T>::width;
#pragma unroll
    for (int v = 0; v < E / W; ++v) {
      const uint64_t col = (static_cast<uint64_t>(v) * THREADS + threadIdx.x) * W;
      if (FULL || col < n) {
        V value;
#pragma unroll
        for (int k = 0; k < W; ++k) vec_set<T>(value, k, y[v * W + k]);
        *reinterpret_cast<V*>(row + col) = value;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t col = column_of<T, THREADS, false>(j);
      if (FULL || col < n) row[col] = y[j];
    }
  }
}

// ----------------------------------------------------- register-row kernels

template <typename T, int THREADS, int E, bool LOG, bool VEC, bool FULL>
__global__ void __launch_bounds__(THREADS)
    forward_row_kernel(T* out, int32_t* undefined, const T* in, uint64_t rows, uint64_t n) {
  for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = in + r * n;
    T x[E];
    load_row<T, THREADS, E, VEC, FULL>(x, row, n);
    SliceStats<T> s;
    stats_init(s);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t col = column_of<T, THREADS, VEC>(j);
      if (FULL || col < n) stats_add(s, x[j], static_cast<int64_t>(col));
    }
    s = block_stats<T, THREADS>(s);
    const bool bad = slice_undefined(s);
    if (threadIdx.x == 0) undefined[r] = bad ? 1 : 0;
    // The results overwrite x in place so one row costs E registers per lane.
    if (bad) {
#pragma unroll
      for (int j = 0; j < E; ++j) x[j] = undefined_value<T, LOG>(s, x[j]);
    } else {
      const T maximum = s.value;
      T local = T(0);
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const uint64_t col = column_of<T, THREADS, VEC>(j);
        if constexpr (LOG) {
          x[j] = x[j] - maximum;
          if (FULL || col < n) local += math_exp(x[j]);
        } else {
          x[j] = math_exp(x[j] - maximum);
          if (FULL || col < n) local += x[j];
        }
      }
      const T total = block_sum<T, THREADS>(local);
      if constexpr (LOG) {
        const T log_sum = math_log(total);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = x[j] - log_sum;
      } else {
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = x[j] / total;
      }
    }
    store_row<T, THREADS, E, VEC, FULL>(out + r * n, x, n);
  }
}

template <typename T, int THREADS, int E, bool LOG, bool VEC, bool FULL>
__global__ void __launch_bounds__(THREADS)
    backward_row_kernel(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                        uint64_t rows, uint64_t n) {
  for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    T* out_row = out + r * n;
    T g[E];
    if (undefined[r] != 0) {
#pragma unroll
      for (int j = 0; j < E; ++j) g[j] = quiet_nan<T>();
      store_row<T, THREADS, E, VEC, FULL>(out_row, g, n);
      continue;
    }
    T y[E];
    load_row<T, THREADS, E, VEC, FULL>(g, gradient + r * n, n);
    load_row<T, THREADS, E, VEC, FULL>(y, saved + r * n, n);
    T local = T(0);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t col = column_of<T, THREADS, VEC>(j);
      if (FULL || col < n) {
        if constexpr (LOG) {
          local += g[j];
        } else {
          local += g[j] * y[j];
        }
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
    store_row<T, THREADS, E, VEC, FULL>(out_row, g, n);
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
    for (uint64_t c = threadIdx.x; c < n; c += kLoopThreads) {
      if constexpr (LOG) {
        out_row[c] = (row[c] - maximum) - log_sum;
      } else {
        out_row[c] = math_exp(row[c] - maximum) / total;
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
    for (uint64_t a = 0; a < axis_extent; ++a) {
      if constexpr (LOG) {
        out_base[a * inner] = (base[a * inner] - maximum) - log_sum;
      } else {
        out_base[a * inner] = math_exp(base[a * inner] - maximum) / total;
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
template <typename T, int THREADS, int E, bool LOG, bool VEC>
void forward_rows(T* out, int32_t* undefined, const T* in, uint64_t rows, uint64_t n,
                  hipStream_t stream) {
  if (n == static_cast<uint64_t>(THREADS) * E) {
    forward_row_kernel<T, THREADS, E, LOG, VEC, true>
        <<<grid_for(rows), THREADS, 0, stream>>>(out, undefined, in, rows, n);
  } else {
    forward_row_kernel<T, THREADS, E, LOG, VEC, false>
        <<<grid_for(rows), THREADS, 0, stream>>>(out, undefined, in, rows, n);
  }
}

template <typename T, int THREADS, int E, bool LOG, bool VEC>
void backward_rows(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                   uint64_t rows, uint64_t n, hipStream_t stream) {
  if (n == static_cast<uint64_t>(THREADS) * E) {
    backward_row_kernel<T, THREADS, E, LOG, VEC, true>
        <<<grid_for(rows), THREADS, 0, stream>>>(out, gradient, saved, undefined, rows, n);
  } else {
    backward_row_kernel<T, THREADS, E, LOG, VEC, false>
        <<<grid_for(rows), THREADS, 0, stream>>>(out, gradient, saved, undefined, rows, n);
  }
}

template <typename T, bool LOG, bool VEC>
bool launch_forward_rows(T* out, int32_t* undefined, const T* in, uint64_t rows, uint64_t n,
                         hipStream_t stream) {
  if (n <= 256 * 4) {
    forward_rows<T, 256, 4, LOG, VEC>(out, undefined, in, rows, n, stream);
  } else if (n <= 256 * 16) {
    forward_rows<T, 256, 16, LOG, VEC>(out, undefined, in, rows, n, stream);
  } else if (n <= 512 * 16) {
    forward_rows<T, 512, 16, LOG, VEC>(out, undefined, in, rows, n, stream);
  } else if (n <= 1024 * 16) {
    forward_rows<T, 1024, 16, LOG, VEC>(out, undefined, in, rows, n, stream);
  } else if (n <= 1024 * 32) {
    forward_rows<T, 1024, 32, LOG, VEC>(out, undefined, in, rows, n, stream);
  } else {
    return false;
  }
  return true;
}

template <typename T, bool LOG, bool VEC>
bool launch_backward_rows(T* out, const T* gradient, const T* saved, const int32_t* undefined,
                          uint64_t rows, uint64_t n, hipStream_t stream) {
  if (n <= 256 * 4) {
    backward_rows<T, 256, 4, LOG, VEC>(out, gradient, saved, undefined, rows, n, stream);
  } else if (n <= 256 * 16) {
    backward_rows<T, 256, 16, LOG, VEC>(out, gradient, saved, undefined, rows, n, stream);
  } else if (n <= 512 * 16) {
    backward_rows<T, 512, 16, LOG, VEC>(out, gradient, saved, undefined, rows, n, stream);
  } else if (n <= 1024 * 16) {
    backward_rows<T, 1024, 16, LOG, VEC>(out, gradient, saved, undefined, rows, n, stream);
  } else if (n <= 1024 * 32) {
    backward_rows<T, 1024, 32, LOG, VEC>(out, gradient, saved, undefined, rows, n, stream);
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
    const bool done = vec ? launch_forward_rows<T, LOG, true>(out, undefined, in, outer, axis, guard.stream)
                          : launch_forward_rows<T, LOG, false>(out, undefined, in, outer, axis, guard.stream);
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
        vec ? launch_backward_rows<T, LOG, true>(out, g, y, undefined, outer, axis, guard.stream)
            : launch_backward_rows<T, LOG, false>(out, g, y, undefined, outer, axis, guard.stream);
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
