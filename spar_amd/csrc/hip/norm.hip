// Fused row normalisation over the last axis: LayerNorm
//   mu = sum(x) / n, xc = x - mu, var = sum(xc * xc) / n, d = sqrt(var + eps),
//   y = (xc / d) * weight + bias
// and RMSNorm (the same without centring or bias)
//   d = sqrt(sum(x * x) / n + eps), y = (x / d) * weight.
//
// Spar composes these from separate ops: RMSNorm::forward is
// multiply(divide(x, sqrt(add_scalar(mean(square(x), -1, true), eps))), w)
// (src/nn/rmsnorm.cpp:50-52), about six tensor passes forward and a dozen
// backward through autograd.  Here the forward reads x once and writes y once;
// the backward reads x and dy once and writes dx once, and the weight / bias
// gradients come from per-workgroup column partials combined in a fixed order.
//
// Each element is computed with the composed path's float operations (mean as
// a sum divided by (T)n, eps rounded to T before the add, IEEE sqrt); only the
// order of the row sums differs (a tree instead of a sequential scan).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.hpp"

namespace spar_hip {
namespace {

constexpr uint64_t kMaxGrid = uint64_t{1} << 20;

template <typename T, int THREADS>
__device__ __forceinline__ T norm_block_sum(T value) {
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

// Two sums at once (one exchange instead of two).
template <typename T, int THREADS>
__device__ __forceinline__ void norm_block_sum2(T& a, T& b) {
  constexpr int kWavesPerBlock = THREADS / kWave;
  __shared__ T lds[2][kWavesPerBlock];
  a = wave_sum(a);
  b = wave_sum(b);
  __syncthreads();
  if (threadIdx.x % kWave == 0) {
    lds[0][threadIdx.x / kWave] = a;
    lds[1][threadIdx.x / kWave] = b;
  }
  __syncthreads();
  a = lds[0][0];
  b = lds[1][0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) {
    a += lds[0][w];
    b += lds[1][w];
  }
}

// Element j of a lane's register array sits at column col(j): 16-byte groups
// interleaved across lanes (VEC) or single elements interleaved (scalar).
template <typename T, int THREADS, bool VEC>
__device__ __forceinline__ uint64_t norm_column(int j) {
  if constexpr (VEC) {
    constexpr int W = Vec16<T>::width;
    return (static_cast<uint64_t>(j / W) * THREADS + threadIdx.x) * W + (j % W);
  } else {
    return static_cast<uint64_t>(j) * THREADS + threadIdx.x;
  }
}

template <typename T, int THREADS, int E, bool VEC, bool FULL>
__device__ __forceinline__ void norm_load(T (&x)[E], const T* row, uint64_t n) {
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
      } else {
#pragma unroll
        for (int k = 0; k < W; ++k) x[v * W + k] = T(0);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t col = norm_column<T, THREADS, false>(j);
      x[j] = (FULL || col < n) ? row[col] : T(0);
    }
  }
}

// Cached loads of a per-column parameter (weight or bias), re-read per row.
template <typename T, int THREADS, int E, bool VEC, bool FULL>
__device__ __forceinline__ void norm_load_parameter(T (&p)[E], const T* parameter, uint64_t n) {
  if constexpr (VEC) {
    using V = typename Vec16<T>::type;
    constexpr int W = Vec16<T>::width;
#pragma unroll
    for (int v = 0; v < E / W; ++v) {
      const uint64_t col = (static_cast<uint64_t>(v) * THREADS + threadIdx.x) * W;
      if (FULL || col < n) {
        const V value = *reinterpret_cast<const V*>(parameter + col);
#pragma unroll
        for (int k = 0; k < W; ++k) p[v * W + k] = vec_get<T>(value, k);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t col = norm_column<T, THREADS, false>(j);
      if (FULL || col < n) p[j] = parameter[col];
    }
  }
}

// NT: non-temporal stores (outputs of 64 MiB or more).
template <typename T, int THREADS, int E, bool VEC, bool FULL, bool NT>
__device__ __forceinline__ void norm_store(T* row, const T (&y)[E], uint64_t n) {
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
        store_vector<NT>(reinterpret_cast<V*>(row + col), value);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t col = norm_column<T, THREADS, false>(j);
      if (FULL || col < n) row[col] = y[j];
    }
  }
}

// An output gradient handed over as factor x one value (the gradient of a
// product whose other operand needs none, fed a single value broadcast): dy
// = value * factor for each present element, with the one rounding the
// product op gives it and the value on the left as the product op has it;
// absent (zero) elements stay zero.
template <typename T, int THREADS, int E, bool VEC, bool FULL>
__device__ __forceinline__ void norm_scale(T (&g)[E], T value, uint64_t n) {
#pragma unroll
  for (int j = 0; j < E; ++j) {
    if (FULL || norm_column<T, THREADS, VEC>(j) < n) g[j] = value * g[j];
  }
}

template <typename T, typename V>
__device__ __forceinline__ V scale_granule(T value, V v) {
  V out;
#pragma unroll
  for (int k = 0; k < Vec16<T>::width; ++k) vec_set<T>(out, k, value * vec_get<T>(v, k));
  return out;
}

// q / d for many q and one d: q0 = q * (1 / d) corrected by one residual
// step through a fused multiply-add (Markstein), within one ulp of the IEEE
// quotient and equal to it in almost all cases.
template <typename T>
struct Divisor {
  T d;
  T r;
  __device__ __forceinline__ explicit Divisor(T value) : d(value), r(T(1) / value) {}
  // `reciprocal` must be T(1) / value, computed once for many Divisors.
  __device__ __forceinline__ Divisor(T value, T reciprocal) : d(value), r(reciprocal) {}
  __device__ __forceinline__ T operator()(T q) const {
    const T q0 = q * r;
    return __builtin_fma(__builtin_fma(-q0, d, q), r, q0);
  }
};

template <>
__device__ __forceinline__ float Divisor<float>::operator()(float q) const {
  const float q0 = q * r;
  return __builtin_fmaf(__builtin_fmaf(-q0, d, q), r, q0);
}

template <typename T> __device__ __forceinline__ T norm_sqrt(T x);
template <> __device__ __forceinline__ float norm_sqrt<float>(float x) { return sqrtf(x); }
template <> __device__ __forceinline__ double norm_sqrt<double>(double x) { return sqrt(x); }

// Forward: the row held in registers.  One workgroup per row (the launcher
// issues grids of at most kMaxGrid rows): without a row loop the compiler
// keeps nothing live across rows, and the kernel measured 5% faster than a
// grid-stride loop on [4096, 8192] and [8192, 8192] (bitwise equal).
template <typename T, int THREADS, int E, bool CENTER, bool VEC, bool FULL, bool NT>
__global__ void __launch_bounds__(THREADS)
    norm_forward_kernel(T* out, T* mean_out, T* denominator_out, const T* in, uint64_t in_stride,
                        const T* weight, const T* bias, uint64_t n, T eps) {
  const T count = static_cast<T>(n);
  {
    const uint64_t r = blockIdx.x;
    T x[E];
    norm_load<T, THREADS, E, VEC, FULL>(x, in + r * in_stride, n);
    T mu = T(0);
    if constexpr (CENTER) {
      T local = T(0);
#pragma unroll
      for (int j = 0; j < E; ++j) local += x[j];  // out-of-range entries are zero
      mu = norm_block_sum<T, THREADS>(local) / count;
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const uint64_t col = norm_column<T, THREADS, VEC>(j);
        x[j] = (FULL || col < n) ? x[j] - mu : T(0);
      }
    }
    T local = T(0);
#pragma unroll
    for (int j = 0; j < E; ++j) local += x[j] * x[j];
    const T variance = norm_block_sum<T, THREADS>(local) / count;
    const T d = norm_sqrt<T>(variance + eps);
    if (threadIdx.x == 0) {
      if constexpr (CENTER) mean_out[r] = mu;
      denominator_out[r] = d;
    }
    const Divisor<T> divide(d);
    T w[E];
    norm_load_parameter<T, THREADS, E, VEC, FULL>(w, weight, n);
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = divide(x[j]) * w[j];
    if constexpr (CENTER) {
      norm_load_parameter<T, THREADS, E, VEC, FULL>(w, bias, n);
#pragma unroll
      for (int j = 0; j < E; ++j) x[j] = x[j] + w[j];
    }
    norm_store<T, THREADS, E, VEC, FULL, NT>(out + r * n, x, n);
  }
}

// ------------------------------------------------ rows down storage columns
//
// The same forward over a view whose rows run down the columns of its
// storage: x[p][q] = in[p + q * pitch] for p < rows, q < n, with pitch >=
// rows (x.transpose(0, 1) of a row-major [n, pitch] block).  A row of x is
// then a column of the storage, and reading it as a row would take one
// 4-byte piece of n different storage rows.  Two passes over x replace the
// transposing copy and the row kernel (four passes):
//
//  1. norm_column_stats_kernel.  A workgroup owns a strip of kStatGroups
//     16-byte groups of adjacent p (128 bytes of each storage row) and one of
//     `splits` ranges of q.  Lane t takes group t % kStatGroups and q rows
//     t / kStatGroups, + kStatRows, ..., R rows in flight, and sums in double
//     s1 = sum(x - k) and s2 = sum((x - k)^2) with the shift k = x[p][0]
//     (RMSNorm: k = 0 and only s2).  The kStatRows lanes of a group are
//     added by a fixed LDS tree; the result is the pair partial[split][p].
//  2. norm_apply_columns_kernel.  Tiles of 32 W values of p by 32 W values
//     of q, staged through LDS as in the transposing elementwise path (XOR
//     swizzle, the next tile's loads in flight during the stores, rotated
//     tile order).  Before its stores a tile adds the partials of its p in
//     split order: mean = k + s1 / n and var = (s2 - s1^2 / n) / n in double,
//     rounded to T, then d = sqrt(var + eps) in T; the tiles of the first q
//     column also write mean and d.  Each element is then computed as the
//     row kernel computes it: y = (x - mean) / d * weight + bias, with the
//     same quotient and the same order of float operations.
//
// The statistics are summed around a shift in double, so they are at least
// as accurate as the row kernel's float sums; the two layouts agree within
// rounding of the statistics, not bit for bit.
constexpr int kStatThreads = 256;
constexpr int kStatGroups = 8;
constexpr int kStatRows = kStatThreads / kStatGroups;
constexpr int kStatBatch = 8;        // q rows in flight per lane
constexpr int kMaxStatSplits = 4;    // partials a tile adds (held in registers)
constexpr int kApplyThreads = 256;
constexpr int kApplyGranules = 32;   // tile side in 16-byte granules
// Inputs up to this size take cached loads in the statistics pass (the
// Infinity Cache holds 256 MB; the margin leaves room for the output).
constexpr uint64_t kCacheReuseBytes = uint64_t{160} << 20;

// The W elements of x[p .. p + W - 1][q] (zero past the last row).
template <typename T, bool VEC>
__device__ __forceinline__ typename Vec16<T>::type load_column_group(const T* in, uint64_t p,
                                                                    uint64_t q, uint64_t pitch,
                                                                    uint64_t rows) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  V v{};
  if constexpr (VEC) {
    // rows is a multiple of W: a group is wholly present or wholly absent
    if (p < rows) v = stream_load(reinterpret_cast<const V*>(in + p + q * pitch));
  } else {
#pragma unroll
    for (int k = 0; k < W; ++k) {
      if (p + k < rows) vec_set<T>(v, k, in[p + k + q * pitch]);
    }
  }
  return v;
}

// CACHED: the statistics pass reads x with ordinary (cached) loads, so that
// an x that fits the Infinity Cache is still there for the apply pass; on
// x^T for x [8192, 4096] float32 the pair took 64.8 us this way against
// 72.9 us with non-temporal loads (the statistics pass alone 25.7 against
// 23.5 us).  Larger inputs take non-temporal loads.
template <typename T, bool CENTER, bool VEC, int R, bool CACHED>
__global__ void __launch_bounds__(kStatThreads)
    norm_column_stats_kernel(double2* partial, const T* in, uint64_t pitch, uint64_t rows,
                             uint64_t n, uint64_t splits, uint64_t segment) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  constexpr int kColumns = kStatGroups * W;
  constexpr int kSums = CENTER ? 2 : 1;
  __shared__ double lds[kSums][kStatRows][kColumns];
  const int group = threadIdx.x % kStatGroups;
  const uint64_t lane_row = threadIdx.x / kStatGroups;
  const uint64_t strips = (rows + kColumns - 1) / kColumns;
  const uint64_t items = strips * splits;
  for (uint64_t item = blockIdx.x; item < items; item += gridDim.x) {
    // strips fastest: workgroups side by side read neighbouring strips of
    // the same storage rows
    const uint64_t split = item / strips;
    const uint64_t strip = item - split * strips;
    const uint64_t p = strip * kColumns + static_cast<uint64_t>(group) * W;
    const uint64_t begin = split * segment;
    const uint64_t end = begin + segment < n ? begin + segment : n;
    double shift[W];
    double s1[W];
    double s2[W];
    {
      const V first = CENTER ? load_column_group<T, VEC>(in, p, 0, pitch, rows) : V{};
#pragma unroll
      for (int k = 0; k < W; ++k) {
        shift[k] = static_cast<double>(vec_get<T>(first, k));
        s1[k] = 0.0;
        s2[k] = 0.0;
      }
    }
    auto add = [&](const V& v) {
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const double d = static_cast<double>(vec_get<T>(v, k)) - shift[k];
        if constexpr (CENTER) s1[k] += d;
        s2[k] = __builtin_fma(d, d, s2[k]);
      }
    };
    // Whether a lane's group has any element is fixed for the whole strip,
    // so it is checked once, not per load, and the rows are walked with a
    // pointer: no 64-bit multiply and no branch around each load, which kept
    // the loads from issuing back to back.
    const uint64_t first_q = begin + lane_row;
    if (p < rows) {
      const uint64_t step = static_cast<uint64_t>(kStatRows) * pitch;
      const T* at = in + p + first_q * pitch;
      uint64_t q = first_q;
      for (; q + static_cast<uint64_t>(R - 1) * kStatRows < end; q += R * kStatRows) {
        V v[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
          if constexpr (VEC) {
            const V* source = reinterpret_cast<const V*>(at + u * step);
            v[u] = CACHED ? *source : stream_load(source);
          } else {
            v[u] = load_column_group<T, false>(in, p, q + u * kStatRows, pitch, rows);
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // all R loads in flight first
#pragma unroll
        for (int u = 0; u < R; ++u) add(v[u]);
        at += R * step;
      }
      for (; q < end; q += kStatRows) add(load_column_group<T, VEC>(in, p, q, pitch, rows));
    }
    __syncthreads();  // the previous item's readers are done with lds
#pragma unroll
    for (int k = 0; k < W; ++k) {
      lds[0][lane_row][group * W + k] = s2[k];
      if constexpr (CENTER) lds[kSums - 1][lane_row][group * W + k] = s1[k];
    }
    __syncthreads();
    for (int half = kStatRows / 2; half > 0; half /= 2) {
      for (int e = threadIdx.x; e < half * kColumns; e += kStatThreads) {
        const int row = e / kColumns;
        const int c = e % kColumns;
#pragma unroll
        for (int s = 0; s < kSums; ++s) lds[s][row][c] += lds[s][row + half][c];
      }
      __syncthreads();
    }
    if (threadIdx.x < kColumns) {
      const uint64_t column = strip * kColumns + threadIdx.x;
      if (column < rows) {
        partial[split * rows + column] =
            double2{CENTER ? lds[kSums - 1][0][threadIdx.x] : 0.0, lds[0][0][threadIdx.x]};
      }
    }
  }
}

template <typename T, bool CENTER, bool VEC, bool NT>
__global__ void __launch_bounds__(kApplyThreads)
    norm_apply_columns_kernel(T* out, T* mean_out, T* denominator_out, const T* in,
                              uint64_t pitch, const T* weight, const T* bias,
                              const double2* partial, uint32_t splits, uint64_t rows, uint64_t n,
                              T eps, FastDiv tiles_q, FastDiv tiles_p, uint32_t tile_count) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  constexpr int G = kApplyGranules;
  constexpr int TP = G * W;
  constexpr int TQ = G * W;
  constexpr int kLoads = TQ * G / kApplyThreads;             // granules staged per lane
  constexpr int kBlocks = (TQ / W) * G / kApplyThreads;      // W x W blocks stored per lane
  static_assert(kApplyThreads % (TQ / W) == 0, "a lane keeps one q granule");
  static_assert(kApplyThreads % G == 0, "a lane keeps its p granule for all its loads");
  __shared__ V lds[TQ][G];
  __shared__ T stat_mean[TP];
  __shared__ T stat_d[TP];
  __shared__ T stat_r[TP];
  const double count = static_cast<double>(n);
  struct Where {
    uint64_t p0, q0;
    bool first_column;
  };
  // q tiles fastest, each q column of tiles rotated along p by its index, so
  // that workgroups side by side differ in both p and q.
  auto locate = [&](uint32_t tile) {
    const uint32_t rest = tiles_q.div(tile);
    const uint32_t tq = tile - rest * tiles_q.divisor;
    const uint32_t rotated = rest + tq % tiles_p.divisor;
    const uint32_t tp = rotated >= tiles_p.divisor ? rotated - tiles_p.divisor : rotated;
    return Where{static_cast<uint64_t>(tp) * TP, static_cast<uint64_t>(tq) * TQ, tq == 0};
  };
  V staged[kLoads];
  double2 parts[kMaxStatSplits];
  T shift = T(0);
  // A lane's staged granules within a tile: p offset (lane % G) W, q offsets
  // lane / G + it * kApplyThreads / G.
  const uint64_t lane_offset = static_cast<uint64_t>(threadIdx.x % G) * W +
                               static_cast<uint64_t>(threadIdx.x / G) * pitch;
  const uint64_t load_step = static_cast<uint64_t>(kApplyThreads / G) * pitch;
  auto load_tile = [&](const Where& w) {
    if (VEC && w.p0 + TP <= rows && w.q0 + TQ <= n) {
      // a whole tile: no bounds checks, pointer steps only
      const T* at = in + w.p0 + w.q0 * pitch + lane_offset;
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        staged[it] = stream_load(reinterpret_cast<const V*>(at + it * load_step));
      }
    } else {
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const int index = it * kApplyThreads + threadIdx.x;
        const uint64_t p = w.p0 + static_cast<uint64_t>(index % G) * W;
        const uint64_t q = w.q0 + index / G;
        staged[it] = q < n ? load_column_group<T, VEC>(in, p, q, pitch, rows) : V{};
      }
    }
    const uint64_t p = w.p0 + threadIdx.x;
    if (threadIdx.x < TP && p < rows) {
#pragma unroll
      for (int s = 0; s < kMaxStatSplits; ++s) {
        if (static_cast<uint32_t>(s) < splits) parts[s] = partial[s * rows + p];
      }
      if constexpr (CENTER) shift = in[p];
    }
  };
  uint32_t tile = blockIdx.x;
  if (tile >= tile_count) return;
  Where cur = locate(tile);
  load_tile(cur);
  while (true) {
    const uint32_t next = tile + gridDim.x;
    __syncthreads();  // the previous tile's LDS readers are done
#pragma unroll
    for (int it = 0; it < kLoads; ++it) {
      const int index = it * kApplyThreads + threadIdx.x;
      const int row = index / G;
      lds[row][(index % G) ^ ((row / W) & 7)] = staged[it];
    }
    {
      const uint64_t p = cur.p0 + threadIdx.x;
      if (threadIdx.x < TP && p < rows) {
        double s1 = 0.0;
        double s2 = 0.0;
#pragma unroll
        for (int s = 0; s < kMaxStatSplits; ++s) {
          if (static_cast<uint32_t>(s) < splits) {
            s1 += parts[s].x;
            s2 += parts[s].y;
          }
        }
        double variance = CENTER ? (s2 - s1 * s1 / count) / count : s2 / count;
        variance = variance > 0.0 ? variance : 0.0;
        const T mu = CENTER ? static_cast<T>(static_cast<double>(shift) + s1 / count) : T(0);
        const T d = norm_sqrt<T>(static_cast<T>(variance) + eps);
        stat_mean[threadIdx.x] = mu;
        stat_d[threadIdx.x] = d;
        stat_r[threadIdx.x] = T(1) / d;
        if (cur.first_column) {
          if constexpr (CENTER) mean_out[p] = mu;
          denominator_out[p] = d;
        }
      }
    }
    __syncthreads();
    // A lane keeps one q granule m for all its blocks: its weight and bias
    // groups are loaded once per tile, before the next tile's loads are
    // issued (the wait counter retires vector loads in issue order, so a
    // load issued after them would wait for them too).
    const int m = threadIdx.x % (TQ / W);
    const uint64_t q = cur.q0 + static_cast<uint64_t>(m) * W;
    T w[W];
    T b[W];
#pragma unroll
    for (int k = 0; k < W; ++k) {
      w[k] = T(0);
      b[k] = T(0);
    }
    if constexpr (VEC) {
      if (q < n) {
        const V wv = *reinterpret_cast<const V*>(weight + q);
#pragma unroll
        for (int k = 0; k < W; ++k) w[k] = vec_get<T>(wv, k);
        if constexpr (CENTER) {
          const V bv = *reinterpret_cast<const V*>(bias + q);
#pragma unroll
          for (int k = 0; k < W; ++k) b[k] = vec_get<T>(bv, k);
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < W; ++k) {
        if (q + k < n) {
          w[k] = weight[q + k];
          if constexpr (CENTER) b[k] = bias[q + k];
        }
      }
    }
    Where following = cur;
    if (next < tile_count) {
      following = locate(next);
      load_tile(following);  // in flight during this tile's stores
    }
#pragma unroll
    for (int it = 0; it < kBlocks; ++it) {
      const int index = it * kApplyThreads + threadIdx.x;
      const int g = index / (TQ / W);  // p granule within the tile
      const uint64_t p = cur.p0 + static_cast<uint64_t>(g) * W;
      if (q >= n || p >= rows) continue;
      T values[W][W];  // [p offset][q offset]
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const V block = lds[m * W + k][g ^ (m & 7)];
#pragma unroll
        for (int i = 0; i < W; ++i) values[i][k] = vec_get<T>(block, i);
      }
#pragma unroll
      for (int i = 0; i < W; ++i) {
        if (!VEC && p + i >= rows) break;
        const T mu = stat_mean[g * W + i];
        const Divisor<T> divide(stat_d[g * W + i], stat_r[g * W + i]);
        V o;
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const T centred = CENTER ? values[i][k] - mu : values[i][k];
          T y = divide(centred) * w[k];
          if constexpr (CENTER) y = y + b[k];
          vec_set<T>(o, k, y);
        }
        T* row = out + (p + i) * n + q;
        if constexpr (VEC) {
          store_vector<NT>(reinterpret_cast<V*>(row), o);
        } else {
#pragma unroll
          for (int k = 0; k < W; ++k) {
            if (q + k < n) row[k] = vec_get<T>(o, k);
          }
        }
      }
    }
    if (next >= tile_count) break;
    tile = next;
    cur = following;
  }
}

// Backward: with xhat = (x - mu) / d (x / d for RMSNorm) and g = dy * w,
//   dx = (g - mean(g) - xhat * mean(g * xhat)) / d     (LayerNorm)
//   dx = (g - xhat * mean(g * xhat)) / d               (RMSNorm)
//   dw = sum over rows of dy * xhat, db = sum over rows of dy.
// Each workgroup walks rows blockIdx.x, + gridDim.x, ... and keeps its dw and
// db partials for its columns in registers; they are written once, as row
// blockIdx.x of the [gridDim.x, n] partial arrays.
template <typename T, int THREADS, int E, bool CENTER, bool VEC, bool FULL, bool NT>
__global__ void __launch_bounds__(THREADS)
    norm_backward_kernel(T* dx, uint64_t dx_stride, T* partial_weight, T* partial_bias,
                         const T* dy, const T* dy_scale, const T* in, uint64_t in_stride,
                         const T* weight, const T* mean, const T* denominator, uint64_t rows,
                         uint64_t n) {
  const T count = static_cast<T>(n);
  const bool scaled = dy_scale != nullptr;  // dy = *dy_scale * factor
  const T value = scaled ? *dy_scale : T(1);
  T acc_w[E];
  T acc_b[CENTER ? E : 1];
#pragma unroll
  for (int j = 0; j < E; ++j) acc_w[j] = T(0);
  if constexpr (CENTER) {
#pragma unroll
    for (int j = 0; j < E; ++j) acc_b[j] = T(0);
  }
  for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    T x[E];
    T g[E];
    norm_load<T, THREADS, E, VEC, FULL>(x, in + r * in_stride, n);
    norm_load<T, THREADS, E, VEC, FULL>(g, dy + r * n, n);
    if (scaled) norm_scale<T, THREADS, E, VEC, FULL>(g, value, n);
    const T mu = CENTER ? mean[r] : T(0);
    const Divisor<T> divide(denominator[r]);
    T sum_g = T(0);
    T sum_gx = T(0);
    // The weight is streamed one 16-byte group at a time (cached loads) so
    // that a whole row of it never occupies registers.
    constexpr int G = VEC ? Vec16<T>::width : 1;
#pragma unroll
    for (int v = 0; v < E / G; ++v) {
      T w[G];
      const uint64_t col0 = norm_column<T, THREADS, VEC>(v * G);
      const bool in_row = FULL || col0 < n;
      if constexpr (VEC) {
        using V = typename Vec16<T>::type;
        const V wv = in_row ? *reinterpret_cast<const V*>(weight + col0) : V{};
#pragma unroll
        for (int k = 0; k < G; ++k) w[k] = vec_get<T>(wv, k);
      } else {
        w[0] = in_row ? weight[col0] : T(0);
      }
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int j = v * G + k;
        x[j] = in_row ? divide(x[j] - mu) : T(0);  // xhat
        acc_w[j] += g[j] * x[j];
        if constexpr (CENTER) acc_b[j] += g[j];
        g[j] = g[j] * w[k];                         // dxhat (zero outside the row)
        sum_g += g[j];
        sum_gx += g[j] * x[j];
      }
    }
    if constexpr (CENTER) {
      norm_block_sum2<T, THREADS>(sum_g, sum_gx);
    } else {
      sum_gx = norm_block_sum<T, THREADS>(sum_gx);
    }
    const T mean_g = CENTER ? sum_g / count : T(0);
    const T mean_gx = sum_gx / count;
#pragma unroll
    for (int j = 0; j < E; ++j) g[j] = divide(g[j] - mean_g - x[j] * mean_gx);
    norm_store<T, THREADS, E, VEC, FULL, NT>(dx + r * dx_stride, g, n);
  }
  norm_store<T, THREADS, E, VEC, FULL, false>(partial_weight + blockIdx.x * n, acc_w, n);
  if constexpr (CENTER) {
    norm_store<T, THREADS, E, VEC, FULL, false>(partial_bias + blockIdx.x * n, acc_b, n);
  }
}

// The same backward with the next row's x and dy loaded while the current
// row's block sums run, and the weight row held in registers: for float32
// rows of up to 16 elements per lane, where the extra registers fit (one
// 512-lane workgroup per CU).  Same operations in the same order, so the same
// bits.  On [4096, 8192] float32: 70.3 us against 74.1 us for two workgroups
// per CU without the prefetch, and half the weight / bias partials.
template <typename T, int THREADS, int E, bool CENTER, bool VEC, bool FULL, bool NT>
__global__ void __launch_bounds__(THREADS)
    norm_backward_pipelined_kernel(T* dx, uint64_t dx_stride, T* partial_weight,
                                   T* partial_bias, const T* dy, const T* dy_scale, const T* in,
                                   uint64_t in_stride, const T* weight, const T* mean,
                                   const T* denominator, uint64_t rows, uint64_t n) {
  const T count = static_cast<T>(n);
  const bool scaled = dy_scale != nullptr;  // dy = *dy_scale * factor
  const T value = scaled ? *dy_scale : T(1);
  T acc_w[E];
  T acc_b[CENTER ? E : 1];
  T w[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    acc_w[j] = T(0);
    w[j] = T(0);
  }
  if constexpr (CENTER) {
#pragma unroll
    for (int j = 0; j < E; ++j) acc_b[j] = T(0);
  }
  norm_load_parameter<T, THREADS, E, VEC, FULL>(w, weight, n);
  uint64_t r = blockIdx.x;
  T x[E];
  T g[E];
  if (r < rows) {
    norm_load<T, THREADS, E, VEC, FULL>(x, in + r * in_stride, n);
    norm_load<T, THREADS, E, VEC, FULL>(g, dy + r * n, n);
  }
  for (; r < rows; r += gridDim.x) {
    const T mu = CENTER ? mean[r] : T(0);
    const Divisor<T> divide(denominator[r]);
    T sum_g = T(0);
    T sum_gx = T(0);
    // The scale is applied here, where the row is consumed: applied when
    // the next row's loads are issued it would wait for them at once.
    if (scaled) norm_scale<T, THREADS, E, VEC, FULL>(g, value, n);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const bool in_row = FULL || norm_column<T, THREADS, VEC>(j) < n;
      x[j] = in_row ? divide(x[j] - mu) : T(0);  // xhat
      acc_w[j] += g[j] * x[j];
      if constexpr (CENTER) acc_b[j] += g[j];
      g[j] = g[j] * w[j];                         // dxhat (zero outside the row)
      sum_g += g[j];
      sum_gx += g[j] * x[j];
    }
    const uint64_t next = r + gridDim.x;
    T next_x[E];
    T next_g[E];
    if (next < rows) {
      norm_load<T, THREADS, E, VEC, FULL>(next_x, in + next * in_stride, n);
      norm_load<T, THREADS, E, VEC, FULL>(next_g, dy + next * n, n);
    }
    if constexpr (CENTER) {
      norm_block_sum2<T, THREADS>(sum_g, sum_gx);
    } else {
      sum_gx = norm_block_sum<T, THREADS>(sum_gx);
    }
    const T mean_g = CENTER ? sum_g / count : T(0);
    const T mean_gx = sum_gx / count;
#pragma unroll
    for (int j = 0; j < E; ++j) g[j] = divide(g[j] - mean_g - x[j] * mean_gx);
    norm_store<T, THREADS, E, VEC, FULL, NT>(dx + r * dx_stride, g, n);
    if (next < rows) {
#pragma unroll
      for (int j = 0; j < E; ++j) {
        x[j] = next_x[j];
        g[j] = next_g[j];
      }
    }
  }
  norm_store<T, THREADS, E, VEC, FULL, false>(partial_weight + blockIdx.x * n, acc_w, n);
  if constexpr (CENTER) {
    norm_store<T, THREADS, E, VEC, FULL, false>(partial_bias + blockIdx.x * n, acc_b, n);
  }
}

// Column sums of [parts, n] partials in a fixed order: a 1024-lane block owns
// 64 columns; wave w sums parts w, w + 16, ... in order and the 16 wave sums
// are added in wave order, so the result does not depend on scheduling.
constexpr int kCombineThreads = 1024;
constexpr int kCombineWaves = kCombineThreads / kWave;

// Column group `group` (64 columns) of [parts, n] partials into out.
template <typename T>
__device__ __forceinline__ void combine_group(T* out, const T* partial, uint64_t parts,
                                              uint64_t n, uint64_t group,
                                              T (&lds)[kCombineWaves][kWave]) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const uint64_t col = group * kWave + lane;
  T total = T(0);
  if (col < n) {
    // Eight loads in flight per lane, added in the same order as one at a
    // time.
    constexpr int kBatch = 8;
    uint64_t p = wave;
    for (; p + (kBatch - 1) * kCombineWaves < parts; p += kBatch * kCombineWaves) {
      T v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) v[u] = partial[(p + u * kCombineWaves) * n + col];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) total += v[u];
    }
    for (; p < parts; p += kCombineWaves) total += partial[p * n + col];
  }
  __syncthreads();
  lds[wave][lane] = total;
  __syncthreads();
  if (wave == 0 && col < n) {
    T sum = lds[0][lane];
#pragma unroll
    for (int w = 1; w < kCombineWaves; ++w) sum += lds[w][lane];
    out[col] = sum;
  }
}

template <typename T>
__global__ void __launch_bounds__(kCombineThreads)
    norm_combine_kernel(T* out, const T* partial, uint64_t parts, uint64_t n) {
  __shared__ T lds[kCombineWaves][kWave];
  const uint64_t groups = (n + kWave - 1) / kWave;
  for (uint64_t group = blockIdx.x; group < groups; group += gridDim.x) {
    combine_group<T>(out, partial, parts, n, group, lds);
  }
}

// The weight and bias partials in one launch: groups [0, groups) of the
// weight, then the bias's, each summed as norm_combine_kernel sums it.
template <typename T>
__global__ void __launch_bounds__(kCombineThreads)
    norm_combine_pair_kernel(T* out_weight, const T* partial_weight, T* out_bias,
                             const T* partial_bias, uint64_t parts, uint64_t n) {
  __shared__ T lds[kCombineWaves][kWave];
  const uint64_t groups = (n + kWave - 1) / kWave;
  for (uint64_t group = blockIdx.x; group < 2 * groups; group += gridDim.x) {
    if (group < groups) {
      combine_group<T>(out_weight, partial_weight, parts, n, group, lds);
    } else {
      combine_group<T>(out_bias, partial_bias, parts, n, group - groups, lds);
    }
  }
}

// ------------------------------------- backward, rows down storage columns
//
// The backward over the forward's column layout, x[p][q] = in[p + q * pitch],
// with dy in rows (dy[p * n + q]).  dx is written in x's layout,
// dx[p + q * stride]; with stride == rows, the storage of a contiguous
// [n, rows] tensor whose transpose is the gradient of the transposed view.
// Three launches take the
// place of a transposing copy of x, the row kernel and a transposing copy of
// dx:
//
//  1. norm_backward_columns_sums_kernel.  Tiles of 32 W values of p by 32 W
//     values of q in the transposed frame: dy goes through LDS (XOR swizzle)
//     and x is read along p; the next tile's x, dy and weight are in flight
//     while the current tile is used.  A workgroup owns one p tile and a run
//     of q tiles (a split of q); each lane keeps one granule of W rows for
//     the run and the sums of g = dy * w and g * xhat over its columns, which
//     at the end the lanes of each granule add (two per wave by a lane
//     exchange, then the waves in order through LDS).  Per block of W
//     columns the lane's partials of dy * xhat and dy over its rows are
//     added across the 32 lanes of its half wave (the tile's p) by a
//     butterfly.  Results: [2, splits, rows] row sums and [tiles_p, n]
//     weight / bias partials.
//  2. norm_backward_columns_finish_kernel: the weight and bias gradients (the
//     partials added in p-tile order, as norm_combine_kernel does) and each
//     row's mean(g) and mean(g * xhat) (splits added in order, then divided
//     by (T)n).
//  3. norm_backward_columns_apply_kernel.  Tiles in the transposed frame: dy
//     goes through LDS, x is read and dx written along p.  Each element is
//     computed with the row kernel's operations in the same order.
//
// Only the order of the sums differs from the row kernel, so the two layouts
// agree within the sums' rounding.  On an input that fits the Infinity Cache
// the sums pass reads x with cached loads and the apply pass finds it there.
// lanes that share one p granule (and take every kBackwardGroups-th q granule)
constexpr int kBackwardGroups = kApplyThreads / kApplyGranules;
// Lanes of a sums-pass workgroup: at 512 a lane's share of a 128 x 128
// float32 tile (8 dy granules, 2 blocks of x) leaves room for a second x set,
// so every tile's x is loaded one tile ahead.
constexpr int kSumsThreads = 512;

// Lane exchanges within a half wave, on 32-bit words (a double as two).
// swap_rows: v_permlane16_swap, which swaps the odd 16-lane rows of its first
// operand with the even rows of its second: for lanes c < 16 of a half wave
// `second` becomes the first operand of lane c + 16, for lanes c >= 16
// `first` becomes the second operand of lane c - 16.
// mirror<CTRL>: a DPP move within 16-lane rows, lane c reading lane
// 15 - c (row_mirror, 0x140), within 8-lane halves 7 - c (row_half_mirror,
// 0x141), or c ^ 2 and c ^ 1 within quads (quad_perm 0x4E and 0xB1).
__device__ __forceinline__ void swap_rows(uint32_t& first, uint32_t& second) {
  const auto swapped = __builtin_amdgcn_permlane16_swap(first, second, false, false);
  first = swapped[0];
  second = swapped[1];
}

template <typename T>
__device__ __forceinline__ void swap_rows(T& first, T& second) {
  if constexpr (sizeof(T) == 4) {
    uint32_t a = __builtin_bit_cast(uint32_t, first);
    uint32_t b = __builtin_bit_cast(uint32_t, second);
    swap_rows(a, b);
    first = __builtin_bit_cast(T, a);
    second = __builtin_bit_cast(T, b);
  } else {
    static_assert(sizeof(T) == 8, "32- or 64-bit values");
    const uint64_t a = __builtin_bit_cast(uint64_t, first);
    const uint64_t b = __builtin_bit_cast(uint64_t, second);
    uint32_t a0 = static_cast<uint32_t>(a), a1 = static_cast<uint32_t>(a >> 32);
    uint32_t b0 = static_cast<uint32_t>(b), b1 = static_cast<uint32_t>(b >> 32);
    swap_rows(a0, b0);
    swap_rows(a1, b1);
    first = __builtin_bit_cast(T, (static_cast<uint64_t>(a1) << 32) | a0);
    second = __builtin_bit_cast(T, (static_cast<uint64_t>(b1) << 32) | b0);
  }
}

template <int CTRL>
__device__ __forceinline__ uint32_t mirror_word(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xF, 0xF, false));
}

template <int CTRL, typename T>
__device__ __forceinline__ T mirror(T x) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, mirror_word<CTRL>(__builtin_bit_cast(uint32_t, x)));
  } else {
    const uint64_t a = __builtin_bit_cast(uint64_t, x);
    const uint64_t lo = mirror_word<CTRL>(static_cast<uint32_t>(a));
    const uint64_t hi = mirror_word<CTRL>(static_cast<uint32_t>(a >> 32));
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}

// Butterfly reduce-scatter over the 32 lanes of a half wave: on entry each
// lane holds NV values (NV divides 32), on exit lane c holds in v[0] the sum
// over the 32 lanes of value c * NV / 32, the 32 / NV lanes that share it
// alike.  Step b pairs lane c with a lane whose bit b differs: c ^ 16 (a row
// swap), then 15 - c, 7 - c, c ^ 2 and c ^ 1 within rows (DPP moves, no
// LDS); the partners' offsets 16, 15, 7, 2, 1 span all 32 lanes, so after
// the five steps every lane's value covers the half wave once.  While more
// than one value is left the lane with bit b set keeps the upper half,
// after that both add.  The row swap exchanges a pair of values at once: a
// lane of the lower row gets its partner's lower value in `upper_half`'s
// place, a lane of the upper row the partner's upper value in `lower`'s, so
// one add gives each lane its kept half.
template <typename T, int NV, int B = 16>
__device__ __forceinline__ void half_wave_reduce_scatter(T (&v)[NV], int c) {
  if constexpr (B >= 1) {
    constexpr int kCtrl = B == 8 ? 0x140 : B == 4 ? 0x141 : B == 2 ? 0x4E : 0xB1;
    if constexpr (NV > 1) {
      constexpr int kHalf = NV / 2;
      T kept[kHalf];
      if constexpr (B == 16) {
#pragma unroll
        for (int j = 0; j < kHalf; ++j) {
          T lower = v[j];
          T upper_half = v[j + kHalf];
          swap_rows(lower, upper_half);
          kept[j] = lower + upper_half;
        }
      } else {
        const bool upper = (c & B) != 0;
#pragma unroll
        for (int j = 0; j < kHalf; ++j) {
          const T send = upper ? v[j] : v[j + kHalf];
          const T keep = upper ? v[j + kHalf] : v[j];
          kept[j] = keep + mirror<kCtrl>(send);
        }
      }
      half_wave_reduce_scatter<T, kHalf, B / 2>(kept, c);
      v[0] = kept[0];
    } else {
      if constexpr (B == 16) {
        T own = v[0];
        T other = v[0];
        swap_rows(own, other);
        v[0] = own + other;
      } else {
        v[0] = v[0] + mirror<kCtrl>(v[0]);
      }
      half_wave_reduce_scatter<T, 1, B / 2>(v, c);
    }
  }
}

// Tile modes of the column backward kernels: scalar loads with per-element
// bounds (any layout), 16-byte granules with per-granule presence (rows and n
// multiples of W), and 16-byte granules of tiles all whole (rows and n
// multiples of the tile side: no presence tests at all).
constexpr int kScalarTiles = 0;
constexpr int kVectorTiles = 1;
constexpr int kWholeTiles = 2;

template <typename T, bool CENTER, int MODE, bool CACHED, int THREADS>
__global__ void __launch_bounds__(THREADS)
    norm_backward_columns_sums_kernel(T* row_partial, T* partial_weight, T* partial_bias,
                                      const T* dy, const T* dy_scale, const T* in,
                                      uint64_t pitch, const T* weight,
                                      const T* mean, const T* denominator, uint64_t rows,
                                      uint64_t n, uint32_t tiles_q, uint32_t splits,
                                      uint32_t split_tiles) {
  constexpr bool VEC = MODE != kScalarTiles;
  constexpr bool WHOLE = MODE == kWholeTiles;
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  constexpr int G = kApplyGranules;
  constexpr int TP = G * W;
  constexpr int TQ = G * W;
  constexpr int kLoads = TP * G / THREADS;             // dy granules staged per lane
  constexpr int kBlocks = (TP / W) * G / THREADS;      // W x W blocks per lane
  constexpr int kGroups = THREADS / G;                 // lanes that share one p granule
  constexpr int kValues = W * 2;                       // column partials per block
  constexpr int kWaves = THREADS / kWave;
  static_assert(THREADS % G == 0 && kGroups * (TP / W) == THREADS, "lane layout");
  static_assert(TP / W == 32 && 32 % kValues == 0, "half-wave reduce-scatter");
  static_assert(kWaves * (TP / W) * 2 * W * sizeof(T) <= sizeof(V) * TP * G, "row sums fit");
  __shared__ V lds[TP][G];
  __shared__ V tile_weight[TQ / W];
  const uint32_t split = blockIdx.x % splits;
  const uint32_t tp = blockIdx.x / splits;
  const uint32_t first_tile = split * split_tiles;
  if (first_tile >= tiles_q) return;  // the whole workgroup
  const uint32_t run = tiles_q - first_tile < split_tiles ? tiles_q - first_tile : split_tiles;
  const uint64_t p0 = static_cast<uint64_t>(tp) * TP;
  // A lane keeps p granule c (W rows) for the whole run and takes q granules
  // g0, g0 + kGroups, ... (one per block) of each tile.
  const int c = threadIdx.x % (TP / W);
  const int g0 = threadIdx.x / (TP / W);
  const uint64_t p = p0 + static_cast<uint64_t>(c) * W;
  T mu[W];
  T d[W];
  T r[W];
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const bool present = p + i < rows;
    mu[i] = CENTER && present ? mean[p + i] : T(0);
    d[i] = present ? denominator[p + i] : T(1);
    r[i] = T(1) / d[i];
  }
  T sum_g[W];
  T sum_gx[W];
#pragma unroll
  for (int i = 0; i < W; ++i) {
    sum_g[i] = T(0);
    sum_gx[i] = T(0);
  }
  // Staged dy granules: q offset (lane % G) W, p offsets lane / G + it *
  // THREADS / G.
  const uint64_t lane_offset = static_cast<uint64_t>(threadIdx.x % G) * W +
                               static_cast<uint64_t>(threadIdx.x / G) * n;
  const uint64_t load_step = static_cast<uint64_t>(THREADS / G) * n;
  const bool scaled = dy_scale != nullptr;  // dy = *dy_scale * factor
  const T value = scaled ? *dy_scale : T(1);
  // Staged granules stay as loaded; the scale is applied when they go to
  // LDS, where the loads have to be waited for anyway (applied at load time
  // it would wait for the next tile's loads at once).  Bit `it` of
  // staged_present marks a granule that exists (absent ones hold zero and
  // must stay zero whatever the scale).
  static_assert(kLoads <= 32, "presence bits");
  uint32_t staged_present = 0;
  V staged[kLoads];
  auto load_tile = [&](uint64_t q0) {
    if constexpr (VEC) {
      // Granules are wholly present or absent (rows and n are multiples of
      // W).  Absent ones load the first element instead and are zeroed, so
      // every load issues unconditionally, back to back.
      const T* at = dy + p0 * n + q0 + lane_offset;
      const bool q_present = q0 + static_cast<uint64_t>(threadIdx.x % G) * W < n;
      const uint64_t first_p = p0 + threadIdx.x / G;
      staged_present = 0;
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const bool present =
            WHOLE ||
            (q_present && first_p + static_cast<uint64_t>(it) * (THREADS / G) < rows);
        const V v = stream_load(reinterpret_cast<const V*>(present ? at + it * load_step : dy));
        staged[it] = present ? v : V{};
        staged_present |= present ? 1U << it : 0U;
      }
    } else {
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const int index = it * THREADS + threadIdx.x;
        const uint64_t pr = p0 + index / G;
        const uint64_t q = q0 + static_cast<uint64_t>(index % G) * W;
        V v{};
        if (pr < rows) {
#pragma unroll
          for (int k = 0; k < W; ++k) {
            if (q + k < n) {
              const T element = dy[pr * n + q + k];
              vec_set<T>(v, k, scaled ? value * element : element);
            }
          }
        }
        staged[it] = v;
      }
    }
  };
  // The run starts at a tile rotated by the p tile, so that workgroups side
  // by side read different q.
  const uint32_t start = tp % run;
  auto tile_q0 = [&](uint32_t step) {
    const uint32_t o = start + step < run ? start + step : start + step - run;
    return static_cast<uint64_t>(first_tile + o) * TQ;
  };
  // The tile's weight, staged in a register like dy and written to LDS with
  // it by the first TQ / W lanes.  Every lane loads granule lane % (TQ / W)
  // (vector tiles: unconditionally, absent granules from the first element
  // and zeroed), so no wave branches around the load.
  V staged_weight{};
  auto load_weight = [&](uint64_t q0) {
    const uint64_t q = q0 + static_cast<uint64_t>(threadIdx.x % (TQ / W)) * W;
    if constexpr (VEC) {
      const bool present = WHOLE || q < n;
      const V wv = *reinterpret_cast<const V*>(present ? weight + q : weight);
      staged_weight = present ? wv : V{};
    } else {
      V wv{};
#pragma unroll
      for (int k = 0; k < W; ++k) {
        if (q + k < n) vec_set<T>(wv, k, weight[q + k]);
      }
      staged_weight = wv;
    }
  };
  // x of the tile at q0: [block][q offset], W values of p each
  auto load_x = [&](V(&x)[kBlocks][W], uint64_t q0) {
    const uint64_t first_q = q0 + static_cast<uint64_t>(g0) * W;
      if constexpr (VEC) {
        const T* at = in + p + first_q * pitch;
#pragma unroll
        for (int it = 0; it < kBlocks; ++it) {
          const uint64_t q = first_q + static_cast<uint64_t>(it) * kGroups * W;
          const bool present = WHOLE || (p < rows && q < n);
#pragma unroll
          for (int k = 0; k < W; ++k) {
            const V* source = reinterpret_cast<const V*>(
                present ? at + (static_cast<uint64_t>(it) * kGroups * W + k) * pitch : in);
            const V v = CACHED ? *source : stream_load(source);
            x[it][k] = present ? v : V{};
          }
        }
      } else {
#pragma unroll
        for (int it = 0; it < kBlocks; ++it) {
          const uint64_t q = first_q + static_cast<uint64_t>(it) * kGroups * W;
#pragma unroll
          for (int k = 0; k < W; ++k) {
            x[it][k] = q + k < n ? load_column_group<T, false>(in, p, q + k, pitch, rows) : V{};
          }
        }
      }
  };
  // One tile: dy (staged) and the weight to LDS, then (PREFETCH) the next
  // tile's x, dy and weight issued, then this tile's sums from x (loaded one
  // tile ago) and LDS.  Two x register sets are used in turn (x, x_next), so
  // no register is copied between tiles: a copy would make the wave wait for
  // the next tile's loads right after issuing them.  The prefetch is a
  // compile-time choice, the last tile's body being the only one without:
  // behind a run-time test the compiler counts the loads of the path that
  // skips it, and the sums would wait for the next tile's first loads.
  auto body = [&](V(&x)[kBlocks][W], V(&x_next)[kBlocks][W], uint32_t step, auto prefetch) {
    const uint64_t q0 = tile_q0(step);
    __syncthreads();  // the previous tile's LDS readers are done
#pragma unroll
    for (int it = 0; it < kLoads; ++it) {
      const int index = it * THREADS + threadIdx.x;
      const int row = index / G;
      V v = staged[it];
      if (VEC && scaled && ((staged_present >> it) & 1U)) v = scale_granule<T>(value, v);
      lds[row][(index % G) ^ ((row / W) & 7)] = v;
    }
    if (threadIdx.x < TQ / W) tile_weight[threadIdx.x] = staged_weight;
    __syncthreads();
    if constexpr (decltype(prefetch)::value) {
      const uint64_t next_q0 = tile_q0(step + 1);
      load_x(x_next, next_q0);
      load_tile(next_q0);
      load_weight(next_q0);
    }
    const uint64_t first_q = q0 + static_cast<uint64_t>(g0) * W;
      // Column partials, block by block: value k * 2 + s is the sum over the
      // lane's W rows of dy * xhat (s = 0) or dy (s = 1) at q row k of the
      // block, then over the 32 lanes of the half wave (the tile's p), after
      // which lane c holds value c / (32 / kValues).  Absent rows and columns
      // hold zero dy and add nothing.
#pragma unroll
      for (int it = 0; it < kBlocks; ++it) {
        const int g = g0 + it * kGroups;
        T grad[W][W];  // [p offset][q offset]
#pragma unroll
        for (int i = 0; i < W; ++i) {
          const V block = lds[c * W + i][g ^ (c & 7)];
#pragma unroll
          for (int k = 0; k < W; ++k) grad[i][k] = vec_get<T>(block, k);
        }
        const V wv = tile_weight[g];  // zero past the last column
        T column[kValues];
        T block_g[W];
        T block_gx[W];
#pragma unroll
        for (int k = 0; k < W; ++k) {
          T dw = T(0);
          T db = T(0);
#pragma unroll
          for (int i = 0; i < W; ++i) {
            const Divisor<T> divide(d[i], r[i]);
            const T xhat = divide(vec_get<T>(x[it][k], i) - mu[i]);
            dw += grad[i][k] * xhat;
            if constexpr (CENTER) db += grad[i][k];
            const T gw = grad[i][k] * vec_get<T>(wv, k);
            if (k == 0) {
              block_g[i] = gw;
              block_gx[i] = gw * xhat;
            } else {
              block_g[i] += gw;
              block_gx[i] += gw * xhat;
            }
          }
          column[k * 2] = dw;
          column[k * 2 + 1] = db;
        }
        // The row sums gather the block's W columns first.  The empty asm
        // pins each sum here: otherwise the compiler sinks these adds to the
        // loop's end and keeps the block's xhat and g * w live until then.
#pragma unroll
        for (int i = 0; i < W; ++i) {
          if constexpr (CENTER) {
            sum_g[i] += block_g[i];
            asm volatile("" : "+v"(sum_g[i]));
          }
          sum_gx[i] += block_gx[i];
          asm volatile("" : "+v"(sum_gx[i]));
        }
        half_wave_reduce_scatter<T, kValues>(column, c);
        constexpr int kLanesPerValue = 32 / kValues;
        const int j = c / kLanesPerValue;
        const int s = j % 2;
        const uint64_t q = first_q + static_cast<uint64_t>(it) * kGroups * W + j / 2;
        if (c % kLanesPerValue == 0 && (WHOLE || q < n) && (CENTER || s == 0)) {
          (s == 0 ? partial_weight : partial_bias)[static_cast<uint64_t>(tp) * n + q] = column[0];
        }
      }
  };
  V xa[kBlocks][W];
  V xb[kBlocks][W];
  load_x(xa, tile_q0(0));
  load_tile(tile_q0(0));
  load_weight(tile_q0(0));
  uint32_t step = 0;
  for (; step + 2 < run; step += 2) {
    body(xa, xb, step, Policy<true>{});
    body(xb, xa, step + 1, Policy<true>{});
  }
  if (step + 1 < run) {
    body(xa, xb, step, Policy<true>{});
    body(xb, xa, step + 1, Policy<false>{});
  } else {
    body(xa, xb, step, Policy<false>{});
  }
  // The row sums over the run: lanes c and c + 32 of a wave, then the waves
  // in order through LDS.
#pragma unroll
  for (int i = 0; i < W; ++i) {
    if constexpr (CENTER) sum_g[i] += __shfl_xor(sum_g[i], 32);
    sum_gx[i] += __shfl_xor(sum_gx[i], 32);
  }
  __syncthreads();  // the last tile's LDS readers are done
  T* red = reinterpret_cast<T*>(&lds[0][0]);  // [kWaves][TP][2]
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave < TP / W) {
#pragma unroll
    for (int i = 0; i < W; ++i) {
      red[(wave * TP + c * W + i) * 2] = sum_g[i];
      red[(wave * TP + c * W + i) * 2 + 1] = sum_gx[i];
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < 2 * TP; t += THREADS) {
    const int s = t / TP;
    const int pl = t % TP;
    const uint64_t row = p0 + pl;
    if (row < rows && (CENTER || s == 1)) {
      T total = red[pl * 2 + s];
#pragma unroll
      for (int v = 1; v < kWaves; ++v) total += red[(v * TP + pl) * 2 + s];
      row_partial[(static_cast<uint64_t>(s) * splits + split) * rows + row] = total;
    }
  }
}

// Weight / bias gradients and the rows' means, in one launch: blocks
// [0, column_blocks) combine the weight partials, the next column_blocks
// (LayerNorm) the bias partials, the rest finish kCombineThreads rows each.
template <typename T, bool CENTER>
__global__ void __launch_bounds__(kCombineThreads)
    norm_backward_columns_finish_kernel(T* weight_gradient, T* bias_gradient, T* row_means,
                                        const T* partial_weight, const T* partial_bias,
                                        uint64_t parts, const T* row_partial, uint64_t splits,
                                        uint64_t rows, uint64_t n, uint64_t column_blocks) {
  __shared__ T lds[kCombineWaves][kWave];
  const uint64_t block = blockIdx.x;
  if (block < column_blocks) {
    combine_group<T>(weight_gradient, partial_weight, parts, n, block, lds);
    return;
  }
  uint64_t rest = block - column_blocks;
  if constexpr (CENTER) {
    if (rest < column_blocks) {
      combine_group<T>(bias_gradient, partial_bias, parts, n, rest, lds);
      return;
    }
    rest -= column_blocks;
  }
  const uint64_t p = rest * kCombineThreads + threadIdx.x;
  if (p >= rows) return;
  const T count = static_cast<T>(n);
  T sum_g = T(0);
  T sum_gx = T(0);
  for (uint64_t s = 0; s < splits; ++s) {
    if constexpr (CENTER) sum_g += row_partial[s * rows + p];
    sum_gx += row_partial[(splits + s) * rows + p];
  }
  row_means[p] = CENTER ? sum_g / count : T(0);
  row_means[rows + p] = sum_gx / count;
}

template <typename T, bool CENTER, int MODE, bool NT>
__global__ void __launch_bounds__(kApplyThreads)
    norm_backward_columns_apply_kernel(T* dx, uint64_t dx_stride, const T* dy,
                                       const T* dy_scale, const T* in, uint64_t pitch,
                                       const T* weight, const T* mean, const T* denominator,
                                       const T* row_means, uint64_t rows, uint64_t n,
                                       FastDiv tiles_p, FastDiv tiles_q, uint32_t tile_count) {
  constexpr bool VEC = MODE != kScalarTiles;
  constexpr bool WHOLE = MODE == kWholeTiles;
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  constexpr int G = kApplyGranules;
  constexpr int TP = G * W;
  constexpr int TQ = G * W;
  constexpr int kLoads = TP * G / kApplyThreads;             // dy granules staged per lane
  constexpr int kBlocks = (TP / W) * G / kApplyThreads;      // W x W blocks per lane
  constexpr int kGroups = kBackwardGroups;
  static_assert(kApplyThreads % G == 0 && kGroups * (TP / W) == kApplyThreads, "lane layout");
  __shared__ V lds[TP][G];
  // p tiles fastest, each p column of tiles rotated along q by its index.
  auto locate = [&](uint32_t tile, uint64_t& p0, uint64_t& q0) {
    const uint32_t rest = tiles_p.div(tile);
    const uint32_t tp = tile - rest * tiles_p.divisor;
    const uint32_t rotated = rest + tp % tiles_q.divisor;
    const uint32_t tq = rotated >= tiles_q.divisor ? rotated - tiles_q.divisor : rotated;
    p0 = static_cast<uint64_t>(tp) * TP;
    q0 = static_cast<uint64_t>(tq) * TQ;
  };
  const bool scaled = dy_scale != nullptr;  // dy = *dy_scale * factor
  const T value = scaled ? *dy_scale : T(1);
  // Staged granules stay as loaded; the scale is applied when they go to
  // LDS, where the loads have to be waited for anyway (applied at load time
  // it would wait for the next tile's loads at once).  Bit `it` of
  // staged_present marks a granule that exists (absent ones hold zero and
  // must stay zero whatever the scale).
  static_assert(kLoads <= 32, "presence bits");
  uint32_t staged_present = 0;
  V staged[kLoads];
  // Staged dy granules: q offset (lane % G) W, p offsets lane / G + it *
  // kApplyThreads / G.
  const uint64_t lane_offset = static_cast<uint64_t>(threadIdx.x % G) * W +
                               static_cast<uint64_t>(threadIdx.x / G) * n;
  const uint64_t load_step = static_cast<uint64_t>(kApplyThreads / G) * n;
  auto load_tile = [&](uint64_t p0, uint64_t q0) {
    if constexpr (VEC) {
      // whole granules; absent ones load the first element and are zeroed
      const T* at = dy + p0 * n + q0 + lane_offset;
      const bool q_present = q0 + static_cast<uint64_t>(threadIdx.x % G) * W < n;
      const uint64_t first_p = p0 + threadIdx.x / G;
      staged_present = 0;
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const bool present =
            WHOLE ||
            (q_present && first_p + static_cast<uint64_t>(it) * (kApplyThreads / G) < rows);
        const V v = stream_load(reinterpret_cast<const V*>(present ? at + it * load_step : dy));
        staged[it] = present ? v : V{};
        staged_present |= present ? 1U << it : 0U;
      }
    } else {
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const int index = it * kApplyThreads + threadIdx.x;
        const uint64_t p = p0 + index / G;
        const uint64_t q = q0 + static_cast<uint64_t>(index % G) * W;
        V v{};
        if (p < rows) {
#pragma unroll
          for (int k = 0; k < W; ++k) {
            if (q + k < n) {
              const T element = dy[p * n + q + k];
              vec_set<T>(v, k, scaled ? value * element : element);
            }
          }
        }
        staged[it] = v;
      }
    }
  };
  // Store-phase layout: a lane keeps p granule c and takes q granules g0,
  // g0 + kGroups, ... (one per block).
  const int c = threadIdx.x % (TP / W);
  const int g0 = threadIdx.x / (TP / W);
  uint32_t tile = blockIdx.x;
  if (tile >= tile_count) return;
  uint64_t p0 = 0;
  uint64_t q0 = 0;
  locate(tile, p0, q0);
  load_tile(p0, q0);
  while (true) {
    const uint32_t next = tile + gridDim.x;
    __syncthreads();  // the previous tile's LDS readers are done
#pragma unroll
    for (int it = 0; it < kLoads; ++it) {
      const int index = it * kApplyThreads + threadIdx.x;
      const int row = index / G;
      V v = staged[it];
      if (VEC && scaled && ((staged_present >> it) & 1U)) v = scale_granule<T>(value, v);
      lds[row][(index % G) ^ ((row / W) & 7)] = v;
    }
    __syncthreads();
    // This tile's x, weight and row statistics, issued before the next
    // tile's dy loads.
    const uint64_t p = p0 + static_cast<uint64_t>(c) * W;
    T mu[W];
    T d[W];
    T mean_g[W];
    T mean_gx[W];
    V x[kBlocks][W];  // [block][q offset], W values of p each
    T w[kBlocks][W];
    if constexpr (VEC) {
      // whole granules; absent ones load the first element instead
      const bool p_present = WHOLE || p < rows;
      const uint64_t at_p = p_present ? p : 0;
      const V dv = *reinterpret_cast<const V*>(denominator + at_p);
      const V gv = *reinterpret_cast<const V*>(row_means + at_p);
      const V xv = *reinterpret_cast<const V*>(row_means + rows + at_p);
      V mv{};
      if constexpr (CENTER) mv = *reinterpret_cast<const V*>(mean + at_p);
#pragma unroll
      for (int i = 0; i < W; ++i) {
        mu[i] = vec_get<T>(mv, i);
        d[i] = p_present ? vec_get<T>(dv, i) : T(1);
        mean_g[i] = vec_get<T>(gv, i);
        mean_gx[i] = vec_get<T>(xv, i);
      }
      const uint64_t first_q = q0 + static_cast<uint64_t>(g0) * W;
      const T* at = in + p + first_q * pitch;
#pragma unroll
      for (int it = 0; it < kBlocks; ++it) {
        const uint64_t q = first_q + static_cast<uint64_t>(it) * kGroups * W;
        const bool present = WHOLE || (p_present && q < n);
        const V wv = *reinterpret_cast<const V*>(present ? weight + q : weight);
#pragma unroll
        for (int k = 0; k < W; ++k) {
          w[it][k] = vec_get<T>(wv, k);
          const V* source = reinterpret_cast<const V*>(
              present ? at + (static_cast<uint64_t>(it) * kGroups * W + k) * pitch : in);
          x[it][k] = *source;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const bool present = p + i < rows;
        mu[i] = CENTER && present ? mean[p + i] : T(0);
        d[i] = present ? denominator[p + i] : T(1);
        mean_g[i] = present ? row_means[p + i] : T(0);
        mean_gx[i] = present ? row_means[rows + p + i] : T(0);
      }
#pragma unroll
      for (int it = 0; it < kBlocks; ++it) {
        const uint64_t q = q0 + static_cast<uint64_t>(g0 + it * kGroups) * W;
#pragma unroll
        for (int k = 0; k < W; ++k) {
          w[it][k] = q + k < n ? weight[q + k] : T(0);
          x[it][k] = q + k < n ? load_column_group<T, false>(in, p, q + k, pitch, rows) : V{};
        }
      }
    }
    uint64_t next_p0 = p0;
    uint64_t next_q0 = q0;
    if (next < tile_count) {
      locate(next, next_p0, next_q0);
      load_tile(next_p0, next_q0);  // in flight during this tile's stores
    }
    T r[W];
#pragma unroll
    for (int i = 0; i < W; ++i) r[i] = T(1) / d[i];
#pragma unroll
    for (int it = 0; it < kBlocks; ++it) {
      const int g = g0 + it * kGroups;
      const uint64_t q = q0 + static_cast<uint64_t>(g) * W;
      if (!WHOLE && (q >= n || p >= rows)) continue;
      T grad[W][W];  // [p offset][q offset]
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const V block = lds[c * W + i][g ^ (c & 7)];
#pragma unroll
        for (int k = 0; k < W; ++k) grad[i][k] = vec_get<T>(block, k);
      }
#pragma unroll
      for (int k = 0; k < W; ++k) {
        if (!WHOLE && q + k >= n) break;
        V o;
#pragma unroll
        for (int i = 0; i < W; ++i) {
          const Divisor<T> divide(d[i], r[i]);
          const T xhat = divide(vec_get<T>(x[it][k], i) - mu[i]);
          const T gw = grad[i][k] * w[it][k];
          vec_set<T>(o, i, divide(gw - mean_g[i] - xhat * mean_gx[i]));
        }
        T* column = dx + p + (q + k) * dx_stride;
        if constexpr (VEC) {
          store_vector<NT>(reinterpret_cast<V*>(column), o);
        } else {
#pragma unroll
          for (int i = 0; i < W; ++i) {
            if (p + i < rows) column[i] = vec_get<T>(o, i);
          }
        }
      }
    }
    if (next >= tile_count) break;
    tile = next;
    p0 = next_p0;
    q0 = next_q0;
  }
}

uint32_t grid_for(uint64_t blocks) {
  if (blocks == 0) blocks = 1;
  return static_cast<uint32_t>(blocks > kMaxGrid ? kMaxGrid : blocks);
}

struct NormArgs {
  void* out;
  void* mean;
  void* denominator;
  const void* input;
  uint64_t input_stride;  // elements between the starts of two input rows
  const void* weight;
  const void* bias;
  uint64_t rows;
  uint64_t n;
  double eps;
  bool center;
};

template <typename T, int THREADS, int E, bool CENTER, bool VEC>
void forward_as(const NormArgs& a, const DeviceGuard& guard) {
  const bool full = a.n == static_cast<uint64_t>(THREADS) * E;
  const T eps = static_cast<T>(a.eps);
  auto launch = [&](auto kernel) {
    for (uint64_t first = 0; first < a.rows; first += kMaxGrid) {
      const uint64_t count = a.rows - first < kMaxGrid ? a.rows - first : kMaxGrid;
      T* mean = a.mean != nullptr ? static_cast<T*>(a.mean) + first : nullptr;  // null for RMSNorm
      kernel<<<static_cast<uint32_t>(count), THREADS, 0, guard.stream>>>(
          static_cast<T*>(a.out) + first * a.n, mean, static_cast<T*>(a.denominator) + first,
          static_cast<const T*>(a.input) + first * a.input_stride, a.input_stride,
          static_cast<const T*>(a.weight), static_cast<const T*>(a.bias), a.n, eps);
    }
  };
  with_policy(stream_output(a.rows * a.n * sizeof(T)), [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    if (full) {
      launch(norm_forward_kernel<T, THREADS, E, CENTER, VEC, true, NT>);
    } else {
      launch(norm_forward_kernel<T, THREADS, E, CENTER, VEC, false, NT>);
    }
  });
}

// Rows down storage columns: statistics pass, then the tiled apply pass.
// The [splits, rows] partials come from the stream-ordered scratch pool.
template <typename T, bool CENTER, bool VEC>
hipError_t forward_columns_as(const NormArgs& a, uint64_t pitch, int device,
                              const DeviceGuard& guard) {
  constexpr int W = Vec16<T>::width;
  constexpr uint64_t kColumns = static_cast<uint64_t>(kStatGroups) * W;
  constexpr uint64_t kTile = static_cast<uint64_t>(kApplyGranules) * W;
  const uint64_t tiles_p = (a.rows + kTile - 1) / kTile;
  const uint64_t tiles_q = (a.n + kTile - 1) / kTile;
  const uint64_t tiles = tiles_p * tiles_q;
  // Splits of q: about one strip workgroup per CU, at most kMaxStatSplits,
  // and at least one full batch of rows per lane.  On x^T for x [8192,
  // 4096] float32 (128 strips) the statistics pass took 23.9 us with 2
  // splits (one workgroup per CU), 26.5 us with 4 and 35.1 us with 1.
  const uint64_t strips = (a.rows + kColumns - 1) / kColumns;
  const uint64_t cus = static_cast<uint64_t>(guard.multiprocessors);
  const uint64_t wanted = cus * 2;
  uint64_t splits = (cus + strips / 2) / strips;
  const uint64_t most = a.n / (static_cast<uint64_t>(kStatRows) * kStatBatch);
  if (splits > most) splits = most;
  if (splits > static_cast<uint64_t>(kMaxStatSplits)) splits = kMaxStatSplits;
  if (splits < 1) splits = 1;
  const uint64_t segment = (a.n + splits - 1) / splits;
  splits = (a.n + segment - 1) / segment;
  void* scratch = nullptr;
  hipError_t error = scratch_allocate(&scratch, splits * a.rows * sizeof(double2), device);
  if (error != hipSuccess) return error;
  auto* partial = static_cast<double2*>(scratch);
  const T* in = static_cast<const T*>(a.input);
  const uint32_t stats_grid = grid_for(strips * splits);
  if (a.rows * a.n * sizeof(T) <= kCacheReuseBytes) {
    norm_column_stats_kernel<T, CENTER, VEC, kStatBatch, true>
        <<<stats_grid, kStatThreads, 0, guard.stream>>>(partial, in, pitch, a.rows, a.n, splits,
                                                        segment);
  } else {
    norm_column_stats_kernel<T, CENTER, VEC, kStatBatch, false>
        <<<stats_grid, kStatThreads, 0, guard.stream>>>(partial, in, pitch, a.rows, a.n, splits,
                                                        segment);
  }
  FastDiv divide_q;
  FastDiv divide_p;
  divide_q.init(static_cast<uint32_t>(tiles_q));
  divide_p.init(static_cast<uint32_t>(tiles_p));
  with_policy(stream_output(a.rows * a.n * sizeof(T)), [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    const auto kernel = norm_apply_columns_kernel<T, CENTER, VEC, NT>;
    // One workgroup per resident slot, each walking tiles; they do not
    // depend on each other, so an unknown occupancy (0) takes two per CU.
    uint64_t slots = resident_blocks(kernel, kApplyThreads, guard);
    if (slots == 0) slots = wanted;
    kernel<<<static_cast<uint32_t>(tiles < slots ? tiles : slots), kApplyThreads, 0,
             guard.stream>>>(static_cast<T*>(a.out), static_cast<T*>(a.mean),
                             static_cast<T*>(a.denominator), in, pitch,
                             static_cast<const T*>(a.weight), static_cast<const T*>(a.bias),
                             partial, static_cast<uint32_t>(splits), a.rows, a.n,
                             static_cast<T>(a.eps), divide_q, divide_p,
                             static_cast<uint32_t>(tiles));
  });
  error = hipGetLastError();
  scratch_release(scratch, device);  // stream-ordered reuse
  return error;
}

struct NormBackwardArgs {
  void* dx;
  uint64_t dx_stride;  // row layout: elements between dx rows; column layout: between q
  void* dweight;
  void* dbias;
  const void* dy;
  const void* dy_scale;  // null, or one element: dy = *dy_scale * dy[i]
  const void* input;
  uint64_t input_stride;
  const void* weight;
  const void* mean;
  const void* denominator;
  uint64_t rows;
  uint64_t n;
  bool center;
};

// Rows down storage columns: sums pass, finish, tiled apply pass.  The
// partials come from the stream-ordered scratch pool.
template <typename T, bool CENTER, int MODE>
hipError_t backward_columns_as(const NormBackwardArgs& a, uint64_t pitch, int device,
                               const DeviceGuard& guard) {
  constexpr int W = Vec16<T>::width;
  constexpr uint64_t kTile = static_cast<uint64_t>(kApplyGranules) * W;
  const uint64_t tiles_p = (a.rows + kTile - 1) / kTile;
  const uint64_t tiles_q = (a.n + kTile - 1) / kTile;
  const uint64_t tiles = tiles_p * tiles_q;
  // Splits of q for the sums pass: about one workgroup per CU.  On x^T for
  // x [8192, 4096] float32 (32 p tiles, 64 q tiles; two workgroups fit a CU)
  // the whole fused backward took 174 us with 8 splits, against 203, 183,
  // 178, 181 and 192 us with 4, 6, 16, 12 and 64.
  const uint64_t cus = static_cast<uint64_t>(guard.multiprocessors);
  uint64_t splits = (cus + tiles_p - 1) / tiles_p;
  if (splits > tiles_q) splits = tiles_q;
  if (splits < 1) splits = 1;
  const uint64_t split_tiles = (tiles_q + splits - 1) / splits;
  splits = (tiles_q + split_tiles - 1) / split_tiles;
  const uint64_t row_partials = 2 * splits * a.rows;
  const uint64_t column_partials = (CENTER ? 2 : 1) * tiles_p * a.n;
  const uint64_t row_means = 2 * a.rows;
  void* scratch = nullptr;
  hipError_t error = scratch_allocate(
      &scratch, (row_partials + column_partials + row_means) * sizeof(T) + 512, device);
  if (error != hipSuccess) return error;
  // three 256-byte aligned pieces
  auto piece = [](void* base, uint64_t offset) {
    return reinterpret_cast<T*>((reinterpret_cast<uintptr_t>(base) + offset + 255) /
                                256 * 256);
  };
  T* row_partial = static_cast<T*>(scratch);
  T* partial_weight = piece(scratch, row_partials * sizeof(T));
  T* partial_bias = CENTER ? partial_weight + tiles_p * a.n : nullptr;
  T* means = piece(partial_weight, column_partials * sizeof(T));
  const T* dy = static_cast<const T*>(a.dy);
  const T* dy_scale = static_cast<const T*>(a.dy_scale);
  const T* in = static_cast<const T*>(a.input);
  const T* weight = static_cast<const T*>(a.weight);
  const T* mean = static_cast<const T*>(a.mean);
  const T* denominator = static_cast<const T*>(a.denominator);
  const uint32_t sums_grid = static_cast<uint32_t>(tiles_p * splits);
  if (a.rows * a.n * sizeof(T) <= kCacheReuseBytes) {
    norm_backward_columns_sums_kernel<T, CENTER, MODE, true, kSumsThreads>
        <<<sums_grid, kSumsThreads, 0, guard.stream>>>(
            row_partial, partial_weight, partial_bias, dy, dy_scale, in, pitch, weight, mean,
            denominator,
            a.rows, a.n, static_cast<uint32_t>(tiles_q), static_cast<uint32_t>(splits),
            static_cast<uint32_t>(split_tiles));
  } else {
    norm_backward_columns_sums_kernel<T, CENTER, MODE, false, kSumsThreads>
        <<<sums_grid, kSumsThreads, 0, guard.stream>>>(
            row_partial, partial_weight, partial_bias, dy, dy_scale, in, pitch, weight, mean,
            denominator,
            a.rows, a.n, static_cast<uint32_t>(tiles_q), static_cast<uint32_t>(splits),
            static_cast<uint32_t>(split_tiles));
  }
  const uint64_t column_blocks = (a.n + kWave - 1) / kWave;
  const uint64_t row_blocks = (a.rows + kCombineThreads - 1) / kCombineThreads;
  norm_backward_columns_finish_kernel<T, CENTER>
      <<<static_cast<uint32_t>((CENTER ? 2 : 1) * column_blocks + row_blocks), kCombineThreads,
         0, guard.stream>>>(static_cast<T*>(a.dweight), static_cast<T*>(a.dbias), means,
                            partial_weight, partial_bias, tiles_p, row_partial, splits, a.rows,
                            a.n, column_blocks);
  FastDiv divide_p;
  FastDiv divide_q;
  divide_p.init(static_cast<uint32_t>(tiles_p));
  divide_q.init(static_cast<uint32_t>(tiles_q));
  with_policy(stream_output(a.rows * a.n * sizeof(T)), [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    const auto kernel = norm_backward_columns_apply_kernel<T, CENTER, MODE, NT>;
    // One workgroup per resident slot, each walking tiles; they do not
    // depend on each other, so an unknown occupancy (0) takes two per CU.
    uint64_t slots = resident_blocks(kernel, kApplyThreads, guard);
    if (slots == 0) slots = 2 * cus;
    kernel<<<static_cast<uint32_t>(tiles < slots ? tiles : slots), kApplyThreads, 0,
             guard.stream>>>(static_cast<T*>(a.dx), a.dx_stride, dy, dy_scale, in, pitch,
                             weight, mean, denominator, means, a.rows, a.n, divide_p, divide_q,
                             static_cast<uint32_t>(tiles));
  });
  error = hipGetLastError();
  scratch_release(scratch, device);  // stream-ordered reuse
  return error;
}

template <typename T, int THREADS, int E, bool CENTER, bool VEC>
hipError_t backward_as(const NormBackwardArgs& a, int device, const DeviceGuard& guard) {
  const bool full = a.n == static_cast<uint64_t>(THREADS) * E;
  const bool stream = stream_output(a.rows * a.n * sizeof(T));
  // float32 rows of up to 16 elements per lane take the prefetching kernel
  // (one workgroup per CU); the others the plain one (two per CU).
  constexpr bool kPipelined = sizeof(T) == 4 && E <= 16;
  // The four instantiations share one register budget, so any of them gives
  // the occupancy bound.
  auto kernel_for = [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    if constexpr (kPipelined) {
      return full ? norm_backward_pipelined_kernel<T, THREADS, E, CENTER, VEC, true, NT>
                  : norm_backward_pipelined_kernel<T, THREADS, E, CENTER, VEC, false, NT>;
    } else {
      return full ? norm_backward_kernel<T, THREADS, E, CENTER, VEC, true, NT>
                  : norm_backward_kernel<T, THREADS, E, CENTER, VEC, false, NT>;
    }
  };
  // Enough rows in flight per CU while keeping the [grid, n] partials small,
  // bounded by occupancy.  The workgroups do not depend on each other, so an
  // unknown occupancy (0) leaves the wanted count.
  const uint64_t resident = stream ? resident_blocks(kernel_for(Policy<true>{}), THREADS, guard)
                                   : resident_blocks(kernel_for(Policy<false>{}), THREADS, guard);
  // The prefetching kernel fills every resident slot (one 512-lane workgroup
  // per CU at 8192 float32 columns, more for shorter rows); the plain one
  // takes two per CU.
  const uint64_t cus = static_cast<uint64_t>(guard.multiprocessors);
  const uint64_t wanted = kPipelined ? (resident != 0 ? resident : cus * 2) : cus * 2;
  uint64_t grid = resident != 0 && resident < wanted ? resident : wanted;
  if (grid > a.rows) grid = a.rows;
  const uint64_t parts = (CENTER ? 2 : 1) * grid * a.n;
  void* scratch = nullptr;
  hipError_t error = scratch_allocate(&scratch, parts * sizeof(T), device);
  if (error != hipSuccess) return error;
  T* partial_weight = static_cast<T*>(scratch);
  T* partial_bias = CENTER ? partial_weight + grid * a.n : nullptr;
  with_policy(stream, [&](auto nt) {
    kernel_for(nt)<<<static_cast<uint32_t>(grid), THREADS, 0, guard.stream>>>(
        static_cast<T*>(a.dx), a.dx_stride, partial_weight, partial_bias,
        static_cast<const T*>(a.dy), static_cast<const T*>(a.dy_scale),
        static_cast<const T*>(a.input), a.input_stride, static_cast<const T*>(a.weight),
        static_cast<const T*>(a.mean), static_cast<const T*>(a.denominator), a.rows, a.n);
  });
  const uint64_t groups = (a.n + kWave - 1) / kWave;
  if constexpr (CENTER) {
    norm_combine_pair_kernel<T><<<grid_for(2 * groups), kCombineThreads, 0, guard.stream>>>(
        static_cast<T*>(a.dweight), partial_weight, static_cast<T*>(a.dbias), partial_bias, grid,
        a.n);
  } else {
    norm_combine_kernel<T><<<grid_for(groups), kCombineThreads, 0, guard.stream>>>(
        static_cast<T*>(a.dweight), partial_weight, grid, a.n);
  }
  error = hipGetLastError();
  scratch_release(scratch, device);  // stream-ordered reuse
  return error;
}

// Register-row configurations (threads, elements per lane) by row length,
// chosen so that the forward (x and one parameter row) and the backward (x,
// g, a parameter row and two accumulators) stay within the VGPR budget of
// their workgroup size.  Rows up to kMaxExtent (float32) / kMaxExtent / 2
// (float64) elements.
constexpr uint64_t kMaxExtent = 16384;

template <typename T, bool CENTER, bool VEC>
bool dispatch_forward(const NormArgs& a, const DeviceGuard& guard) {
  const uint64_t n = a.n;
  if (n <= 256 * 4) {
    forward_as<T, 256, 4, CENTER, VEC>(a, guard);
    return true;
  }
  if (n <= 256 * 16) {
    forward_as<T, 256, 16, CENTER, VEC>(a, guard);
    return true;
  }
  // 8192 float32: 512 lanes x 16 (60 VGPRs, four workgroups per CU, 1024
  // rows at once) took 47.8-49 us on [4096, 8192] LayerNorm against
  // 49.8-51.5 us for 256 x 32 (74 VGPRs, six per CU: 4096 rows in 2.7
  // rounds); 1024 x 8 took 51-55 us.
  if (n <= 512 * 16) {
    forward_as<T, 512, 16, CENTER, VEC>(a, guard);
    return true;
  }
  if constexpr (sizeof(T) == 4) {
    if (n <= 1024 * 16) {
      forward_as<T, 1024, 16, CENTER, VEC>(a, guard);
      return true;
    }
  }
  return false;
}

template <typename T, bool CENTER, bool VEC>
hipError_t dispatch_backward(const NormBackwardArgs& a, int device, const DeviceGuard& guard,
                             bool& handled) {
  const uint64_t n = a.n;
  handled = true;
  if (n <= 256 * 4) return backward_as<T, 256, 4, CENTER, VEC>(a, device, guard);
  if (n <= 256 * 16) return backward_as<T, 256, 16, CENTER, VEC>(a, device, guard);
  if (n <= 512 * 16) return backward_as<T, 512, 16, CENTER, VEC>(a, device, guard);
  if constexpr (sizeof(T) == 4) {
    // 512 lanes (two waves per SIMD, 256 VGPRs each) rather than 1024 (128)
    if (n <= 512 * 32) return backward_as<T, 512, 32, CENTER, VEC>(a, device, guard);
  }
  handled = false;
  return hipSuccess;
}

bool aligned_rows(const void* p, uint64_t n, int width) {
  return p == nullptr || (aligned16(p) && n % static_cast<uint64_t>(width) == 0);
}

}  // namespace
}  // namespace spar_hip

using namespace spar_hip;

extern "C" uint64_t spar_hip_norm_max_extent(int dtype) {
  return dtype == SPAR_HIP_FLOAT32 ? kMaxExtent : dtype == SPAR_HIP_FLOAT64 ? kMaxExtent / 2 : 0;
}

extern "C" SparHipStatus spar_hip_launch_norm_forward(void* output, void* mean, void* denominator,
                                                      const void* input, uint64_t input_row_stride,
                                                      uint64_t input_column_stride,
                                                      const void* weight, const void* bias,
                                                      uint64_t rows, uint64_t extent,
                                                      double epsilon, int center, int dtype,
                                                      int device) {
  // Row layout: elements of a row adjacent, rows input_row_stride >= extent
  // apart.  Column layout: rows adjacent (row stride 1), a row's elements
  // input_column_stride >= rows apart.
  const bool row_layout = input_column_stride == 1 && input_row_stride >= extent;
  const bool column_layout =
      input_column_stride != 1 && input_row_stride == 1 && input_column_stride >= rows;
  if (!valid_float_dtype(dtype) || (center != 0 && center != 1) || extent == 0 ||
      extent > spar_hip_norm_max_extent(dtype) || !(epsilon >= 0.0) ||
      !(row_layout || column_layout) ||
      (rows != 0 && (output == nullptr || denominator == nullptr || input == nullptr ||
                     weight == nullptr || (center && (mean == nullptr || bias == nullptr))))) {
    return invalid();
  }
  if (rows == 0) return ok();
  const int width = dtype == SPAR_HIP_FLOAT32 ? 4 : 2;
  if (column_layout) {
    const uint64_t tile = static_cast<uint64_t>(kApplyGranules) * width;
    const uint64_t tiles = ((rows + tile - 1) / tile) * ((extent + tile - 1) / tile);
    if (tiles > kIndex32Limit) return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const NormArgs a{output,  mean, denominator, input,   input_row_stride,
                   weight,  bias, rows,        extent,  epsilon,
                   center != 0};
  const bool parameters_vec = aligned_rows(output, extent, width) && extent % width == 0 &&
                              aligned_rows(weight, extent, width) &&
                              aligned_rows(bias, extent, width);
  if (column_layout) {
    const bool vec = parameters_vec && aligned_rows(input, input_column_stride, width) &&
                     rows % static_cast<uint64_t>(width) == 0;
    hipError_t error = hipSuccess;
    auto run = [&](auto tag, auto center_tag, auto vec_tag) {
      using T = decltype(tag);
      error = forward_columns_as<T, decltype(center_tag)::value, decltype(vec_tag)::value>(
          a, input_column_stride, device, guard);
    };
    auto with_vec = [&](auto tag, auto center_tag) {
      if (vec) {
        run(tag, center_tag, std::true_type{});
      } else {
        run(tag, center_tag, std::false_type{});
      }
    };
    auto with_center = [&](auto tag) {
      if (center) {
        with_vec(tag, std::true_type{});
      } else {
        with_vec(tag, std::false_type{});
      }
    };
    if (dtype == SPAR_HIP_FLOAT32) {
      with_center(float{});
    } else {
      with_center(double{});
    }
    if (error != hipSuccess) return runtime(error);
    return finish(guard);
  }
  const bool vec = parameters_vec && aligned_rows(input, input_row_stride, width);
  bool done = false;
  if (dtype == SPAR_HIP_FLOAT32) {
    if (center) {
      done = vec ? dispatch_forward<float, true, true>(a, guard)
                 : dispatch_forward<float, true, false>(a, guard);
    } else {
      done = vec ? dispatch_forward<float, false, true>(a, guard)
                 : dispatch_forward<float, false, false>(a, guard);
    }
  } else {
    if (center) {
      done = vec ? dispatch_forward<double, true, true>(a, guard)
                 : dispatch_forward<double, true, false>(a, guard);
    } else {
      done = vec ? dispatch_forward<double, false, true>(a, guard)
                 : dispatch_forward<double, false, false>(a, guard);
    }
  }
  if (!done) return invalid();
  return finish(guard);
}

namespace {

SparHipStatus norm_backward(void* input_gradient, uint64_t input_gradient_stride,
                            void* weight_gradient, void* bias_gradient,
                            const void* output_gradient, const void* output_gradient_scale,
                            const void* input, uint64_t input_row_stride,
                            uint64_t input_column_stride, const void* weight, const void* mean,
                            const void* denominator, uint64_t rows, uint64_t extent, int center,
                            int dtype, int device) {
  // The forward's two layouts.  dx takes the input's layout: rows
  // input_gradient_stride apart (row layout), or dx[p + q * stride] (column
  // layout; stride == rows packs it).
  const bool row_layout = input_column_stride == 1 && input_row_stride >= extent &&
                          input_gradient_stride >= extent;
  const bool column_layout = input_column_stride != 1 && input_row_stride == 1 &&
                             input_column_stride >= rows && input_gradient_stride >= rows;
  if (!valid_float_dtype(dtype) || (center != 0 && center != 1) || extent == 0 ||
      extent > spar_hip_norm_max_extent(dtype) || !(row_layout || column_layout) ||
      (rows != 0 &&
       (input_gradient == nullptr || weight_gradient == nullptr || output_gradient == nullptr ||
        input == nullptr || weight == nullptr || denominator == nullptr ||
        (center && (mean == nullptr || bias_gradient == nullptr))))) {
    return invalid();
  }
  const int width = dtype == SPAR_HIP_FLOAT32 ? 4 : 2;
  if (column_layout) {
    const uint64_t tile = static_cast<uint64_t>(kApplyGranules) * width;
    const uint64_t tiles = ((rows + tile - 1) / tile) * ((extent + tile - 1) / tile);
    if (tiles > kIndex32Limit) return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (rows == 0) {
    // no rows: the parameter gradients are zero (fill kernels, no memset)
    const uint64_t bytes = extent * (dtype == SPAR_HIP_FLOAT32 ? 4 : 8);
    SparHipStatus status = spar_hip_zero(weight_gradient, bytes, device);
    if (status.code == 0 && center) status = spar_hip_zero(bias_gradient, bytes, device);
    return status;
  }
  const NormBackwardArgs a{input_gradient,   input_gradient_stride, weight_gradient,
                           bias_gradient,    output_gradient,       output_gradient_scale,
                           input,            input_row_stride,      weight,
                           mean,             denominator,           rows,
                           extent,           center != 0};
  if (column_layout) {
    const bool vec = aligned_rows(output_gradient, extent, width) && extent % width == 0 &&
                     aligned_rows(weight, extent, width) &&
                     aligned_rows(input, input_column_stride, width) &&
                     aligned_rows(input_gradient, input_gradient_stride, width) &&
                     rows % static_cast<uint64_t>(width) == 0 &&
                     aligned16(denominator) && (!center || aligned16(mean));
    // every tile whole: rows and extent multiples of the tile side
    const uint64_t tile = static_cast<uint64_t>(kApplyGranules) * width;
    const bool whole = vec && rows % tile == 0 && extent % tile == 0;
    hipError_t error = hipSuccess;
    auto run = [&](auto tag, auto center_tag, auto mode_tag) {
      using T = decltype(tag);
      error = backward_columns_as<T, decltype(center_tag)::value, decltype(mode_tag)::value>(
          a, input_column_stride, device, guard);
    };
    auto with_vec = [&](auto tag, auto center_tag) {
      if (whole) {
        run(tag, center_tag, std::integral_constant<int, kWholeTiles>{});
      } else if (vec) {
        run(tag, center_tag, std::integral_constant<int, kVectorTiles>{});
      } else {
        run(tag, center_tag, std::integral_constant<int, kScalarTiles>{});
      }
    };
    auto with_center = [&](auto tag) {
      if (center) {
        with_vec(tag, std::true_type{});
      } else {
        with_vec(tag, std::false_type{});
      }
    };
    if (dtype == SPAR_HIP_FLOAT32) {
      with_center(float{});
    } else {
      with_center(double{});
    }
    if (error != hipSuccess) return runtime(error);
    return finish(guard);
  }
  const bool vec = aligned_rows(input_gradient, input_gradient_stride, width) &&
                   aligned_rows(output_gradient, extent, width) &&
                   aligned_rows(input, input_row_stride, width) && extent % width == 0 &&
                   aligned_rows(weight, extent, width);
  bool handled = false;
  hipError_t error = hipSuccess;
  if (dtype == SPAR_HIP_FLOAT32) {
    if (center) {
      error = vec ? dispatch_backward<float, true, true>(a, device, guard, handled)
                  : dispatch_backward<float, true, false>(a, device, guard, handled);
    } else {
      error = vec ? dispatch_backward<float, false, true>(a, device, guard, handled)
                  : dispatch_backward<float, false, false>(a, device, guard, handled);
    }
  } else {
    if (center) {
      error = vec ? dispatch_backward<double, true, true>(a, device, guard, handled)
                  : dispatch_backward<double, true, false>(a, device, guard, handled);
    } else {
      error = vec ? dispatch_backward<double, false, true>(a, device, guard, handled)
                  : dispatch_backward<double, false, false>(a, device, guard, handled);
    }
  }
  if (!handled) return invalid();
  if (error != hipSuccess) return runtime(error);
  return finish(guard);
}

}  // namespace

extern "C" SparHipStatus spar_hip_launch_norm_backward(
    void* input_gradient, uint64_t input_gradient_stride, void* weight_gradient,
    void* bias_gradient, const void* output_gradient, const void* input,
    uint64_t input_row_stride, uint64_t input_column_stride, const void* weight, const void* mean,
    const void* denominator, uint64_t rows, uint64_t extent, int center, int dtype, int device) {
  return norm_backward(input_gradient, input_gradient_stride, weight_gradient, bias_gradient,
                       output_gradient, nullptr, input, input_row_stride, input_column_stride,
                       weight, mean, denominator, rows, extent, center, dtype, device);
}

extern "C" SparHipStatus spar_hip_launch_norm_backward_scaled(
    void* input_gradient, uint64_t input_gradient_stride, void* weight_gradient,
    void* bias_gradient, const void* output_gradient, const void* output_gradient_scale,
    const void* input, uint64_t input_row_stride, uint64_t input_column_stride,
    const void* weight, const void* mean, const void* denominator, uint64_t rows,
    uint64_t extent, int center, int dtype, int device) {
  if (output_gradient_scale == nullptr && rows != 0) return invalid();
  return norm_backward(input_gradient, input_gradient_stride, weight_gradient, bias_gradient,
                       output_gradient, output_gradient_scale, input, input_row_stride,
                       input_column_stride, weight, mean, denominator, rows, extent, center,
                       dtype, device);
}
