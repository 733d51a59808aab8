// Contiguous elementwise kernels: binary, compare, scalar, unary, fills,
// gradient accumulation and the seeded generators.
//
// Replaces kernels K1-K3, K9, K10 of src/backend/cuda_kernels.cu (:113-191,
// :249-266).  Design for CDNA4: each 256-thread workgroup streams one tile of
// 256 x UNROLL 16-byte vectors per operand, issuing every load of the tile
// before the first store so that UNROLL independent 128-bit loads per lane
// are in flight; the tiles are laid out so consecutive lanes touch
// consecutive 16-byte words (fully coalesced 1 KiB per wave per load).  The
// grid has one workgroup per tile (tens of thousands at the benchmark shapes,
// far more than the 256 CUs), and a tile loop keeps launches within the grid
// limit for any size.  Pointers that are not 16-byte aligned take a scalar
// grid-stride kernel.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.hpp"
#include "ops.hpp"

namespace spar_hip {
namespace {

// One 16-byte vector per lane per tile and one tile per single-wave
// workgroup: on MI355X this beats deeper per-lane unrolling and larger
// workgroups for streaming kernels (many short workgroups keep every CU's
// memory pipeline full until the end of the grid).  A broadcast add over
// x[32768, 4096] (1 GiB moved, steady state) took 161 / 162 / 165 / 169 us
// with workgroups of 64 / 128 / 256 / 512 lanes.
constexpr int kThreads = 256;        // grid-stride scalar kernels
constexpr int kVectorThreads = 64;   // streaming vector kernels
constexpr int kUnroll = 1;
constexpr uint64_t kMaxGrid = uint64_t{1} << 20;

template <typename T, typename F, bool NT>
__global__ void __launch_bounds__(kVectorThreads)
    map1_vec_kernel(T* out, const T* in, uint64_t count, F f) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  const uint64_t vectors = count / W;
  constexpr int U = VectorsPerLane<F>::value;
  const uint64_t tile = static_cast<uint64_t>(kVectorThreads) * U;
  const V* in_v = reinterpret_cast<const V*>(in);
  V* out_v = reinterpret_cast<V*>(out);
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile; base < vectors;
       base += static_cast<uint64_t>(gridDim.x) * tile) {
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads + threadIdx.x;
      if (i < vectors) r[u] = stream_load(in_v + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads + threadIdx.x;
      if (i < vectors) {
        V o;
#pragma unroll
        for (int k = 0; k < W; ++k) vec_set<T>(o, k, f(vec_get<T>(r[u], k)));
        store_vector<NT>(out_v + i, o);
      }
    }
  }
  if (blockIdx.x == 0) {
    const uint64_t i = vectors * W + threadIdx.x;
    if (i < count) out[i] = f(in[i]);
  }
}

template <typename T, typename F, bool NT>
__global__ void __launch_bounds__(kVectorThreads)
    map2_vec_kernel(T* out, const T* a, const T* b, uint64_t count, F f) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  const uint64_t vectors = count / W;
  const uint64_t tile = static_cast<uint64_t>(kVectorThreads) * kUnroll;
  const V* a_v = reinterpret_cast<const V*>(a);
  const V* b_v = reinterpret_cast<const V*>(b);
  V* out_v = reinterpret_cast<V*>(out);
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile; base < vectors;
       base += static_cast<uint64_t>(gridDim.x) * tile) {
    V ra[kUnroll];
    V rb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads + threadIdx.x;
      if (i < vectors) {
        ra[u] = stream_load(a_v + i);
        rb[u] = stream_load(b_v + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads + threadIdx.x;
      if (i < vectors) {
        V o;
#pragma unroll
        for (int k = 0; k < W; ++k) {
          vec_set<T>(o, k, f(vec_get<T>(ra[u], k), vec_get<T>(rb[u], k)));
        }
        store_vector<NT>(out_v + i, o);
      }
    }
  }
  if (blockIdx.x == 0) {
    const uint64_t i = vectors * W + threadIdx.x;
    if (i < count) out[i] = f(a[i], b[i]);
  }
}

template <typename T, typename F>
__global__ void __launch_bounds__(kThreads)
    map1_scalar_kernel(T* out, const T* in, uint64_t count, F f) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride) {
    out[i] = f(in[i]);
  }
}

template <typename T, typename F>
__global__ void __launch_bounds__(kThreads)
    map2_scalar_kernel(T* out, const T* a, const T* b, uint64_t count, F f) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride) {
    out[i] = f(a[i], b[i]);
  }
}

uint32_t vector_grid(uint64_t count, int width, int vectors_per_lane = kUnroll) {
  const uint64_t vectors = count / static_cast<uint64_t>(width);
  const uint64_t tile = static_cast<uint64_t>(kVectorThreads) * vectors_per_lane;
  uint64_t blocks = (vectors + tile - 1) / tile;
  if (blocks == 0) blocks = 1;
  if (blocks > kMaxGrid) blocks = kMaxGrid;
  return static_cast<uint32_t>(blocks);
}

uint32_t scalar_grid(uint64_t count, const DeviceGuard& guard) {
  uint64_t blocks = (count + kThreads - 1) / kThreads;
  const uint64_t cap = static_cast<uint64_t>(guard.multiprocessors) * 16;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  return static_cast<uint32_t>(blocks);
}

// GELU of contiguous float32 with the tail table in LDS (ops.hpp).  One
// 512-lane workgroup per CU copies the table to LDS once and walks tiles of
// kGeluLoopVectors 16-byte vectors per lane, t = blockIdx.x, + gridDim.x, ...
// with two register sets used in turn: the loads of tile t + gridDim.x are
// issued before tile t is computed and stored, and no register is copied from
// one set to the other.  A loop that moved the prefetched set into the
// working set at the end of each iteration made the wave wait for those
// loads there, so the prefetch overlapped nothing: on [8192, 8192] N(0,1)
// that loop measured 73.1% of HBM bandwidth and a single-chunk-per-workgroup
// form (which copies the table per 32 KiB chunk) 73.2%; this one 75.1-76.1%,
// on [4096, 4096] 63.8% (chunks) against 69.9%.  A prefetch past the last
// whole tile reads the last whole tile again (every path issues the same
// loads, so the compiler's wait counts stay exact); it is not stored.
// Leftover vectors and the count % 4 trailing elements come after the loop.
// On the same inputs a plain copy in this loop reaches 78.5% and in
// single-wave workgroups 83%: the LDS table is what keeps GELU in the loop
// (read from global memory instead, GELU took 150 us on [8192, 8192]).
constexpr int kGeluThreads = 512;
constexpr int kGeluLoopVectors = 2;
// The table's pieces keep their global layout in LDS, two 16-byte units
// apart (18 KiB); padding them to three units measured no faster.
constexpr int kGeluLdsStride = 2;

template <bool NT>
__global__ void __launch_bounds__(kGeluThreads)
    gelu_table_kernel(float* out, const float* in, uint64_t count) {
  __shared__ f64x2 table[kGeluPieces * kGeluLdsStride];
  const f64x2* units = reinterpret_cast<const f64x2*>(kGeluTable);  // two per piece
  for (int k = threadIdx.x; k < kGeluPieces * 2; k += kGeluThreads) {
    table[(k / 2) * kGeluLdsStride + k % 2] = units[k];
  }
  const uint64_t vectors = count / 4;
  constexpr uint64_t kTile = static_cast<uint64_t>(kGeluThreads) * kGeluLoopVectors;
  const uint64_t whole = vectors / kTile;
  const f32x4* src = reinterpret_cast<const f32x4*>(in) + threadIdx.x;
  f32x4* dst = reinterpret_cast<f32x4*>(out) + threadIdx.x;
  f32x4 a[kGeluLoopVectors];
  f32x4 b[kGeluLoopVectors];
  auto load = [&](f32x4(&r)[kGeluLoopVectors], uint64_t tile) {
    const f32x4* at = src + (tile < whole ? tile : whole - 1) * kTile;
#pragma unroll
    for (int u = 0; u < kGeluLoopVectors; ++u) r[u] = stream_load(at + u * kGeluThreads);
  };
  auto emit = [&](const f32x4(&r)[kGeluLoopVectors], uint64_t tile) {
    f32x4* at = dst + tile * kTile;
#pragma unroll
    for (int u = 0; u < kGeluLoopVectors; ++u) {
      store_vector<NT>(at + u * kGeluThreads, gelu_float4<kGeluLdsStride>(r[u], table));
    }
  };
  uint64_t t = blockIdx.x;
  if (t < whole) load(a, t);  // uniform over the workgroup
  __syncthreads();            // the table is in LDS
  if (t < whole) {
    while (true) {
      const uint64_t t1 = t + gridDim.x;
      load(b, t1);
      emit(a, t);
      if (t1 >= whole) break;
      const uint64_t t2 = t1 + gridDim.x;
      load(a, t2);
      emit(b, t1);
      if (t2 >= whole) break;
      t = t2;
    }
  }
  const f32x4* rest = reinterpret_cast<const f32x4*>(in);
  f32x4* rest_out = reinterpret_cast<f32x4*>(out);
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kGeluThreads;
  for (uint64_t i = whole * kTile + static_cast<uint64_t>(blockIdx.x) * kGeluThreads + threadIdx.x;
       i < vectors; i += stride) {
    rest_out[i] = gelu_float4<kGeluLdsStride>(rest[i], table);
  }
  if (blockIdx.x == 0) {
    const uint64_t i = vectors * 4 + threadIdx.x;
    if (i < count) out[i] = gelu_float<kGeluLdsStride>(in[i], table);
  }
}

void launch_gelu_table(float* out, const float* in, uint64_t count, const DeviceGuard& guard) {
  with_policy(stream_output(count * sizeof(float)), [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    // one workgroup per CU (two or four per CU measured 1-3% slower)
    constexpr uint64_t kTile = static_cast<uint64_t>(kGeluThreads) * kGeluLoopVectors;
    const uint64_t tiles = (count / 4 + kTile - 1) / kTile;
    const uint64_t slots = static_cast<uint64_t>(guard.multiprocessors);
    const uint64_t grid = tiles == 0 ? 1 : tiles < slots ? tiles : slots;
    gelu_table_kernel<NT><<<static_cast<uint32_t>(grid), kGeluThreads, 0, guard.stream>>>(
        out, in, count);
  });
}

template <typename T, typename F>
void launch_map1(T* out, const T* in, uint64_t count, F f, const DeviceGuard& guard) {
  if constexpr (std::is_same_v<T, float> && std::is_same_v<F, GeluOp>) {
    if (aligned16(out) && aligned16(in)) {
      launch_gelu_table(out, in, count, guard);
      return;
    }
  }
  if (aligned16(out) && aligned16(in)) {
    with_policy(stream_output(count * sizeof(T)), [&](auto nt) {
      map1_vec_kernel<T, F, decltype(nt)::value>
          <<<vector_grid(count, Vec16<T>::width, VectorsPerLane<F>::value), kVectorThreads, 0,
             guard.stream>>>(out, in, count, f);
    });
  } else {
    map1_scalar_kernel<T, F><<<scalar_grid(count, guard), kThreads, 0, guard.stream>>>(
        out, in, count, f);
  }
}

template <typename T, typename F>
void launch_map2(T* out, const T* a, const T* b, uint64_t count, F f, const DeviceGuard& guard) {
  if (aligned16(out) && aligned16(a) && aligned16(b)) {
    with_policy(stream_output(count * sizeof(T)), [&](auto nt) {
      map2_vec_kernel<T, F, decltype(nt)::value>
          <<<vector_grid(count, Vec16<T>::width), kVectorThreads, 0, guard.stream>>>(out, a, b,
                                                                                    count, f);
    });
  } else {
    map2_scalar_kernel<T, F><<<scalar_grid(count, guard), kThreads, 0, guard.stream>>>(
        out, a, b, count, f);
  }
}


// How a fill derives its value from scalar[0] (or the host value): as is,
// times a factor (the reference's fill_from_scalar: g * scale), or divided by
// a divisor (the CPU mean backward's g / (T)n).  All in T.
enum class FillScale : int { kNone = 0, kMultiply = 1, kDivide = 2 };

// Writes one value to every element.  The vector form stores 16 bytes per
// lane over the aligned body and needs a 16-byte aligned output.
template <typename T>
__device__ __forceinline__ T fill_value(const T* scalar, T value, T factor, FillScale mode) {
  const T v = scalar != nullptr ? scalar[0] : value;
  if (mode == FillScale::kMultiply) return v * factor;
  if (mode == FillScale::kDivide) return v / factor;
  return v;
}

template <typename T, bool NT>
__global__ void __launch_bounds__(kVectorThreads)
    fill_vec_kernel(T* out, uint64_t count, const T* scalar, T value, T factor, FillScale mode) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  const T v = fill_value(scalar, value, factor, mode);
  V o;
#pragma unroll
  for (int k = 0; k < W; ++k) vec_set<T>(o, k, v);
  const uint64_t vectors = count / W;
  V* out_v = reinterpret_cast<V*>(out);
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kVectorThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kVectorThreads + threadIdx.x; i < vectors;
       i += stride) {
    store_vector<NT>(out_v + i, o);
  }
  if (blockIdx.x == 0) {
    const uint64_t i = vectors * W + threadIdx.x;
    if (i < count) out[i] = v;
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads)
    fill_scalar_kernel(T* out, uint64_t count, const T* scalar, T value, T factor, FillScale mode) {
  const T v = fill_value(scalar, value, factor, mode);
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride) {
    out[i] = v;
  }
}

template <typename T>
void launch_fill_values(T* out, uint64_t count, const T* scalar, T value, T factor, FillScale mode,
                        const DeviceGuard& guard) {
  if (aligned16(out)) {
    with_policy(stream_output(count * sizeof(T)), [&](auto nt) {
      fill_vec_kernel<T, decltype(nt)::value>
          <<<vector_grid(count, Vec16<T>::width), kVectorThreads, 0, guard.stream>>>(
              out, count, scalar, value, factor, mode);
    });
  } else {
    fill_scalar_kernel<T><<<scalar_grid(count, guard), kThreads, 0, guard.stream>>>(
        out, count, scalar, value, factor, mode);
  }
}

// Fills output with scalar[0] (a device element) scaled by `factor` in T.
SparHipStatus fill_from_device_scalar(void* output, const void* scalar, uint64_t count, int dtype,
                                      double factor, FillScale mode, int device) {
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (dtype == SPAR_HIP_FLOAT32) {
    launch_fill_values(static_cast<float*>(output), count, static_cast<const float*>(scalar), 0.0F,
                       static_cast<float>(factor), mode, guard);
  } else {
    launch_fill_values(static_cast<double*>(output), count, static_cast<const double*>(scalar),
                       0.0, factor, mode, guard);
  }
  return finish(guard);
}

// SplitMix64 draw `index` (0-based) of Random(seed): the generator adds the
// golden-ratio increment before mixing (src/core/random.cpp:22-28), so draw i
// mixes seed + (i + 1) * increment.
__device__ __forceinline__ uint64_t splitmix_draw(uint64_t seed, uint64_t index) {
  uint64_t value = seed + (index + 1) * 0x9E3779B97F4A7C15ULL;
  value = (value ^ (value >> 30U)) * 0xBF58476D1CE4E5B9ULL;
  value = (value ^ (value >> 27U)) * 0x94D049BB133111EBULL;
  return value ^ (value >> 31U);
}

__device__ __forceinline__ double uniform_double_draw(uint64_t seed, uint64_t index) {
  return static_cast<double>(splitmix_draw(seed, index) >> 11U) / 9007199254740992.0;
}

__global__ void __launch_bounds__(kThreads)
    uniform_f32_kernel(float* out, uint64_t count, uint64_t seed, float low, float width) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride) {
    const float u = static_cast<float>(splitmix_draw(seed, i) >> 40U) / 16777216.0F;
    out[i] = low + width * u;
  }
}

__global__ void __launch_bounds__(kThreads)
    uniform_f64_kernel(double* out, uint64_t count, uint64_t seed, double low, double width) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride) {
    out[i] = low + width * uniform_double_draw(seed, i);
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads)
    normal_kernel(T* out, uint64_t count, uint64_t seed, double mean, double stddev) {
  const uint64_t pairs = (count + 1) / 2;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  const double two_pi = 6.283185307179586476925286766559;
  for (uint64_t k = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; k < pairs;
       k += stride) {
    const double u0 = uniform_double_draw(seed, 2 * k);
    const double u1 = uniform_double_draw(seed, 2 * k + 1);
    const double radius = sqrt(-2.0 * log(1.0 - u0));
    const double angle = two_pi * u1;
    out[2 * k] = static_cast<T>(mean + stddev * (radius * cos(angle)));
    if (2 * k + 1 < count) out[2 * k + 1] = static_cast<T>(mean + stddev * (radius * sin(angle)));
  }
}

// ---------------------------------------------------------------- window embed
//
// output[o][e][i] = e in [start, start + length) ? input[o][e - start][i] : 0
// for the row-major output [outer, extent, inner] and the contiguous window
// input [outer, length, inner]: narrow's gradient scattered into a zeroed
// tensor of the base's shape in one pass (the zero fill and the window's
// strided assign wrote the window twice).  Each lane handles G elements at a
// time, G = 16 / sizeof(element) when every group lies inside one window row
// or outside it and the input groups stay 16-byte aligned (VEC), else 1;
// one 32-bit invariant-divisor division pair per group.
template <typename E, bool VEC>
__global__ void __launch_bounds__(kThreads)
    window_embed_kernel(E* output, const E* input, uint64_t groups, uint32_t length,
                        uint32_t start, FastDiv inner, FastDiv extent) {
  constexpr int G = VEC ? static_cast<int>(16 / sizeof(E)) : 1;
  using V = typename Vec16<E>::type;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t group = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
       group < groups; group += stride) {
    const uint32_t element = static_cast<uint32_t>(group) * G;
    const uint32_t row = inner.div(element);
    const uint32_t i = element - row * inner.divisor;
    const uint32_t o = extent.div(row);
    const uint32_t e = row - o * extent.divisor;
    const bool inside = e >= start && e - start < length;
    const uint64_t from = (static_cast<uint64_t>(o) * length + (e - start)) * inner.divisor + i;
    if constexpr (VEC) {
      V value{};
      if (inside) value = stream_load(reinterpret_cast<const V*>(input + from));
      *reinterpret_cast<V*>(output + element) = value;
    } else {
      output[element] = inside ? input[from] : E(0);
    }
  }
}

template <typename E>
void launch_window_embed(E* output, const E* input, uint64_t outer, uint64_t extent,
                         uint64_t inner, uint64_t start, uint64_t length,
                         const DeviceGuard& guard) {
  constexpr uint64_t G = 16 / sizeof(E);
  const uint64_t count = outer * extent * inner;
  // Groups of G elements stay in one row and keep the input aligned when
  // rows are multiples of G, or when the narrowed axis is the last one and
  // its window starts and ends on group boundaries.
  const bool vec = aligned16(output) && aligned16(input) &&
                   (inner % G == 0 || (inner == 1 && extent % G == 0 && start % G == 0 &&
                                       length % G == 0));
  FastDiv divide_inner;
  FastDiv divide_extent;
  divide_inner.init(static_cast<uint32_t>(inner));
  divide_extent.init(static_cast<uint32_t>(extent));
  const uint64_t groups = vec ? count / G : count;
  uint64_t blocks = (groups + kThreads - 1) / kThreads;
  const uint64_t cap = static_cast<uint64_t>(guard.multiprocessors) * 16;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  if (vec) {
    window_embed_kernel<E, true><<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(
        output, input, groups, static_cast<uint32_t>(length), static_cast<uint32_t>(start),
        divide_inner, divide_extent);
  } else {
    window_embed_kernel<E, false><<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(
        output, input, groups, static_cast<uint32_t>(length), static_cast<uint32_t>(start),
        divide_inner, divide_extent);
  }
}

// A box of a contiguous tensor embedded in zeros: the output (contiguous,
// extents E[0..R-1]) takes the input (contiguous, extents L) at coordinates
// c with S[a] <= c[a] < S[a] + L[a] on every axis, zero elsewhere -- the
// gradient of a chain of narrows, in one pass.  Axes are coalesced on the
// host (R <= kMaxBoxAxes); indices are 32-bit.  VEC: groups of G elements
// along the innermost axis, whose extent, start and length are multiples of
// G, so a group is wholly inside or outside and its input stays aligned.
constexpr int kMaxBoxAxes = 4;

struct BoxGeometry {
  FastDiv extent[kMaxBoxAxes];    // output extents, outermost first
  uint32_t start[kMaxBoxAxes];
  uint32_t length[kMaxBoxAxes];
  uint32_t in_stride[kMaxBoxAxes];  // input elements per step along the axis
};

template <typename E, bool VEC, int R>
__global__ void __launch_bounds__(kThreads)
    box_embed_kernel(E* output, const E* input, uint64_t groups, BoxGeometry box) {
  constexpr int G = VEC ? static_cast<int>(16 / sizeof(E)) : 1;
  using V = typename Vec16<E>::type;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t group = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
       group < groups; group += stride) {
    const uint32_t element = static_cast<uint32_t>(group) * G;
    uint32_t rest = element;
    bool inside = true;
    uint32_t from = 0;
#pragma unroll
    for (int a = R - 1; a >= 0; --a) {
      const uint32_t outer = box.extent[a].div(rest);
      const uint32_t c = rest - outer * box.extent[a].divisor;
      rest = outer;
      inside = inside && c >= box.start[a] && c - box.start[a] < box.length[a];
      from += (c - box.start[a]) * box.in_stride[a];
    }
    if constexpr (VEC) {
      V value{};
      if (inside) value = stream_load(reinterpret_cast<const V*>(input + from));
      *reinterpret_cast<V*>(output + element) = value;
    } else {
      output[element] = inside ? input[from] : E(0);
    }
  }
}

// Only the zeros around a box, which a producer writes in place: a
// workgroup per row of the last axis (rows decoded once, not per element).
// A row inside the box on every outer axis gets its two margins along the
// last axis, any other row all of it.  VEC: 16-byte groups (the last axis's
// extent, start and length are multiples of G).
template <typename E, bool VEC, int R>
__global__ void __launch_bounds__(kThreads)
    box_border_kernel(E* output, uint64_t rows, BoxGeometry box) {
  constexpr uint32_t G = VEC ? static_cast<uint32_t>(16 / sizeof(E)) : 1;
  using V = typename Vec16<E>::type;
  const uint32_t extent = box.extent[R - 1].divisor / G;
  const uint32_t first = box.start[R - 1] / G;
  const uint32_t last = first + box.length[R - 1] / G;
  for (uint64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    uint32_t rest = static_cast<uint32_t>(row);
    bool inside = true;
#pragma unroll
    for (int a = R - 2; a >= 0; --a) {
      const uint32_t outer = box.extent[a].div(rest);
      const uint32_t c = rest - outer * box.extent[a].divisor;
      rest = outer;
      inside = inside && c >= box.start[a] && c - box.start[a] < box.length[a];
    }
    E* base = output + row * box.extent[R - 1].divisor;
    // the groups [0, first) and [last, extent) of an inside row, all others'
    const uint32_t gap_begin = inside ? first : extent;
    const uint32_t gap_end = inside ? last : extent;
    const uint32_t zeros = extent - (gap_end - gap_begin);
    for (uint32_t k = threadIdx.x; k < zeros; k += kThreads) {
      const uint32_t g = k < gap_begin ? k : k + (gap_end - gap_begin);
      if constexpr (VEC) {
        reinterpret_cast<V*>(base)[g] = V{};
      } else {
        base[g] = E(0);
      }
    }
  }
}

template <typename E>
void launch_box_embed(E* output, const E* input, int rank, const uint64_t* extents,
                      const uint64_t* starts, const uint64_t* lengths, uint64_t count,
                      const DeviceGuard& guard) {
  constexpr uint64_t G = 16 / sizeof(E);
  BoxGeometry box{};
  uint32_t in_stride = 1;
  for (int a = rank - 1; a >= 0; --a) {
    box.extent[a].init(static_cast<uint32_t>(extents[a]));
    box.start[a] = static_cast<uint32_t>(starts[a]);
    box.length[a] = static_cast<uint32_t>(lengths[a]);
    box.in_stride[a] = in_stride;
    in_stride *= static_cast<uint32_t>(lengths[a]);
  }
  const int last = rank - 1;
  const bool vec = aligned16(output) && aligned16(input) && extents[last] % G == 0 &&
                   starts[last] % G == 0 && lengths[last] % G == 0;
  const uint64_t groups = vec ? count / G : count;
  uint64_t blocks = (groups + kThreads - 1) / kThreads;
  const uint64_t cap = static_cast<uint64_t>(guard.multiprocessors) * 16;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  auto launch = [&](auto kernel) {
    kernel<<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(output, input, groups,
                                                                          box);
  };
  if (input == nullptr) {
    // border only: a workgroup per row of the last axis
    const uint64_t rows = count / extents[last];
    uint64_t row_blocks = rows < cap ? rows : cap;
    if (row_blocks == 0) row_blocks = 1;
    auto border = [&](auto kernel) {
      kernel<<<static_cast<uint32_t>(row_blocks), kThreads, 0, guard.stream>>>(output, rows,
                                                                                box);
    };
    auto border_rank = [&](auto vec_tag) {
      constexpr bool VEC = decltype(vec_tag)::value;
      switch (rank) {
        case 1: border(box_border_kernel<E, VEC, 1>); break;
        case 2: border(box_border_kernel<E, VEC, 2>); break;
        case 3: border(box_border_kernel<E, VEC, 3>); break;
        default: border(box_border_kernel<E, VEC, 4>); break;
      }
    };
    if (vec) {
      border_rank(std::true_type{});
    } else {
      border_rank(std::false_type{});
    }
    return;
  }
  auto with_rank = [&](auto vec_tag) {
    constexpr bool VEC = decltype(vec_tag)::value;
    switch (rank) {
      case 1: launch(box_embed_kernel<E, VEC, 1>); break;
      case 2: launch(box_embed_kernel<E, VEC, 2>); break;
      case 3: launch(box_embed_kernel<E, VEC, 3>); break;
      default: launch(box_embed_kernel<E, VEC, 4>); break;
    }
  };
  if (vec) {
    with_rank(std::true_type{});
  } else {
    with_rank(std::false_type{});
  }
}

}  // namespace
}  // namespace spar_hip

using namespace spar_hip;

extern "C" SparHipStatus spar_hip_launch_binary(void* output, const void* left, const void* right,
                                                uint64_t count, int dtype, int operation,
                                                int device) {
  if (!valid_float_dtype(dtype) || operation < SPAR_HIP_ADD ||
      operation > SPAR_HIP_GREATER_EQUAL ||
      (count != 0 && (output == nullptr || left == nullptr || right == nullptr))) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  dispatch_binary(operation, [&](auto op) {
    if (dtype == SPAR_HIP_FLOAT32) {
      launch_map2(static_cast<float*>(output), static_cast<const float*>(left),
                  static_cast<const float*>(right), count, op, guard);
    } else {
      launch_map2(static_cast<double*>(output), static_cast<const double*>(left),
                  static_cast<const double*>(right), count, op, guard);
    }
  });
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_scalar(void* output, const void* input, uint64_t count,
                                                int dtype, int operation, double scalar,
                                                int device) {
  if (!valid_float_dtype(dtype) || operation < SPAR_HIP_ADD || operation > SPAR_HIP_DIVIDE ||
      (count != 0 && (output == nullptr || input == nullptr))) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  dispatch_binary(operation, [&](auto op) {
    using Op = decltype(op);
    if (dtype == SPAR_HIP_FLOAT32) {
      launch_map1(static_cast<float*>(output), static_cast<const float*>(input), count,
                  BindRight<Op, float>{op, static_cast<float>(scalar)}, guard);
    } else {
      launch_map1(static_cast<double*>(output), static_cast<const double*>(input), count,
                  BindRight<Op, double>{op, scalar}, guard);
    }
  });
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_unary(void* output, const void* input, uint64_t count,
                                               int dtype, int operation, int device) {
  if (!valid_float_dtype(dtype) || operation < SPAR_HIP_NEGATE || operation > SPAR_HIP_GELU_DERIVATIVE ||
      (count != 0 && (output == nullptr || input == nullptr))) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  dispatch_unary(operation, [&](auto op) {
    if (dtype == SPAR_HIP_FLOAT32) {
      launch_map1(static_cast<float*>(output), static_cast<const float*>(input), count, op, guard);
    } else {
      launch_map1(static_cast<double*>(output), static_cast<const double*>(input), count, op,
                  guard);
    }
  });
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_fill_from_scalar(void* output, const void* scalar,
                                                          uint64_t count, int dtype, double scale,
                                                          int device) {
  if (!valid_float_dtype(dtype) || scalar == nullptr || (count != 0 && output == nullptr)) {
    return invalid();
  }
  return fill_from_device_scalar(output, scalar, count, dtype, scale, FillScale::kMultiply, device);
}

extern "C" SparHipStatus spar_hip_launch_fill_from_scalar_divided(void* output,
                                                                  const void* scalar,
                                                                  uint64_t count, int dtype,
                                                                  double divisor, int device) {
  if (!valid_float_dtype(dtype) || scalar == nullptr || (count != 0 && output == nullptr) ||
      !(divisor > 0.0)) {
    return invalid();
  }
  const FillScale mode = divisor == 1.0 ? FillScale::kNone : FillScale::kDivide;
  return fill_from_device_scalar(output, scalar, count, dtype, divisor, mode, device);
}

extern "C" SparHipStatus spar_hip_launch_window_embed(void* output, const void* input,
                                                      uint64_t outer, uint64_t extent,
                                                      uint64_t inner, uint64_t start,
                                                      uint64_t length, uint64_t element_size,
                                                      int device) {
  if ((element_size != 4 && element_size != 8) || start > extent || length > extent - start) {
    return invalid();
  }
  uint64_t count = 0;
  if (__builtin_mul_overflow(outer, extent, &count) ||
      __builtin_mul_overflow(count, inner, &count)) {
    return invalid();
  }
  if (count == 0) return ok();
  // 32-bit element indices inside the kernel
  if (count > kIndex32Limit || output == nullptr || (length != 0 && input == nullptr)) {
    return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (element_size == 4) {
    launch_window_embed(static_cast<int32_t*>(output), static_cast<const int32_t*>(input),
                        outer, extent, inner, start, length, guard);
  } else {
    launch_window_embed(static_cast<int64_t*>(output), static_cast<const int64_t*>(input),
                        outer, extent, inner, start, length, guard);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_box_embed(void* output, const void* input, int rank,
                                                   const uint64_t* extents,
                                                   const uint64_t* starts,
                                                   const uint64_t* lengths,
                                                   uint64_t element_size, int device) {
  if ((element_size != 4 && element_size != 8) || rank < 1 || rank > SPAR_HIP_MAX_RANK ||
      extents == nullptr || starts == nullptr || lengths == nullptr) {
    return invalid();
  }
  uint64_t count = 1;
  uint64_t inside = 1;
  for (int a = 0; a < rank; ++a) {
    if (starts[a] > extents[a] || lengths[a] > extents[a] - starts[a] ||
        __builtin_mul_overflow(count, extents[a], &count)) {
      return invalid();
    }
    inside *= lengths[a];  // <= count
  }
  if (count == 0) return ok();
  // 32-bit element indices inside the kernel
  // (input null: the zeros around the box only)
  if (count > kIndex32Limit || output == nullptr) return invalid();
  // Coalesce: drop axes of extent 1 and merge neighbours that are both whole.
  uint64_t e[SPAR_HIP_MAX_RANK];
  uint64_t st[SPAR_HIP_MAX_RANK];
  uint64_t len[SPAR_HIP_MAX_RANK];
  int r = 0;
  for (int a = 0; a < rank; ++a) {
    if (extents[a] == 1) continue;
    const bool whole = starts[a] == 0 && lengths[a] == extents[a];
    if (r > 0 && whole && st[r - 1] == 0 && len[r - 1] == e[r - 1]) {
      e[r - 1] *= extents[a];
      len[r - 1] = e[r - 1];
      continue;
    }
    e[r] = extents[a];
    st[r] = starts[a];
    len[r] = lengths[a];
    ++r;
  }
  if (r == 0) {  // a single element
    e[0] = 1;
    st[0] = 0;
    len[0] = 1;
    r = 1;
  }
  // status 1: more box axes than the kernel takes, or an empty box (the
  // caller fills zeros itself)
  if (r > kMaxBoxAxes || inside == 0) return invalid();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (element_size == 4) {
    launch_box_embed(static_cast<int32_t*>(output), static_cast<const int32_t*>(input), r, e, st,
                     len, count, guard);
  } else {
    launch_box_embed(static_cast<int64_t*>(output), static_cast<const int64_t*>(input), r, e,
                     st, len, count, guard);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_fill(void* output, uint64_t count, int dtype,
                                              double value, int device) {
  if (!valid_float_dtype(dtype) && dtype != SPAR_HIP_INT32 && dtype != SPAR_HIP_INT64) {
    return invalid();
  }
  if (count != 0 && output == nullptr) return invalid();
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  switch (dtype) {
    case SPAR_HIP_FLOAT32:
      launch_fill_values<float>(static_cast<float*>(output), count, nullptr,
                                static_cast<float>(value), 1.0F, FillScale::kNone, guard);
      break;
    case SPAR_HIP_FLOAT64:
      launch_fill_values<double>(static_cast<double*>(output), count, nullptr, value, 1.0,
                                 FillScale::kNone, guard);
      break;
    case SPAR_HIP_INT32:
      launch_fill_values<int32_t>(static_cast<int32_t*>(output), count, nullptr,
                                  static_cast<int32_t>(value), 1, FillScale::kNone, guard);
      break;
    default:
      launch_fill_values<int64_t>(static_cast<int64_t*>(output), count, nullptr,
                                  static_cast<int64_t>(value), 1, FillScale::kNone, guard);
      break;
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_add_in_place(void* destination, const void* source,
                                                      uint64_t count, int dtype, int device) {
  if (!valid_float_dtype(dtype) || (count != 0 && (destination == nullptr || source == nullptr))) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (dtype == SPAR_HIP_FLOAT32) {
    float* dst = static_cast<float*>(destination);
    launch_map2(dst, static_cast<const float*>(dst), static_cast<const float*>(source), count,
                AddOp{}, guard);
  } else {
    double* dst = static_cast<double*>(destination);
    launch_map2(dst, static_cast<const double*>(dst), static_cast<const double*>(source), count,
                AddOp{}, guard);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_random_uniform(void* output, uint64_t count, int dtype,
                                                 uint64_t seed, double low, double high,
                                                 int device) {
  if (!valid_float_dtype(dtype) || !(low < high) || (count != 0 && output == nullptr)) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (dtype == SPAR_HIP_FLOAT32) {
    // random.cpp:59-63: low and width are rounded to float once.
    uniform_f32_kernel<<<scalar_grid(count, guard), kThreads, 0, guard.stream>>>(
        static_cast<float*>(output), count, seed, static_cast<float>(low),
        static_cast<float>(high - low));
  } else {
    uniform_f64_kernel<<<scalar_grid(count, guard), kThreads, 0, guard.stream>>>(
        static_cast<double*>(output), count, seed, low, high - low);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_random_normal(void* output, uint64_t count, int dtype,
                                                uint64_t seed, double mean, double stddev,
                                                int device) {
  if (!valid_float_dtype(dtype) || !(stddev >= 0.0) || (count != 0 && output == nullptr)) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const uint64_t pairs = (count + 1) / 2;
  if (dtype == SPAR_HIP_FLOAT32) {
    normal_kernel<float><<<scalar_grid(pairs, guard), kThreads, 0, guard.stream>>>(
        static_cast<float*>(output), count, seed, mean, stddev);
  } else {
    normal_kernel<double><<<scalar_grid(pairs, guard), kThreads, 0, guard.stream>>>(
        static_cast<double*>(output), count, seed, mean, stddev);
  }
  return finish(guard);
}
