// Strided layouts: materialising views (strided copy) and binary operations
// over broadcast/strided operands without materialising them.
//
// Replaces K11 strided_copy_kernel and the expand().contiguous() + K1 chain
// of the reference (src/backend/cuda_kernels.cu:268-285, :1145-1191;
// src/ops/elementwise.cpp:26-31).  Geometry is coalesced on the host and
// passed by value (no per-call device metadata).  Three kernels:
//   * row-vector: the innermost (coalesced) axis is contiguous or broadcast
//     for every operand and a multiple of the 16-byte vector width - e.g. a
//     bias [C] or a scale [B,1,C] against x [B,T,C]; 128-bit loads/stores,
//     broadcast operands are re-read from cache, not HBM;
//   * tiled: an operand is contiguous along an outer axis only (a transposed
//     view); 64x64 tiles are staged through LDS so both the operand reads and
//     the output writes are coalesced;
//   * generic: per-element index decode with invariant-divisor division.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "layout.hpp"
#include "ops.hpp"

namespace spar_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 1;  // one 16-byte group per lane per tile (see elementwise.hip)
constexpr uint64_t kMaxGrid = uint64_t{1} << 20;

struct CopyOp {
  template <typename T> __device__ __forceinline__ T operator()(T x) const { return x; }
};

// ------------------------------------------------------------ generic path

template <int NOPS, bool kIndex32>
__device__ __forceinline__ void decode(uint64_t e, const KernelGeometry& g, uint64_t (&off)[2]) {
  off[0] = g.offsets[0];
  off[1] = g.offsets[1];
  if constexpr (kIndex32) {
    uint32_t rem = static_cast<uint32_t>(e);
#pragma unroll
    for (int k = 0; k < kMaxRank; ++k) {
      if (k < g.rank) {
        const uint32_t q = g.divisors[k].div(rem);
        const uint32_t c = rem - q * g.divisors[k].divisor;
        rem = q;
        off[0] += static_cast<uint64_t>(c) * g.strides[0][k];
        if constexpr (NOPS == 2) off[1] += static_cast<uint64_t>(c) * g.strides[1][k];
      }
    }
  } else {
    uint64_t rem = e;
#pragma unroll
    for (int k = 0; k < kMaxRank; ++k) {
      if (k < g.rank) {
        const uint64_t q = rem / g.extents[k];
        const uint64_t c = rem - q * g.extents[k];
        rem = q;
        off[0] += c * g.strides[0][k];
        if constexpr (NOPS == 2) off[1] += c * g.strides[1][k];
      }
    }
  }
}

template <typename T, int NOPS, bool kIndex32, typename F>
__global__ void __launch_bounds__(kThreads)
    generic_kernel(T* out, const T* a, const T* b, uint64_t count, KernelGeometry g, F f) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; e < count;
       e += stride) {
    uint64_t off[2];
    decode<NOPS, kIndex32>(e, g, off);
    if constexpr (NOPS == 1) {
      out[e] = f(a[off[0]]);
    } else {
      out[e] = f(a[off[0]], b[off[1]]);
    }
  }
}

// -------------------------------------------------------- row-vector path

// The innermost axis has extent `inner` (a multiple of W); each operand's
// inner stride is 0 (broadcast) or 1 (contiguous).  Rows are decoded from the
// outer axes of `g` (g.rank - 1 axes, innermost first starting at index 1).
struct RowGeometry {
  KernelGeometry g;        // full coalesced geometry (axis 0 = innermost)
  FastDiv groups_per_row;  // inner / W
  int inner_unit[2];       // 1 if the operand is contiguous along the inner axis
};

// Offsets of row `row` (the outer axes of g, innermost first from index 1).
template <int NOPS>
__device__ __forceinline__ void row_offsets(const KernelGeometry& g, uint32_t row, uint64_t& off0,
                                            uint64_t& off1) {
  off0 = g.offsets[0];
  off1 = g.offsets[1];
  uint32_t rem = row;
#pragma unroll
  for (int k = 1; k < kMaxRank; ++k) {
    if (k < g.rank) {
      const uint32_t q = g.divisors[k].div(rem);
      const uint64_t c = rem - q * g.divisors[k].divisor;
      rem = q;
      off0 += c * g.strides[0][k];
      if constexpr (NOPS == 2) off1 += c * g.strides[1][k];
    }
  }
}

// How a row kernel reads one operand's 16-byte group at (row offset, column):
//   kStreamGroup: contiguous along the row and read once (non-temporal load);
//   kCachedGroup: contiguous along the row and broadcast across rows, so it is
//                 re-read for every row (ordinary, cached load);
//   kSplatGroup:  broadcast along the row (inner stride 0): one value splat.
// The mode is a template parameter of the long-row kernel so that its loads
// form straight-line code: with a run-time choice per operand the compiler
// waits for every outstanding load before the next one is issued.
constexpr int kStreamGroup = 0;
constexpr int kCachedGroup = 1;
constexpr int kSplatGroup = 2;

template <typename T, int MODE>
__device__ __forceinline__ typename Vec16<T>::type row_group(const T* base, uint64_t row_offset,
                                                             uint64_t column) {
  using V = typename Vec16<T>::type;
  V v;
  if constexpr (MODE == kSplatGroup) {
    const T s = base[row_offset];
#pragma unroll
    for (int k = 0; k < Vec16<T>::width; ++k) vec_set<T>(v, k, s);
  } else {
    v = load_vector_policy<MODE == kStreamGroup>(
        reinterpret_cast<const V*>(base + row_offset + column));
  }
  return v;
}

// Run-time form for the short-row kernel: contiguous operands stream
// (non-temporal), operands broadcast along the row are splat.
template <typename T>
__device__ __forceinline__ typename Vec16<T>::type row_group_any(const T* base,
                                                                 uint64_t row_offset,
                                                                 uint64_t column, int inner_unit) {
  using V = typename Vec16<T>::type;
  V v;
  if (inner_unit) {
    v = stream_load(reinterpret_cast<const V*>(base + row_offset + column));
  } else {
    const T s = base[row_offset];
#pragma unroll
    for (int k = 0; k < Vec16<T>::width; ++k) vec_set<T>(v, k, s);
  }
  return v;
}

template <typename T, int NOPS, typename F>
__device__ __forceinline__ typename Vec16<T>::type apply_group(F f, const typename Vec16<T>::type& ra,
                                                               const typename Vec16<T>::type& rb) {
  typename Vec16<T>::type o;
#pragma unroll
  for (int k = 0; k < Vec16<T>::width; ++k) {
    if constexpr (NOPS == 1) {
      vec_set<T>(o, k, f(vec_get<T>(ra, k)));
    } else {
      vec_set<T>(o, k, f(vec_get<T>(ra, k), vec_get<T>(rb, k)));
    }
  }
  return o;
}

// Short rows: each lane decodes the row of its own group.  NT: non-temporal
// output stores.
template <typename T, int NOPS, typename F, bool NT>
__global__ void __launch_bounds__(kThreads)
    row_vector_kernel(T* out, const T* a, const T* b, uint64_t groups, RowGeometry rg, F f) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  const KernelGeometry& g = rg.g;
  const uint64_t tile = static_cast<uint64_t>(kThreads) * kUnroll;
  V* out_v = reinterpret_cast<V*>(out);
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile; base < groups;
       base += static_cast<uint64_t>(gridDim.x) * tile) {
    V ra[kUnroll];
    V rb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t group = base + static_cast<uint64_t>(u) * kThreads + threadIdx.x;
      if (group < groups) {
        const uint32_t row = rg.groups_per_row.div(static_cast<uint32_t>(group));
        const uint32_t column = (static_cast<uint32_t>(group) - row * rg.groups_per_row.divisor) * W;
        uint64_t off0, off1;
        row_offsets<NOPS>(g, row, off0, off1);
        ra[u] = row_group_any<T>(a, off0, column, rg.inner_unit[0]);
        if constexpr (NOPS == 2) rb[u] = row_group_any<T>(b, off1, column, rg.inner_unit[1]);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t group = base + static_cast<uint64_t>(u) * kThreads + threadIdx.x;
      if (group < groups) store_vector<NT>(out_v + group, apply_group<T, NOPS>(f, ra[u], rb[u]));
    }
  }
}

// Row-segment variant for long rows of a view of rank <= 3: a single-wave
// workgroup t owns 64 groups (one per lane) of row t / column_tiles.  The
// row's operand offsets come from its two outer coordinates, (row mod e1,
// row / e1), with one multiply-shift division in scalar registers; each lane
// then only adds its column.  One group per lane and many short workgroups
// measured fastest on MI355X for x[32768, 4096] + bias[4096] (steady state,
// 1 GiB moved): with 256-lane workgroups, 168 us against 174 us for two
// consecutive rows per workgroup, 178 us for four, and 173 / 183 us for two /
// four column segments of one row; a minimal kernel of this shape took 161 /
// 162 / 165 / 169 us with workgroups of 64 / 128 / 256 / 512 lanes.
// Requires tiles and rows below 2^31.
constexpr int kRowTileThreads = 64;

struct RowTileGeometry {
  uint64_t inner;        // row length (elements), a multiple of W
  uint32_t tiles;        // column tiles x rows
  FastDiv column_tiles;  // kRowTileThreads-group segments per row
  FastDiv outer1;        // extent of the axis above the row (1 for a single row)
  uint64_t offsets[2];
  uint64_t stride1[2];   // operand strides of that axis
  uint64_t stride2[2];   // operand strides of the axis above it (0 when absent)
};

template <typename T, int NOPS, typename F, bool NT, int MODE_A, int MODE_B>
__global__ void __launch_bounds__(kRowTileThreads)
    row_tile_kernel(T* out, const T* a, const T* b, RowTileGeometry rg, F f) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  for (uint32_t tile = blockIdx.x; tile < rg.tiles; tile += gridDim.x) {
    const uint32_t row = rg.column_tiles.div(tile);
    const uint64_t column =
        (static_cast<uint64_t>(tile - row * rg.column_tiles.divisor) * kRowTileThreads +
         threadIdx.x) * W;
    const uint32_t c2 = rg.outer1.div(row);
    const uint32_t c1 = row - c2 * rg.outer1.divisor;
    const uint64_t off0 = rg.offsets[0] + c1 * rg.stride1[0] + c2 * rg.stride2[0];
    const uint64_t off1 = rg.offsets[1] + c1 * rg.stride1[1] + c2 * rg.stride2[1];
    if (column < rg.inner) {
      V ra;
      V rb{};  // unused by one-operand ops
      ra = row_group<T, MODE_A>(a, off0, column);
      if constexpr (NOPS == 2) rb = row_group<T, MODE_B>(b, off1, column);
      store_vector<NT>(reinterpret_cast<V*>(out + row * rg.inner + column),
                       apply_group<T, NOPS>(f, ra, rb));
    }
  }
}

// ------------------------------------------------------------- tiled path

// Output axes p (an outer axis) and q (the innermost axis) are tiled; the
// remaining axes form the batch.  Operands flagged `staged` are contiguous
// along p and are read p-fastest into LDS; others are read q-fastest.
struct TileGeometry {
  uint64_t extent_p, extent_q;
  uint64_t out_stride_p;          // output (contiguous) stride of axis p
  uint64_t stride_p[2], stride_q[2];
  int staged[2];
  int batch_rank;
  uint64_t batch_extents[kMaxRank];  // innermost first
  uint64_t batch_out_strides[kMaxRank];
  uint64_t batch_strides[2][kMaxRank];
  uint64_t offsets[2];
  uint64_t tiles_p, tiles_q;
};

template <typename T, int NOPS, int TILE, typename F>
__global__ void __launch_bounds__(kThreads)
    tiled_kernel(T* out, const T* a, const T* b, uint64_t tile_count, TileGeometry tg, F f) {
  __shared__ T tile[NOPS][TILE][TILE + 1];
  constexpr int kRowsPerPass = kThreads / TILE;
  const int tx = threadIdx.x % TILE;
  const int ty = threadIdx.x / TILE;
  const T* operands[2] = {a, b};
  for (uint64_t block = blockIdx.x; block < tile_count; block += gridDim.x) {
    uint64_t rem = block;
    const uint64_t tq = rem % tg.tiles_q;
    rem /= tg.tiles_q;
    const uint64_t tp = rem % tg.tiles_p;
    rem /= tg.tiles_p;
    uint64_t out_base = 0;
    uint64_t base[2] = {tg.offsets[0], tg.offsets[1]};
    for (int k = 0; k < tg.batch_rank; ++k) {
      const uint64_t c = rem % tg.batch_extents[k];
      rem /= tg.batch_extents[k];
      out_base += c * tg.batch_out_strides[k];
      base[0] += c * tg.batch_strides[0][k];
      base[1] += c * tg.batch_strides[1][k];
    }
    const uint64_t p0 = tp * TILE;
    const uint64_t q0 = tq * TILE;
#pragma unroll
    for (int op = 0; op < NOPS; ++op) {
      if (tg.staged[op]) {
        for (int j = ty; j < TILE; j += kRowsPerPass) {
          const uint64_t p = p0 + tx;
          const uint64_t q = q0 + j;
          if (p < tg.extent_p && q < tg.extent_q) {
            tile[op][j][tx] = operands[op][base[op] + p * tg.stride_p[op] + q * tg.stride_q[op]];
          }
        }
      }
    }
    __syncthreads();
    for (int j = ty; j < TILE; j += kRowsPerPass) {
      const uint64_t p = p0 + j;
      const uint64_t q = q0 + tx;
      if (p < tg.extent_p && q < tg.extent_q) {
        T v[2];
#pragma unroll
        for (int op = 0; op < NOPS; ++op) {
          v[op] = tg.staged[op]
                      ? tile[op][tx][j]
                      : operands[op][base[op] + p * tg.stride_p[op] + q * tg.stride_q[op]];
        }
        T result;
        if constexpr (NOPS == 1) {
          result = f(v[0]);
        } else {
          result = f(v[0], v[1]);
        }
        out[out_base + p * tg.out_stride_p + q] = result;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- dispatch

// ------------------------------------------- vector tiled path (transpose)

// Vector form of the tiled path for 16-byte aligned layouts.  A tile covers
// 32 W values of p by 32 W values of q (128 x 128 float32, 64 x 64 float64),
// W elements per 16-byte granule.  Staged operands (contiguous along p) are
// read in granules along p -- 32 lanes cover 512 contiguous bytes of one
// source row -- and kept in LDS as [q][granule]; the store phase reads W
// granules from W consecutive q rows, transposes the W x W block in
// registers and writes W output rows of one granule each, so 32 lanes write
// 512 contiguous bytes of an output row.  LDS granules are XOR-swizzled by
// (q / W) mod 8: the 32 lanes writing one q row hit a permutation of that
// row's granules, and 8 lanes of the store phase, which read one granule
// index from rows W m + k of 8 consecutive m, hit 8 different bank groups.
// Measured on MI355X for x^T - mu over x [8192, 4096] float32 (cold cache):
// ~4.9 TB/s, against ~1.8 TB/s for the scalar 64 x 65 tile above.  Back to
// back over rotated inputs, the rotated tile order (see locate) and
// non-temporal stores for outputs of 64 MiB or more took the same op from
// 57.4 us to 46.2 us (5.8 TB/s); each alone gave 53.5 (stores) and 50.1 us
// (order).
//
// The grid is the resident workgroups, each walking tiles; the staged loads
// of a workgroup's next tile are issued right after its current tile lands in
// LDS, so they fly while the current tile is transposed and stored.  Steady
// state on [4096, 8192] outputs, against one tile per workgroup: x^T - mu
// 65.1 -> 61.6 us, copy of x^T 63.4 -> 60.0 us, x^T + y^T 97.8 -> 87.2 us.
constexpr int kVecTileGranules = 32;

struct VecTileGeometry {
  uint64_t extent_p, extent_q;
  uint64_t out_stride_p;
  uint64_t stride_p[2], stride_q[2];
  int mode[2];  // kStaged, kAlongQ (contiguous along q), kFixedQ (stride 0 along q), kGather
  int slot[2];  // LDS slot of a staged operand
  int batch_rank;
  uint64_t batch_extents[kMaxRank];  // innermost first
  uint64_t batch_out_strides[kMaxRank];
  uint64_t batch_strides[2][kMaxRank];
  uint64_t offsets[2];
  FastDiv tiles_q;
  FastDiv tiles_p;
  uint32_t tile_count;
};

constexpr int kStaged = 0;
constexpr int kAlongQ = 1;
constexpr int kFixedQ = 2;
constexpr int kGather = 3;

template <typename T, int NOPS, int NSTAGED, typename F, bool NT>
__global__ void __launch_bounds__(kThreads)
    vec_tiled_kernel(T* out, const T* a, const T* b, VecTileGeometry tg, F f) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  constexpr int G = kVecTileGranules;
  constexpr int TP = G * W;
  constexpr int TQ = G * W;
  constexpr int kLoads = TQ * G / kThreads;       // granules staged per lane
  static_assert(kThreads % G == 0, "a lane keeps its p granule for all its loads");
  constexpr int kBlocks = (TQ / W) * G / kThreads;  // W x W blocks stored per lane
  __shared__ V lds[NSTAGED][TQ][G];
  const T* operands[2] = {a, b};
  // Where a tile lives: its output base, operand bases and first p and q.
  struct Where {
    uint64_t out_base;
    uint64_t base[2];
    uint64_t p0, q0;
  };
  // Tiles are numbered q fastest, then p, then batch, and each q column of
  // tiles is rotated along p by its q index (tile (tq, r) covers p tile
  // (r + tq) mod tiles_p): workgroups running side by side then differ in both
  // p and q, so neither the staged reads (512-byte pieces of rows 16 KiB
  // apart in the C5 base) nor the stores gather on the same DRAM channels.
  auto locate = [&](uint32_t tile) {
    Where w;
    const uint32_t rest = tg.tiles_q.div(tile);
    const uint32_t tq = tile - rest * tg.tiles_q.divisor;
    const uint32_t batch = tg.tiles_p.div(rest);
    const uint32_t rotated = rest - batch * tg.tiles_p.divisor + tq % tg.tiles_p.divisor;
    const uint32_t tp =
        rotated >= tg.tiles_p.divisor ? rotated - tg.tiles_p.divisor : rotated;
    w.out_base = 0;
    w.base[0] = tg.offsets[0];
    w.base[1] = tg.offsets[1];
    uint64_t coordinate = batch;
    for (int k = 0; k < tg.batch_rank; ++k) {
      const uint64_t c = coordinate % tg.batch_extents[k];
      coordinate /= tg.batch_extents[k];
      w.out_base += c * tg.batch_out_strides[k];
      w.base[0] += c * tg.batch_strides[0][k];
      w.base[1] += c * tg.batch_strides[1][k];
    }
    w.p0 = static_cast<uint64_t>(tp) * TP;
    w.q0 = static_cast<uint64_t>(tq) * TQ;
    return w;
  };
  // Staged operands in registers; with two, operand op uses slot op.
  V staged[NSTAGED][kLoads];
  auto load_tile = [&](const Where& w) {
    const bool whole = w.p0 + TP <= tg.extent_p && w.q0 + TQ <= tg.extent_q;
#pragma unroll
    for (int op = 0; op < NOPS; ++op) {
      if (tg.mode[op] != kStaged) continue;
      const int s = NSTAGED == 1 ? 0 : op;
      if (whole) {
        // a whole tile: no bounds checks; lane offset (lane % G) W along p,
        // lane / G + it * kThreads / G along q
        const T* at = operands[op] + w.base[op] + w.p0 + w.q0 * tg.stride_q[op] +
                      static_cast<uint64_t>(threadIdx.x % G) * W +
                      static_cast<uint64_t>(threadIdx.x / G) * tg.stride_q[op];
        const uint64_t step = static_cast<uint64_t>(kThreads / G) * tg.stride_q[op];
#pragma unroll
        for (int it = 0; it < kLoads; ++it) {
          staged[s][it] = stream_load(reinterpret_cast<const V*>(at + it * step));
        }
        continue;
      }
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const int index = it * kThreads + threadIdx.x;
        const uint64_t p = w.p0 + static_cast<uint64_t>(index % G) * W;
        const uint64_t q = w.q0 + index / G;
        staged[s][it] = V{};
        if (p < tg.extent_p && q < tg.extent_q) {
          staged[s][it] = stream_load(
              reinterpret_cast<const V*>(operands[op] + w.base[op] + p + q * tg.stride_q[op]));
        }
      }
    }
  };
  uint32_t tile = blockIdx.x;
  if (tile >= tg.tile_count) return;
  Where cur = locate(tile);
  load_tile(cur);
  while (true) {
    const uint32_t next = tile + gridDim.x;
    __syncthreads();  // the previous tile's LDS readers are done
#pragma unroll
    for (int op = 0; op < NOPS; ++op) {
      if (tg.mode[op] != kStaged) continue;
      const int s = NSTAGED == 1 ? 0 : op;
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const int index = it * kThreads + threadIdx.x;
        const int row = index / G;
        lds[tg.slot[op]][row][(index % G) ^ ((row / W) & 7)] = staged[s][it];
      }
    }
    __syncthreads();
    const uint64_t out_base = cur.out_base;
    const uint64_t base[2] = {cur.base[0], cur.base[1]};
    const uint64_t p0 = cur.p0;
    const uint64_t q0 = cur.q0;
    // An operand fixed along q (x^T - mu's mu) is read into registers before
    // the next tile's staged loads are issued.  Vector memory operations
    // complete in issue order as far as the wait counter goes, so a read
    // issued after those loads could only be waited for together with them,
    // and the store phase would stall until the next tile had landed.  Other
    // direct operands are read in the store phase: holding their W x W
    // blocks as well would take the kernel past 128 VGPRs, to one wave per
    // SIMD.
    constexpr bool kDirect = NOPS == 2 && NSTAGED == 1;
    const int direct_op = tg.mode[0] == kStaged ? 1 : 0;
    const bool fixed_direct = kDirect && tg.mode[direct_op] == kFixedQ;
    T fixed[kDirect ? kBlocks : 1][W];
    if constexpr (kDirect) {
      if (fixed_direct) {
        const int op = direct_op;
#pragma unroll
        for (int it = 0; it < kBlocks; ++it) {
          const int index = it * kThreads + threadIdx.x;
          const int m = index % (TQ / W);
          const int g = index / (TQ / W);
          const uint64_t q = q0 + static_cast<uint64_t>(m) * W;
          const uint64_t p = p0 + static_cast<uint64_t>(g) * W;
          if (q >= tg.extent_q || p >= tg.extent_p) continue;
#pragma unroll
          for (int i = 0; i < W; ++i) fixed[it][i] = operands[op][base[op] + (p + i) * tg.stride_p[op]];
        }
      }
    }
    Where following = cur;
    if (next < tg.tile_count) {
      following = locate(next);
      load_tile(following);  // in flight during this tile's store phase
    }

#pragma unroll
    for (int it = 0; it < kBlocks; ++it) {
      const int index = it * kThreads + threadIdx.x;
      const int m = index % (TQ / W);  // q granule within the tile
      const int g = index / (TQ / W);  // p granule within the tile
      const uint64_t q = q0 + static_cast<uint64_t>(m) * W;
      const uint64_t p = p0 + static_cast<uint64_t>(g) * W;
      if (q >= tg.extent_q || p >= tg.extent_p) continue;
      T values[2][W][W];  // [operand][p offset][q offset]
#pragma unroll
      for (int op = 0; op < NOPS; ++op) {
        if (tg.mode[op] == kStaged) {
#pragma unroll
          for (int k = 0; k < W; ++k) {
            const V block = lds[tg.slot[op]][m * W + k][g ^ (m & 7)];
#pragma unroll
            for (int i = 0; i < W; ++i) values[op][i][k] = vec_get<T>(block, i);
          }
        } else if (tg.mode[op] == kFixedQ) {
          if constexpr (kDirect) {
#pragma unroll
            for (int i = 0; i < W; ++i) {
#pragma unroll
              for (int k = 0; k < W; ++k) values[op][i][k] = fixed[it][i];
            }
          }
        } else if (tg.mode[op] == kAlongQ) {
#pragma unroll
          for (int i = 0; i < W; ++i) {
            const V row = *reinterpret_cast<const V*>(operands[op] + base[op] +
                                                       (p + i) * tg.stride_p[op] + q);
#pragma unroll
            for (int k = 0; k < W; ++k) values[op][i][k] = vec_get<T>(row, k);
          }
        } else {
#pragma unroll
          for (int i = 0; i < W; ++i) {
#pragma unroll
            for (int k = 0; k < W; ++k) {
              values[op][i][k] = operands[op][base[op] + (p + i) * tg.stride_p[op] +
                                              (q + k) * tg.stride_q[op]];
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < W; ++i) {
        V o;
#pragma unroll
        for (int k = 0; k < W; ++k) {
          if constexpr (NOPS == 1) {
            vec_set<T>(o, k, f(values[0][i][k]));
          } else {
            vec_set<T>(o, k, f(values[0][i][k], values[1][i][k]));
          }
        }
        store_vector<NT>(reinterpret_cast<V*>(out + out_base + (p + i) * tg.out_stride_p + q), o);
      }
    }
    if (next >= tg.tile_count) break;
    tile = next;
    cur = following;
  }
}

template <int M>
struct GroupMode {
  static constexpr int value = M;
};

// Calls body(GroupMode<mode>{}) for a run-time row-group mode.
template <typename Body>
void with_group_mode(int mode, Body&& body) {
  if (mode == kSplatGroup) {
    body(GroupMode<kSplatGroup>{});
  } else if (mode == kCachedGroup) {
    body(GroupMode<kCachedGroup>{});
  } else {
    body(GroupMode<kStreamGroup>{});
  }
}

uint32_t capped_grid(uint64_t work, uint64_t per_block) {
  uint64_t blocks = (work + per_block - 1) / per_block;
  if (blocks == 0) blocks = 1;
  if (blocks > kMaxGrid) blocks = kMaxGrid;
  return static_cast<uint32_t>(blocks);
}

// Launches the vector tiled kernel for output axes p (where some operand is
// contiguous) and q (the innermost); returns false when the layout does not
// meet its alignment rules, leaving the scalar tiled kernel to run.
template <typename T, int NOPS, typename F>
bool launch_vec_tiled(T* out, const T* a, const T* b, const MultiView& view, int p_axis, F f,
                      const DeviceGuard& guard) {
  constexpr int W = Vec16<T>::width;
  constexpr uint64_t kTile = static_cast<uint64_t>(kVecTileGranules) * W;
  const int last = view.rank - 1;
  VecTileGeometry tg{};
  tg.extent_p = view.extents[p_axis];
  tg.extent_q = view.extents[last];
  if (tg.extent_p % W != 0 || tg.extent_q % W != 0 || !aligned16(out)) return false;
  uint64_t out_strides[kMaxRank];
  uint64_t running = 1;
  for (int axis = view.rank - 1; axis >= 0; --axis) {
    out_strides[axis] = running;
    running *= view.extents[axis];
  }
  tg.out_stride_p = out_strides[p_axis];
  const T* bases[2] = {a, b};
  int staged = 0;
  for (int op = 0; op < 2; ++op) tg.mode[op] = kGather;
  for (int op = 0; op < NOPS; ++op) {
    const uint64_t sp = view.strides[op][p_axis];
    const uint64_t sq = view.strides[op][last];
    tg.stride_p[op] = sp;
    tg.stride_q[op] = sq;
    tg.offsets[op] = view.offsets[op];
    bool aligned = aligned16(bases[op]) && view.offsets[op] % W == 0;
    for (int axis = 0; axis < view.rank; ++axis) {
      if (axis != p_axis && axis != last && view.strides[op][axis] % W != 0) aligned = false;
    }
    if (sp == 1 && sq != 0 && sq != 1) {
      if (!aligned || sq % W != 0) return false;
      tg.mode[op] = kStaged;
      tg.slot[op] = staged++;
    } else if (sq == 1 && aligned && sp % W == 0) {
      tg.mode[op] = kAlongQ;
    } else if (sq == 0) {
      tg.mode[op] = kFixedQ;
    }
  }
  if (staged == 0) return false;
  uint64_t batch_count = 1;
  for (int axis = view.rank - 1; axis >= 0; --axis) {
    if (axis == p_axis || axis == last) continue;
    const int k = tg.batch_rank++;
    tg.batch_extents[k] = view.extents[axis];
    tg.batch_out_strides[k] = out_strides[axis];
    for (int op = 0; op < NOPS; ++op) tg.batch_strides[op][k] = view.strides[op][axis];
    batch_count *= view.extents[axis];
  }
  const uint64_t tiles_p = (tg.extent_p + kTile - 1) / kTile;
  const uint64_t tiles_q = (tg.extent_q + kTile - 1) / kTile;
  const uint64_t tiles = tiles_p * tiles_q * batch_count;
  if (tiles > kIndex32Limit) return false;
  tg.tiles_p.init(static_cast<uint32_t>(tiles_p));
  tg.tiles_q.init(static_cast<uint32_t>(tiles_q));
  tg.tile_count = static_cast<uint32_t>(tiles);
  // Three workgroups per resident slot (two slots per CU with one staged
  // operand, one with two), each walking tiles: the workgroups beyond the
  // resident ones start as others finish.  On x^T - mu for x [8192, 4096]
  // float32 (2048 tiles) one per slot took 48.8-49.5 us, three 47.0-48.0
  // and four to eight no less.  Without an occupancy answer the view takes
  // another kernel (same values).
  auto launch = [&](auto kernel) {
    const uint64_t slots = 3 * resident_blocks(kernel, kThreads, guard);
    if (slots == 0) return false;
    kernel<<<static_cast<uint32_t>(tiles < slots ? tiles : slots), kThreads, 0, guard.stream>>>(
        out, a, b, tg, f);
    return true;
  };
  bool launched = false;
  with_policy(stream_output(view_numel(view) * sizeof(T)), [&](auto nt) {
    constexpr bool NT = decltype(nt)::value;
    launched = staged == 1 ? launch(vec_tiled_kernel<T, NOPS, 1, F, NT>)
                           : launch(vec_tiled_kernel<T, NOPS, 2, F, NT>);
  });
  return launched;
}

// Chooses and launches the kernel for a coalesced view; out is contiguous.
template <typename T, int NOPS, typename F>
void launch_view(T* out, const T* a, const T* b, const MultiView& view, F f,
                 const DeviceGuard& guard) {
  constexpr int W = Vec16<T>::width;
  const uint64_t count = view_numel(view);
  const int last = view.rank - 1;
  const uint64_t inner = view.extents[last];

  bool index32 = count <= kIndex32Limit;
  for (int op = 0; op < NOPS; ++op) {
    if (view_span(view, op) > kIndex32Limit) {
      // offsets stay 64-bit in every kernel; only coordinates need 32 bits
    }
  }

  // Row-vector path.
  bool row_ok = index32 && inner % W == 0 && aligned16(out);
  int inner_unit[2] = {0, 0};
  for (int op = 0; op < NOPS && row_ok; ++op) {
    const uint64_t s = view.strides[op][last];
    const T* base = op == 0 ? a : b;
    if (s == 1) {
      inner_unit[op] = 1;
      if (!aligned16(base) || view.offsets[op] % W != 0) row_ok = false;
      for (int axis = 0; axis < last; ++axis) {
        if (view.strides[op][axis] % W != 0) row_ok = false;
      }
    } else if (s != 0) {
      row_ok = false;
    }
  }
  if (row_ok) {
    RowGeometry rg{};
    rg.g = kernel_geometry(view);
    rg.groups_per_row.init(static_cast<uint32_t>(inner / W));
    rg.inner_unit[0] = inner_unit[0];
    rg.inner_unit[1] = inner_unit[1];
    // An operand with a zero stride on some axis of extent > 1 is re-read:
    // it takes cached loads; every other operand streams.
    bool reused[2] = {false, false};
    for (int op = 0; op < NOPS; ++op) {
      for (int axis = 0; axis < view.rank; ++axis) {
        if (view.strides[op][axis] == 0 && view.extents[axis] > 1) reused[op] = true;
      }
    }
    int mode[2] = {kStreamGroup, kStreamGroup};
    for (int op = 0; op < NOPS; ++op) {
      mode[op] = !inner_unit[op] ? kSplatGroup : reused[op] ? kCachedGroup : kStreamGroup;
    }
    const uint64_t groups = count / W;
    const uint64_t groups_per_row = inner / W;
    const uint64_t rows = count / inner;
    const bool long_rows = groups_per_row >= kRowTileThreads && view.rank <= 3 &&
                           !(NOPS == 2 && mode[0] == kSplatGroup && mode[1] == kSplatGroup);
    with_policy(stream_output(count * sizeof(T)), [&](auto nt) {
      constexpr bool NT = decltype(nt)::value;
      if (!long_rows) {
        row_vector_kernel<T, NOPS, F, NT>
            <<<capped_grid(groups, static_cast<uint64_t>(kThreads) * kUnroll), kThreads, 0,
               guard.stream>>>(out, a, b, groups, rg, f);
        return;
      }
      // Long rows: one single-wave workgroup per 64-group row segment.
      RowTileGeometry tg{};
      tg.inner = inner;
      const uint64_t column_tiles = (groups_per_row + kRowTileThreads - 1) / kRowTileThreads;
      tg.tiles = static_cast<uint32_t>(column_tiles * rows);  // <= count / 128
      tg.column_tiles.init(static_cast<uint32_t>(column_tiles));
      // Outer axes: axis1 directly above the row, axis2 above it (rank 3).
      const int axis1 = view.rank - 2;
      tg.outer1.init(axis1 >= 0 ? static_cast<uint32_t>(view.extents[axis1]) : 1U);
      for (int op = 0; op < NOPS; ++op) {
        tg.offsets[op] = view.offsets[op];
        tg.stride1[op] = axis1 >= 0 ? view.strides[op][axis1] : 0;
        tg.stride2[op] = view.rank == 3 ? view.strides[op][0] : 0;
      }
      with_group_mode(mode[0], [&](auto mode_a) {
        with_group_mode(NOPS == 2 ? mode[1] : kStreamGroup, [&](auto mode_b) {
          constexpr int MA = decltype(mode_a)::value;
          constexpr int MB = decltype(mode_b)::value;
          if constexpr ((NOPS == 1 && MB != kStreamGroup) ||
                        (MA == kSplatGroup && MB == kSplatGroup)) {
            return;  // never selected (see long_rows and the NOPS == 1 mode above)
          } else {
            row_tile_kernel<T, NOPS, F, NT, MA, MB>
                <<<capped_grid(tg.tiles, 1), kRowTileThreads, 0, guard.stream>>>(out, a, b, tg, f);
          }
        });
      });
    });
    return;
  }

  // Tiled path: some operand is strided along q but contiguous along an
  // outer axis p.
  if (view.rank >= 2) {
    int p_axis = -1;
    for (int op = 0; op < NOPS && p_axis < 0; ++op) {
      const uint64_t sq = view.strides[op][last];
      if (sq == 0 || sq == 1) continue;
      for (int axis = last - 1; axis >= 0; --axis) {
        if (view.strides[op][axis] == 1) {
          p_axis = axis;
          break;
        }
      }
    }
    if (p_axis >= 0) {
      if (launch_vec_tiled<T, NOPS>(out, a, b, view, p_axis, f, guard)) return;
      constexpr int TILE = sizeof(T) == 4 ? 64 : 32;
      TileGeometry tg{};
      tg.extent_p = view.extents[p_axis];
      tg.extent_q = inner;
      uint64_t out_strides[kMaxRank];
      uint64_t running = 1;
      for (int axis = view.rank - 1; axis >= 0; --axis) {
        out_strides[axis] = running;
        running *= view.extents[axis];
      }
      tg.out_stride_p = out_strides[p_axis];
      for (int op = 0; op < NOPS; ++op) {
        tg.stride_p[op] = view.strides[op][p_axis];
        tg.stride_q[op] = view.strides[op][last];
        tg.staged[op] = (tg.stride_p[op] == 1 && tg.stride_q[op] != 1 && tg.stride_q[op] != 0);
        tg.offsets[op] = view.offsets[op];
      }
      tg.batch_rank = 0;
      uint64_t batch_count = 1;
      for (int axis = view.rank - 1; axis >= 0; --axis) {
        if (axis == p_axis || axis == last) continue;
        const int k = tg.batch_rank++;
        tg.batch_extents[k] = view.extents[axis];
        tg.batch_out_strides[k] = out_strides[axis];
        for (int op = 0; op < NOPS; ++op) tg.batch_strides[op][k] = view.strides[op][axis];
        batch_count *= view.extents[axis];
      }
      tg.tiles_p = (tg.extent_p + TILE - 1) / TILE;
      tg.tiles_q = (tg.extent_q + TILE - 1) / TILE;
      const uint64_t tiles = tg.tiles_p * tg.tiles_q * batch_count;
      tiled_kernel<T, NOPS, TILE, F><<<capped_grid(tiles, 1), kThreads, 0, guard.stream>>>(
          out, a, b, tiles, tg, f);
      return;
    }
  }

  // Generic path.
  const KernelGeometry g = kernel_geometry(view);
  uint64_t blocks = (count + kThreads - 1) / kThreads;
  const uint64_t cap = static_cast<uint64_t>(guard.multiprocessors) * 32;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  if (index32) {
    generic_kernel<T, NOPS, true, F><<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(
        out, a, b, count, g, f);
  } else {
    generic_kernel<T, NOPS, false, F>
        <<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(out, a, b, count, g, f);
  }
}

template <typename T>
void launch_copy(void* destination, const void* source, const MultiView& view,
                 const DeviceGuard& guard) {
  launch_view<T, 1>(static_cast<T*>(destination), static_cast<const T*>(source),
                    static_cast<const T*>(nullptr), view, CopyOp{}, guard);
}

}  // namespace
}  // namespace spar_hip

using namespace spar_hip;

extern "C" SparHipStatus spar_hip_launch_strided_copy(void* destination, const void* source,
                                                      uint64_t rank, const uint64_t* extents,
                                                      const uint64_t* strides,
                                                      uint64_t storage_offset, uint64_t count,
                                                      uint64_t element_size, int device) {
  if ((element_size != 4U && element_size != 8U) ||
      (count != 0 && (destination == nullptr || source == nullptr)) ||
      (rank != 0 && (extents == nullptr || strides == nullptr)) || rank > kMaxRank) {
    return invalid();
  }
  if (count == 0) return ok();
  MultiView view;
  view.rank = static_cast<int>(rank);
  view.operands = 1;
  uint64_t product = 1;
  for (uint64_t axis = 0; axis < rank; ++axis) {
    view.extents[axis] = extents[axis];
    view.strides[0][axis] = strides[axis];
    product *= extents[axis];
  }
  view.offsets[0] = storage_offset;
  if (product != count) return invalid();
  coalesce(view);
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  // The payload is moved as 4- or 8-byte words (float / double bit patterns).
  if (element_size == 4U) {
    launch_copy<float>(destination, source, view, guard);
  } else {
    launch_copy<double>(destination, source, view, guard);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_strided_binary(void* output, const void* left,
                                                        const uint64_t* left_strides,
                                                        uint64_t left_offset, const void* right,
                                                        const uint64_t* right_strides,
                                                        uint64_t right_offset, uint64_t rank,
                                                        const uint64_t* extents, int dtype,
                                                        int operation, int device) {
  if (!valid_float_dtype(dtype) || operation < SPAR_HIP_ADD ||
      operation > SPAR_HIP_GREATER_EQUAL || rank > kMaxRank ||
      (rank != 0 && (extents == nullptr || left_strides == nullptr || right_strides == nullptr))) {
    return invalid();
  }
  MultiView view;
  view.rank = static_cast<int>(rank);
  view.operands = 2;
  uint64_t count = 1;
  for (uint64_t axis = 0; axis < rank; ++axis) {
    view.extents[axis] = extents[axis];
    view.strides[0][axis] = left_strides[axis];
    view.strides[1][axis] = right_strides[axis];
    count *= extents[axis];
  }
  view.offsets[0] = left_offset;
  view.offsets[1] = right_offset;
  if (count == 0) return ok();
  if (output == nullptr || left == nullptr || right == nullptr) return invalid();
  coalesce(view);
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  dispatch_binary(operation, [&](auto op) {
    if (dtype == SPAR_HIP_FLOAT32) {
      launch_view<float, 2>(static_cast<float*>(output), static_cast<const float*>(left),
                            static_cast<const float*>(right), view, op, guard);
    } else {
      launch_view<double, 2>(static_cast<double*>(output), static_cast<const double*>(left),
                             static_cast<const double*>(right), view, op, guard);
    }
  });
  return finish(guard);
}

namespace spar_hip {
namespace {

// Scatter of a contiguous source into a strided destination view: element e
// of the source goes to the destination offset decoded from e.
template <typename T, bool kIndex32>
__global__ void __launch_bounds__(kThreads)
    scatter_kernel(T* destination, const T* source, uint64_t count, KernelGeometry g) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; e < count;
       e += stride) {
    uint64_t off[2];
    decode<1, kIndex32>(e, g, off);
    destination[off[0]] = source[e];
  }
}

template <typename T>
void launch_scatter(void* destination, const void* source, const MultiView& view,
                    const DeviceGuard& guard) {
  const uint64_t count = view_numel(view);
  const KernelGeometry g = kernel_geometry(view);
  uint64_t blocks = (count + kThreads - 1) / kThreads;
  const uint64_t cap = static_cast<uint64_t>(guard.multiprocessors) * 32;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  if (count <= kIndex32Limit) {
    scatter_kernel<T, true><<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(
        static_cast<T*>(destination), static_cast<const T*>(source), count, g);
  } else {
    scatter_kernel<T, false><<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(
        static_cast<T*>(destination), static_cast<const T*>(source), count, g);
  }
}

}  // namespace
}  // namespace spar_hip

extern "C" SparHipStatus spar_hip_launch_strided_assign(void* destination, uint64_t rank,
                                                        const uint64_t* extents,
                                                        const uint64_t* strides,
                                                        uint64_t storage_offset,
                                                        const void* source,
                                                        uint64_t element_size, int device) {
  if ((element_size != 4U && element_size != 8U) || rank > kMaxRank ||
      (rank != 0 && (extents == nullptr || strides == nullptr))) {
    return invalid();
  }
  MultiView view;
  view.rank = static_cast<int>(rank);
  view.operands = 1;
  uint64_t count = 1;
  for (uint64_t axis = 0; axis < rank; ++axis) {
    view.extents[axis] = extents[axis];
    view.strides[0][axis] = strides[axis];
    count *= extents[axis];
  }
  view.offsets[0] = storage_offset;
  if (count == 0) return ok();
  if (destination == nullptr || source == nullptr) return invalid();
  coalesce(view);
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (element_size == 4U) {
    launch_scatter<float>(destination, source, view, guard);
  } else {
    launch_scatter<double>(destination, source, view, guard);
  }
  return finish(guard);
}
