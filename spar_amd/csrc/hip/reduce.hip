// Reductions: full, row (reduced axis contiguous), column (kept axis
// contiguous, reduced axis strided), generic; broadcast-gradient sums and the
// fused product-sum used by the multiply backward rule.
//
// Replaces K4-K6 and K12 of the reference (src/backend/cuda_kernels.cu:193-247,
// :287-311, :457-480) and the permute().contiguous() staging of
// src/ops/reduction.cpp:167-185 and src/core/tensor.cpp:604-623.
//
// CDNA4 design:
//   * row reduction: a 256-thread workgroup per row segment, 128-bit loads,
//     per-lane accumulation, wave64 butterfly (DPP/ds_swizzle via __shfl_xor)
//     and one LDS exchange across the 4 waves.  Long rows with few outputs
//     (a full reduction is one row) are split over many workgroups and
//     finished by a second, fixed-order pass (deterministic, no atomics);
//   * column reduction: lanes own 4 adjacent output columns (one float4),
//     rows are split across workgroups so that 8192 columns still fill 256
//     CUs; partials [outer, splits, inner] are combined in split order;
//   * argmax/max carry (value, index) pairs with the rule "NaN first, then
//     larger value, then smaller index", which reproduces the first-occurrence
//     result of a sequential scan bit for bit (including -0.0 vs +0.0).
#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "layout.hpp"

namespace spar_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr uint64_t kMaxGrid = uint64_t{1} << 20;

enum class Kind { Sum, Max };

// Accumulator: a running sum, or a (value, index) pair for max/argmax.
template <typename T, Kind K> struct Acc;

template <typename T> struct Acc<T, Kind::Sum> {
  T value;
  __device__ __forceinline__ void init() { value = T(0); }
  __device__ __forceinline__ void add(T x, int64_t) { value += x; }
  __device__ __forceinline__ void merge(const Acc& other) { value += other.value; }
  __device__ __forceinline__ void wave_reduce() { value = wave_sum(value); }
  __device__ __forceinline__ void seal(int64_t) {}
};

// Every kernel feeds one accumulator its elements in increasing index order.
// Under the max rule (NaN first, then the larger value, ties to the smaller
// index) a later element therefore wins only if it is NaN or strictly
// larger, and a NaN best is never displaced: one compare-and-select per
// element.  Starting from the identity (-inf, none), a -inf element never
// wins, so an accumulator over a non-empty range that took nothing saw only
// -inf; seal(first index of the range) records that answer.  Sealing any
// accumulator of a block with the block's first index is safe: the claim
// (-inf, first) loses to every real element and is exact when all are -inf.
template <typename T> struct Acc<T, Kind::Max> {
  ArgMax<T> best;
  __device__ __forceinline__ void init() { best = argmax_identity<T>(); }
  __device__ __forceinline__ void add(T x, int64_t index) {
    const bool take = !(x <= best.value) && best.value == best.value;
    best.value = take ? x : best.value;
    best.index = take ? index : best.index;
  }
  // The full rule, as selects: NaN first (the earlier of two NaNs), then
  // the larger value, then the earlier index.
  __device__ __forceinline__ void merge(const Acc& other) {
    const T v = other.best.value;
    const T b = best.value;
    const bool earlier = other.best.index < best.index;
    const bool better = v > b || (v == b && earlier) || (v != v && (b == b || earlier));
    best.value = better ? v : b;
    best.index = better ? other.best.index : best.index;
  }
  __device__ __forceinline__ void wave_reduce() { best = wave_argmax(best); }
  __device__ __forceinline__ void seal(int64_t first) {
    if (best.index == INT64_MAX) best.index = first;
  }
};

// Accumulator of the streaming row and column scans: the same rules as Acc,
// but max/argmax keep a 32-bit index relative to the start of the scanned
// range, which saves 64-bit index arithmetic on every element (the planner
// keeps every range below kMaxScanRange elements).  finish(base) rebases it
// into an Acc.
constexpr uint64_t kMaxScanRange = uint64_t{1} << 31;

template <typename T, Kind K> struct ScanAcc;

// Each has two forms of add: `add`, the exact rule, and `add_ordered`, which
// is exact when no element is NaN.  The streaming kernels scan with
// add_ordered, note whether any element was NaN (one unordered compare per
// pair of elements), and rescan with `add` only the lanes that saw one.
template <typename T> struct ScanAcc<T, Kind::Sum> {
  T value;
  __device__ __forceinline__ void init() { value = T(0); }
  __device__ __forceinline__ void add(T x, uint32_t) { value += x; }
  __device__ __forceinline__ void add_ordered(T x, uint32_t) { value += x; }
  __device__ __forceinline__ Acc<T, Kind::Sum> finish(int64_t) const {
    Acc<T, Kind::Sum> acc;
    acc.value = value;
    return acc;
  }
};

template <typename T> struct ScanAcc<T, Kind::Max> {
  T value;
  uint32_t index;
  __device__ __forceinline__ void init() {
    value = argmax_identity<T>().value;
    index = UINT32_MAX;
  }
  __device__ __forceinline__ void add(T x, uint32_t i) {
    const bool take = !(x <= value) && value == value;
    value = take ? x : value;
    index = take ? i : index;
  }
  // Without NaNs the value never becomes NaN, and a later element wins only
  // if it is strictly larger: one ordered compare and two selects.
  __device__ __forceinline__ void add_ordered(T x, uint32_t i) {
    const bool take = x > value;
    value = take ? x : value;
    index = take ? i : index;
  }
  __device__ __forceinline__ Acc<T, Kind::Max> finish(int64_t base) const {
    Acc<T, Kind::Max> acc;
    acc.best.value = value;
    acc.best.index = index == UINT32_MAX ? INT64_MAX : base + static_cast<int64_t>(index);
    return acc;
  }
};

// Max without its index, for a scan whose accumulator covers one contiguous
// range in order (a column scan's split): the first occurrence of the
// maximum is then fixed by the compare rule alone, ties included (-0 before
// +0 stays -0), and the range's position orders it against other ranges.
// One compare and one select per element.
template <typename T> struct ScanPeak {
  T value;
  __device__ __forceinline__ void init() { value = argmax_identity<T>().value; }
  __device__ __forceinline__ void add(T x, uint32_t) {
    value = !(x <= value) && value == value ? x : value;
  }
  __device__ __forceinline__ void add_ordered(T x, uint32_t) { value = x > value ? x : value; }
  // The index is the range's first; only the value is kept.
  __device__ __forceinline__ Acc<T, Kind::Max> finish(int64_t base) const {
    Acc<T, Kind::Max> acc;
    acc.best.value = value;
    acc.best.index = base;
    return acc;
  }
};

// Column scans of a max without argmax use ScanPeak (INDEX false).
template <typename T, Kind K, bool INDEX>
using ColumnScan = std::conditional_t<K == Kind::Max && !INDEX, ScanPeak<T>, ScanAcc<T, K>>;

// Reads one element: the input itself, or the product of two inputs that
// share strides (each product rounded to T, as multiply() would store it).
template <typename T, int NIN>
__device__ __forceinline__ T load_value(const T* a, const T* b, uint64_t offset) {
  if constexpr (NIN == 1) {
    return a[offset];
  } else {
    return a[offset] * b[offset];
  }
}

template <typename T, int NIN>
__device__ __forceinline__ typename Vec16<T>::type load_vector(const T* a, const T* b,
                                                               uint64_t offset) {
  using V = typename Vec16<T>::type;
  V va = stream_load(reinterpret_cast<const V*>(a + offset));
  if constexpr (NIN == 2) {
    const V vb = stream_load(reinterpret_cast<const V*>(b + offset));
#pragma unroll
    for (int k = 0; k < Vec16<T>::width; ++k) {
      vec_set<T>(va, k, vec_get<T>(va, k) * vec_get<T>(vb, k));
    }
  }
  return va;
}

// Block-wide combine of per-thread accumulators; every thread gets the result.
template <typename T, Kind K>
__device__ __forceinline__ Acc<T, K> block_reduce(Acc<T, K> acc) {
  __shared__ Acc<T, K> lds[kWaves];
  acc.wave_reduce();
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  __syncthreads();
  if (lane == 0) lds[wave] = acc;
  __syncthreads();
  Acc<T, K> total = lds[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) total.merge(lds[w]);
  return total;
}

// Where a reduction writes: final outputs, or partials for a second pass.
// A max/argmax partial keeps its index relative to the first index of its
// split (every split is below kMaxScanRange elements), as 32 bits: the
// combine adds split x segment back.  Sealed partials always hold an index.
template <typename T>
struct Sink {
  T* values;                  // final values (Sum/Mean/Max) or partial values
  int64_t* indices;           // argmax output (may be null)
  uint32_t* partial_indices;  // max/argmax partial indices, relative to the split
  int operation;              // SPAR_HIP_SUM / MEAN / MAX / ARGMAX
  T mean_divisor;             // (T)count for MEAN
  int partial;                // 1: write raw partials (values + relative indices)
};

// Writes one result; `first` is the first index of the accumulator's split.
template <typename T, Kind K>
__device__ __forceinline__ void sink_write(const Sink<T>& sink, uint64_t slot, const Acc<T, K>& acc,
                                           int64_t first) {
  if constexpr (K == Kind::Sum) {
    T v = acc.value;
    if (!sink.partial && sink.operation == SPAR_HIP_MEAN) v = v / sink.mean_divisor;
    sink.values[slot] = v;
  } else {
    if (sink.partial) {
      sink.values[slot] = acc.best.value;
      sink.partial_indices[slot] = static_cast<uint32_t>(acc.best.index - first);
    } else if (sink.operation == SPAR_HIP_ARGMAX) {
      sink.indices[slot] = acc.best.index;
    } else {
      sink.values[slot] = acc.best.value;
    }
  }
}

// Reads partial `slot` of split `split` (splits of `segment` elements).
// Without stored indices (INDEX false: a max of contiguous splits) the
// split's number stands in for the index: it orders equal maxima of
// different splits the way their first occurrences are ordered.
template <typename T, Kind K, bool INDEX = true>
__device__ __forceinline__ Acc<T, K> partial_read(const T* values, const uint32_t* indices,
                                                  uint64_t slot, uint64_t split, uint64_t segment) {
  Acc<T, K> acc;
  if constexpr (K == Kind::Sum) {
    acc.value = values[slot];
  } else if constexpr (INDEX) {
    acc.best.value = values[slot];
    acc.best.index = static_cast<int64_t>(split * segment + indices[slot]);
  } else {
    acc.best.value = values[slot];
    acc.best.index = static_cast<int64_t>(split);
  }
  return acc;
}

// Row offsets: the kept axes (innermost first) with their strides.
struct RowMap {
  int rank;
  FastDiv divisors[kMaxRank];
  uint64_t extents[kMaxRank];
  uint64_t strides[kMaxRank];
  uint64_t offset;
  int index32;
};

__device__ __forceinline__ uint64_t row_offset(const RowMap& map, uint64_t row) {
  uint64_t off = map.offset;
  if (map.index32) {
    uint32_t rem = static_cast<uint32_t>(row);
#pragma unroll
    for (int k = 0; k < kMaxRank; ++k) {
      if (k < map.rank) {
        const uint32_t q = map.divisors[k].div(rem);
        off += static_cast<uint64_t>(rem - q * map.divisors[k].divisor) * map.strides[k];
        rem = q;
      }
    }
  } else {
    uint64_t rem = row;
    for (int k = 0; k < map.rank; ++k) {
      const uint64_t q = rem / map.extents[k];
      off += (rem - q * map.extents[k]) * map.strides[k];
      rem = q;
    }
  }
  return off;
}

// --------------------------------------------------------------- row kernel

// Block b reduces segment (b % splits) of row (b / splits); the reduced axis
// is contiguous (stride 1) with length n.  VEC: 16-byte loads (row starts and
// segment length aligned to the vector width).
template <typename T, Kind K, int NIN, bool VEC>
__global__ void __launch_bounds__(kThreads)
    row_kernel(const T* a, const T* b, uint64_t rows, uint64_t n, uint64_t splits,
               uint64_t segment, RowMap map, Sink<T> sink) {
  constexpr int W = Vec16<T>::width;
  for (uint64_t block = blockIdx.x; block < rows * splits; block += gridDim.x) {
    const uint64_t row = block / splits;
    const uint64_t split = block - row * splits;
    const uint64_t begin = split * segment;
    const uint64_t end = begin + segment < n ? begin + segment : n;
    const uint64_t base = row_offset(map, row);
    // Indices relative to `begin` (segments are below kMaxScanRange).
    ScanAcc<T, K> scan[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) scan[u].init();
    if constexpr (VEC) {
      // Ordered scan; `unordered` records whether this lane saw a NaN (for
      // max/argmax: one unordered compare per pair of elements).
      bool unordered = false;
      constexpr uint32_t step = static_cast<uint32_t>(kThreads) * W;
      uint64_t i = begin + static_cast<uint64_t>(threadIdx.x) * W;
      for (; i + 3 * step < end; i += 4 * step) {
        typename Vec16<T>::type v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = load_vector<T, NIN>(a, b, base + i + u * step);
        const uint32_t relative = static_cast<uint32_t>(i - begin);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
          for (int k = 0; k < W; ++k) {
            scan[u].add_ordered(vec_get<T>(v[u], k), relative + u * step + k);
            if constexpr (K == Kind::Max) {
              if (u % 2 == 1) {
                unordered |= __builtin_isunordered(vec_get<T>(v[u], k), vec_get<T>(v[u - 1], k));
              }
            }
          }
        }
      }
      for (; i < end; i += step) {
        const auto v = load_vector<T, NIN>(a, b, base + i);
        const uint32_t relative = static_cast<uint32_t>(i - begin);
#pragma unroll
        for (int k = 0; k < W; ++k) {
          scan[0].add_ordered(vec_get<T>(v, k), relative + k);
          if constexpr (K == Kind::Max) unordered |= __builtin_isunordered(vec_get<T>(v, k), T(0));
        }
      }
      if constexpr (K == Kind::Max) {
        // A lane that saw a NaN rescans its elements, in increasing index
        // order, with the exact rule (the block merge does not depend on how
        // elements are split among the lane's accumulators).
        if (unordered) {
#pragma unroll
          for (int u = 0; u < 4; ++u) scan[u].init();
          for (uint64_t j = begin + static_cast<uint64_t>(threadIdx.x) * W; j < end; j += step) {
            const auto v = load_vector<T, NIN>(a, b, base + j);
            const uint32_t relative = static_cast<uint32_t>(j - begin);
#pragma unroll
            for (int k = 0; k < W; ++k) scan[0].add(vec_get<T>(v, k), relative + k);
          }
        }
      }
    } else {
      for (uint64_t i = begin + threadIdx.x; i < end; i += kThreads) {
        scan[0].add(load_value<T, NIN>(a, b, base + i), static_cast<uint32_t>(i - begin));
      }
    }
    Acc<T, K> acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = scan[u].finish(static_cast<int64_t>(begin));
    acc[0].merge(acc[1]);
    acc[2].merge(acc[3]);
    acc[0].merge(acc[2]);
    Acc<T, K> total = block_reduce<T, K>(acc[0]);
    if (begin < end) total.seal(static_cast<int64_t>(begin));
    if (threadIdx.x == 0) sink_write<T, K>(sink, block, total, static_cast<int64_t>(begin));
  }
}

// One long contiguous row (a full reduction), interleaved: block b's lanes
// take the 16-byte vectors b * kThreads + lane, then every gridDim.x *
// kThreads vectors after, four loads in flight, so that at any moment the
// whole grid reads one contiguous window of the row.  Each lane's four load
// slots keep their own accumulators, each fed in increasing index order
// (max/argmax indices are the elements' own, below kMaxScanRange), merged in
// slot order; the block's result goes to partial b (combined by
// combine_rows_kernel).  A lane that saw a NaN rescans its elements in index
// order with the exact rule, as row_kernel does.  On 2^25 float32 elements
// the sum over 512 such blocks and the combine took 22.8 us against 25.1 us
// for 2048 blocks each scanning a contiguous 64 KiB segment, and on 2^28
// 156-162 us against 172 us on the same box.  The row's start and length
// are multiples of W.
constexpr uint64_t kInterleavedBlocksPerCu = 2;

template <typename T, Kind K, int NIN>
__global__ void __launch_bounds__(kThreads)
    interleaved_row_kernel(const T* a, const T* b, uint64_t base, uint64_t n, Sink<T> sink) {
  constexpr int W = Vec16<T>::width;
  const uint64_t vectors = n / W;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  const uint64_t first = static_cast<uint64_t>(blockIdx.x) * kThreads;
  ScanAcc<T, K> scan[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) scan[u].init();
  bool unordered = false;
  uint64_t i = first + threadIdx.x;
  for (; i + 3 * stride < vectors; i += 4 * stride) {
    typename Vec16<T>::type v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = load_vector<T, NIN>(a, b, base + (i + u * stride) * W);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t element = static_cast<uint32_t>((i + u * stride) * W);
#pragma unroll
      for (int k = 0; k < W; ++k) {
        scan[u].add_ordered(vec_get<T>(v[u], k), element + k);
        if constexpr (K == Kind::Max) {
          if (u % 2 == 1) {
            unordered |= __builtin_isunordered(vec_get<T>(v[u], k), vec_get<T>(v[u - 1], k));
          }
        }
      }
    }
  }
  for (; i < vectors; i += stride) {
    const auto v = load_vector<T, NIN>(a, b, base + i * W);
    const uint32_t element = static_cast<uint32_t>(i * W);
#pragma unroll
    for (int k = 0; k < W; ++k) {
      scan[0].add_ordered(vec_get<T>(v, k), element + k);
      if constexpr (K == Kind::Max) unordered |= __builtin_isunordered(vec_get<T>(v, k), T(0));
    }
  }
  if constexpr (K == Kind::Max) {
    if (unordered) {
#pragma unroll
      for (int u = 0; u < 4; ++u) scan[u].init();
      for (uint64_t j = first + threadIdx.x; j < vectors; j += stride) {
        const auto v = load_vector<T, NIN>(a, b, base + j * W);
        const uint32_t element = static_cast<uint32_t>(j * W);
#pragma unroll
        for (int k = 0; k < W; ++k) scan[0].add(vec_get<T>(v, k), element + k);
      }
    }
  }
  Acc<T, K> acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) acc[u] = scan[u].finish(0);
  acc[0].merge(acc[1]);
  acc[2].merge(acc[3]);
  acc[0].merge(acc[2]);
  Acc<T, K> total = block_reduce<T, K>(acc[0]);
  // a block that saw only -inf answers with its first element
  total.seal(static_cast<int64_t>(first * W));
  if (threadIdx.x == 0) sink_write<T, K>(sink, blockIdx.x, total, 0);
}

// Short rows (n <= kNarrowRow): one lane per row, scanning its n elements in
// index order with the exact rule, so a sum is the CPU loop's in-order sum
// and a max / argmax keeps the first maximum and the first NaN.  The row
// kernel would give every such row a whole workgroup and a block-wide
// combine, about a microsecond per row whatever its length.
constexpr uint64_t kNarrowRow = 32;

template <typename T, Kind K, int NIN>
__global__ void __launch_bounds__(kThreads)
    narrow_row_kernel(const T* a, const T* b, uint64_t rows, uint64_t n, uint64_t stride,
                      RowMap map, Sink<T> sink) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t row = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; row < rows;
       row += step) {
    const uint64_t base = row_offset(map, row);
    ScanAcc<T, K> scan;
    scan.init();
    for (uint64_t i = 0; i < n; ++i) {
      scan.add(load_value<T, NIN>(a, b, base + i * stride), static_cast<uint32_t>(i));
    }
    Acc<T, K> acc = scan.finish(0);
    if (n > 0) acc.seal(0);  // a row of only -inf: its first element
    sink_write<T, K>(sink, row, acc, 0);
  }
}

// Second pass after row splits: one block per output reduces its `parts`
// consecutive partials with a fixed tree.
template <typename T, Kind K>
__global__ void __launch_bounds__(kThreads)
    combine_rows_kernel(const T* part_values, const uint32_t* part_indices, uint64_t outputs,
                        uint64_t parts, uint64_t segment, Sink<T> sink) {
  for (uint64_t o = blockIdx.x; o < outputs; o += gridDim.x) {
    Acc<T, K> acc;
    acc.init();
    // Batches of 8 partials: every load of a batch is issued before the first
    // merge, as in combine_columns_kernel.
    constexpr int kBatch = 8;
    for (uint64_t s0 = threadIdx.x; s0 < parts; s0 += kThreads * kBatch) {
      Acc<T, K> part[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const uint64_t s = s0 + static_cast<uint64_t>(j) * kThreads;
        if (s < parts) {
          part[j] = partial_read<T, K>(part_values, part_indices, o * parts + s, s, segment);
        } else {
          part[j].init();
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) acc.merge(part[j]);
    }
    const Acc<T, K> total = block_reduce<T, K>(acc);
    if (threadIdx.x == 0) sink_write<T, K>(sink, o, total, 0);
  }
}

// ------------------------------------------------------------ column kernel

// Input element (o, r, i) at map-offset(o) + r * reduced_stride + i, with the
// inner axis contiguous.  A block owns 64 * W adjacent columns (each lane W
// of them, one 16-byte load per row when VEC); its four waves walk the rows
// of the block's segment interleaved (wave w takes rows w, w+4, ...), so a
// wave reads 1 KiB contiguous per row.  The four wave partials are combined
// through LDS in wave order.  Block b covers column block cb, split s, outer o.
template <typename T, Kind K, int NIN, bool VEC>
__global__ void __launch_bounds__(kThreads)
    column_kernel(const T* a, const T* b, uint64_t outer, uint64_t n, uint64_t reduced_stride,
                  uint64_t inner, uint64_t column_blocks, uint64_t splits, uint64_t segment,
                  RowMap map, Sink<T> sink) {
  constexpr int W = VEC ? Vec16<T>::width : 1;
  __shared__ Acc<T, K> lds[kWaves][kWave * W];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const uint64_t total_blocks = outer * splits * column_blocks;
  for (uint64_t block = blockIdx.x; block < total_blocks; block += gridDim.x) {
    const uint64_t cb = block % column_blocks;
    const uint64_t rest = block / column_blocks;
    const uint64_t split = rest % splits;
    const uint64_t o = rest / splits;
    const uint64_t column = (cb * kWave + lane) * W;
    const uint64_t begin = split * segment;
    const uint64_t end = begin + segment < n ? begin + segment : n;
    Acc<T, K> acc[W];
#pragma unroll
    for (int k = 0; k < W; ++k) acc[k].init();
    if (column < inner) {
      const uint64_t base = row_offset(map, o) + column;
      uint64_t r = begin + wave;
      if constexpr (VEC) {
        for (; r + 3 * kWaves < end; r += 4 * kWaves) {
          typename Vec16<T>::type v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            v[u] = load_vector<T, NIN>(a, b, base + (r + u * kWaves) * reduced_stride);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int k = 0; k < W; ++k) {
              acc[k].add(vec_get<T>(v[u], k), static_cast<int64_t>(r + u * kWaves));
            }
          }
        }
        for (; r < end; r += kWaves) {
          const auto v = load_vector<T, NIN>(a, b, base + r * reduced_stride);
#pragma unroll
          for (int k = 0; k < W; ++k) acc[k].add(vec_get<T>(v, k), static_cast<int64_t>(r));
        }
      } else {
        for (; r < end; r += kWaves) {
          acc[0].add(load_value<T, NIN>(a, b, base + r * reduced_stride), static_cast<int64_t>(r));
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < W; ++k) lds[wave][lane * W + k] = acc[k];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int k = 0; k < W; ++k) {
        if (column + k < inner) {
          Acc<T, K> total = lds[0][lane * W + k];
#pragma unroll
          for (int w = 1; w < kWaves; ++w) total.merge(lds[w][lane * W + k]);
          if (begin < end) total.seal(static_cast<int64_t>(begin));
          // Output slot: final [outer, inner]; partial [outer, splits, inner].
          const uint64_t slot = sink.partial ? (o * splits + split) * inner + column + k
                                             : o * inner + column + k;
          sink_write<T, K>(sink, slot, total, static_cast<int64_t>(begin));
        }
      }
    }
  }
}

// Max/argmax in one pass when the kept axis is contiguous and wide enough to
// give every CU its own strip of columns (the kernel also sums, but slower
// than the split scan): a workgroup owns the 128
// bytes (kStripGroups 16-byte groups) of adjacent columns of one strip and
// every row.  Lane t takes group t % kStripGroups and rows t / kStripGroups,
// + kStripRows, ... in increasing order, R rows in flight, so each lane's
// accumulators see their elements in index order; the lanes of a column then
// merge through a fixed LDS tree (for max/argmax under the full (NaN, value,
// index) rule, whose result does not depend on the merge order).  No
// partials and no second kernel: on [8192, 8192] over axis 0 the 256 strips
// read 128-byte pieces of every row side by side, and the argmax took 42.0
// us against 50.2 us for the split scan plus combine (steady state, MI355X).
// Lanes that saw a NaN rescan their rows with the exact rule, as the other
// scans do.  The rows are walked with a pointer (no 64-bit multiply per
// load).
constexpr int kStripGroups = 8;
constexpr int kStripRows = kThreads / kStripGroups;

template <typename T, Kind K, int NIN, int R>
__global__ void __launch_bounds__(kThreads)
    column_strip_kernel(const T* a, const T* b, uint64_t outer, uint64_t n,
                        uint64_t reduced_stride, uint64_t inner, RowMap map, Sink<T> sink) {
  constexpr int W = Vec16<T>::width;
  constexpr int kColumns = kStripGroups * W;
  using V = typename Vec16<T>::type;
  __shared__ Acc<T, K> lds[kStripRows][kColumns];
  const int group = threadIdx.x % kStripGroups;
  const uint32_t first_row = threadIdx.x / kStripGroups;
  const uint64_t strips_per_outer = (inner + kColumns - 1) / kColumns;
  const uint64_t strips = outer * strips_per_outer;
  const uint64_t step = static_cast<uint64_t>(kStripRows) * reduced_stride;
  for (uint64_t strip = blockIdx.x; strip < strips; strip += gridDim.x) {
    const uint64_t o = strip / strips_per_outer;
    const uint64_t column = (strip - o * strips_per_outer) * kColumns + group * W;
    const bool present = column < inner;  // inner is a multiple of W
    const uint64_t base = row_offset(map, o) + column;
    ScanAcc<T, K> scan[W];
#pragma unroll
    for (int k = 0; k < W; ++k) scan[k].init();
    bool unordered = false;
    if (present) {
      uint64_t offset = base + first_row * reduced_stride;
      uint64_t r = first_row;
      for (; r + static_cast<uint64_t>(R - 1) * kStripRows < n; r += R * kStripRows) {
        V v[R];
#pragma unroll
        for (int u = 0; u < R; ++u) v[u] = load_vector<T, NIN>(a, b, offset + u * step);
        offset += R * step;
        // All R loads in flight before the first add or compare.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < R; ++u) {
#pragma unroll
          for (int k = 0; k < W; ++k) {
            scan[k].add_ordered(vec_get<T>(v[u], k), static_cast<uint32_t>(r + u * kStripRows));
            if constexpr (K == Kind::Max) {
              if (u % 2 == 1) {
                unordered |= __builtin_isunordered(vec_get<T>(v[u], k), vec_get<T>(v[u - 1], k));
              }
            }
          }
        }
      }
      for (; r < n; r += kStripRows, offset += step) {
        const V v = load_vector<T, NIN>(a, b, offset);
#pragma unroll
        for (int k = 0; k < W; ++k) {
          scan[k].add_ordered(vec_get<T>(v, k), static_cast<uint32_t>(r));
          if constexpr (K == Kind::Max) unordered |= __builtin_isunordered(vec_get<T>(v, k), T(0));
        }
      }
      if constexpr (K == Kind::Max) {
        if (unordered) {
#pragma unroll
          for (int k = 0; k < W; ++k) scan[k].init();
          for (uint64_t row = first_row; row < n; row += kStripRows) {
            const V v = load_vector<T, NIN>(a, b, base + row * reduced_stride);
#pragma unroll
            for (int k = 0; k < W; ++k) scan[k].add(vec_get<T>(v, k), static_cast<uint32_t>(row));
          }
        }
      }
    }
    __syncthreads();  // the previous strip's readers are done with lds
#pragma unroll
    for (int k = 0; k < W; ++k) {
      Acc<T, K> acc = scan[k].finish(0);
      if (first_row < n) acc.seal(static_cast<int64_t>(first_row));
      lds[first_row][group * W + k] = acc;
    }
    __syncthreads();
    for (int half = kStripRows / 2; half > 0; half /= 2) {
      for (int e = threadIdx.x; e < half * kColumns; e += kThreads) {
        const int row = e / kColumns;
        const int c = e % kColumns;
        Acc<T, K> acc = lds[row][c];
        acc.merge(lds[row + half][c]);
        lds[row][c] = acc;
      }
      __syncthreads();
    }
    if (threadIdx.x < kColumns) {
      const uint64_t c = column - group * W + threadIdx.x;
      if (c < inner) sink_write<T, K>(sink, o * inner + c, lds[0][threadIdx.x], 0);
    }
  }
}

// Wide rows (inner >= 256 vectors): each wave owns VPL x 64 x W adjacent
// columns (lane l holds the 16-byte groups l, l + 64, ..., so one row of the
// wave's columns is VPL x 1 KiB contiguous) and walks every row of the
// block's segment, R rows in flight; no cross-wave combine is needed.  A
// block's four waves cover 4 x VPL x 64 x W adjacent columns.  Measured on
// MI355X (steady state, two kernels including the combine):
//
//   shape (reduced axis first)      VPL=1, R=4, 2 blocks/CU   VPL=4, R=2, 1 block/CU
//   [8192, 8192]  axis 0            47.1 us                    42.4 us
//   [32768, 4096] axis 0            81.3 us                    80.9 us
//   [32, 1024, 4096] G*x, axis 1    162.8 us                   155.7 us
//   [8192, 4096]  axis 0            26.5 us                    25.8 us
//
// With VPL = 4, more rows in flight lost: R = 3 and 4 took 46 us on
// [8192, 8192] axis 0 (R = 2: 44 us), and the C2 sums over [32, 1024, 4096]
// 86 us against 81 us (dbias; R = 4 took dscale from 164 to 283 us).
// VPL = 4 needs the row length to be a multiple of 4 x 256 groups; other
// wide rows take VPL = 1.  A max without argmax (INDEX false) scans values
// only and writes value-only partials.
template <typename T, Kind K, int NIN, int VPL, int R, bool INDEX = true>
__global__ void __launch_bounds__(kThreads)
    column_wide_kernel(const T* a, const T* b, uint64_t outer, uint64_t n,
                       uint64_t reduced_stride, uint64_t inner, uint64_t column_blocks,
                       uint64_t splits, uint64_t segment, RowMap map, Sink<T> sink) {
  constexpr int W = Vec16<T>::width;
  constexpr uint64_t kGroupStride = static_cast<uint64_t>(kWave) * W;  // columns between a lane's groups
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const uint64_t total_blocks = outer * splits * column_blocks;
  for (uint64_t block = blockIdx.x; block < total_blocks; block += gridDim.x) {
    const uint64_t cb = block % column_blocks;
    const uint64_t rest = block / column_blocks;
    const uint64_t split = rest % splits;
    const uint64_t o = rest / splits;
    const uint64_t column = ((cb * kWaves + wave) * VPL * kWave + lane) * W;
    // inner is a multiple of W, and of 256 x VPL x W when VPL > 1: every group exists
    if (column >= inner) continue;
    const uint64_t begin = split * segment;
    const uint64_t end = begin + segment < n ? begin + segment : n;
    ColumnScan<T, K, INDEX> scan[VPL][W];
#pragma unroll
    for (int g = 0; g < VPL; ++g) {
#pragma unroll
      for (int k = 0; k < W; ++k) scan[g][k].init();
    }
    const uint64_t base = row_offset(map, o) + column;
    using V = typename Vec16<T>::type;
    auto load_batch = [&](V (&v)[R][VPL], uint64_t first) {
#pragma unroll
      for (int u = 0; u < R; ++u) {
#pragma unroll
        for (int g = 0; g < VPL; ++g) {
          v[u][g] = load_vector<T, NIN>(a, b, base + (first + u) * reduced_stride + g * kGroupStride);
        }
      }
    };
    // Ordered scan; `unordered` records whether this lane saw a NaN (for
    // max/argmax: one unordered compare per pair of rows).
    bool unordered = false;
    auto scan_batch = [&](const V (&v)[R][VPL], uint64_t first) {
      const uint32_t relative = static_cast<uint32_t>(first - begin);
#pragma unroll
      for (int u = 0; u < R; ++u) {
#pragma unroll
        for (int g = 0; g < VPL; ++g) {
#pragma unroll
          for (int k = 0; k < W; ++k) {
            scan[g][k].add_ordered(vec_get<T>(v[u][g], k), relative + u);
            if constexpr (K == Kind::Max) {
              if (u % 2 == 1 || u == R - 1) {
                const T x = vec_get<T>(v[u][g], k);
                const T y = vec_get<T>(v[u - (u % 2)][g], k);
                unordered |= __builtin_isunordered(x, y);
              }
            }
          }
        }
      }
    };
    uint64_t r = begin;
    for (; r + (R - 1) < end; r += R) {
      V v[R][VPL];
      load_batch(v, r);
      // Keep all R x VPL loads in flight: without this barrier the scheduler
      // interleaves the max/argmax compare-and-selects with the loads to save
      // registers and leaves about three loads outstanding.
      __builtin_amdgcn_sched_barrier(0);
      scan_batch(v, r);
    }
    for (; r < end; ++r) {
      const uint32_t relative = static_cast<uint32_t>(r - begin);
#pragma unroll
      for (int g = 0; g < VPL; ++g) {
        const auto v = load_vector<T, NIN>(a, b, base + r * reduced_stride + g * kGroupStride);
#pragma unroll
        for (int k = 0; k < W; ++k) {
          scan[g][k].add_ordered(vec_get<T>(v, k), relative);
          if constexpr (K == Kind::Max) unordered |= __builtin_isunordered(vec_get<T>(v, k), T(0));
        }
      }
    }
    if constexpr (K == Kind::Max) {
      // A lane that saw a NaN rescans its columns with the exact rule.
      if (unordered) {
#pragma unroll
        for (int g = 0; g < VPL; ++g) {
#pragma unroll
          for (int k = 0; k < W; ++k) scan[g][k].init();
        }
        for (uint64_t row = begin; row < end; ++row) {
          const uint32_t relative = static_cast<uint32_t>(row - begin);
#pragma unroll
          for (int g = 0; g < VPL; ++g) {
            const auto v = load_vector<T, NIN>(a, b, base + row * reduced_stride + g * kGroupStride);
#pragma unroll
            for (int k = 0; k < W; ++k) scan[g][k].add(vec_get<T>(v, k), relative);
          }
        }
      }
    }
#pragma unroll
    for (int g = 0; g < VPL; ++g) {
      const uint64_t c = column + g * kGroupStride;
      Acc<T, K> total[W];
#pragma unroll
      for (int k = 0; k < W; ++k) {
        total[k] = scan[g][k].finish(static_cast<int64_t>(begin));
        if (begin < end) total[k].seal(static_cast<int64_t>(begin));
      }
      if (sink.partial) {
        // Partials [outer, splits, inner]: the group's W values (and W
        // relative indices) go out as one vector store each.
        const uint64_t slot = (o * splits + split) * inner + c;
        V values;
        uint32_t indices[W];
#pragma unroll
        for (int k = 0; k < W; ++k) {
          if constexpr (K == Kind::Sum) {
            vec_set<T>(values, k, total[k].value);
          } else {
            vec_set<T>(values, k, total[k].best.value);
            indices[k] = static_cast<uint32_t>(total[k].best.index - static_cast<int64_t>(begin));
          }
        }
        *reinterpret_cast<V*>(sink.values + slot) = values;
        if constexpr (K == Kind::Max && INDEX) {
          if constexpr (W == 4) {
            *reinterpret_cast<i32x4*>(sink.partial_indices + slot) =
                i32x4{static_cast<int32_t>(indices[0]), static_cast<int32_t>(indices[1]),
                      static_cast<int32_t>(indices[2]), static_cast<int32_t>(indices[3])};
          } else {
#pragma unroll
            for (int k = 0; k < W; ++k) sink.partial_indices[slot + k] = indices[k];
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < W; ++k) {
          sink_write<T, K>(sink, o * inner + c + k, total[k], static_cast<int64_t>(begin));
        }
      }
    }
  }
}

// Second pass after column splits.  A 1024-lane block holds 16 / P groups of
// P waves; each group owns 64 columns of one outer index, its wave p combines
// splits p, p + P, ... in order, and the group's P results are combined by a
// fixed tree, so the result is deterministic.  P grows with the number of
// splits: few splits need no split parallelism, and a block of 16 waves on
// one column range would then be mostly idle.
//
// The combine is short (a few microseconds after the split pass), so its
// latency chain is what it costs:
//   * a wave issues a batch of B partials at once.  EXACT launches have
//     splits a multiple of P x B, so no load has a bounds test and slots step
//     by the uniform P x inner from the batch's first (one 64-bit add per
//     address); other split counts test each slot.  After the 256-split pass
//     over [8192, 4096] (steady state, back to back) the pass plus combine
//     took 26.3 us with two batches of 8 tested loads and about 24.3 us with
//     one exact batch of 16: a bounds test per load kept the batch from going
//     out back to back (the compiler branches around each load).
//   * after one barrier the group's first wave reads the P results from LDS
//     and evaluates the tree in registers: the same pairs in the same order
//     as a tree through LDS with a barrier per level, so the same bits.
constexpr int kCombineThreads = 1024;
constexpr int kCombineWaves = kCombineThreads / kWave;

template <typename T, Kind K, int P, int B, bool EXACT, bool INDEX>
__global__ void __launch_bounds__(kCombineThreads)
    combine_columns_kernel(const T* part_values, const uint32_t* part_indices, uint64_t outer,
                           uint64_t splits, uint64_t segment, uint64_t inner, Sink<T> sink) {
  constexpr int kGroups = kCombineWaves / P;
  __shared__ Acc<T, K> lds[kCombineWaves][kWave];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int group = wave / P;
  const int p = wave % P;
  const uint64_t ranges = (inner + kWave - 1) / kWave;  // 64-column ranges per outer index
  const uint64_t blocks = outer * ((ranges + kGroups - 1) / kGroups);
  const uint64_t step = static_cast<uint64_t>(P) * inner;  // slots between a wave's partials
  for (uint64_t block = blockIdx.x; block < blocks; block += gridDim.x) {
    const uint64_t range = block * kGroups + group;  // over outer x ranges, ranges padded
    const uint64_t o = range / (((ranges + kGroups - 1) / kGroups) * kGroups);
    const uint64_t r = range - o * (((ranges + kGroups - 1) / kGroups) * kGroups);
    const uint64_t i = r * kWave + lane;
    const bool valid = r < ranges && i < inner;
    Acc<T, K> acc;
    acc.init();
    if (valid) {
      for (uint64_t s0 = p; s0 < splits; s0 += static_cast<uint64_t>(P) * B) {
        Acc<T, K> part[B];
        const uint64_t first = (o * splits + s0) * inner + i;
#pragma unroll
        for (int j = 0; j < B; ++j) {
          const uint64_t s = s0 + static_cast<uint64_t>(j) * P;
          if (EXACT || s < splits) {
            part[j] = partial_read<T, K, INDEX>(part_values, part_indices,
                                                first + static_cast<uint64_t>(j) * step, s,
                                                segment);
          } else {
            part[j].init();
          }
        }
#pragma unroll
        for (int j = 0; j < B; ++j) acc.merge(part[j]);
      }
    }
    if constexpr (P > 1) {
      if (block != blockIdx.x) __syncthreads();  // the previous range's readers are done
      lds[wave][lane] = acc;
      __syncthreads();
      if (p == 0) {
        // Level `half` merges result q + half into result q, q < half.
        Acc<T, K> tree[P];
#pragma unroll
        for (int q = 0; q < P; ++q) tree[q] = lds[wave + q][lane];
#pragma unroll
        for (int half = P / 2; half > 0; half /= 2) {
#pragma unroll
          for (int q = 0; q < half; ++q) tree[q].merge(tree[q + half]);
        }
        acc = tree[0];
      }
    }
    if (p == 0 && valid) sink_write<T, K>(sink, o * inner + i, acc, 0);
  }
}

// ----------------------------------------------------------- generic kernel

// One wave per output; lanes stride over the flattened reduced sub-space and
// decode its coordinates (reduced axes, innermost first).
struct ReducedMap {
  int rank;
  uint64_t extents[kMaxRank];
  uint64_t strides[kMaxRank];
  uint64_t count;
};

template <typename T, Kind K, int NIN>
__global__ void __launch_bounds__(kThreads)
    generic_kernel(const T* a, const T* b, uint64_t outputs, RowMap map, ReducedMap red,
                   Sink<T> sink) {
  const uint64_t wave = (static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x) / kWave;
  const int lane = threadIdx.x % kWave;
  const uint64_t waves = static_cast<uint64_t>(gridDim.x) * kWaves;
  for (uint64_t o = wave; o < outputs; o += waves) {
    const uint64_t base = row_offset(map, o);
    Acc<T, K> acc;
    acc.init();
    for (uint64_t j = lane; j < red.count; j += kWave) {
      uint64_t rem = j;
      uint64_t off = base;
      for (int k = 0; k < red.rank; ++k) {
        const uint64_t q = rem / red.extents[k];
        off += (rem - q * red.extents[k]) * red.strides[k];
        rem = q;
      }
      acc.add(load_value<T, NIN>(a, b, off), static_cast<int64_t>(j));
    }
    acc.wave_reduce();
    if (red.count != 0) acc.seal(0);
    if (lane == 0) sink_write<T, K>(sink, o, acc, 0);
  }
}

// ------------------------------------------------------------------ planner

// A reduction over a permuted, coalesced view: kept axes (output order) and
// reduced axes (flattened-index order), each innermost last.
struct Plan {
  int kept_rank = 0;
  uint64_t kept_extents[kMaxRank];
  uint64_t kept_strides[kMaxRank];
  int red_rank = 0;
  uint64_t red_extents[kMaxRank];
  uint64_t red_strides[kMaxRank];
  uint64_t offset = 0;
  uint64_t outputs = 1;
  uint64_t reduced = 1;
};

// Merges neighbours in a list of (extent, stride) axes (row-major order) and
// drops extent-1 axes.
void coalesce_list(int& rank, uint64_t* extents, uint64_t* strides) {
  int out = 0;
  for (int axis = 0; axis < rank; ++axis) {
    if (extents[axis] == 1) continue;
    if (out > 0 && strides[out - 1] == strides[axis] * extents[axis]) {
      extents[out - 1] *= extents[axis];
      strides[out - 1] = strides[axis];
      continue;
    }
    extents[out] = extents[axis];
    strides[out] = strides[axis];
    ++out;
  }
  rank = out;
}

RowMap make_row_map(const Plan& plan, int kept_axes_used) {
  // kept axes [0, kept_axes_used) in output order; innermost first in the map
  RowMap map{};
  map.rank = kept_axes_used;
  map.offset = plan.offset;
  uint64_t rows = 1;
  for (int k = 0; k < kept_axes_used; ++k) {
    const int axis = kept_axes_used - 1 - k;
    map.extents[k] = plan.kept_extents[axis];
    map.strides[k] = plan.kept_strides[axis];
    rows *= plan.kept_extents[axis];
  }
  map.index32 = rows <= kIndex32Limit;
  for (int k = 0; k < map.rank; ++k) {
    map.divisors[k].init(static_cast<uint32_t>(map.index32 ? map.extents[k] : 1));
  }
  return map;
}

uint32_t grid_for(uint64_t blocks) {
  if (blocks == 0) blocks = 1;
  return static_cast<uint32_t>(blocks > kMaxGrid ? kMaxGrid : blocks);
}

// Where a split reduction keeps its partial results.  With `fixed` null the
// caching allocator supplies them for the duration of the launch; otherwise
// they are carved from the caller's fixed region of `capacity` bytes (values
// first, then 32-bit indices at the next 256-byte boundary), and a plan that
// needs more is refused before anything is launched: run_plan sets
// `exceeded` and returns hipErrorInvalidValue.  The flag, not the error
// code, tells the caller it was the capacity check, so a real error from
// the runtime is never reported as a refusal.
struct Workspace {
  void* fixed = nullptr;
  uint64_t capacity = 0;
  mutable bool exceeded = false;
};

uint64_t align256(uint64_t bytes) { return (bytes + 255) / 256 * 256; }

template <typename T, Kind K, int NIN>
hipError_t run_plan(const Plan& plan, const T* a, const T* b, void* output, int operation,
                    int device, const DeviceGuard& guard, const Workspace& workspace) {
  constexpr int W = Vec16<T>::width;
  Sink<T> sink{};
  sink.operation = operation;
  sink.mean_divisor = static_cast<T>(plan.reduced);
  const bool argmax = operation == SPAR_HIP_ARGMAX;
  const int cus = guard.multiprocessors;
  const uint64_t target_blocks = static_cast<uint64_t>(cus) * 8;

  auto final_sink = [&]() {
    Sink<T> s = sink;
    s.partial = 0;
    s.values = argmax ? nullptr : static_cast<T*>(output);
    s.indices = argmax ? static_cast<int64_t*>(output) : nullptr;
    return s;
  };

  // Scratch for partial results (values, plus indices for max/argmax unless
  // the partials are value-only), from the allocator or the fixed workspace.
  auto with_partials = [&](uint64_t slots, auto&& body, bool value_only = false) -> hipError_t {
    const bool indexed = K == Kind::Max && !value_only;
    void* values = nullptr;
    void* indices = nullptr;
    if (workspace.fixed != nullptr) {
      const uint64_t value_bytes = align256(slots * sizeof(T));
      const uint64_t needed = value_bytes + (indexed ? slots * sizeof(uint32_t) : 0);
      if (needed > workspace.capacity) {
        workspace.exceeded = true;  // nothing enqueued
        return hipErrorInvalidValue;
      }
      values = workspace.fixed;
      indices = indexed ? static_cast<unsigned char*>(workspace.fixed) + value_bytes : nullptr;
    } else {
      hipError_t error = scratch_allocate(&values, slots * sizeof(T), device);
      if (error != hipSuccess) return error;
      if (indexed) {
        error = scratch_allocate(&indices, slots * sizeof(uint32_t), device);
        if (error != hipSuccess) {
          scratch_release(values, device);
          return error;
        }
      }
    }
    Sink<T> partial = sink;
    partial.partial = 1;
    partial.values = static_cast<T*>(values);
    partial.indices = nullptr;
    partial.partial_indices = static_cast<uint32_t*>(indices);
    body(partial);
    if (workspace.fixed == nullptr) {
      scratch_release(values, device);
      scratch_release(indices, device);
    }
    return hipSuccess;
  };

  const bool row_case = plan.red_rank == 1 && plan.red_strides[0] == 1;
  const bool column_case = !row_case && plan.red_rank == 1 && plan.kept_rank >= 1 &&
                           plan.kept_strides[plan.kept_rank - 1] == 1;

  if (plan.red_rank == 0) {
    // Nothing is reduced (all reduced extents are 1): a reduction of one
    // element per output.
    Plan single = plan;
    single.red_rank = 1;
    single.red_extents[0] = 1;
    single.red_strides[0] = 1;
    return run_plan<T, K, NIN>(single, a, b, output, operation, device, guard, workspace);
  }

  if (row_case) {
    const uint64_t rows = plan.outputs;
    const uint64_t n = plan.red_extents[0];
    const RowMap map = make_row_map(plan, plan.kept_rank);
    if (n <= kNarrowRow) {
      narrow_row_kernel<T, K, NIN><<<grid_for((rows + kThreads - 1) / kThreads), kThreads, 0,
                                     guard.stream>>>(a, b, rows, n, 1, map, final_sink());
      return hipSuccess;
    }
    bool vec = n % W == 0 && plan.offset % W == 0 && aligned16(a) && (NIN == 1 || aligned16(b));
    for (int k = 0; k < plan.kept_rank; ++k) {
      if (plan.kept_strides[k] % W != 0) vec = false;
    }
    // Split long rows when there are too few rows to fill the device, and
    // keep every segment below kMaxScanRange elements.
    uint64_t splits = 1;
    const uint64_t min_segment = static_cast<uint64_t>(kThreads) * W * 8;
    if (rows < target_blocks && n >= 2 * min_segment) {
      splits = (target_blocks + rows - 1) / rows;
      const uint64_t max_splits = n / min_segment;
      if (splits > max_splits) splits = max_splits;
      if (splits < 1) splits = 1;
    }
    const uint64_t range_splits = (n + kMaxScanRange / 2 - 1) / (kMaxScanRange / 2);
    if (splits < range_splits) splits = range_splits;
    // A full reduction of a long contiguous row: interleaved blocks.
    if (rows == 1 && vec && splits > 1 && n < kMaxScanRange) {
      uint64_t blocks = static_cast<uint64_t>(cus) * kInterleavedBlocksPerCu;
      if (blocks > splits) blocks = splits;
      const uint64_t base = map.offset;  // row 0
      return with_partials(blocks, [&](const Sink<T>& partial) {
        interleaved_row_kernel<T, K, NIN><<<static_cast<uint32_t>(blocks), kThreads, 0,
                                            guard.stream>>>(a, b, base, n, partial);
        // partial b's index is the element's own: segment 0
        combine_rows_kernel<T, K><<<1, kThreads, 0, guard.stream>>>(
            partial.values, partial.partial_indices, 1, blocks, 0, final_sink());
      });
    }
    uint64_t segment = (n + splits - 1) / splits;
    if (vec) segment = (segment + W - 1) / W * W;
    splits = (n + segment - 1) / segment;
    auto launch = [&](const Sink<T>& s) {
      if (vec) {
        row_kernel<T, K, NIN, true><<<grid_for(rows * splits), kThreads, 0, guard.stream>>>(
            a, b, rows, n, splits, segment, map, s);
      } else {
        row_kernel<T, K, NIN, false><<<grid_for(rows * splits), kThreads, 0, guard.stream>>>(
            a, b, rows, n, splits, segment, map, s);
      }
    };
    if (splits == 1) {
      launch(final_sink());
      return hipSuccess;
    }
    return with_partials(rows * splits, [&](const Sink<T>& partial) {
      launch(partial);
      combine_rows_kernel<T, K><<<grid_for(rows), kThreads, 0, guard.stream>>>(
          partial.values, partial.partial_indices, rows, splits, segment, final_sink());
    });
  }

  if (column_case) {
    const uint64_t inner = plan.kept_extents[plan.kept_rank - 1];
    const uint64_t outer = plan.outputs / inner;
    const uint64_t n = plan.red_extents[0];
    const uint64_t reduced_stride = plan.red_strides[0];
    const RowMap map = make_row_map(plan, plan.kept_rank - 1);
    bool vec = inner % W == 0 && plan.offset % W == 0 && reduced_stride % W == 0 &&
               aligned16(a) && (NIN == 1 || aligned16(b));
    for (int k = 0; k < plan.kept_rank - 1; ++k) {
      if (plan.kept_strides[k] % W != 0) vec = false;
    }
    // Max/argmax over rows wide enough for a 128-byte strip per CU: one pass
    // with no partials.  (Sums stay on the split scan: on [8192, 8192] over
    // axis 0 strips took 47.0 us against 45.5 us, while the strip max took
    // 44.2 us.)
    if constexpr (K == Kind::Max) {
      constexpr uint64_t kStripColumns = static_cast<uint64_t>(kStripGroups) * W;
      const uint64_t strips = outer * ((inner + kStripColumns - 1) / kStripColumns);
      if (vec && n < kMaxScanRange && n >= static_cast<uint64_t>(kStripRows) * 8 &&
          strips >= static_cast<uint64_t>(cus)) {
        column_strip_kernel<T, K, NIN, 8><<<grid_for(strips), kThreads, 0, guard.stream>>>(
            a, b, outer, n, reduced_stride, inner, map, final_sink());
        return hipSuccess;
      }
    }
    // Wide rows: waves own columns.  Rows of whole 4-group blocks take 4
    // groups per lane, 2 rows in flight, one block per CU and >= 16 rows per
    // split; other wide rows 1 group per lane, 4 rows in flight, 2 blocks per
    // CU and >= 64 rows per split.  Narrow rows: waves interleave rows (8
    // blocks per CU, >= 16 rows per wave).
    const bool wide = vec && inner / W >= static_cast<uint64_t>(kWaves) * kWave;
    const bool quad = wide && (inner / W) % (static_cast<uint64_t>(kThreads) * 4) == 0;
    const uint64_t columns_per_block = static_cast<uint64_t>(kWave) * (vec ? W : 1) *
                                       (wide ? kWaves : 1) * (quad ? 4 : 1);
    const uint64_t column_blocks = (inner + columns_per_block - 1) / columns_per_block;
    const uint64_t base_blocks = outer * column_blocks;
    uint64_t splits = 1;
    const uint64_t min_rows = quad ? 16 : wide ? 64 : 16 * kWaves;
    const uint64_t wanted_blocks = static_cast<uint64_t>(cus) * (quad ? 1 : wide ? 2 : 8);
    if (base_blocks < wanted_blocks && n >= 2 * min_rows) {
      splits = (wanted_blocks + base_blocks - 1) / base_blocks;
      if (splits > n / min_rows) splits = n / min_rows;
      if (splits < 1) splits = 1;
    }
    const uint64_t range_splits = (n + kMaxScanRange / 2 - 1) / (kMaxScanRange / 2);
    if (splits < range_splits) splits = range_splits;
    const uint64_t segment = (n + splits - 1) / splits;
    splits = (n + segment - 1) / segment;
    // A max without argmax over wide rows scans and combines values only.
    const bool value_only = K == Kind::Max && operation == SPAR_HIP_MAX && wide;
    auto launch = [&](const Sink<T>& s) {
      const uint32_t grid = grid_for(outer * splits * column_blocks);
      auto launch_wide = [&](auto index) {
        constexpr bool INDEX = decltype(index)::value;
        if (quad) {
          column_wide_kernel<T, K, NIN, 4, 2, INDEX><<<grid, kThreads, 0, guard.stream>>>(
              a, b, outer, n, reduced_stride, inner, column_blocks, splits, segment, map, s);
        } else {
          column_wide_kernel<T, K, NIN, 1, 4, INDEX><<<grid, kThreads, 0, guard.stream>>>(
              a, b, outer, n, reduced_stride, inner, column_blocks, splits, segment, map, s);
        }
      };
      if (wide) {
        if constexpr (K == Kind::Max) {
          if (value_only) {
            launch_wide(std::false_type{});
            return;
          }
        }
        launch_wide(std::true_type{});
      } else if (vec) {
        column_kernel<T, K, NIN, true><<<grid, kThreads, 0, guard.stream>>>(
            a, b, outer, n, reduced_stride, inner, column_blocks, splits, segment, map, s);
      } else {
        column_kernel<T, K, NIN, false><<<grid, kThreads, 0, guard.stream>>>(
            a, b, outer, n, reduced_stride, inner, column_blocks, splits, segment, map, s);
      }
    };
    if (splits == 1) {
      launch(final_sink());
      return hipSuccess;
    }
    return with_partials(outer * splits * inner, [&](const Sink<T>& partial) {
      launch(partial);
      const uint64_t ranges = (inner + kWave - 1) / kWave;
      auto combine = [&](auto kernel, uint64_t groups) {
        kernel<<<grid_for(outer * ((ranges + groups - 1) / groups)), kCombineThreads, 0,
                 guard.stream>>>(partial.values, partial.partial_indices, outer, splits, segment,
                                 inner, final_sink());
      };
      // Waves per column range P and batch B: the exact kernels when the
      // splits are a multiple of P x B (256 and 128 splits over wide rows,
      // 8 for C2's per-batch sums), tested loads otherwise.
      auto combine_all = [&](auto index) {
        constexpr bool INDEX = decltype(index)::value;
        if (splits >= 128) {
          if (splits % 256 == 0) {
            combine(combine_columns_kernel<T, K, 16, 16, true, INDEX>, 1);
          } else if (splits % 128 == 0) {
            combine(combine_columns_kernel<T, K, 16, 8, true, INDEX>, 1);
          } else {
            combine(combine_columns_kernel<T, K, 16, 16, false, INDEX>, 1);
          }
        } else if (splits >= 16) {
          if (splits % 32 == 0) {
            combine(combine_columns_kernel<T, K, 4, 8, true, INDEX>, 4);
          } else {
            combine(combine_columns_kernel<T, K, 4, 16, false, INDEX>, 4);
          }
        } else if (splits % 8 == 0) {
          combine(combine_columns_kernel<T, K, 1, 8, true, INDEX>, 16);
        } else {
          combine(combine_columns_kernel<T, K, 1, 16, false, INDEX>, 16);
        }
      };
      if constexpr (K == Kind::Max) {
        if (value_only) {
          combine_all(std::false_type{});
          return;
        }
      }
      combine_all(std::true_type{});
    }, value_only);
  }

  // Generic: one wave per output.
  const RowMap map = make_row_map(plan, plan.kept_rank);
  ReducedMap red{};
  red.rank = plan.red_rank;
  red.count = plan.reduced;
  for (int k = 0; k < plan.red_rank; ++k) {
    red.extents[k] = plan.red_extents[plan.red_rank - 1 - k];
    red.strides[k] = plan.red_strides[plan.red_rank - 1 - k];
  }
  generic_kernel<T, K, NIN><<<grid_for((plan.outputs + kWaves - 1) / kWaves), kThreads, 0,
                              guard.stream>>>(a, b, plan.outputs, map, red, final_sink());
  return hipSuccess;
}

template <typename T, int NIN>
hipError_t dispatch_plan(const Plan& plan, const void* a, const void* b, void* output,
                         int operation, int device, const DeviceGuard& guard,
                         const Workspace& workspace) {
  const T* ta = static_cast<const T*>(a);
  const T* tb = static_cast<const T*>(b);
  if (operation == SPAR_HIP_SUM || operation == SPAR_HIP_MEAN) {
    return run_plan<T, Kind::Sum, NIN>(plan, ta, tb, output, operation, device, guard,
                                       workspace);
  }
  return run_plan<T, Kind::Max, NIN>(plan, ta, tb, output, operation, device, guard, workspace);
}

// Builds a plan from a view and a reduced-axis mask.
Plan make_plan(uint64_t rank, const uint64_t* extents, const uint64_t* strides, uint64_t offset,
               uint32_t mask) {
  Plan plan;
  plan.offset = offset;
  for (uint64_t axis = 0; axis < rank; ++axis) {
    if ((mask >> axis) & 1U) {
      plan.red_extents[plan.red_rank] = extents[axis];
      plan.red_strides[plan.red_rank] = strides[axis];
      ++plan.red_rank;
      plan.reduced *= extents[axis];
    } else {
      plan.kept_extents[plan.kept_rank] = extents[axis];
      plan.kept_strides[plan.kept_rank] = strides[axis];
      ++plan.kept_rank;
      plan.outputs *= extents[axis];
    }
  }
  coalesce_list(plan.kept_rank, plan.kept_extents, plan.kept_strides);
  coalesce_list(plan.red_rank, plan.red_extents, plan.red_strides);
  return plan;
}

// Runs a plan on `device`'s stream.  `fixed_workspace`, when given, returns
// the device's fixed partial-result region (it is called with the device
// current) and no memory is allocated.
template <typename FixedWorkspace>
SparHipStatus execute_with(const Plan& plan, const void* a, const void* b, int nin, void* output,
                           int dtype, int operation, int device, FixedWorkspace&& fixed_workspace) {
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  Workspace workspace;
  if (const hipError_t error = fixed_workspace(workspace); error != hipSuccess) {
    return runtime(error);
  }
  hipError_t error;
  if (dtype == SPAR_HIP_FLOAT32) {
    error = nin == 1
                ? dispatch_plan<float, 1>(plan, a, b, output, operation, device, guard, workspace)
                : dispatch_plan<float, 2>(plan, a, b, output, operation, device, guard, workspace);
  } else {
    error = nin == 1
                ? dispatch_plan<double, 1>(plan, a, b, output, operation, device, guard, workspace)
                : dispatch_plan<double, 2>(plan, a, b, output, operation, device, guard, workspace);
  }
  if (workspace.exceeded) {
    return {SPAR_HIP_STATUS_WORKSPACE_EXCEEDED, static_cast<int>(hipErrorInvalidValue)};
  }
  if (error != hipSuccess) return runtime(error);
  return finish(guard);
}

SparHipStatus execute(const Plan& plan, const void* a, const void* b, int nin, void* output,
                      int dtype, int operation, int device) {
  return execute_with(plan, a, b, nin, output, dtype, operation, device,
                      [](Workspace&) { return hipSuccess; });
}

// Validates an axis reduction request and builds its plan.  Returns false
// with `status` set when the request is finished without a launch (an
// empty output, an empty reduced domain zero-filled) or invalid.
bool axis_reduction_plan(Plan& plan, SparHipStatus& status, void* output, const void* input,
                         uint64_t rank, const uint64_t* extents, const uint64_t* strides,
                         uint64_t storage_offset, uint32_t reduced_mask, int dtype, int operation,
                         int device);

bool valid_reduction(int operation) {
  return operation >= SPAR_HIP_SUM && operation <= SPAR_HIP_ARGMAX;
}

// Gradient view + mask for reducing a contiguous gradient to a right-aligned
// original shape: leading axes and axes where the original extent is 1 (and
// the gradient's is not) are reduced.
bool broadcast_plan(Plan& plan, uint64_t gradient_rank, const uint64_t* gradient_extents,
                    uint64_t original_rank, const uint64_t* original_extents) {
  if (gradient_rank > kMaxRank || original_rank > gradient_rank) return false;
  uint64_t strides[kMaxRank];
  uint64_t running = 1;
  for (uint64_t axis = gradient_rank; axis > 0; --axis) {
    strides[axis - 1] = running;
    running *= gradient_extents[axis - 1];
  }
  const uint64_t leading = gradient_rank - original_rank;
  uint32_t mask = 0;
  for (uint64_t axis = 0; axis < gradient_rank; ++axis) {
    if (axis < leading) {
      mask |= 1U << axis;
      continue;
    }
    const uint64_t original = original_extents[axis - leading];
    if (original == gradient_extents[axis]) continue;
    if (original != 1) return false;
    mask |= 1U << axis;
  }
  plan = make_plan(gradient_rank, gradient_extents, strides, 0, mask);
  return true;
}

}  // namespace
}  // namespace spar_hip

using namespace spar_hip;

extern "C" SparHipStatus spar_hip_launch_reduction(void* output, const void* input, uint64_t count,
                                                   int dtype, int operation, int device) {
  if (!valid_float_dtype(dtype) || !valid_reduction(operation) || output == nullptr ||
      (count != 0 && input == nullptr) || (operation != SPAR_HIP_SUM && count == 0)) {
    return invalid();
  }
  if (count == 0) {
    // sum of nothing is 0 (reduction.cpp:21-30)
    const uint64_t bytes = dtype == SPAR_HIP_FLOAT32 ? 4 : 8;
    return spar_hip_zero(output, bytes, device);
  }
  uint64_t extents[1] = {count};
  uint64_t strides[1] = {1};
  const Plan plan = make_plan(1, extents, strides, 0, 1U);
  return execute(plan, input, nullptr, 1, output, dtype, operation, device);
}

extern "C" SparHipStatus spar_hip_launch_row_reduction(void* output, const void* input,
                                                       uint64_t row_count,
                                                       uint64_t reduction_count, int dtype,
                                                       int operation, int device) {
  if (!valid_float_dtype(dtype) || !valid_reduction(operation) ||
      (row_count != 0 && output == nullptr) ||
      (row_count != 0 && reduction_count != 0 && input == nullptr) ||
      (operation != SPAR_HIP_SUM && reduction_count == 0)) {
    return invalid();
  }
  if (row_count == 0) return ok();
  if (reduction_count == 0) {
    const uint64_t bytes = row_count * (dtype == SPAR_HIP_FLOAT32 ? 4 : 8);
    return spar_hip_zero(output, bytes, device);
  }
  uint64_t extents[2] = {row_count, reduction_count};
  uint64_t strides[2] = {reduction_count, 1};
  const Plan plan = make_plan(2, extents, strides, 0, 2U);
  return execute(plan, input, nullptr, 1, output, dtype, operation, device);
}

namespace spar_hip {
namespace {

bool axis_reduction_plan(Plan& plan, SparHipStatus& status, void* output, const void* input,
                         uint64_t rank, const uint64_t* extents, const uint64_t* strides,
                         uint64_t storage_offset, uint32_t reduced_mask, int dtype, int operation,
                         int device) {
  if (!valid_float_dtype(dtype) || !valid_reduction(operation) || rank > kMaxRank ||
      (rank != 0 && (extents == nullptr || strides == nullptr)) ||
      (rank < 32 && (reduced_mask >> rank) != 0)) {
    status = invalid();
    return false;
  }
  uint64_t outputs = 1;
  uint64_t reduced = 1;
  for (uint64_t axis = 0; axis < rank; ++axis) {
    if ((reduced_mask >> axis) & 1U) {
      reduced *= extents[axis];
    } else {
      outputs *= extents[axis];
    }
  }
  if (outputs == 0) {
    status = ok();
    return false;
  }
  if (output == nullptr) {
    status = invalid();
    return false;
  }
  if (reduced == 0) {
    status = operation != SPAR_HIP_SUM
                 ? invalid()
                 : spar_hip_zero(output, outputs * (dtype == SPAR_HIP_FLOAT32 ? 4 : 8), device);
    return false;
  }
  if (input == nullptr) {
    status = invalid();
    return false;
  }
  plan = make_plan(rank, extents, strides, storage_offset, reduced_mask);
  return true;
}

// The no-allocation entry point's partial results: one fixed array per
// device, resident until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host it names a stand-in, not device memory):
// the first call on each device, with that device current, resolves the
// device's own address with hipGetSymbolAddress, and launches use that.
static __device__ __align__(256) unsigned char scratch[SPAR_HIP_NO_ALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxScratchDevices] = {};

hipError_t scratch_address(int device, void** address) {
  if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* resolved = nullptr;
    const hipError_t error = hipGetSymbolAddress(&resolved, HIP_SYMBOL(scratch));
    if (error != hipSuccess) return error;
    if (resolved == nullptr) return hipErrorInvalidSymbol;
    g_scratch_address[device] = resolved;
  }
  *address = g_scratch_address[device];
  return hipSuccess;
}

}  // namespace
}  // namespace spar_hip

extern "C" SparHipStatus spar_hip_launch_axis_reduction(void* output, const void* input,
                                                        uint64_t rank, const uint64_t* extents,
                                                        const uint64_t* strides,
                                                        uint64_t storage_offset,
                                                        uint32_t reduced_mask, int dtype,
                                                        int operation, int device) {
  Plan plan;
  SparHipStatus status{};
  if (!axis_reduction_plan(plan, status, output, input, rank, extents, strides, storage_offset,
                           reduced_mask, dtype, operation, device)) {
    return status;
  }
  return execute(plan, input, nullptr, 1, output, dtype, operation, device);
}

extern "C" SparHipStatus spar_hip_launch_axis_reduction_no_alloc(
    void* output, const void* input, uint64_t rank, const uint64_t* extents,
    const uint64_t* strides, uint64_t storage_offset, uint32_t reduced_mask, int dtype,
    int operation, int device) {
  Plan plan;
  SparHipStatus status{};
  if (!axis_reduction_plan(plan, status, output, input, rank, extents, strides, storage_offset,
                           reduced_mask, dtype, operation, device)) {
    return status;
  }
  return execute_with(plan, input, nullptr, 1, output, dtype, operation, device,
                      [device](Workspace& workspace) {
                        void* address = nullptr;
                        const hipError_t error = scratch_address(device, &address);
                        if (error != hipSuccess) return error;
                        workspace.fixed = address;
                        workspace.capacity = SPAR_HIP_NO_ALLOC_SCRATCH_BYTES;
                        return hipSuccess;
                      });
}

extern "C" SparHipStatus spar_hip_launch_broadcast_reduce(
    void* destination, const void* gradient, uint64_t gradient_rank,
    const uint64_t* gradient_extents, uint64_t original_rank, const uint64_t* original_extents,
    const uint64_t* original_strides, uint64_t count, int dtype, int device) {
  (void)original_strides;  // the destination is always contiguous
  if (!valid_float_dtype(dtype) || original_rank > gradient_rank ||
      gradient_rank > kMaxRank || (count != 0 && (destination == nullptr || gradient == nullptr)) ||
      (gradient_rank != 0 && gradient_extents == nullptr) ||
      (original_rank != 0 && original_extents == nullptr)) {
    return invalid();
  }
  uint64_t product = 1;
  for (uint64_t axis = 0; axis < gradient_rank; ++axis) product *= gradient_extents[axis];
  if (product != count) return invalid();
  uint64_t original_count = 1;
  for (uint64_t axis = 0; axis < original_rank; ++axis) original_count *= original_extents[axis];
  if (count == 0) {
    if (original_count == 0 || destination == nullptr) return ok();
    return spar_hip_zero(destination, original_count * (dtype == SPAR_HIP_FLOAT32 ? 4 : 8), device);
  }
  Plan plan;
  if (!broadcast_plan(plan, gradient_rank, gradient_extents, original_rank, original_extents)) {
    return invalid();
  }
  return execute(plan, gradient, nullptr, 1, destination, dtype, SPAR_HIP_SUM, device);
}

extern "C" SparHipStatus spar_hip_launch_multiply_reduce(
    void* destination, const void* gradient, const void* factor, uint64_t gradient_rank,
    const uint64_t* gradient_extents, uint64_t original_rank, const uint64_t* original_extents,
    uint64_t count, int dtype, int device) {
  if (!valid_float_dtype(dtype) || original_rank > gradient_rank || gradient_rank > kMaxRank ||
      (count != 0 && (destination == nullptr || gradient == nullptr || factor == nullptr)) ||
      (gradient_rank != 0 && gradient_extents == nullptr) ||
      (original_rank != 0 && original_extents == nullptr)) {
    return invalid();
  }
  uint64_t product = 1;
  for (uint64_t axis = 0; axis < gradient_rank; ++axis) product *= gradient_extents[axis];
  if (product != count) return invalid();
  uint64_t original_count = 1;
  for (uint64_t axis = 0; axis < original_rank; ++axis) original_count *= original_extents[axis];
  if (count == 0) {
    if (original_count == 0 || destination == nullptr) return ok();
    return spar_hip_zero(destination, original_count * (dtype == SPAR_HIP_FLOAT32 ? 4 : 8), device);
  }
  Plan plan;
  if (!broadcast_plan(plan, gradient_rank, gradient_extents, original_rank, original_extents)) {
    return invalid();
  }
  return execute(plan, gradient, factor, 2, destination, dtype, SPAR_HIP_SUM, device);
}
