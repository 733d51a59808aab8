// Host-side view geometry for the strided kernels: dimension coalescing and
// the checks that select a vectorised or tiled kernel.
#pragma once

#include <stdint.h>

#include "common.hpp"

namespace spar_hip {

// Up to two operands that share one logical shape (`extents`); each has its
// own strides and storage offset (elements).  The output is contiguous.
struct MultiView {
  int rank = 0;
  int operands = 1;
  uint64_t extents[kMaxRank] = {};
  uint64_t strides[2][kMaxRank] = {};
  uint64_t offsets[2] = {};
};

inline uint64_t view_numel(const MultiView& view) {
  uint64_t count = 1;
  for (int axis = 0; axis < view.rank; ++axis) count *= view.extents[axis];
  return count;
}

// Removes extent-1 axes and merges neighbours (a, a+1) whenever every operand
// satisfies stride[a] == stride[a+1] * extent[a+1]; the logical row-major
// order of elements is unchanged, so the output stays contiguous.
inline void coalesce(MultiView& view) {
  MultiView out;
  out.operands = view.operands;
  out.offsets[0] = view.offsets[0];
  out.offsets[1] = view.offsets[1];
  for (int axis = 0; axis < view.rank; ++axis) {
    if (view.extents[axis] == 1) continue;
    if (out.rank > 0) {
      const int last = out.rank - 1;
      bool mergeable = true;
      for (int op = 0; op < view.operands; ++op) {
        if (out.strides[op][last] != view.strides[op][axis] * view.extents[axis]) mergeable = false;
      }
      if (mergeable) {
        out.extents[last] *= view.extents[axis];
        for (int op = 0; op < view.operands; ++op) out.strides[op][last] = view.strides[op][axis];
        continue;
      }
    }
    out.extents[out.rank] = view.extents[axis];
    for (int op = 0; op < view.operands; ++op) out.strides[op][out.rank] = view.strides[op][axis];
    ++out.rank;
  }
  if (out.rank == 0) {  // a single element
    out.rank = 1;
    out.extents[0] = 1;
    for (int op = 0; op < view.operands; ++op) out.strides[op][0] = 1;
  }
  view = out;
}

// Largest storage index any operand can touch, plus one.
inline uint64_t view_span(const MultiView& view, int op) {
  uint64_t last = view.offsets[op];
  for (int axis = 0; axis < view.rank; ++axis) {
    last += (view.extents[axis] - 1) * view.strides[op][axis];
  }
  return last + 1;
}

// Geometry passed to kernels: extents as fast divisors (innermost first) and
// per-operand strides, in the coalesced rank.
struct KernelGeometry {
  int rank;
  FastDiv divisors[kMaxRank];     // divisors[k] divides by extent of axis rank-1-k
  uint64_t extents[kMaxRank];     // innermost first
  uint64_t strides[2][kMaxRank];  // innermost first
  uint64_t offsets[2];
};

inline KernelGeometry kernel_geometry(const MultiView& view) {
  KernelGeometry g{};
  g.rank = view.rank;
  for (int k = 0; k < view.rank; ++k) {
    const int axis = view.rank - 1 - k;
    g.extents[k] = view.extents[axis];
    g.divisors[k].init(static_cast<uint32_t>(view.extents[axis] > 0xFFFFFFFFull
                                                  ? 1
                                                  : view.extents[axis]));
    for (int op = 0; op < view.operands; ++op) g.strides[op][k] = view.strides[op][axis];
  }
  g.offsets[0] = view.offsets[0];
  g.offsets[1] = view.offsets[1];
  return g;
}

}  // namespace spar_hip
