// Optimizer-side kernels: the AdamW update, the scaled sum-of-squares summary
// behind the global gradient norm, and in-place gradient scaling.
//
// Replaces kernels K16-K18 of src/backend/cuda_kernels.cu (gradient_norm_kernel
// :390-424, scale_in_place_kernel :426-433, adamw_kernel :435-455) behind the
// same entry points (cuda_kernels.hpp:118-128).  All three are HBM-bound
// streams; the arithmetic is IEEE double exactly as the reference's CPU loops
// write it (optim/adamw.cpp:50-60, training/gradients.cpp:107-111), so the
// updated values are the CPU path's bits.
//
// Design for CDNA4:
//  * AdamW and scaling read and write 16-byte vectors per lane in tiles of
//    consecutive vectors, the layout of the elementwise kernels.  AdamW
//    moves 28 bytes per fp32 element (four reads, three writes) and spends
//    about 70 fp64 operations on it (two IEEE divides, one correctly rounded
//    square root): on MI355X that is under half of the fp64 rate at the HBM
//    bound, so the update stays memory-bound without approximating a divide.
//  * The norm summary reads the gradient once across the whole chip (the
//    reference runs one 256-thread block).  Each lane keeps a power-of-two
//    scaled sum of squares: for fp32 input every square is exact in double
//    and no sum of them can overflow, so the scale exponent stays 0; for fp64
//    input the exponent tracks the largest element so far and rescaling is an
//    exact ldexp rather than the reference's division per element.  A lane
//    whose sum turns out non-finite saw an infinity or NaN and re-reads its
//    own elements with the reference's per-element classification, so the
//    common case carries no per-element flag work.  Block partials are
//    combined in a fixed order by one block, so the result is deterministic.
#include <hip/hip_runtime.h>

#include <math.h>

#include "common.hpp"

namespace spar_hip {
namespace {

constexpr int kThreads = 256;
// Streaming kernels use single-wave workgroups (see elementwise.hip).
constexpr int kVectorThreads = 64;
constexpr uint64_t kMaxGrid = uint64_t{1} << 20;

uint32_t tile_grid(uint64_t vectors) {
  uint64_t blocks = (vectors + kVectorThreads - 1) / kVectorThreads;
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

// ------------------------------------------------------------------ AdamW

// Per-launch constants of one AdamW step.  `one_minus_beta*` and
// `decay_factor` (1 - lr * weight_decay) are the values the reference forms
// per element and per call; forming them once gives the same doubles.
struct AdamwStep {
  double learning_rate;
  double beta1;
  double beta2;
  double epsilon;
  double first_correction;
  double second_correction;
  double one_minus_beta1;
  double one_minus_beta2;
  double decay_factor;
};

// optim/adamw.cpp:50-60 for one element.  The moments are rounded to T when
// stored and read back before the bias correction, as the reference's loop
// does; every operation is a separately rounded IEEE double operation (the
// library is compiled without contraction).
template <typename T>
__device__ __forceinline__ void adamw_element(T& parameter, T gradient, T& first, T& second,
                                              const AdamwStep& s) {
  const double g = static_cast<double>(gradient);
  first = static_cast<T>(s.beta1 * static_cast<double>(first) + s.one_minus_beta1 * g);
  second = static_cast<T>(s.beta2 * static_cast<double>(second) + s.one_minus_beta2 * g * g);
  const double corrected_first = static_cast<double>(first) / s.first_correction;
  const double corrected_second = static_cast<double>(second) / s.second_correction;
  const double decayed = static_cast<double>(parameter) * s.decay_factor;
  parameter = static_cast<T>(decayed - s.learning_rate * corrected_first /
                                           (sqrt(corrected_second) + s.epsilon));
}

// Each workgroup updates a tile of 2 x 256 16-byte vectors of every array,
// issuing all eight loads of a lane (grouped by array) before its first
// store.  Measured on MI355X over 124M fp32 elements: two vectors per lane
// beat one (5.90 vs 5.76 TB/s) and four (5.47); a variant with the same
// traffic and no arithmetic runs no faster, so the double math is hidden.
constexpr int kAdamwUnroll = 2;

template <typename T, bool NT>
__global__ void __launch_bounds__(kVectorThreads)
    adamw_vec_kernel(T* parameter, const T* gradient, T* first, T* second, uint64_t count,
                     AdamwStep step) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  constexpr int U = kAdamwUnroll;
  const uint64_t vectors = count / W;
  V* p_v = reinterpret_cast<V*>(parameter);
  const V* g_v = reinterpret_cast<const V*>(gradient);
  V* m_v = reinterpret_cast<V*>(first);
  V* s_v = reinterpret_cast<V*>(second);
  const uint64_t tile = static_cast<uint64_t>(kVectorThreads) * U;
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile + threadIdx.x; base < vectors;
       base += static_cast<uint64_t>(gridDim.x) * tile) {
    V p[U], g[U], m[U], s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads;
      if (i < vectors) p[u] = stream_load(p_v + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads;
      if (i < vectors) g[u] = stream_load(g_v + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads;
      if (i < vectors) m[u] = stream_load(m_v + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads;
      if (i < vectors) s[u] = stream_load(s_v + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kVectorThreads;
      if (i >= vectors) continue;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        T pk = vec_get<T>(p[u], k), mk = vec_get<T>(m[u], k), sk = vec_get<T>(s[u], k);
        adamw_element(pk, vec_get<T>(g[u], k), mk, sk, step);
        vec_set<T>(p[u], k, pk);
        vec_set<T>(m[u], k, mk);
        vec_set<T>(s[u], k, sk);
      }
      store_vector<NT>(m_v + i, m[u]);
      store_vector<NT>(s_v + i, s[u]);
      store_vector<NT>(p_v + i, p[u]);
    }
  }
  if (blockIdx.x == 0) {
    const uint64_t i = vectors * W + threadIdx.x;
    if (i < count) adamw_element(parameter[i], gradient[i], first[i], second[i], step);
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads)
    adamw_scalar_kernel(T* parameter, const T* gradient, T* first, T* second, uint64_t count,
                        AdamwStep step) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride) {
    adamw_element(parameter[i], gradient[i], first[i], second[i], step);
  }
}

template <typename T>
void launch_adamw(T* parameter, const T* gradient, T* first, T* second, uint64_t count,
                  const AdamwStep& step, const DeviceGuard& guard) {
  if (aligned16(parameter) && aligned16(gradient) && aligned16(first) && aligned16(second)) {
    const uint64_t vectors = count / Vec16<T>::width;
    with_policy(stream_output(3 * count * sizeof(T)), [&](auto nt) {
      adamw_vec_kernel<T, decltype(nt)::value>
          <<<tile_grid((vectors + kAdamwUnroll - 1) / kAdamwUnroll), kVectorThreads, 0,
             guard.stream>>>(
              parameter, gradient, first, second, count, step);
    });
  } else {
    adamw_scalar_kernel<T><<<scalar_grid(count, guard), kThreads, 0, guard.stream>>>(
        parameter, gradient, first, second, count, step);
  }
}

// ---------------------------------------------------------------- scaling

// training/gradients.cpp:107-111: v = (T)((double)v * factor).
template <typename T>
__device__ __forceinline__ T scaled(T value, double factor) {
  return static_cast<T>(static_cast<double>(value) * factor);
}

template <typename T, bool NT>
__global__ void __launch_bounds__(kVectorThreads)
    scale_vec_kernel(T* values, uint64_t count, double factor) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  const uint64_t vectors = count / W;
  V* v_v = reinterpret_cast<V*>(values);
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kVectorThreads + threadIdx.x;
       i < vectors; i += static_cast<uint64_t>(gridDim.x) * kVectorThreads) {
    V v = stream_load(v_v + i);
#pragma unroll
    for (int k = 0; k < W; ++k) vec_set<T>(v, k, scaled(vec_get<T>(v, k), factor));
    store_vector<NT>(v_v + i, v);
  }
  if (blockIdx.x == 0) {
    const uint64_t i = vectors * W + threadIdx.x;
    if (i < count) values[i] = scaled(values[i], factor);
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads)
    scale_scalar_kernel(T* values, uint64_t count, double factor) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride) {
    values[i] = scaled(values[i], factor);
  }
}

template <typename T>
void launch_scale(T* values, uint64_t count, double factor, const DeviceGuard& guard) {
  if (aligned16(values)) {
    with_policy(stream_output(count * sizeof(T)), [&](auto nt) {
      scale_vec_kernel<T, decltype(nt)::value>
          <<<tile_grid(count / Vec16<T>::width), kVectorThreads, 0, guard.stream>>>(values, count,
                                                                                    factor);
    });
  } else {
    scale_scalar_kernel<T><<<scalar_grid(count, guard), kThreads, 0, guard.stream>>>(
        values, count, factor);
  }
}

// ----------------------------------------------------------- norm summary

// Exponent of a sum that holds no element yet: below every double's, so it
// never wins a max, and rescaling by it flushes only zeros.
constexpr int kNoExponent = -4096;

// Sum of squares of finite elements held as sum * 2^(2 * exponent), plus the
// largest finite magnitude and the infinity / NaN flags.
struct NormPartial {
  double sum;
  double maximum;
  int32_t exponent;
  int32_t flags;  // bit 0: an infinity was seen, bit 1: a NaN was seen
};

__device__ __forceinline__ NormPartial empty_partial() {
  return NormPartial{0.0, 0.0, kNoExponent, 0};
}

__device__ __forceinline__ NormPartial merge(NormPartial a, const NormPartial& b) {
  const int32_t e = a.exponent > b.exponent ? a.exponent : b.exponent;
  a.sum = ldexp(a.sum, 2 * (a.exponent - e)) + ldexp(b.sum, 2 * (b.exponent - e));
  a.exponent = e;
  a.maximum = fmax(a.maximum, b.maximum);
  a.flags |= b.flags;
  return a;
}

// One element into a lane's partial.  CAREFUL applies the reference's
// classification (gradients.cpp:30-40): infinities and NaNs set their flags
// and are left out of the sum and maximum.  The fast form omits it; a
// non-finite element then makes the lane's sum non-finite, which sends the
// lane to the careful form.
template <bool CAREFUL>
__device__ __forceinline__ void accumulate(NormPartial& p, float x) {
  // Squares of floats are exact in double and a sum of at most 2^64 of them
  // stays below 2^320: the exponent stays 0 and no rescaling is needed.
  float a = fabsf(x);
  if constexpr (CAREFUL) {
    if (x != x) p.flags |= 2;
    if (a == __builtin_huge_valf()) p.flags |= 1;
    if (!(a < __builtin_huge_valf())) a = 0.0f;
  }
  const double d = static_cast<double>(a);
  p.sum = fma(d, d, p.sum);
  p.maximum = fmax(p.maximum, d);
}

template <bool CAREFUL>
__device__ __forceinline__ void accumulate(NormPartial& p, double x) {
  double a = fabs(x);
  if constexpr (CAREFUL) {
    if (x != x) p.flags |= 2;
    if (a == __builtin_huge_val()) p.flags |= 1;
    if (!(a < __builtin_huge_val())) a = 0.0;
  }
  // v_frexp_exp: a = m * 2^e with m in [0.5, 1) for finite nonzero a.
  const int e = a == 0.0 ? kNoExponent : __builtin_amdgcn_frexp_exp(a);
  const int32_t top = p.exponent > e ? p.exponent : e;
  const double t = ldexp(a, -top);
  p.sum = fma(t, t, ldexp(p.sum, 2 * (p.exponent - top)));
  p.exponent = top;
  p.maximum = fmax(p.maximum, a);
}

// One lane's elements of [begin, end): 16-byte vectors strided by the block,
// two in flight (with the many short segments below, deeper unrolling
// measured no faster).
template <typename T, bool CAREFUL>
__device__ __forceinline__ NormPartial lane_summary(const T* gradient, uint64_t begin,
                                                    uint64_t end) {
  using V = typename Vec16<T>::type;
  constexpr int W = Vec16<T>::width;
  NormPartial p = empty_partial();
  if constexpr (sizeof(T) == 4) p.exponent = 0;
  const V* g_v = reinterpret_cast<const V*>(gradient);
  const uint64_t step = kThreads;
  uint64_t i = begin / W + threadIdx.x;
  const uint64_t stop = end / W;
  for (; i + step < stop; i += 2 * step) {
    const V v0 = stream_load(g_v + i);
    const V v1 = stream_load(g_v + i + step);
#pragma unroll
    for (int k = 0; k < W; ++k) accumulate<CAREFUL>(p, vec_get<T>(v0, k));
#pragma unroll
    for (int k = 0; k < W; ++k) accumulate<CAREFUL>(p, vec_get<T>(v1, k));
  }
  for (; i < stop; i += step) {
    const V v = stream_load(g_v + i);
#pragma unroll
    for (int k = 0; k < W; ++k) accumulate<CAREFUL>(p, vec_get<T>(v, k));
  }
  return p;
}

__device__ __forceinline__ NormPartial wave_merge(NormPartial p) {
#pragma unroll
  for (int lane_mask = kWave / 2; lane_mask > 0; lane_mask >>= 1) {
    NormPartial other;
    other.sum = __shfl_xor(p.sum, lane_mask, kWave);
    other.maximum = __shfl_xor(p.maximum, lane_mask, kWave);
    other.exponent = __shfl_xor(p.exponent, lane_mask, kWave);
    other.flags = __shfl_xor(p.flags, lane_mask, kWave);
    p = merge(p, other);
  }
  return p;
}

// Block partials as separate arrays, so that the combine reads them coalesced.
struct PartialArrays {
  double* sum;
  double* maximum;
  int32_t* exponent;
  int32_t* flags;
};

// Block b summarises elements [b * segment, min((b + 1) * segment, count))
// (segments are multiples of the vector width; the unaligned tail of the last
// vector goes to block 0's first lanes) into partial b.
template <typename T>
__global__ void __launch_bounds__(kThreads)
    norm_partial_kernel(PartialArrays partials, const T* gradient, uint64_t count,
                        uint64_t segment) {
  constexpr int W = Vec16<T>::width;
  const uint64_t body = count / W * W;
  const uint64_t begin = static_cast<uint64_t>(blockIdx.x) * segment;
  const uint64_t end = begin + segment < body ? begin + segment : body;
  NormPartial p = empty_partial();
  if (begin < end) {
    p = lane_summary<T, false>(gradient, begin, end);
    if (!(p.sum < __builtin_huge_val())) p = lane_summary<T, true>(gradient, begin, end);
  }
  if (blockIdx.x == 0 && body + threadIdx.x < count) {
    NormPartial q = empty_partial();
    if constexpr (sizeof(T) == 4) q.exponent = 0;
    accumulate<true>(q, gradient[body + threadIdx.x]);
    p = merge(p, q);
  }
  p = wave_merge(p);
  __shared__ NormPartial waves[kThreads / kWave];
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) waves[wave] = p;
  __syncthreads();
  if (threadIdx.x == 0) {
    NormPartial total = waves[0];
#pragma unroll
    for (int w = 1; w < kThreads / kWave; ++w) total = merge(total, waves[w]);
    partials.sum[blockIdx.x] = total.sum;
    partials.maximum[blockIdx.x] = total.maximum;
    partials.exponent[blockIdx.x] = total.exponent;
    partials.flags[blockIdx.x] = total.flags;
  }
}

constexpr int kCombineThreads = 1024;
constexpr int kCombineWaves = kCombineThreads / kWave;
constexpr int kCombineBatch = 16;

// Combines `parts` partials in a fixed order and writes the summary in the
// reference's form (SparCudaNormSummary): scale = the largest finite
// magnitude, scaled_sum_squares = sum of (x / scale)^2; {0, 1} when no finite
// nonzero element was seen, as the reference's initial state.  RESCALE (fp64
// partials): two passes, the common exponent, maximum and flags first, then
// every partial's sum rescaled to that exponent, so neither pass is a chain
// of dependent merges.  fp32 partials all have exponent 0 (or hold nothing),
// so the rescale is the identity and one pass adds the same values in the
// same order: the same bits, one round trip to the partials instead of two.
template <bool RESCALE>
__global__ void __launch_bounds__(kCombineThreads)
    norm_combine_kernel(SparHipNormSummary* summary, PartialArrays partials, uint64_t parts) {
  __shared__ int32_t wave_top[kCombineWaves];
  __shared__ int32_t wave_flags[kCombineWaves];
  __shared__ double wave_maximum[kCombineWaves];
  __shared__ double wave_total[kCombineWaves];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  // fp32 partials that hold elements all have exponent 0, so theirs is 0
  int32_t top = RESCALE ? kNoExponent : 0;
  int32_t flags = 0;
  double maximum = 0.0;
  double sum = 0.0;
  // The partials come from every XCD: each batch issues all of a thread's
  // loads before using any, so a pass costs about one round trip.
  for (uint64_t base = threadIdx.x; base < parts; base += kCombineThreads * kCombineBatch) {
    int32_t e[kCombineBatch], f[kCombineBatch];
    double m[kCombineBatch];
    double v[RESCALE ? 1 : kCombineBatch];
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      const uint64_t i = base + static_cast<uint64_t>(k) * kCombineThreads;
      const bool in = i < parts;
      if constexpr (RESCALE) e[k] = in ? partials.exponent[i] : kNoExponent;
      m[k] = in ? partials.maximum[i] : 0.0;
      f[k] = in ? partials.flags[i] : 0;
      if constexpr (!RESCALE) v[k] = in ? partials.sum[i] : 0.0;
    }
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      if constexpr (RESCALE) top = max(top, e[k]);
      maximum = fmax(maximum, m[k]);
      flags |= f[k];
      if constexpr (!RESCALE) sum += v[k];
    }
  }
#pragma unroll
  for (int lane_mask = kWave / 2; lane_mask > 0; lane_mask >>= 1) {
    top = max(top, __shfl_xor(top, lane_mask, kWave));
    maximum = fmax(maximum, __shfl_xor(maximum, lane_mask, kWave));
    flags |= __shfl_xor(flags, lane_mask, kWave);
  }
  if (lane == 0) {
    wave_top[wave] = top;
    wave_maximum[wave] = maximum;
    wave_flags[wave] = flags;
  }
  __syncthreads();
  top = wave_top[0];
  maximum = wave_maximum[0];
  flags = wave_flags[0];
#pragma unroll
  for (int w = 1; w < kCombineWaves; ++w) {
    top = max(top, wave_top[w]);
    maximum = fmax(maximum, wave_maximum[w]);
    flags |= wave_flags[w];
  }
  if constexpr (RESCALE) {
    for (uint64_t base = threadIdx.x; base < parts; base += kCombineThreads * kCombineBatch) {
      int32_t e[kCombineBatch];
      double v[kCombineBatch];
#pragma unroll
      for (int k = 0; k < kCombineBatch; ++k) {
        const uint64_t i = base + static_cast<uint64_t>(k) * kCombineThreads;
        const bool in = i < parts;
        e[k] = in ? partials.exponent[i] : top;
        v[k] = in ? partials.sum[i] : 0.0;
      }
#pragma unroll
      for (int k = 0; k < kCombineBatch; ++k) sum += ldexp(v[k], 2 * (e[k] - top));
    }
  }
  sum = wave_sum(sum);
  if (lane == 0) wave_total[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    double total = wave_total[0];
#pragma unroll
    for (int w = 1; w < kCombineWaves; ++w) total += wave_total[w];
    SparHipNormSummary out;
    if (maximum == 0.0) {
      out.scale = 0.0;
      out.scaled_sum_squares = 1.0;
    } else {
      // maximum = r * 2^top with r in [0.5, 1) for fp64 input (top = 0 for
      // fp32); sum * 2^(2 top) / maximum^2 = sum / r^2.
      const double r = ldexp(maximum, -top);
      out.scale = maximum;
      out.scaled_sum_squares = total / r / r;
    }
    out.has_infinity = flags & 1;
    out.has_nan = (flags >> 1) & 1;
    *summary = out;
  }
}

template <typename T>
hipError_t launch_norm_summary(SparHipNormSummary* device_summary, const T* gradient,
                               uint64_t count, int device, const DeviceGuard& guard) {
  constexpr int W = Vec16<T>::width;
  const uint64_t body = count / W * W;
  // Segments of at least four vectors per lane and up to 64 blocks per CU:
  // over 124M fp32 elements 16384 short segments read at 6.7 TB/s where
  // 2048 long ones reach 6.1 TB/s.
  const uint64_t min_segment = static_cast<uint64_t>(kThreads) * W * 4;
  const uint64_t max_blocks = static_cast<uint64_t>(guard.multiprocessors) * 64;
  uint64_t blocks = (body + min_segment - 1) / min_segment;
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks == 0) blocks = 1;
  uint64_t segment = (body + blocks - 1) / blocks;
  segment = (segment + W - 1) / W * W;
  if (segment == 0) segment = W;
  blocks = body == 0 ? 1 : (body + segment - 1) / segment;
  void* scratch = nullptr;
  hipError_t error = scratch_allocate(&scratch, blocks * 24, device);
  if (error != hipSuccess) return error;
  char* bytes = static_cast<char*>(scratch);
  PartialArrays partials{reinterpret_cast<double*>(bytes),
                         reinterpret_cast<double*>(bytes + 8 * blocks),
                         reinterpret_cast<int32_t*>(bytes + 16 * blocks),
                         reinterpret_cast<int32_t*>(bytes + 20 * blocks)};
  norm_partial_kernel<T><<<static_cast<uint32_t>(blocks), kThreads, 0, guard.stream>>>(
      partials, gradient, count, segment);
  norm_combine_kernel<(sizeof(T) > 4)>
      <<<1, kCombineThreads, 0, guard.stream>>>(device_summary, partials, blocks);
  scratch_release(scratch, device);  // stream-ordered reuse
  return hipGetLastError();
}

}  // namespace
}  // namespace spar_hip

using namespace spar_hip;

extern "C" SparHipStatus spar_hip_launch_adamw(void* parameter, const void* gradient,
                                               void* first_moment, void* second_moment,
                                               uint64_t count, int dtype, double learning_rate,
                                               double beta1, double beta2, double epsilon,
                                               double weight_decay, double first_correction,
                                               double second_correction, int device) {
  if (!valid_float_dtype(dtype) ||
      (count != 0 && (parameter == nullptr || gradient == nullptr || first_moment == nullptr ||
                      second_moment == nullptr))) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  AdamwStep step;
  step.learning_rate = learning_rate;
  step.beta1 = beta1;
  step.beta2 = beta2;
  step.epsilon = epsilon;
  step.first_correction = first_correction;
  step.second_correction = second_correction;
  step.one_minus_beta1 = 1.0 - beta1;
  step.one_minus_beta2 = 1.0 - beta2;
  step.decay_factor = 1.0 - learning_rate * weight_decay;
  if (dtype == SPAR_HIP_FLOAT32) {
    launch_adamw(static_cast<float*>(parameter), static_cast<const float*>(gradient),
                 static_cast<float*>(first_moment), static_cast<float*>(second_moment), count,
                 step, guard);
  } else {
    launch_adamw(static_cast<double*>(parameter), static_cast<const double*>(gradient),
                 static_cast<double*>(first_moment), static_cast<double*>(second_moment), count,
                 step, guard);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_scale_in_place(void* values, uint64_t count, int dtype,
                                                        double factor, int device) {
  if (!valid_float_dtype(dtype) || !isfinite(factor) || (count != 0 && values == nullptr)) {
    return invalid();
  }
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (dtype == SPAR_HIP_FLOAT32) {
    launch_scale(static_cast<float*>(values), count, factor, guard);
  } else {
    launch_scale(static_cast<double*>(values), count, factor, guard);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_launch_gradient_norm_summary(SparHipNormSummary* summary,
                                                               const void* gradient,
                                                               uint64_t count, int dtype,
                                                               int device) {
  if (summary == nullptr || !valid_float_dtype(dtype) || (count != 0 && gradient == nullptr)) {
    return invalid();
  }
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  if (count == 0) {
    norm_combine_kernel<true><<<1, kCombineThreads, 0, guard.stream>>>(
        summary, PartialArrays{nullptr, nullptr, nullptr, nullptr}, 0);
    return finish(guard);
  }
  const hipError_t error =
      dtype == SPAR_HIP_FLOAT32
          ? launch_norm_summary(summary, static_cast<const float*>(gradient), count, device, guard)
          : launch_norm_summary(summary, static_cast<const double*>(gradient), count, device,
                                guard);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_gradient_norm_summary(SparHipNormSummary* host_summary,
                                                        const void* gradient, uint64_t count,
                                                        int dtype, int device) {
  if (host_summary == nullptr || !valid_float_dtype(dtype) ||
      (count != 0 && gradient == nullptr)) {
    return invalid();
  }
  *host_summary = SparHipNormSummary{0.0, 1.0, 0, 0};
  if (count == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  void* scratch = nullptr;
  hipError_t error = scratch_allocate(&scratch, sizeof(SparHipNormSummary), device);
  if (error != hipSuccess) return runtime(error);
  SparHipNormSummary* device_summary = static_cast<SparHipNormSummary*>(scratch);
  error = dtype == SPAR_HIP_FLOAT32
              ? launch_norm_summary(device_summary, static_cast<const float*>(gradient), count,
                                    device, guard)
              : launch_norm_summary(device_summary, static_cast<const double*>(gradient), count,
                                    device, guard);
  SparHipStatus status = error == hipSuccess ? ok() : runtime(error);
  if (status.code == 0) {
    status = spar_hip_copy_device_to_host(host_summary, device_summary,
                                          sizeof(SparHipNormSummary), device);
  }
  scratch_release(scratch, device);
  return status;
}
