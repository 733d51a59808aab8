/*
 * spar_hip.h — the C ABI of Spar's MI355X (gfx950) device backend.
 *
 * This header is the drop-in boundary that replaces Spar's CUDA launcher ABI
 * (src/backend/cuda_kernels.hpp:1-135) and the device runtime that core/storage
 * and core/tensor call (src/backend/cuda_runtime.cppm:14-36).  It is plain C:
 * raw pointers, 64-bit counts and integer tags, no C++ or torch types, so the
 * C++ host layer (or a ctypes/FFI binding) includes it in a global module
 * fragment exactly as src/backend/cuda_ops.cppm:1-5 includes cuda_kernels.hpp.
 *
 * Conventions shared by every entry point:
 *   - Status: {code, hip_error}.  code 0 = success, 1 = invalid argument
 *     (rejected on the host before any device API call), 2 = HIP runtime error
 *     (hip_error holds the hipError_t value).  Same meaning as SparCudaStatus
 *     (cuda_kernels.hpp:41-44, cuda_kernels.cu:12-22).
 *   - count == 0 returns success without touching the device, as the reference
 *     launchers do (e.g. cuda_kernels.cu:718-720).
 *   - Every launch is enqueued on the backend's single stream for `device`
 *     and returns without waiting.  Work is stream-ordered; host<->device
 *     copies and spar_hip_synchronize() are the synchronisation points.  The
 *     reference instead synchronised after every launch (cuda_kernels.cu:39-49).
 *   - Device pointers come from spar_hip_allocate (or any allocation visible to
 *     the device); element pointers must be aligned to their element size.
 *   - Strides and offsets are in elements, never bytes.
 *   - Geometry (extents/strides, rank <= SPAR_HIP_MAX_RANK) is passed to the
 *     kernels by value; no launcher allocates metadata on the device
 *     (the reference cudaMalloc'd it per call: cuda_kernels.cu:1165-1190).
 */
#ifndef SPAR_HIP_H
#define SPAR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPAR_HIP_MAX_RANK 8

/* Element types; values equal SparCudaDType (cuda_kernels.hpp:10-15). */
enum SparHipDType {
  SPAR_HIP_FLOAT32 = 0,
  SPAR_HIP_FLOAT64 = 1,
  SPAR_HIP_INT32 = 2,
  SPAR_HIP_INT64 = 3,
};

/* Binary operations.  0-3 equal SparCudaBinaryOp (cuda_kernels.hpp:17-22).
 * 4-9 are comparisons, which the reference does not have: they write 1 or 0
 * in the input dtype (there is no Bool dtype, src/core/dtype.cppm:8-13) and
 * follow IEEE-754 ordered comparison, so NaN compares unequal to everything. */
enum SparHipBinaryOp {
  SPAR_HIP_ADD = 0,
  SPAR_HIP_SUBTRACT = 1,
  SPAR_HIP_MULTIPLY = 2,
  SPAR_HIP_DIVIDE = 3,
  SPAR_HIP_EQUAL = 4,
  SPAR_HIP_NOT_EQUAL = 5,
  SPAR_HIP_LESS = 6,
  SPAR_HIP_LESS_EQUAL = 7,
  SPAR_HIP_GREATER = 8,
  SPAR_HIP_GREATER_EQUAL = 9,
};

/* Unary operations.  0-7 equal SparCudaUnaryOp (cuda_kernels.hpp:24-33).
 * TANH and GELU are additions: gelu(x) = 0.5 * x * erfc(-x * (1/sqrt(2))),
 * evaluated in double precision and rounded once to the element type.
 * GELU_DERIVATIVE (used by the gelu backward rule) is
 * 0.5 * erfc(-x / sqrt(2)) + x * exp(-x*x/2) / sqrt(2 pi), evaluated the same way. */
enum SparHipUnaryOp {
  SPAR_HIP_NEGATE = 0,
  SPAR_HIP_SQUARE = 1,
  SPAR_HIP_RECIPROCAL = 2,
  SPAR_HIP_EXP = 3,
  SPAR_HIP_LOG = 4,
  SPAR_HIP_SQRT = 5,
  SPAR_HIP_SIGMOID = 6,
  SPAR_HIP_SILU = 7,
  SPAR_HIP_TANH = 8,
  SPAR_HIP_GELU = 9,
  SPAR_HIP_GELU_DERIVATIVE = 10,
};

/* Reductions.  0-2 equal SparCudaReductionOp (cuda_kernels.hpp:35-39).
 * ARGMAX writes int64 indices.  MAX and ARGMAX share one rule: a NaN wins
 * (the first NaN in logical order), otherwise the first element equal to the
 * maximum wins, so max(-0.0, +0.0) is -0.0 when -0.0 comes first — the result
 * of the reference's sequential `value > result` scan (reduction.cpp:44-60). */
enum SparHipReductionOp {
  SPAR_HIP_SUM = 0,
  SPAR_HIP_MEAN = 1,
  SPAR_HIP_MAX = 2,
  SPAR_HIP_ARGMAX = 3,
};

/* Status code of spar_hip_launch_axis_reduction_no_alloc when the reduction
 * needs more partial-result memory than its fixed workspace holds; nothing
 * was enqueued.  (Codes 0-2 are listed at the top of this header.) */
#define SPAR_HIP_STATUS_WORKSPACE_EXCEEDED 3

/* Bytes of the fixed per-device workspace of
 * spar_hip_launch_axis_reduction_no_alloc (8 MiB). */
#define SPAR_HIP_NO_ALLOC_SCRATCH_BYTES (8u << 20)

/* Replaces struct SparCudaStatus (cuda_kernels.hpp:41-44). */
struct SparHipStatus {
  int code;
  int hip_error;
};

/* Allocator statistics for one device (no reference counterpart: the
 * reference called cudaMalloc/cudaFree per tensor, cuda_runtime.cppm:121-159). */
struct SparHipMemoryStats {
  uint64_t bytes_in_use;      /* bytes handed out and not yet returned      */
  uint64_t bytes_cached;      /* bytes held in free lists for reuse          */
  uint64_t bytes_reserved;    /* bytes obtained from hipMalloc in total      */
  uint64_t device_allocations;/* number of hipMalloc calls made              */
  uint64_t cache_hits;        /* allocations served from a free list         */
};

/* Summary of a gradient's sum of squares; replaces struct SparCudaNormSummary
 * (cuda_kernels.hpp:99-104), same fields and layout: the norm is
 * scale * sqrt(scaled_sum_squares) over the finite elements, with scale the
 * largest finite magnitude ({0, 1} when there is none), and the flags record
 * infinities and NaNs (training/gradients.cpp:27-97). */
struct SparHipNormSummary {
  double scale;
  double scaled_sum_squares;
  int has_infinity;
  int has_nan;
};

/* ---------------------------------------------------------------- runtime */

/* Number of visible HIP devices (replaces the cudaGetDeviceCount check in
 * spar::detail::cuda::validate_device, cuda_runtime.cppm:109-120). */
struct SparHipStatus spar_hip_device_count(int* count);

/* Compute units (CUs) of `device`, as the launchers size their grids and
 * split their reductions (256 on MI355X).  A reduction's partial results,
 * and so whether spar_hip_launch_axis_reduction_no_alloc can take it,
 * depend on this count.  No reference counterpart. */
struct SparHipStatus spar_hip_multiprocessor_count(int* count, int device);

/* Caching device allocator: size-classed free lists over hipMalloc, reuse is
 * stream-ordered on the backend's single stream.  Replaces cuda::allocate /
 * cuda::deallocate (cuda_runtime.cppm:121-159).  bytes == 0 yields NULL. */
struct SparHipStatus spar_hip_allocate(void** pointer, uint64_t bytes, int device);
struct SparHipStatus spar_hip_deallocate(void* pointer, int device);
/* Synchronises the device and returns every cached block to the driver. */
struct SparHipStatus spar_hip_empty_cache(int device);
struct SparHipStatus spar_hip_memory_stats(struct SparHipMemoryStats* stats, int device);

/* Zero-fill of device bytes with a fill kernel (cuda::zero,
 * cuda_runtime.cppm:161-174, used cudaMemset). */
struct SparHipStatus spar_hip_zero(void* destination, uint64_t bytes, int device);

/* Reads `bytes` (a multiple of 16, 16-byte aligned) with ordinary cached
 * loads; `sink` (4 bytes, may be NULL) is never written for real data.
 * Benchmarks call it on a buffer larger than the L2 and Infinity Cache to
 * evict and write back cached lines before a timed launch.  No reference
 * counterpart (Spar has no benchmarking support). */
struct SparHipStatus spar_hip_touch(const void* buffer, uint64_t bytes, void* sink, int device);

/* Copies (cuda_runtime.cppm:176-237).  Host<->device copies return after the
 * copy has completed (the host buffer may be reused at once); device-to-device
 * copies are stream-ordered.  Cross-device copies use hipMemcpyPeerAsync on the
 * destination's stream, ordered after the source stream's pending work, and
 * the source stream waits for the copy; the host does not wait (the reference
 * stages them through host memory, cuda_runtime.cppm:226-228). */
struct SparHipStatus spar_hip_copy_host_to_device(void* destination, const void* source,
                                                  uint64_t bytes, int device);
struct SparHipStatus spar_hip_copy_device_to_host(void* destination, const void* source,
                                                  uint64_t bytes, int device);
struct SparHipStatus spar_hip_copy_device_to_device(void* destination, int destination_device,
                                                    const void* source, int source_device,
                                                    uint64_t bytes);

/* Waits for all work enqueued on the backend's stream for `device`. */
struct SparHipStatus spar_hip_synchronize(int device);
/* Returns the backend's hipStream_t for `device` (for interoperation). */
struct SparHipStatus spar_hip_stream(void** stream, int device);

/* Event timing on the backend's stream (no reference counterpart; Spar has no
 * tracing).  Elapsed time is in milliseconds between two recorded events. */
struct SparHipStatus spar_hip_event_create(void** event);
struct SparHipStatus spar_hip_event_destroy(void* event);
struct SparHipStatus spar_hip_event_record(void* event, int device);
struct SparHipStatus spar_hip_event_elapsed(float* milliseconds, void* start, void* stop);

/* Replaces spar_cuda_error_string (cuda_kernels.hpp:129). */
const char* spar_hip_error_string(int hip_error);

/* ------------------------------------------------ contiguous elementwise */

/* output[i] = left[i] op right[i] over `count` contiguous elements.
 * Replaces spar_cuda_launch_binary (cuda_kernels.hpp:46-47); comparisons
 * (ops 4-9) are additions. */
struct SparHipStatus spar_hip_launch_binary(void* output, const void* left, const void* right,
                                            uint64_t count, int dtype, int operation, int device);

/* output[i] = input[i] op (T)scalar.  For float32 the double scalar is
 * rounded to float before the operation, as the CPU path does
 * (src/ops/scalar.cpp:40-47).  Replaces spar_cuda_launch_scalar
 * (cuda_kernels.hpp:48-49). */
struct SparHipStatus spar_hip_launch_scalar(void* output, const void* input, uint64_t count,
                                            int dtype, int operation, double scalar, int device);

/* output[i] = op(input[i]).  Replaces spar_cuda_launch_unary
 * (cuda_kernels.hpp:50-51); TANH and GELU are additions. */
struct SparHipStatus spar_hip_launch_unary(void* output, const void* input, uint64_t count,
                                           int dtype, int operation, int device);

/* output[i] = scalar[0] * (T)scale, with scalar a device pointer to one
 * element: the reference's semantics.  Replaces
 * spar_cuda_launch_fill_from_scalar (cuda_kernels.hpp:85-87,
 * cuda_kernels.cu:249-257, :1093-1118); its callers pass scale 1 for sum
 * backward and 1.0 / n for mean backward (src/ops/reduction.cpp:201-204,
 * :265-268). */
struct SparHipStatus spar_hip_launch_fill_from_scalar(void* output, const void* scalar,
                                                      uint64_t count, int dtype, double scale,
                                                      int device);

/* output[i] = scalar[0] / (T)divisor, divisor > 0.  The CPU path's mean
 * backward divides the gradient by (T)n (src/ops/reduction.cpp:263-277),
 * which differs in the last bit from multiplying by the rounded reciprocal;
 * this form reproduces the CPU bits.  No counterpart in the reference's
 * C ABI; the Tensor layer's sum/mean backward calls it. */
struct SparHipStatus spar_hip_launch_fill_from_scalar_divided(void* output, const void* scalar,
                                                              uint64_t count, int dtype,
                                                              double divisor, int device);

/* output[i] = (T)value for a host value (ones/full on the device,
 * src/core/tensor.cppm:168-178 staged these through the host). */
struct SparHipStatus spar_hip_launch_fill(void* output, uint64_t count, int dtype, double value,
                                          int device);

/* destination[i] += source[i].  Replaces spar_cuda_launch_add_in_place
 * (cuda_kernels.hpp:88-89). */
struct SparHipStatus spar_hip_launch_add_in_place(void* destination, const void* source,
                                                  uint64_t count, int dtype, int device);

/* ------------------------------------------------------- strided layouts */

/* Materialises a strided view (rank, extents, strides, storage_offset) into a
 * contiguous row-major destination.  element_size is 4 or 8.  Same arguments
 * as spar_cuda_launch_strided_copy (cuda_kernels.hpp:90-94); rank must be
 * <= SPAR_HIP_MAX_RANK. */
struct SparHipStatus spar_hip_launch_strided_copy(void* destination, const void* source,
                                                  uint64_t rank, const uint64_t* extents,
                                                  const uint64_t* strides,
                                                  uint64_t storage_offset, uint64_t count,
                                                  uint64_t element_size, int device);

/* Scatter: writes the contiguous `source` (rank, extents) into the strided
 * destination view (destination base, strides, storage_offset).  Used for
 * gradients of narrowed views and value copies into views (the reference's
 * copy_tensor_values, src/core/tensor.cpp:514-537, needed a contiguous
 * destination). */
struct SparHipStatus spar_hip_launch_strided_assign(void* destination, uint64_t rank,
                                                    const uint64_t* extents,
                                                    const uint64_t* strides,
                                                    uint64_t storage_offset, const void* source,
                                                    uint64_t element_size, int device);

/* The gradient of a narrowed view, scattered into a fresh tensor of the
 * base's shape in one pass: for the row-major output [outer, extent, inner]
 * and the contiguous window input [outer, length, inner] (the narrowed axis
 * has `extent` elements, the window starts at `start`),
 *   output[o][e][i] = start <= e < start + length ? input[o][e - start][i] : 0.
 * Elements are copied as bits (element_size 4 or 8).  No reference
 * counterpart: narrow is this library's addition to the view model, and its
 * backward would otherwise take a zero fill plus the window's strided copy,
 * writing the window twice.  Outputs up to 2^31 - 1 elements. */
struct SparHipStatus spar_hip_launch_window_embed(void* output, const void* input, uint64_t outer,
                                                  uint64_t extent, uint64_t inner, uint64_t start,
                                                  uint64_t length, uint64_t element_size,
                                                  int device);

/* The same for a box of several axes at once: output (contiguous, `rank`
 * extents) = zeros except the box starts[a] <= c[a] < starts[a] + lengths[a]
 * on every axis, which holds input (contiguous, extents `lengths`).  The
 * gradient of a chain of narrows in one pass; no reference counterpart.
 * With input NULL only the zeros are written and the box is left as it is
 * (the border of a gradient whose box a producer writes in place).
 * element_size 4 or 8; outputs of at most 2^31 - 1 elements; after dropping
 * axes of extent 1 and merging neighbouring whole axes, at most 4 axes.
 * Status 1 for other shapes and for an empty box (length 0 on some axis). */
struct SparHipStatus spar_hip_launch_box_embed(void* output, const void* input, int rank,
                                               const uint64_t* extents, const uint64_t* starts,
                                               const uint64_t* lengths, uint64_t element_size,
                                               int device);

/* Binary op over the broadcast shape `extents` (rank dims) without
 * materialising either operand: each operand is read through its own strides
 * (0 on broadcast axes) and storage offset; output is contiguous row-major.
 * Replaces the expand().contiguous() + binary chain of the reference
 * (src/ops/elementwise.cpp:26-31). */
struct SparHipStatus spar_hip_launch_strided_binary(void* output, const void* left,
                                                    const uint64_t* left_strides,
                                                    uint64_t left_offset, const void* right,
                                                    const uint64_t* right_strides,
                                                    uint64_t right_offset, uint64_t rank,
                                                    const uint64_t* extents, int dtype,
                                                    int operation, int device);

/* ------------------------------------------------------------ reductions */

/* Full reduction of `count` contiguous elements to one element (ARGMAX: one
 * int64).  Replaces spar_cuda_launch_reduction (cuda_kernels.hpp:52-53).  A
 * grid of partial reductions is combined by a second pass in a fixed order,
 * so results are deterministic.  MEAN/MAX/ARGMAX reject count == 0. */
struct SparHipStatus spar_hip_launch_reduction(void* output, const void* input, uint64_t count,
                                               int dtype, int operation, int device);

/* Reduces each of `row_count` contiguous rows of `reduction_count` elements.
 * Replaces spar_cuda_launch_row_reduction (cuda_kernels.hpp:54-56), which
 * accepted SUM/MEAN only; MAX and ARGMAX (int64 output) are additions. */
struct SparHipStatus spar_hip_launch_row_reduction(void* output, const void* input,
                                                   uint64_t row_count, uint64_t reduction_count,
                                                   int dtype, int operation, int device);

/* Axis reduction of a strided view without materialising it.  The input view
 * is (rank, extents, strides, storage_offset); reduced_mask bit k set means
 * axis k is reduced.  The output is the contiguous tensor of the kept axes in
 * order (keepdim only changes the shape, not the layout).  MEAN divides the
 * sum by (T)(product of the reduced extents).  ARGMAX writes int64 indices
 * into the flattened reduced sub-space (row-major over the reduced axes).
 * Replaces the permute().contiguous() + row_reduction chain
 * (src/ops/reduction.cpp:167-185). */
struct SparHipStatus spar_hip_launch_axis_reduction(void* output, const void* input,
                                                    uint64_t rank, const uint64_t* extents,
                                                    const uint64_t* strides,
                                                    uint64_t storage_offset,
                                                    uint32_t reduced_mask, int dtype,
                                                    int operation, int device);

/* spar_hip_launch_axis_reduction without any allocation: same arguments,
 * same kernels, same results bit for bit.  No counterpart in the reference;
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Split reductions keep their partial results in a fixed workspace of
 * SPAR_HIP_NO_ALLOC_SCRATCH_BYTES per device, a static device array held
 * until the process ends, instead of allocator scratch.  A reduction whose
 * partials do not fit (values rounded up to 256 bytes, plus 4 bytes per
 * partial for max/argmax indices) returns SPAR_HIP_STATUS_WORKSPACE_EXCEEDED
 * before anything is enqueued; on MI355X every [8192, 8192] float32 or
 * float64 reduction fits.  The partials are written before they are read,
 * so nothing needs clearing between calls.
 *
 * Every call on a device shares that device's workspace.  Calls issued from
 * one host thread are ordered on the backend stream and do not interfere;
 * calls that overlap on one device (several host threads, or captured work
 * replayed concurrently with other calls) race on it.  The first call on a
 * device resolves the workspace's address; the backend stream is created by
 * the first call of any entry point on the device. */
struct SparHipStatus spar_hip_launch_axis_reduction_no_alloc(
    void* output, const void* input, uint64_t rank, const uint64_t* extents,
    const uint64_t* strides, uint64_t storage_offset, uint32_t reduced_mask, int dtype,
    int operation, int device);

/* Sums a contiguous gradient of shape gradient_extents over its broadcast
 * axes into the contiguous original shape (right-aligned numpy rules).  The
 * destination is overwritten (the reference required a zeroed destination and
 * used atomicAdd, cuda_kernels.cu:287-311; this is deterministic).  Same
 * arguments as spar_cuda_launch_broadcast_reduce (cuda_kernels.hpp:95-98). */
struct SparHipStatus spar_hip_launch_broadcast_reduce(
    void* destination, const void* gradient, uint64_t gradient_rank,
    const uint64_t* gradient_extents, uint64_t original_rank, const uint64_t* original_extents,
    const uint64_t* original_strides, uint64_t count, int dtype, int device);

/* Fused broadcast_reduce of a product: destination = reduce_to_original(
 * gradient * factor) where gradient and factor are contiguous with
 * gradient_extents.  Each product is rounded to T before it is summed, exactly
 * like multiply() followed by reduce_gradient_to_shape() in the multiply
 * backward rule (src/ops/elementwise.cpp:159-166), but in one HBM pass. */
struct SparHipStatus spar_hip_launch_multiply_reduce(
    void* destination, const void* gradient, const void* factor, uint64_t gradient_rank,
    const uint64_t* gradient_extents, uint64_t original_rank, const uint64_t* original_extents,
    uint64_t count, int dtype, int device);

/* --------------------------------------------------------------- softmax */

/* Softmax (logarithmic = 0) or log-softmax (1) over slices (outer, axis,
 * inner) of a contiguous input, with the reference's special cases: a slice
 * with NaN or with only -inf becomes all NaN; k > 0 entries of +inf share the
 * mass (1/k, log: -log k) and the rest are 0 (log: -inf).  undefined_slices
 * (int32, outer*inner) is set to 1 for those slices.  Replaces
 * spar_cuda_launch_probability_forward (cuda_kernels.hpp:57-60). */
struct SparHipStatus spar_hip_launch_probability_forward(void* output, int32_t* undefined_slices,
                                                         const void* input, uint64_t outer,
                                                         uint64_t axis_extent, uint64_t inner,
                                                         int dtype, int logarithmic, int device);

/* Backward of the above: softmax dx = y * (g - sum(g*y)); log-softmax
 * dx = g - exp(lp) * sum(g); undefined slices become NaN.  Replaces
 * spar_cuda_launch_probability_backward (cuda_kernels.hpp:61-63). */
struct SparHipStatus spar_hip_launch_probability_backward(
    void* output, const void* gradient, const void* saved_output, const int32_t* undefined_slices,
    uint64_t outer, uint64_t axis_extent, uint64_t inner, int dtype, int logarithmic, int device);

/* ------------------------------------------------ fused row normalisation */

/* Largest row length the fused normalisation kernels accept for `dtype`
 * (16384 float32, 8192 float64; 0 for other dtypes).  Longer rows take the
 * composed ops.  No reference counterpart. */
uint64_t spar_hip_norm_max_extent(int dtype);

/* LayerNorm (center = 1) or RMSNorm (center = 0) over the last axis of a
 * [rows, extent] strided input, fused:
 *   LayerNorm: mu = sum(x)/n, xc = x - mu, d = sqrt(sum(xc*xc)/n + eps),
 *              y = (xc / d) * weight + bias
 *   RMSNorm:   d = sqrt(sum(x*x)/n + eps), y = (x / d) * weight
 * Element x[r][c] is input[r * input_row_stride + c * input_column_stride],
 * in one of two layouts:
 *   rows:    input_column_stride == 1 and input_row_stride >= extent (extent
 *            for a contiguous input, more for a block of a wider tensor);
 *   columns: input_row_stride == 1 and input_column_stride >= rows (the
 *            transpose of a row-major [extent, input_column_stride] block);
 *            a statistics pass and a tiled apply pass, no transposing copy.
 * Writes y [rows, extent] (contiguous), d [rows] and, for LayerNorm, mu
 * [rows] (`mean` and `bias` are ignored and may be NULL for RMSNorm).
 * Replaces the composed forward of RMSNorm, multiply(divide(x,
 * sqrt(add_scalar(mean(square(x), -1, true), eps))), weight)
 * (src/nn/rmsnorm.cpp:50-52), and the same chain with centring and a bias;
 * the reference has no fused kernel for it. */
struct SparHipStatus spar_hip_launch_norm_forward(void* output, void* mean, void* denominator,
                                                  const void* input, uint64_t input_row_stride,
                                                  uint64_t input_column_stride,
                                                  const void* weight, const void* bias,
                                                  uint64_t rows, uint64_t extent, double epsilon,
                                                  int center, int dtype, int device);

/* Backward of the above from the saved mu and d: writes dx, d weight
 * [extent] and, for LayerNorm, d bias [extent] (sums over rows in a fixed
 * order).  The input is in one of the forward's layouts, and dx is written
 * in the same one:
 *   - rows input_row_stride >= extent apart with a row's elements adjacent
 *     (input_column_stride 1): dx row p starts at
 *     input_gradient[p * input_gradient_stride], input_gradient_stride >=
 *     extent (extent: contiguous [rows, extent]; larger: a block of a wider
 *     tensor, such as the gradient of a narrowed view written in place);
 *   - rows adjacent (input_row_stride 1) with a row's elements
 *     input_column_stride >= rows apart: element (p, q) of dx at
 *     input_gradient[p + q * input_gradient_stride], input_gradient_stride >=
 *     rows (rows: a contiguous [extent, rows] block, whose transpose is the
 *     gradient of a transposed view).
 * output_gradient is contiguous [rows, extent] in both.  Replaces the
 * autograd backward of the composed chain. */
struct SparHipStatus spar_hip_launch_norm_backward(
    void* input_gradient, uint64_t input_gradient_stride, void* weight_gradient,
    void* bias_gradient, const void* output_gradient, const void* input,
    uint64_t input_row_stride, uint64_t input_column_stride, const void* weight,
    const void* mean, const void* denominator, uint64_t rows,
    uint64_t extent, int center, int dtype, int device);

/* The same backward with the output gradient given as a product: dy[i] =
 * output_gradient_scale[0] * output_gradient[i], output_gradient_scale one
 * element of `dtype` in device memory, each product formed in the kernels
 * with the single rounding (and operand order) of the multiply op.  This is
 * the gradient a product y * c hands y when c needs no gradient and the
 * product's own gradient is one value broadcast, as in loss = sum(y * c):
 * the reference's autograd materialises dy with a multiply kernel
 * (src/ops/elementwise.cpp:159-166, then K1 of cuda_kernels.cu) before the
 * normalisation's backward reads it; here no dy is written.  Returns status
 * 1 for a NULL scale with rows > 0. */
struct SparHipStatus spar_hip_launch_norm_backward_scaled(
    void* input_gradient, uint64_t input_gradient_stride, void* weight_gradient,
    void* bias_gradient, const void* output_gradient, const void* output_gradient_scale,
    const void* input, uint64_t input_row_stride, uint64_t input_column_stride,
    const void* weight, const void* mean, const void* denominator, uint64_t rows,
    uint64_t extent, int center, int dtype, int device);

/* --------------------------------------------- cross entropy (log-softmax + NLL) */

/* Sets *invalid_target (host memory) to 1 if any of `count` class indices
 * (target_dtype SPAR_HIP_INT32 or SPAR_HIP_INT64) is negative or >= classes,
 * else 0.  Synchronises.  Replaces spar_cuda_validate_targets
 * (cuda_kernels.hpp:105-107). */
struct SparHipStatus spar_hip_validate_targets(int32_t* invalid_target, const void* targets,
                                               uint64_t count, uint64_t classes,
                                               int target_dtype, int device);

/* output[i] = -log_probabilities[row(i) * classes + target(i)]: row(i) = i and
 * target(i) = targets[i], or for the language-model form (language_model = 1)
 * with sequences of sequence_length, i = b * (T-1) + t reads row b*T + t and
 * target targets[b*T + t + 1].  Replaces spar_cuda_launch_nll_forward
 * (cuda_kernels.hpp:108-112). */
struct SparHipStatus spar_hip_launch_nll_forward(void* output, const void* log_probabilities,
                                                 const void* targets, uint64_t output_count,
                                                 uint64_t classes, uint64_t sequence_length,
                                                 int dtype, int target_dtype, int language_model,
                                                 int device);

/* Scatter of the above's gradient into a zeroed [rows, classes] output:
 * output[row(i) * classes + target(i)] = 0 - gradient[i].  Replaces
 * spar_cuda_launch_nll_backward (cuda_kernels.hpp:113-117). */
struct SparHipStatus spar_hip_launch_nll_backward(void* output, const void* gradient,
                                                  const void* targets, uint64_t output_count,
                                                  uint64_t classes, uint64_t sequence_length,
                                                  int dtype, int target_dtype, int language_model,
                                                  int device);

/* Fused log_softmax -> NLL forward over logits [logits_rows, classes]:
 * losses (one per target, indexed as above) = -log_softmax(row)[target],
 * computed with log-softmax's operations; saves each row's maximum and
 * log of its exp-sum, and its undefined flag (log-softmax's special cases).
 * *invalid_target (device memory) is set to 1 if a target is out of range;
 * that target's loss is NaN and its logit is not read.  Replaces
 * log_softmax + select_nll_cuda in cross_entropy / language_model_cross_entropy
 * (cross_entropy.cpp:146-214) without materialising the log-probabilities;
 * the reference has no fused kernel. */
struct SparHipStatus spar_hip_launch_cross_entropy_forward(
    void* losses, void* row_max, void* row_log_sum, int32_t* undefined_rows,
    int32_t* invalid_target, const void* logits, const void* targets, uint64_t logits_rows,
    uint64_t classes, uint64_t sequence_length, int dtype, int target_dtype, int language_model,
    int device);

/* Its backward: logits_gradient = g - exp(lp) * g_t with g the NLL gradient
 * (g_t = 0 - loss_gradient at the target, zero elsewhere) and lp recomputed
 * from the saved row statistics -- the reference's nll_gradient followed by
 * log_softmax's backward (softmax.cpp:406-444), in one pass. */
struct SparHipStatus spar_hip_launch_cross_entropy_backward(
    void* logits_gradient, const void* loss_gradient, const void* logits, const void* row_max,
    const void* row_log_sum, const int32_t* undefined_rows, const void* targets,
    uint64_t logits_rows, uint64_t classes, uint64_t sequence_length, int dtype,
    int target_dtype, int language_model, int device);

/* ---------------------------------------------- optimizer and gradient norm */

/* Summary of `count` contiguous gradient elements (Float32 or Float64) into
 * *host_summary.  Synchronises.  The same function as the reference's
 * StableSumSquares over the elements up to rounding (the reference's own
 * CUDA kernel combines in another order than its CPU loop too).  Replaces
 * spar_cuda_gradient_norm_summary (cuda_kernels.hpp:118-120). */
struct SparHipStatus spar_hip_gradient_norm_summary(struct SparHipNormSummary* host_summary,
                                                    const void* gradient, uint64_t count,
                                                    int dtype, int device);

/* The same summary written to *summary in device memory on the device's
 * stream, without synchronising, so a caller can summarise many gradients and
 * read them back with one copy (no reference counterpart; the reference
 * synchronises per gradient, training/gradients.cpp:119). */
struct SparHipStatus spar_hip_launch_gradient_norm_summary(struct SparHipNormSummary* summary,
                                                           const void* gradient, uint64_t count,
                                                           int dtype, int device);

/* values[i] = (T)((double)values[i] * factor) in place; factor must be
 * finite.  Replaces spar_cuda_launch_scale_in_place (cuda_kernels.hpp:121-122). */
struct SparHipStatus spar_hip_launch_scale_in_place(void* values, uint64_t count, int dtype,
                                                    double factor, int device);

/* One AdamW step over `count` contiguous elements, in place on the parameter
 * and both moments, with the bias corrections 1 - beta^step supplied by the
 * caller: per element, in double, m = (T)(beta1 m + (1 - beta1) g),
 * v = (T)(beta2 v + (1 - beta2) g g), p = (T)(p (1 - lr wd) -
 * lr (m / c1) / (sqrt(v / c2) + eps)), each operation rounded as written
 * (optim/adamw.cpp:37-61), so results are the CPU path's bits.  Replaces
 * spar_cuda_launch_adamw (cuda_kernels.hpp:123-128). */
struct SparHipStatus spar_hip_launch_adamw(void* parameter, const void* gradient,
                                           void* first_moment, void* second_moment,
                                           uint64_t count, int dtype, double learning_rate,
                                           double beta1, double beta2, double epsilon,
                                           double weight_decay, double first_correction,
                                           double second_correction, int device);

/* ------------------------------------------------------ random generation */

/* Fills `count` contiguous elements with Spar's SplitMix64 stream for `seed`
 * (src/core/random.cpp:22-38): element i uses draw i of Random(seed).
 * UNIFORM: low + (high-low) * uniform (random.cpp:40-80).  The device result is
 * bit-identical to the host generator for float32 and float64. */
struct SparHipStatus spar_hip_random_uniform(void* output, uint64_t count, int dtype,
                                             uint64_t seed, double low, double high, int device);

/* Normal samples by the Box-Muller transform on uniform_double draws (the
 * reference has no normal sampler): pair k uses draws 2k and 2k+1,
 * r = sqrt(-2 log(1 - u0)), element 2k = mean + stddev * r * cos(2 pi u1),
 * element 2k+1 = mean + stddev * r * sin(2 pi u1), computed in double and
 * rounded to T.  Same definition as the host spar::random_normal; the device
 * log/sin/cos may differ from the host libm in the last bit of the double,
 * so values can differ from the host generator by one float32 ulp. */
struct SparHipStatus spar_hip_random_normal(void* output, uint64_t count, int dtype,
                                            uint64_t seed, double mean, double stddev,
                                            int device);

#ifdef __cplusplus
}
#endif

#endif /* SPAR_HIP_H */
