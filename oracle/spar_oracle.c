/*
 * spar_oracle.c — CPU restatement of Spar's CPU path for the elementwise,
 * broadcast and reduction ops.  TEST INFRASTRUCTURE ONLY: it is the reference
 * that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare
 * the HIP backend against.  Nothing in spar_amd/ links or calls it.
 *
 * Each loop follows the reference loop it cites (paths relative to the
 * reference's src/), in the same element order and with the same fp32 (or
 * fp64) operations, so results are the reference algorithm's bits.  Build
 * flags: gcc -O2 -ffp-contract=off, no -march=native (x86-64 baseline, SSE
 * arithmetic, no FMA), as the reference's own CPU build would compute.
 *
 * Views are (base pointer, rank, extents, strides, offset) in elements, with
 * logical row-major indexing exactly as Tensor::logical_storage_index
 * (core/tensor.cpp:405-415).
 *
 * Functions for ops the reference lacks (tanh, gelu, compare, axis max,
 * argmax) implement the semantics this backend defines for them; their
 * headers say "build-defined".
 */
#include "spar_oracle.h"

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* core/tensor.cpp:405-415 */
static uint64_t logical_storage_index(uint64_t logical, uint64_t rank, const uint64_t* extents,
                                      const uint64_t* strides, uint64_t offset) {
  uint64_t storage = offset;
  for (uint64_t index = rank; index > 0; --index) {
    const uint64_t axis = index - 1;
    const uint64_t extent = extents[axis];
    const uint64_t coordinate = logical % extent;
    logical /= extent;
    storage += coordinate * strides[axis];
  }
  return storage;
}

static uint64_t numel_of(uint64_t rank, const uint64_t* extents) {
  uint64_t count = 1;
  for (uint64_t axis = 0; axis < rank; ++axis) count *= extents[axis];
  return count;
}

/* ------------------------------------------------------------- random */

/* core/random.cpp:22-28 */
uint64_t spar_oracle_next_u64(uint64_t* state) {
  *state += 0x9E3779B97F4A7C15ULL;
  uint64_t value = *state;
  value = (value ^ (value >> 30U)) * 0xBF58476D1CE4E5B9ULL;
  value = (value ^ (value >> 27U)) * 0x94D049BB133111EBULL;
  return value ^ (value >> 31U);
}

/* core/random.cpp:30-33 */
float spar_oracle_uniform_float(uint64_t* state) {
  return (float)(spar_oracle_next_u64(state) >> 40U) / 16777216.0F;
}

/* core/random.cpp:35-38 */
double spar_oracle_uniform_double(uint64_t* state) {
  return (double)(spar_oracle_next_u64(state) >> 11U) / 9007199254740992.0;
}

/* core/random.cpp:58-65 (Float32 branch of random_uniform) */
void spar_oracle_random_uniform_f32(float* out, uint64_t count, uint64_t* state, double low,
                                    double high) {
  const float low_value = (float)low;
  const float width = (float)(high - low);
  for (uint64_t i = 0; i < count; ++i) out[i] = low_value + width * spar_oracle_uniform_float(state);
}

/* core/random.cpp:66-71 (Float64 branch of random_uniform) */
void spar_oracle_random_uniform_f64(double* out, uint64_t count, uint64_t* state, double low,
                                    double high) {
  const double width = high - low;
  for (uint64_t i = 0; i < count; ++i) out[i] = low + width * spar_oracle_uniform_double(state);
}

/* Build-defined normal sampler (the reference has none): Box-Muller on
 * consecutive uniform_double draws, element 2k from cos, 2k+1 from sin. */
#define SPAR_TWO_PI 6.283185307179586476925286766559
void spar_oracle_random_normal_f32(float* out, uint64_t count, uint64_t* state, double mean,
                                   double stddev) {
  for (uint64_t k = 0; 2 * k < count; ++k) {
    const double u0 = spar_oracle_uniform_double(state);
    const double u1 = spar_oracle_uniform_double(state);
    const double radius = sqrt(-2.0 * log(1.0 - u0));
    const double angle = SPAR_TWO_PI * u1;
    out[2 * k] = (float)(mean + stddev * (radius * cos(angle)));
    if (2 * k + 1 < count) out[2 * k + 1] = (float)(mean + stddev * (radius * sin(angle)));
  }
}

void spar_oracle_random_normal_f64(double* out, uint64_t count, uint64_t* state, double mean,
                                   double stddev) {
  for (uint64_t k = 0; 2 * k < count; ++k) {
    const double u0 = spar_oracle_uniform_double(state);
    const double u1 = spar_oracle_uniform_double(state);
    const double radius = sqrt(-2.0 * log(1.0 - u0));
    const double angle = SPAR_TWO_PI * u1;
    out[2 * k] = mean + stddev * (radius * cos(angle));
    if (2 * k + 1 < count) out[2 * k + 1] = mean + stddev * (radius * sin(angle));
  }
}

/* ------------------------------------------------------------ layouts */

/* optim/adamw.cpp:48-49 */
double spar_oracle_adamw_correction(double beta, uint64_t step) {
  return 1.0 - pow(beta, (double)step);
}

/* Tensor::materialize_cpu_logical (core/tensor.cpp:142-167), by payload size. */
void spar_oracle_strided_copy(void* out, const void* base, uint64_t element_size, uint64_t rank,
                              const uint64_t* extents, const uint64_t* strides, uint64_t offset) {
  const uint64_t count = numel_of(rank, extents);
  for (uint64_t i = 0; i < count; ++i) {
    const uint64_t s = logical_storage_index(i, rank, extents, strides, offset);
    memcpy((char*)out + i * element_size, (const char*)base + s * element_size, element_size);
  }
}

/* ------------------------------------------------- per-type functions */

#define SPAR_ORACLE_TYPE float
#define SPAR_ORACLE_SUFFIX f32
#define SPAR_EXP expf
#define SPAR_LOG logf
#define SPAR_SQRT sqrtf
#define SPAR_TANH tanhf
#include "spar_oracle_typed.inc"
#undef SPAR_ORACLE_TYPE
#undef SPAR_ORACLE_SUFFIX
#undef SPAR_EXP
#undef SPAR_LOG
#undef SPAR_SQRT
#undef SPAR_TANH

#define SPAR_ORACLE_TYPE double
#define SPAR_ORACLE_SUFFIX f64
#define SPAR_EXP exp
#define SPAR_LOG log
#define SPAR_SQRT sqrt
#define SPAR_TANH tanh
#include "spar_oracle_typed.inc"
