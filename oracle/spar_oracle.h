/*
 * spar_oracle.h — CPU restatement of Spar's CPU path (see spar_oracle.c).
 * TEST INFRASTRUCTURE ONLY: used by tests/, smoke() and bench.py's CPU
 * baseline as the reference results are compared with; the product never
 * links it.
 */
#ifndef SPAR_ORACLE_H
#define SPAR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint64_t spar_oracle_next_u64(uint64_t* state);
float spar_oracle_uniform_float(uint64_t* state);
double spar_oracle_uniform_double(uint64_t* state);
void spar_oracle_random_uniform_f32(float* out, uint64_t count, uint64_t* state, double low, double high);
void spar_oracle_random_uniform_f64(double* out, uint64_t count, uint64_t* state, double low, double high);
void spar_oracle_random_normal_f32(float* out, uint64_t count, uint64_t* state, double mean, double stddev);
void spar_oracle_random_normal_f64(double* out, uint64_t count, uint64_t* state, double mean, double stddev);
/* 1 - beta^step, the AdamW bias correction (optim/adamw.cpp:48-49). */
double spar_oracle_adamw_correction(double beta, uint64_t step);
void spar_oracle_strided_copy(void* out, const void* base, uint64_t element_size, uint64_t rank,
                              const uint64_t* extents, const uint64_t* strides, uint64_t offset);

#define SPAR_ORACLE_DECLARE(T, S)                                                                  \
  void spar_oracle_binary_##S(T* out, const T* a, const uint64_t* a_strides, uint64_t a_offset,   \
                              const T* b, const uint64_t* b_strides, uint64_t b_offset,           \
                              uint64_t rank, const uint64_t* extents, int op);                    \
  void spar_oracle_scalar_##S(T* out, const T* in, uint64_t count, int op, double value);         \
  void spar_oracle_unary_##S(T* out, const T* in, uint64_t count, int op);                        \
  T spar_oracle_sum_##S(const T* base, uint64_t rank, const uint64_t* extents,                    \
                        const uint64_t* strides, uint64_t offset);                                \
  T spar_oracle_mean_##S(const T* base, uint64_t rank, const uint64_t* extents,                   \
                         const uint64_t* strides, uint64_t offset);                               \
  T spar_oracle_max_##S(const T* base, uint64_t rank, const uint64_t* extents,                    \
                        const uint64_t* strides, uint64_t offset);                                \
  void spar_oracle_axis_sum_##S(T* out, uint64_t out_count, const T* base, uint64_t rank,         \
                                const uint64_t* extents, const uint64_t* strides,                 \
                                uint64_t offset, uint32_t mask);                                  \
  void spar_oracle_axis_max_##S(T* out, int64_t* indices, uint64_t out_count, const T* base,      \
                                uint64_t rank, const uint64_t* extents, const uint64_t* strides,  \
                                uint64_t offset, uint32_t mask, unsigned char* scratch);          \
  void spar_oracle_reduce_gradient_##S(T* out, const T* base, uint64_t rank,                      \
                                       const uint64_t* extents, const uint64_t* strides,          \
                                       uint64_t offset, uint64_t original_rank,                   \
                                       const uint64_t* original_extents);                         \
  void spar_oracle_add_in_place_##S(T* destination, const T* source, uint64_t count);             \
  void spar_oracle_fill_##S(T* out, uint64_t count, T value);                                     \
  void spar_oracle_softmax_axis_##S(T* out, unsigned char* undefined, const T* base,              \
                                    uint64_t rank, const uint64_t* extents,                       \
                                    const uint64_t* strides, uint64_t offset, uint64_t axis);     \
  void spar_oracle_softmax_full_##S(T* out, const T* in, uint64_t count);                         \
  int spar_oracle_softmax_full_undefined_##S(const T* in, uint64_t count);                        \
  void spar_oracle_softmax_axis_backward_##S(T* out, const T* gradient, const T* output,          \
                                             const unsigned char* undefined, uint64_t rank,       \
                                             const uint64_t* extents, uint64_t axis);             \
  void spar_oracle_softmax_full_backward_##S(T* out, const T* gradient, const T* output,          \
                                             uint64_t count, int undefined_derivative);           \
  void spar_oracle_log_softmax_##S(T* out, unsigned char* undefined, const T* base,               \
                                   uint64_t rank, const uint64_t* extents,                        \
                                   const uint64_t* strides, uint64_t offset, int64_t axis);       \
  void spar_oracle_log_softmax_backward_##S(T* out, const T* gradient,                            \
                                            const T* log_probabilities,                           \
                                            const unsigned char* undefined, uint64_t outer,       \
                                            uint64_t axis_extent, uint64_t inner);

SPAR_ORACLE_DECLARE(float, f32)
SPAR_ORACLE_DECLARE(double, f64)

#undef SPAR_ORACLE_DECLARE

#ifdef __cplusplus
}
#endif

#endif
