/*
 * CPU baseline: the reference's scalar CPU quantized_matmul as its
 * documentation describes it (docs/core/quantized-inference.md:114-128):
 * one specialised scalar loop per bit width and dtype pair, the packed word
 * decoded inside the dot product, ordered f32 accumulation, bf16 widened to
 * f32, no weight cache, no SIMD, no threads of its own.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py times it as the CPU path beside the GPU
 * (single-threaded like the reference, AFFON_CPU_THREADS=1 at
 * src/config.zig:70-74, and split over output rows on all host cores), and
 * tests/test_oracle.py checks it. The product library never links it.
 *
 * Arithmetic per (m, n): for each k in order, w = s*q + b then acc += x*w,
 * every product and sum rounded separately (built with -ffp-contract=off),
 * which is the rounding sequence of oracle_quantized_matmul. So the two agree
 * bit for bit (checked on every bit width, dtype pair and a crossing-word
 * group). What differs is only the loop structure: scale and bias are loaded
 * once per group, the word index and lane shift come from shifts and masks
 * (P = 32/bits is a power of two), and no dtype or bit-width test sits in the
 * inner loop.
 */
#include "oracle.h"

#include <string.h>

static inline float widen_bf16(uint16_t v) {
  uint32_t u = (uint32_t)v << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

#define LOAD_F32(p, i) (((const float*)(p))[i])
#define LOAD_BF16(p, i) widen_bf16(((const uint16_t*)(p))[i])

/* One specialised loop: BITS fixed, LOADX / LOADP the activation and
 * parameter loads. Groups are walked in order; inside a group each k takes
 * its code from word k >> LOG_P at lane (k & (P-1)). */
#define DEFINE_LOOP(NAME, BITS, LOG_P, LOADX, LOADP)                                                      \
  static void NAME(const void* x, const uint32_t* packed, const void* scales, const void* biases,       \
                   float* out, size_t M, size_t K, size_t N, size_t group, size_t n_begin, size_t n_end) { \
    const size_t words = K >> (LOG_P);                                                                   \
    const size_t groups = K / group;                                                                     \
    const uint32_t mask = (1u << (BITS)) - 1u;                                                           \
    for (size_t n = n_begin; n < n_end; ++n) {                                                           \
      const uint32_t* row = packed + n * words;                                                          \
      const size_t prow = n * groups;                                                                    \
      for (size_t m = 0; m < M; ++m) {                                                                   \
        const size_t xrow = m * K;                                                                       \
        float acc = 0.0f;                                                                                \
        size_t k = 0;                                                                                    \
        for (size_t g = 0; g < groups; ++g) {                                                            \
          const float s = LOADP(scales, prow + g);                                                       \
          const float b = LOADP(biases, prow + g);                                                       \
          const size_t end = k + group;                                                                  \
          for (; k < end; ++k) {                                                                         \
            const uint32_t word = row[k >> (LOG_P)];                                                     \
            const float q = (float)((word >> ((k & ((1u << (LOG_P)) - 1u)) * (BITS))) & mask);           \
            const float w = s * q + b;                                                                   \
            acc += LOADX(x, xrow + k) * w;                                                               \
          }                                                                                              \
        }                                                                                                \
        out[m * N + n] = acc;                                                                            \
      }                                                                                                  \
    }                                                                                                    \
  }

#define DEFINE_BITS(BITS, LOG_P)                                                 \
  DEFINE_LOOP(loop_##BITS##_ff, BITS, LOG_P, LOAD_F32, LOAD_F32)                 \
  DEFINE_LOOP(loop_##BITS##_fb, BITS, LOG_P, LOAD_F32, LOAD_BF16)                \
  DEFINE_LOOP(loop_##BITS##_bf, BITS, LOG_P, LOAD_BF16, LOAD_F32)                \
  DEFINE_LOOP(loop_##BITS##_bb, BITS, LOG_P, LOAD_BF16, LOAD_BF16)

DEFINE_BITS(2, 4)
DEFINE_BITS(4, 3)
DEFINE_BITS(8, 2)

typedef void (*loop_fn)(const void*, const uint32_t*, const void*, const void*, float*, size_t, size_t, size_t,
                        size_t, size_t, size_t);

int baseline_quantized_matmul(const void* x, int x_dtype, const uint32_t* packed, const void* scales,
                              const void* biases, int param_dtype, float* out, size_t M, size_t K, size_t N,
                              unsigned bits, size_t group_size, size_t n_begin, size_t n_end) {
  static const loop_fn loops[3][4] = {
      {loop_2_ff, loop_2_fb, loop_2_bf, loop_2_bb},
      {loop_4_ff, loop_4_fb, loop_4_bf, loop_4_bb},
      {loop_8_ff, loop_8_fb, loop_8_bf, loop_8_bb},
  };
  const int b = bits == 2 ? 0 : bits == 4 ? 1 : bits == 8 ? 2 : -1;
  if (b < 0 || group_size == 0 || K % group_size != 0 || K % (32u / bits) != 0) return 1;
  if (n_end > N) n_end = N;
  loops[b][2 * (x_dtype == ORACLE_BF16) + (param_dtype == ORACLE_BF16)](x, packed, scales, biases, out, M, K, N,
                                                                         group_size, n_begin, n_end);
  return 0;
}
