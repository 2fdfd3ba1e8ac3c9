/*
 * CPU oracle for quantize / dequantize / quantized_matmul.
 *
 * TEST INFRASTRUCTURE ONLY: the checker, never the product. Built by
 * oracle/Makefile with -ffp-contract=off so that every product and sum is
 * rounded separately, as the reference's scalar Zig kernel does in its default
 * strict float mode.
 *
 * What pins each function (the checks live in tests/test_oracle.py):
 *   oracle_quantized_matmul      every exact known-answer test of the reference
 *                                (test/e2e/program/operations/quantized-matmul.test.ts:7-204,
 *                                 src/support/compute_core_cyna_smoke.zig:970-984),
 *                                the closed form g*G*(G-1)/2 (quantized-matmul.test.ts:180),
 *                                an independent f64 brute force over little-endian bytes,
 *                                and the special cases bits=8,s=1,b=0 (integer matmul)
 *                                and g=K (y = s*(x.q) + b*sum(x)).
 *                                Bit-level agreement with the absent Zig kernel on
 *                                non-integer inputs is parity unpinned (its source is
 *                                not in the reference tree); parity there is by tolerance.
 *   oracle_quantized_matmul_f64  same checks in f64.
 *   oracle_bf16_from_f32         every upper half-word combined with the low halves that
 *                                decide rounding (ties, both sides, extremes) against the
 *                                reference's RNE formula (probe-capabilities.py:112-115),
 *                                and 300,000 values (random, subnormal, random bit patterns)
 *                                against torch's float32 -> bfloat16 conversion.
 *   oracle_randn / mulberry32    the uniform stream for six seeds against an independent
 *                                restatement of program.ts:1385-1394 with JS int32 semantics
 *                                written out (Math.imul, ToInt32); Box-Muller pairing and
 *                                moments. The f64 log/sin/cos come from libm here and from
 *                                V8 in the reference: bit-level agreement of every normal is
 *                                parity unpinned (a last-ulp f64 difference almost never
 *                                survives the rounding to f32).
 *   oracle_quantize              build-defined contract (no reference op exists):
 *                                invariants q in range, group min -> 0, group max -> 2^bits-1,
 *                                |dequant - w| <= scale/2 (+ bf16 parameter rounding),
 *                                constant groups, round-trip of already-quantized rows,
 *                                exact ties (w-b)/s = k + 1/2 to the even code, and
 *                                quotients near a tie that follow the division where
 *                                a reciprocal-multiply would round the other way.
 *   oracle_dequantize            the affine formula of docs/core/quantized-inference.md:59-61
 *                                on hand-built words with known nibbles.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

static inline uint32_t f32_bits(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float bits_f32(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* probe-capabilities.py:112-115: bits += 0x7fff + ((bits >> 16) & 1); keep the top half. */
uint16_t oracle_bf16_from_f32(float value) {
  uint32_t u = f32_bits(value);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oracle_f32_from_bf16(uint16_t value) { return bits_f32((uint32_t)value << 16); }

void oracle_bf16_from_f32_array(const float* values, uint16_t* out, size_t count) {
  for (size_t i = 0; i < count; ++i) out[i] = oracle_bf16_from_f32(values[i]);
}

static inline float load_value(const void* base, int dtype, size_t index) {
  if (dtype == ORACLE_BF16) return oracle_f32_from_bf16(((const uint16_t*)base)[index]);
  return ((const float*)base)[index];
}

static inline void store_value(void* base, int dtype, size_t index, float value) {
  if (dtype == ORACLE_BF16) ((uint16_t*)base)[index] = oracle_bf16_from_f32(value);
  else ((float*)base)[index] = value;
}

/* program.ts:1385-1394. JS performs the arithmetic on int32 / uint32 values;
 * uint32 wrapping arithmetic gives the same bits. */
double oracle_mulberry32_next(uint32_t* state) {
  *state += 0x6d2b79f5u;
  uint32_t next = *state;
  next = (next ^ (next >> 15)) * (next | 1u);
  next ^= next + (next ^ (next >> 7)) * (next | 61u);
  return (double)(next ^ (next >> 14)) / 4294967296.0;
}

/* program.ts:1396-1422: Box-Muller with a cached spare, cos first. */
void oracle_randn(uint32_t seed, double mean, double std, size_t count, float* f32_out, uint16_t* bf16_out) {
  uint32_t state = seed;
  int have_spare = 0;
  double spare = 0.0;
  const double two_pi = 2.0 * 3.141592653589793;
  for (size_t i = 0; i < count; ++i) {
    double normal;
    if (have_spare) {
      normal = spare;
      have_spare = 0;
    } else {
      double u1 = oracle_mulberry32_next(&state);
      double radius = sqrt(-2.0 * log(u1 > 2.220446049250313e-16 ? u1 : 2.220446049250313e-16));
      double angle = two_pi * oracle_mulberry32_next(&state);
      spare = radius * sin(angle);
      have_spare = 1;
      normal = radius * cos(angle);
    }
    float value = (float)(mean + std * normal);
    if (f32_out) f32_out[i] = value;
    if (bf16_out) bf16_out[i] = oracle_bf16_from_f32(value);
  }
}

static inline unsigned unpack(const uint32_t* row, size_t k, unsigned bits) {
  const unsigned per_word = 32u / bits;
  const uint32_t word = row[k / per_word];
  return (word >> ((k % per_word) * bits)) & ((1u << bits) - 1u);
}

void oracle_quantized_matmul(const void* x, int x_dtype, const uint32_t* packed,
                             const void* scales, const void* biases, int param_dtype,
                             float* out, size_t M, size_t K, size_t N,
                             unsigned bits, size_t group_size, size_t n_begin, size_t n_end) {
  const size_t words = K / (32u / bits);
  const size_t groups = K / group_size;
  for (size_t n = n_begin; n < n_end && n < N; ++n) {
    const uint32_t* row = packed + n * words;
    for (size_t m = 0; m < M; ++m) {
      float acc = 0.0f;
      for (size_t k = 0; k < K; ++k) {
        const size_t g = n * groups + k / group_size;
        const float s = load_value(scales, param_dtype, g);
        const float b = load_value(biases, param_dtype, g);
        const float q = (float)unpack(row, k, bits);
        const float w = s * q + b;
        acc += load_value(x, x_dtype, m * K + k) * w;
      }
      out[m * N + n] = acc;
    }
  }
}

void oracle_quantized_matmul_f64(const void* x, int x_dtype, const uint32_t* packed,
                                 const void* scales, const void* biases, int param_dtype,
                                 double* out, size_t M, size_t K, size_t N,
                                 unsigned bits, size_t group_size) {
  const size_t words = K / (32u / bits);
  const size_t groups = K / group_size;
  for (size_t n = 0; n < N; ++n) {
    const uint32_t* row = packed + n * words;
    for (size_t m = 0; m < M; ++m) {
      double acc = 0.0;
      for (size_t k = 0; k < K; ++k) {
        const size_t g = n * groups + k / group_size;
        const double w = (double)load_value(scales, param_dtype, g) * (double)unpack(row, k, bits) +
                         (double)load_value(biases, param_dtype, g);
        acc += (double)load_value(x, x_dtype, m * K + k) * w;
      }
      out[m * N + n] = acc;
    }
  }
}

void oracle_quantize(const void* weights, int weight_dtype, size_t N, size_t K,
                     unsigned bits, size_t group_size, int param_dtype,
                     uint32_t* packed, void* scales, void* biases) {
  const unsigned per_word = 32u / bits;
  const unsigned max_q = (1u << bits) - 1u;
  const size_t words = K / per_word;
  const size_t groups = K / group_size;
  memset(packed, 0, N * words * sizeof(uint32_t));
  for (size_t n = 0; n < N; ++n) {
    for (size_t g = 0; g < groups; ++g) {
      const size_t k0 = g * group_size;
      float mn = load_value(weights, weight_dtype, n * K + k0);
      float mx = mn;
      for (size_t k = k0 + 1; k < k0 + group_size; ++k) {
        const float v = load_value(weights, weight_dtype, n * K + k);
        mn = v < mn ? v : mn;
        mx = v > mx ? v : mx;
      }
      const float scale = (mx - mn) / (float)max_q + 0.0f;
      const float bias = mn + 0.0f;
      store_value(scales, param_dtype, n * groups + g, scale);
      store_value(biases, param_dtype, n * groups + g, bias);
      const float s = load_value(scales, param_dtype, n * groups + g);
      const float b = load_value(biases, param_dtype, n * groups + g);
      for (size_t k = k0; k < k0 + group_size; ++k) {
        unsigned q = 0;
        if (s != 0.0f) {
          float r = rintf((load_value(weights, weight_dtype, n * K + k) - b) / s);
          if (!(r >= 0.0f)) r = 0.0f;
          if (r > (float)max_q) r = (float)max_q;
          q = (unsigned)r;
        }
        packed[n * words + k / per_word] |= (uint32_t)q << ((k % per_word) * bits);
      }
    }
  }
}

void oracle_dequantize(const uint32_t* packed, const void* scales, const void* biases,
                       int param_dtype, size_t N, size_t K, unsigned bits, size_t group_size,
                       int out_dtype, void* out) {
  const size_t words = K / (32u / bits);
  const size_t groups = K / group_size;
  for (size_t n = 0; n < N; ++n) {
    for (size_t k = 0; k < K; ++k) {
      const size_t g = n * groups + k / group_size;
      const float s = load_value(scales, param_dtype, g);
      const float b = load_value(biases, param_dtype, g);
      const float w = s * (float)unpack(packed + n * words, k, bits) + b;
      store_value(out, out_dtype, n * K + k, w);
    }
  }
}
