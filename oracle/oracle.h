/*
 * CPU oracle for the affine group-wise weight-quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests, the smoke
 * check and the benchmark's CPU-baseline leg load it. The product library
 * (affon_amd/libaffon_rocm.so) never links, loads or calls it.
 *
 * It restates the reference's scalar CPU semantics. The reference kernel
 * itself (compute/src/backend/cpu/quantized_matmul.zig, an un-vendored path
 * dependency) is absent, so the restatement follows its documented contract:
 *   docs/core/quantized-inference.md:45-67   (packed format, affine formula)
 *   docs/core/quantized-inference.md:114-128 (scalar loop, ordered f32
 *                                             accumulation, bf16 widened)
 *   test/parity/fixtures/quantized_fixture.py:36-45 (peer formula)
 *   test/parity/reference/check-cuda-quantized-general.py:71-78 (f64 oracle)
 * Every function below names what pins it; see the header of qmm_oracle.c.
 */
#ifndef AFFON_ORACLE_H
#define AFFON_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F32 = 0, ORACLE_BF16 = 1 };

/* f32 -> bf16 round-to-nearest-even on the bit pattern
 * (test/parity/reference/probe-capabilities.py:112-115). NaN is kept quiet. */
uint16_t oracle_bf16_from_f32(float value);
float oracle_f32_from_bf16(uint16_t value);
void oracle_bf16_from_f32_array(const float* values, uint16_t* out, size_t count);

/* mulberry32 stream (src/js/compute/program.ts:1385-1394): next uniform in [0,1). */
double oracle_mulberry32_next(uint32_t* state);

/* Tensor.randn / initializedValue "normal" (src/js/compute/program.ts:339-345,1396-1422):
 * fills count values of mean + std * normal(), Box-Muller with a cached spare,
 * each double rounded to f32. When bf16_out is non-null it also receives
 * RNE_bf16 of each f32 value (src/js/compute/native.zig:1166). */
void oracle_randn(uint32_t seed, double mean, double std, size_t count, float* f32_out, uint16_t* bf16_out);

/* quantized_matmul, scalar and ordered: for each (m, n) an f32 accumulator
 * over k = 0..K-1 of x[m,k] * (s * q + b), every product and sum rounded
 * separately (no fused multiply-add). Contiguous row-major operands:
 * x [M,K], packed [N,K/P], scales/biases [N,K/g], out [M,N] f32.
 * Rows n in [n_begin, n_end) are computed (lets a caller split N across
 * threads for the multi-core CPU baseline). */
void oracle_quantized_matmul(const void* x, int x_dtype, const uint32_t* packed,
                             const void* scales, const void* biases, int param_dtype,
                             float* out, size_t M, size_t K, size_t N,
                             unsigned bits, size_t group_size, size_t n_begin, size_t n_end);

/* The same product evaluated in f64 (the reference checker's float64 oracle). */
void oracle_quantized_matmul_f64(const void* x, int x_dtype, const uint32_t* packed,
                                 const void* scales, const void* biases, int param_dtype,
                                 double* out, size_t M, size_t K, size_t N,
                                 unsigned bits, size_t group_size);

/* Affine group-wise quantize of a contiguous [N,K] f32 or bf16 matrix.
 * Build-defined contract (the reference has no quantize op):
 *   mn/mx = min/max of the group, scale = (mx - mn) / (2^bits - 1), bias = mn,
 *   both canonicalised (+0.0f added so -0 becomes +0) and stored in
 *   param_dtype (bf16: RNE); q = clamp(rint((w - bias_stored) / scale_stored),
 *   0, 2^bits - 1) with IEEE f32 division, q = 0 when scale_stored == 0.
 * Values are packed least-significant bits first (docs/core/quantized-inference.md:62). */
void oracle_quantize(const void* weights, int weight_dtype, size_t N, size_t K,
                     unsigned bits, size_t group_size, int param_dtype,
                     uint32_t* packed, void* scales, void* biases);

/* Dequantize: w[n,k] = s * q + b with separate f32 rounding of the product and
 * the sum (docs/core/quantized-inference.md:59-61), stored as out_dtype. */
void oracle_dequantize(const uint32_t* packed, const void* scales, const void* biases,
                       int param_dtype, size_t N, size_t K, unsigned bits, size_t group_size,
                       int out_dtype, void* out);

/* The CPU baseline (cpu_baseline.c): the same product as
 * oracle_quantized_matmul, bit for bit, in one specialised scalar loop per
 * bit width and dtype pair (docs/core/quantized-inference.md:114-128).
 * Returns 0, or 1 for arguments it does not take. */
int baseline_quantized_matmul(const void* x, int x_dtype, const uint32_t* packed, const void* scales,
                              const void* biases, int param_dtype, float* out, size_t M, size_t K, size_t N,
                              unsigned bits, size_t group_size, size_t n_begin, size_t n_end);

#ifdef __cplusplus
}
#endif
#endif
