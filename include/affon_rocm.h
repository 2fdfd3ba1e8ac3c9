/*
 * affon_rocm.h — C ABI of the MI355X (gfx950) weight-quantized linear path.
 *
 * This library is the `rocm` device backend for Affon's `quantized_matmul`
 * operation plus the quantize / dequantize kernels that produce and expand its
 * packed format. Every entry point is plain C: pointers, sizes and status codes.
 *
 * Packed format (docs/core/quantized-inference.md:45-67): logical weight [N,K]
 * row-major, P = 32/bits values per u32 word, first value in the least
 * significant bits; scales and biases [N, K/group_size] (f32 or bf16);
 * weight[n,k] = scales[n,k/g] * q + biases[n,k/g].
 *
 * Status codes follow the reference C ABI convention
 * (src/support/compute_core_cyna.zig:1041-1043): 0 ok, 1 invalid shape, any
 * other value a core failure. This library refines "other" into 2 (core
 * failure), 3 (unsupported: e.g. no gfx950 device, or a forced implementation
 * that cannot run the shape) and 4 (HIP runtime error). affon_rocm_last_error()
 * returns the message of the last failure on the calling thread.
 * On any non-zero status the output buffer is left untouched
 * (src/support/compute_core_cyna_smoke.zig:979-983).
 */
#ifndef AFFON_ROCM_H
#define AFFON_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  AFFON_ROCM_OK = 0,
  AFFON_ROCM_INVALID_SHAPE = 1,
  AFFON_ROCM_CORE_FAILURE = 2,
  AFFON_ROCM_UNSUPPORTED = 3,
  AFFON_ROCM_HIP_ERROR = 4
};

/* Element types (src/js/compute/program.ts:5 ProgramDType subset). */
enum { AFFON_ROCM_F32 = 0, AFFON_ROCM_BF16 = 1, AFFON_ROCM_U32 = 2 };

/* Physical implementations of quantized_matmul. AUTO selects by shape and
 * layout the way the reference compiler selects among its candidates
 * (docs/core/quantized-inference.md:132-140); the others force one candidate
 * and return AFFON_ROCM_UNSUPPORTED if it cannot run the problem. */
enum {
  AFFON_ROCM_IMPL_AUTO = 0,
  AFFON_ROCM_IMPL_GENERIC = 1,   /* rocm_quantized_matmul.generic: any view, any group */
  AFFON_ROCM_IMPL_GEMV = 2,      /* rocm_quantized_matmul.gemv: VALU decode, small M */
  AFFON_ROCM_IMPL_GEMV_MFMA = 3, /* rocm_quantized_matmul.gemv_mfma: bf16 x, any M (row tiles of 32) */
  AFFON_ROCM_IMPL_MFMA = 4       /* rocm_quantized_matmul.mfma: prefill GEMM, bf16 x */
};

/* Numerical policies (src/js/compute/program.ts:7 NumericalPolicy). */
enum {
  AFFON_ROCM_BACKEND_EQUIVALENT = 0, /* accepts exact and reassociated candidates */
  AFFON_ROCM_EXACT_ONLY = 1,         /* only candidates bit-identical to the ordered CPU loop */
  AFFON_ROCM_APPROXIMATE = 2         /* also accepts bf16 rounding of decoded weights */
};

typedef struct affon_rocm_session affon_rocm_session;

/* A rank-two device tensor view: logical element [i,j] lives at byte
 * byte_offset + (i*stride[0] + j*stride[1]) * element_size from data.
 * buffer_bytes is the size of the allocation behind data; every element the
 * view names must lie inside it (views: docs/core/quantized-inference.md:47-49). */
typedef struct {
  const void* data;
  size_t buffer_bytes;
  size_t byte_offset;
  int64_t shape[2];
  int64_t stride[2];
  int32_t dtype;
} affon_rocm_view;

/* One quantized_matmul: output[M,N] (f32, contiguous) = input[M,K] . dequant(packed)^T.
 * Mirrors OpTag.quantized_matmul with OpOptions{bits, group_size}
 * (src/js/compute/native.zig:739,746) and the operand contract of
 * src/js/compute/program.ts:481-494. */
typedef struct {
  affon_rocm_view input;   /* [M,K]   f32 | bf16 */
  affon_rocm_view packed;  /* [N,K/P] u32 */
  affon_rocm_view scales;  /* [N,K/g] f32 | bf16 */
  affon_rocm_view biases;  /* [N,K/g] same dtype as scales */
  float* output;           /* [M,N] f32 row-major */
  size_t output_bytes;     /* must be >= M*N*4 */
  uint32_t bits;           /* 2, 4 or 8 */
  uint32_t group_size;     /* > 0, divides K */
  int32_t implementation;  /* AFFON_ROCM_IMPL_* */
  int32_t numerical_policy;/* AFFON_ROCM_BACKEND_EQUIVALENT etc. */
} affon_rocm_qmm_desc;

/* ---- device and session (replaces the compute.Session slot per backend,
 *      src/js/compute/native.zig:240-252; one HIP stream per session) ---- */

/* Number of visible gfx950 devices (0 when none). */
int affon_rocm_device_count(int* count);
/* Opens a session on device ordinal: sets the device and creates one stream. */
int affon_rocm_session_create(int device, affon_rocm_session** out);
int affon_rocm_session_destroy(affon_rocm_session* session);
/* The session's hipStream_t, for callers that record events around its work. */
void* affon_rocm_session_stream(affon_rocm_session* session);

int affon_rocm_alloc(affon_rocm_session* session, size_t bytes, void** out);
int affon_rocm_free(affon_rocm_session* session, void* ptr);
/* Copies are ordered on the session stream and complete before returning. */
int affon_rocm_memcpy_h2d(affon_rocm_session* session, void* dst, const void* src, size_t bytes);
int affon_rocm_memcpy_d2h(affon_rocm_session* session, void* dst, const void* src, size_t bytes);
int affon_rocm_memcpy_d2d(affon_rocm_session* session, void* dst, const void* src, size_t bytes);
/* Waits for all work enqueued on the session stream (host readback boundary,
 * docs/core/backend-support.md:69). */
int affon_rocm_synchronize(affon_rocm_session* session);

/* Message of the last failure on this thread ("" when none). */
const char* affon_rocm_last_error(void);

/* ---- quantized_matmul ---- */

/* Validates (same rules as src/js/compute/program.ts:483-493 and
 * src/support/compute_core_cyna.zig:1012-1022, overflow-checked), selects a
 * physical implementation and enqueues it on the session stream. Nothing is
 * written when validation fails. Replaces compute.Session.run for
 * OpTag.quantized_matmul (src/js/compute/native.zig:1406). */
int affon_rocm_quantized_matmul(affon_rocm_session* session, const affon_rocm_qmm_desc* desc);

/* The same operation without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The
 * scratch that affon_rocm_quantized_matmul keeps in the session's growable
 * workspace (split-K partial sums; the reassociated prefill GEMM's per-group
 * activation sums) goes instead to a static 33 MiB device array (one per
 * GPU, held until the process ends), whose address is looked up on the first
 * call on each device. Same selection, kernels and results as
 * affon_rocm_quantized_matmul; a shape whose plan needs more than 33 MiB of
 * scratch is rejected with AFFON_ROCM_UNSUPPORTED before anything is
 * enqueued (the output is untouched). Every call on a GPU
 * shares that GPU's array, so calls that overlap on one GPU (other streams,
 * other sessions, other threads) race. */
int affon_rocm_quantized_matmul_noalloc(affon_rocm_session* session, const affon_rocm_qmm_desc* desc);

/* Measurement helper, no counterpart in the reference: enqueues one launch
 * that reads every whole 16-byte chunk of `count` (1..4) 16-byte-aligned
 * device buffers once and nothing else, with the geometry of the M = 1
 * decode kernel (256-thread workgroups, four 16-byte loads per lane issued
 * before any wait). Its period is the floor a decode launch reading the same
 * weights can reach. `sink` (one device word) is written at most once. */
int affon_rocm_read_floor(affon_rocm_session* session, const void* const* buffers, const uint64_t* bytes, int count,
                          void* sink);

/* Measurement helpers, no counterpart in the reference: the parts a decode
 * launch's period is made of. affon_rocm_read_floor_geometry reads `bytes`
 * (a multiple of 16) of one 16-byte-aligned device buffer once: every wave
 * reads `kib_per_wave` (1, 2, 4 or 8) contiguous KiB with one 16-byte load per
 * lane per KiB, all issued before any wait, in workgroups of `threads` (64 to
 * 1024, a multiple of 64); then issues `valu_per_wave` (a multiple of 8, at
 * most 4096) dependent f32 multiply-adds on its data; then, when
 * `store_every` > 0, every store_every-th wave writes 8 bytes to `sink`,
 * which must hold 8 * ceil(waves / store_every) bytes (sink_bytes; waves =
 * ceil(bytes / (1024 * kib_per_wave))). affon_rocm_empty_launch enqueues a
 * kernel that does nothing, on `blocks` workgroups of `threads`. */
typedef struct {
  int32_t kib_per_wave;
  int32_t threads;
  int32_t valu_per_wave;
  int32_t store_every;
} affon_rocm_floor_geometry;
int affon_rocm_read_floor_geometry(affon_rocm_session* session, const void* buffer, uint64_t bytes, void* sink,
                                   uint64_t sink_bytes, const affon_rocm_floor_geometry* geometry);
int affon_rocm_empty_launch(affon_rocm_session* session, uint32_t blocks, uint32_t threads);

/* Capability detail, no counterpart in the reference: validates like
 * affon_rocm_quantized_matmul, then writes to *supported whether the guard of
 * one physical kernel behind the candidates accepts the problem (1) or not
 * (0). Kernel names: "generic", "gemv" (the gemv candidate), "gemv1" (its
 * M = 1 kernel), "gemv_mfma", "mfma", "gemm_re" (the group-scaling
 * reassociated prefill GEMM), "gemm_re32" (the reassociated prefill GEMM for
 * groups of 32), "gemm_pair" (the 4-bit prefill GEMM); another name is
 * AFFON_ROCM_INVALID_SHAPE. Enqueues nothing. */
int affon_rocm_kernel_supports(const affon_rocm_qmm_desc* desc, const char* kernel, int* supported);

/* Runs validation and selection only and writes the selected implementation
 * id (e.g. "rocm_quantized_matmul.gemv") into id (capacity cap, NUL-terminated).
 * Mirrors the compiler's implementation_id in executable explanations
 * (src/js/compute/native.zig:1314-1322). */
int affon_rocm_quantized_matmul_select(const affon_rocm_qmm_desc* desc, char* id, size_t cap);

/* ---- fused output epilogues (no reference counterpart: the reference
 *      authors a linear layer's output bias and the SiLU-gated feed-forward
 *      product as separate ops after quantized_matmul,
 *      docs/core/quantized-inference.md:37-42 `add(projected, output_bias)` and
 *      packages/@affon/models/src/llama/model.ts:82
 *      `mul(silu(matmul(h, gate)), matmul(h, up))`) ---- */
enum {
  AFFON_ROCM_EPILOGUE_NONE = 0,      /* plain quantized_matmul */
  AFFON_ROCM_EPILOGUE_BIAS = 1,      /* output[m,n] = qmm[m,n] + bias[n], one f32 add */
  AFFON_ROCM_EPILOGUE_SILU_GATE = 2  /* output[m,n] = silu(gate[m,n]) * up[m,n], silu(g) = g / (1 + e^-g) */
};

typedef struct {
  int32_t kind;           /* AFFON_ROCM_EPILOGUE_* */
  /* BIAS: N contiguous f32 | bf16 device elements, element-aligned. */
  const void* bias;
  size_t bias_bytes;
  int32_t bias_dtype;
  /* SILU_GATE: the up projection. The descriptor's packed/scales/biases are
   * the gate projection; these views have the same shapes and dtypes. */
  affon_rocm_view up_packed;
  affon_rocm_view up_scales;
  affon_rocm_view up_biases;
} affon_rocm_qmm_epilogue;

/* quantized_matmul with an output epilogue applied by the kernel that stores
 * each output element. Validation and implementation selection are those of
 * affon_rocm_quantized_matmul (plus the epilogue's operands); implementation
 * and numerical_policy apply to every launch. SILU_GATE runs as one launch
 * when the selected kernel computes rows of both projections together (the
 * M = 1 gemv kernel, with equal strides), otherwise as two launches: the gate
 * projection into output, then the up projection, whose kernel stores
 * silu(output) * up. */
int affon_rocm_quantized_matmul_fused(affon_rocm_session* session, const affon_rocm_qmm_desc* desc,
                                      const affon_rocm_qmm_epilogue* epilogue);

/* Plan of a fused call: the implementation id of each launch with its
 * epilogue in brackets, launches separated by ';'
 * (e.g. "rocm_quantized_matmul.gemv[silu_gate]"). */
int affon_rocm_quantized_matmul_fused_select(const affon_rocm_qmm_desc* desc, const affon_rocm_qmm_epilogue* epilogue,
                                             char* id, size_t cap);

/* Several quantized_matmul calls that read the same input (a decoder block's
 * query, key and value projections) as one call (no reference counterpart:
 * the reference runs one matmul per projection,
 * packages/@affon/models/src/llama/model.ts:73-75). descs[i] may differ only
 * in packed, scales, biases and output; input, bits, group_size,
 * implementation and numerical_policy are shared. epilogues is null or holds
 * count entries, each AFFON_ROCM_EPILOGUE_NONE or _BIAS. Results equal count
 * separate calls. They run as one launch when count <= 4, the strides are
 * equal and every call selects the same kernel that takes groups: the M = 1
 * gemv kernel, or the LDS-tiled gemv_mfma kernel (bf16 decode batches the
 * virtual-row kernels do not take). */
int affon_rocm_quantized_matmul_grouped(affon_rocm_session* session, const affon_rocm_qmm_desc* descs,
                                        const affon_rocm_qmm_epilogue* epilogues, size_t count);

/* Plan of a grouped call: "<id>[grouped:<count>]" (",bias]" when any call
 * adds an output bias) for one launch, else each call's plan separated by ';'. */
int affon_rocm_quantized_matmul_grouped_select(const affon_rocm_qmm_desc* descs,
                                               const affon_rocm_qmm_epilogue* epilogues, size_t count, char* id,
                                               size_t cap);

/* JSON array describing every registered candidate: id, version, numerical
 * class and guard (capability registration for the rocm backend). */
const char* affon_rocm_quantized_matmul_capabilities(void);

/* Host-pointer drop-in with the exact signature of the reference C ABI
 * compute_core_run_quantized_matmul_f32 (src/support/compute_core_cyna.zig:29-45):
 * f32 activation [rows,depth], u32 weights [columns, depth/P], f32 scales and
 * biases [columns, depth/group_size], f32 output [rows, columns]. Counts must
 * match exactly. Copies through device memory of the default session on
 * device 0 and returns after the result is in output. */
int compute_core_run_quantized_matmul_f32(const float* activation, size_t activation_count,
                                          const uint32_t* weights, size_t weight_count,
                                          const float* scales, size_t scale_count,
                                          const float* biases, size_t bias_count,
                                          float* output, size_t output_count,
                                          size_t rows, size_t depth, size_t columns,
                                          size_t bits, size_t group_size);

/* ---- quantize / dequantize (no reference counterpart: the reference packs
 *      only in test harnesses, test/parity/fixtures/quantized_fixture.py:10-13,
 *      and states dequantization as a formula, docs/core/quantized-inference.md:59-61) ---- */

/* Affine group-wise quantize of a contiguous device matrix weights[rows, columns]
 * (f32 or bf16) into packed[rows, columns/P] u32 and scales/biases
 * [rows, columns/group_size] of param_dtype. Per group: scale =
 * (max - min) / (2^bits - 1), bias = min (signed zeros canonicalised to +0),
 * both stored as param_dtype (bf16: round to nearest even), q =
 * clamp(rint((w - bias) / scale), 0, 2^bits - 1) from the stored scale and
 * bias with IEEE f32 division, q = 0 when the stored scale is 0. min and
 * max are a comparison scan from each group's first value: a NaN there gives
 * a NaN scale and bias and codes 0; a later NaN is skipped and takes code 0. */
int affon_rocm_quantize(affon_rocm_session* session, const void* weights, int32_t weight_dtype,
                        int64_t rows, int64_t columns, uint32_t bits, uint32_t group_size,
                        uint32_t* packed, void* scales, void* biases, int32_t param_dtype);

/* Dequantize packed[rows, columns/P] with scales/biases [rows, columns/g]
 * into out[rows, columns] of out_dtype (f32, or bf16 rounded to nearest even):
 * w = scale * q + bias with the product and the sum each rounded in f32. */
int affon_rocm_dequantize(affon_rocm_session* session, const uint32_t* packed, const void* scales,
                          const void* biases, int32_t param_dtype, int64_t rows, int64_t columns,
                          uint32_t bits, uint32_t group_size, void* out, int32_t out_dtype);

/* ---- the other ops of a decode step (test/parity/catalogs/cuda-apertus-decode-ops.json:1-26) ----
 * Contiguous rank-two device tensors [rows, cols] of dtype f32 or bf16;
 * arithmetic in f32, bf16 results rounded to nearest even; the result has
 * the input's dtype and shape (index_select: the selected shape). */

/* rms_norm along the last axis: out[r,c] = x[r,c] / sqrt(mean_c(x[r,:]^2) + epsilon).
 * Replaces compute.Session.run for OpTag.rms_norm (src/js/compute/native.zig:739;
 * op src/js/ops.ts:99, epsilon default 1e-5). */
int affon_rocm_rms_norm(affon_rocm_session* session, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                        float epsilon, void* out);

/* softmax along the last axis: out[r,c] = exp(x[r,c] - max_r) / sum_c exp(x[r,c] - max_r).
 * Replaces compute.Session.run for OpTag.softmax (native.zig:739; op src/js/ops.ts:97). */
int affon_rocm_softmax(affon_rocm_session* session, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                       void* out);

/* index_select along axis 0 (out[i,:] = x[index[i],:], out [count, cols]) or
 * axis 1 (out[:,i] = x[:,index[i]], out [rows, count]) with count device i64
 * indices; an index outside [0, size) selects zeros. Replaces
 * compute.Session.run for OpTag.index_select (native.zig:739; op
 * src/js/ops.ts:119; zero fill test/parity/reference/probe-capabilities.py:150-153). */
int affon_rocm_index_select(affon_rocm_session* session, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                            int32_t axis, const int64_t* index, int64_t count, void* out);

#ifdef __cplusplus
}
#endif

#endif /* AFFON_ROCM_H */
