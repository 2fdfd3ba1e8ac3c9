// Affine group-wise quantize and dequantize for the packed u32 format.
//
// The reference has no quantize op (it packs only in test harnesses,
// test/parity/fixtures/quantized_fixture.py:10-13) and states dequantization
// as a formula (docs/core/quantized-inference.md:59-61). The quantizer here is
// this library's contract, chosen so that CPU and GPU agree bit for bit:
// min / max by comparison, signed zeros canonicalised by adding +0.0f,
// IEEE f32 division (hipcc's default correctly rounded divide), rint half to
// even, no contraction, scale and bias rounded to their storage dtype before
// the codes are computed from them.

#include "device.h"
#include "internal.h"

// No fused multiply-add anywhere in this file (also built with
// -ffp-contract=off): dequantization rounds the product and the sum separately.
#pragma clang fp contract(off)

namespace affon {
namespace {

template <typename WT>
__device__ __forceinline__ float load_weight(const uint8_t* base, int64_t index) {
  return WT::load(base, index);
}

__device__ __forceinline__ float stored_param(float v, bool bf16) {
  return bf16 ? bf16_bits_to_f32(f32_to_bf16_bits(v)) : v;
}

__device__ __forceinline__ void store_param(void* base, int64_t index, float v, bool bf16) {
  if (bf16)
    static_cast<uint16_t*>(base)[index] = f32_to_bf16_bits(v);
  else
    static_cast<float*>(base)[index] = v;
}

__device__ __forceinline__ uint32_t clamp_code(float r, float max_q) {
  // fmaxf returns the other operand for a NaN: NaN and negative values give 0.
  return static_cast<uint32_t>(fminf(fmaxf(r, 0.0f), max_q));
}

__device__ __forceinline__ uint32_t code(float w, float s, float b, float max_q) {
  if (s == 0.0f) return 0u;
  return clamp_code(rintf((w - b) / s), max_q);
}

// One thread per packed word; the WPG = g/P threads of a group sit in one
// aligned lane group (WPG a power of two <= 64) and combine min/max with
// butterfly shuffles. Reads are contiguous per thread and across lanes.
//
// The codes clamp(rint((w - b) / s)) take one division per thread instead of
// one per value. With inv = 1/s correctly rounded (s in [2^-125, 2^125], so
// inv is normal) and qt = (w - b) * inv rounded, qt lies within
// 1.5 * 2^-23 * |q| of the exact quotient q, and the correctly rounded
// quotient RN(q) within 2^-24 * |q|. While |qt| <= 2^BITS, both lie within
// kNear = 2^BITS * 2^-20 of each other, so when qt is farther than kNear from
// every half-integer, rint gives the same integer for both. Past that range
// both clamp to the same end code, and NaN and infinite quotients clamp alike.
// A thread with a value nearer a half-integer, or a scale outside the range
// (zero, subnormal, huge, NaN), recomputes its word with the division.
template <int BITS, typename WT, int WPG>
__global__ __launch_bounds__(256) void quantize_words_kernel(const uint8_t* weights, int64_t total_words,
                                                             uint32_t* packed, void* scales, void* biases,
                                                             bool bf16_params) {
  constexpr int P = 32 / BITS;
  constexpr float kMaxQ = static_cast<float>((1u << BITS) - 1u);
  constexpr float kNear = static_cast<float>(1u << BITS) * 0x1p-20f;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool active = t < total_words;
  // Threads past the end belong to lane groups that hold no real word
  // (total_words is a multiple of WPG), so they may read any valid word.
  const int64_t tt = active ? t : total_words - 1;
  float v[P];
#pragma unroll
  for (int i = 0; i < P; ++i) v[i] = load_weight<WT>(weights, tt * P + i);
  // The group's min / max as a comparison scan from its first value gives
  // them: NaN when that value is NaN, otherwise over the values that are not
  // NaN (fminf / fmaxf skip a NaN operand).
  float mn = v[0], mx = v[0];
#pragma unroll
  for (int i = 1; i < P; ++i) {
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
  }
#pragma unroll
  for (int offset = 1; offset < WPG; offset <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, offset));
    mx = fmaxf(mx, __shfl_xor(mx, offset));
  }
  const float first = __shfl(v[0], 0, WPG);
  if (first != first) mn = mx = first;
  const float scale = (mx - mn) / kMaxQ + 0.0f;
  const float bias = mn + 0.0f;
  const float s = stored_param(scale, bf16_params);
  const float b = stored_param(bias, bf16_params);
  if (!active) return;
  if ((t & (WPG - 1)) == 0) {
    store_param(scales, t / WPG, scale, bf16_params);
    store_param(biases, t / WPG, bias, bf16_params);
  }
  const float inv = 1.0f / s;
  float d[P], r[P];
  float worst = 0.0f;  // the largest |qt - rint(qt)| of the word
#pragma unroll
  for (int i = 0; i < P; ++i) {
    d[i] = v[i] - b;
    const float qt = d[i] * inv;
    r[i] = rintf(qt);
    worst = fmaxf(worst, fabsf(qt - r[i]));
  }
  if (!(s >= 0x1p-125f && s <= 0x1p125f) || worst >= 0.5f - kNear) {
#pragma unroll
    for (int i = 0; i < P; ++i) r[i] = s == 0.0f ? 0.0f : rintf(d[i] / s);
  }
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < P; ++i) word |= clamp_code(r[i], kMaxQ) << (i * BITS);
  packed[t] = word;
}

// General layout, first pass: one thread per group writes scale and bias.
template <typename WT>
__global__ __launch_bounds__(256) void quantize_params_kernel(const uint8_t* weights, int64_t total_groups,
                                                              int64_t group, float max_q, void* scales, void* biases,
                                                              bool bf16_params) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total_groups) return;
  const int64_t base = t * group;
  float mn = load_weight<WT>(weights, base), mx = mn;
  for (int64_t i = 1; i < group; ++i) {
    const float v = load_weight<WT>(weights, base + i);
    mn = v < mn ? v : mn;
    mx = v > mx ? v : mx;
  }
  store_param(scales, t, (mx - mn) / max_q + 0.0f, bf16_params);
  store_param(biases, t, mn + 0.0f, bf16_params);
}

template <typename T>
__device__ __forceinline__ float load_param(const void* base, int64_t index) {
  return T::load(static_cast<const uint8_t*>(base), index);
}

// General layout, second pass: one thread per word reads the stored
// parameters of each value's group (groups may cross word boundaries).
template <typename WT, typename PT>
__global__ __launch_bounds__(256) void quantize_codes_kernel(const uint8_t* weights, int64_t total_words,
                                                             int64_t group, int bits, uint32_t* packed,
                                                             const void* scales, const void* biases) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total_words) return;
  const int per_word = 32 / bits;
  const float max_q = static_cast<float>((1u << bits) - 1u);
  uint32_t word = 0;
  for (int i = 0; i < per_word; ++i) {
    const int64_t e = t * per_word + i;  // flat element index; groups never straddle rows
    const int64_t g = e / group;
    const float s = load_param<PT>(scales, g);
    const float b = load_param<PT>(biases, g);
    word |= code(load_weight<WT>(weights, e), s, b, max_q) << (i * bits);
  }
  packed[t] = word;
}

template <typename PT, typename OT>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint32_t* packed, const void* scales, const void* biases,
                                                         int64_t total_words, int64_t group, int bits, void* out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total_words) return;
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const uint32_t word = packed[t];
  for (int i = 0; i < per_word; ++i) {
    const int64_t e = t * per_word + i;
    const int64_t g = e / group;
    const float s = load_param<PT>(scales, g);
    const float b = load_param<PT>(biases, g);
    const float w = s * static_cast<float>((word >> (i * bits)) & mask) + b;
    if constexpr (OT::bytes == 2)
      static_cast<uint16_t*>(out)[e] = f32_to_bf16_bits(w);
    else
      static_cast<float*>(out)[e] = w;
  }
}

// One thread per packed word when a group holds whole words (wpg of them:
// the group index is t >> wpg_shift for a power of two, else a 32-bit
// division, the word count then below 2^32): the word's scale and bias are
// read once, and its P values leave as 16-byte stores (the output is 16-byte
// aligned). The arithmetic is the general kernel's, s * q + b with two
// roundings.
template <int BITS, typename PT, typename OT>
__global__ __launch_bounds__(256) void dequantize_words_kernel(const uint32_t* packed, const void* scales,
                                                               const void* biases, int64_t total_words, int wpg_shift,
                                                               uint32_t wpg, void* out) {
  constexpr int P = 32 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total_words) return;
  const uint32_t word = packed[t];
  const int64_t g = wpg_shift >= 0 ? t >> wpg_shift : static_cast<int64_t>(static_cast<uint32_t>(t) / wpg);
  const float s = load_param<PT>(scales, g);
  const float b = load_param<PT>(biases, g);
  uint32_t bits_out[P * OT::bytes / 4];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const float w = s * static_cast<float>((word >> (i * BITS)) & kMask) + b;
    if constexpr (OT::bytes == 2) {
      const uint32_t h = f32_to_bf16_bits(w);
      bits_out[i / 2] = (i % 2 == 0) ? h : (bits_out[i / 2] | (h << 16));
    } else {
      bits_out[i] = __float_as_uint(w);
    }
  }
  constexpr int kWords = P * OT::bytes / 4;  // 32-bit words of output per packed word
  if constexpr (kWords % 4 == 0) {
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(out) + t * (kWords / 4);
#pragma unroll
    for (int j = 0; j < kWords / 4; ++j)
      dst[j] = u32x4_t{bits_out[4 * j], bits_out[4 * j + 1], bits_out[4 * j + 2], bits_out[4 * j + 3]};
  } else {
    static_assert(kWords == 2, "8-bit codes to bf16: 8 bytes per word");
    reinterpret_cast<u32x2_t*>(out)[t] = u32x2_t{bits_out[0], bits_out[1]};
  }
}

unsigned blocks_for(int64_t threads) { return static_cast<unsigned>((threads + 255) / 256); }

template <int BITS, typename WT, int WPG>
hipError_t launch_words(const void* weights, int64_t total_words, uint32_t* packed, void* scales, void* biases,
                        bool bf16, hipStream_t stream) {
  hipLaunchKernelGGL((quantize_words_kernel<BITS, WT, WPG>), dim3(blocks_for(total_words)), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(weights), total_words, packed, scales, biases, bf16);
  return hipGetLastError();
}

// wpg: words per group, a power of two <= 64.
template <int BITS, typename WT>
hipError_t launch_words_wpg(const void* weights, int64_t total_words, int wpg, uint32_t* packed, void* scales,
                            void* biases, bool bf16, hipStream_t stream) {
  switch (wpg) {
    case 1: return launch_words<BITS, WT, 1>(weights, total_words, packed, scales, biases, bf16, stream);
    case 2: return launch_words<BITS, WT, 2>(weights, total_words, packed, scales, biases, bf16, stream);
    case 4: return launch_words<BITS, WT, 4>(weights, total_words, packed, scales, biases, bf16, stream);
    case 8: return launch_words<BITS, WT, 8>(weights, total_words, packed, scales, biases, bf16, stream);
    case 16: return launch_words<BITS, WT, 16>(weights, total_words, packed, scales, biases, bf16, stream);
    case 32: return launch_words<BITS, WT, 32>(weights, total_words, packed, scales, biases, bf16, stream);
    default: return launch_words<BITS, WT, 64>(weights, total_words, packed, scales, biases, bf16, stream);
  }
}

template <typename WT>
hipError_t launch_words_bits(int bits, const void* weights, int64_t total_words, int wpg, uint32_t* packed,
                             void* scales, void* biases, bool bf16, hipStream_t stream) {
  switch (bits) {
    case 2: return launch_words_wpg<2, WT>(weights, total_words, wpg, packed, scales, biases, bf16, stream);
    case 4: return launch_words_wpg<4, WT>(weights, total_words, wpg, packed, scales, biases, bf16, stream);
    default: return launch_words_wpg<8, WT>(weights, total_words, wpg, packed, scales, biases, bf16, stream);
  }
}

template <typename WT>
hipError_t launch_general(const void* weights, int64_t rows, int64_t columns, int bits, int64_t group,
                          uint32_t* packed, void* scales, void* biases, bool bf16, hipStream_t stream) {
  const int64_t total_groups = rows * (columns / group);
  const int64_t total_words = rows * (columns / (32 / bits));
  const float max_q = static_cast<float>((1u << bits) - 1u);
  const auto* w = static_cast<const uint8_t*>(weights);
  hipLaunchKernelGGL((quantize_params_kernel<WT>), dim3(blocks_for(total_groups)), dim3(256), 0, stream, w,
                     total_groups, group, max_q, scales, biases, bf16);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (bf16)
    hipLaunchKernelGGL((quantize_codes_kernel<WT, BF16>), dim3(blocks_for(total_words)), dim3(256), 0, stream, w,
                       total_words, group, bits, packed, scales, biases);
  else
    hipLaunchKernelGGL((quantize_codes_kernel<WT, F32>), dim3(blocks_for(total_words)), dim3(256), 0, stream, w,
                       total_words, group, bits, packed, scales, biases);
  return hipGetLastError();
}

template <int BITS, typename PT, typename OT>
hipError_t launch_dequantize_words(const uint32_t* packed, const void* scales, const void* biases,
                                   int64_t total_words, int wpg_shift, uint32_t wpg, void* out, hipStream_t stream) {
  hipLaunchKernelGGL((dequantize_words_kernel<BITS, PT, OT>), dim3(blocks_for(total_words)), dim3(256), 0, stream,
                     packed, scales, biases, total_words, wpg_shift, wpg, out);
  return hipGetLastError();
}

template <typename PT, typename OT>
hipError_t launch_dequantize_words_bits(int bits, const uint32_t* packed, const void* scales, const void* biases,
                                        int64_t total_words, int wpg_shift, uint32_t wpg, void* out,
                                        hipStream_t stream) {
  switch (bits) {
    case 2: return launch_dequantize_words<2, PT, OT>(packed, scales, biases, total_words, wpg_shift, wpg, out, stream);
    case 4: return launch_dequantize_words<4, PT, OT>(packed, scales, biases, total_words, wpg_shift, wpg, out, stream);
    default:
      return launch_dequantize_words<8, PT, OT>(packed, scales, biases, total_words, wpg_shift, wpg, out, stream);
  }
}

}  // namespace

hipError_t quantize_launch(const void* weights, int weight_dtype, int64_t rows, int64_t columns, int bits,
                           int64_t group, uint32_t* packed, void* scales, void* biases, int param_dtype,
                           hipStream_t stream) {
  const int per_word = 32 / bits;
  const bool bf16 = param_dtype == AFFON_ROCM_BF16;
  const int64_t total_words = rows * (columns / per_word);
  const int64_t wpg = group % per_word == 0 ? group / per_word : 0;
  const bool fast = wpg > 0 && wpg <= 64 && (wpg & (wpg - 1)) == 0;
  if (fast) {
    if (weight_dtype == AFFON_ROCM_BF16)
      return launch_words_bits<BF16>(bits, weights, total_words, static_cast<int>(wpg), packed, scales, biases, bf16,
                                     stream);
    return launch_words_bits<F32>(bits, weights, total_words, static_cast<int>(wpg), packed, scales, biases, bf16,
                                  stream);
  }
  if (weight_dtype == AFFON_ROCM_BF16)
    return launch_general<BF16>(weights, rows, columns, bits, group, packed, scales, biases, bf16, stream);
  return launch_general<F32>(weights, rows, columns, bits, group, packed, scales, biases, bf16, stream);
}

hipError_t dequantize_launch(const uint32_t* packed, const void* scales, const void* biases, int param_dtype,
                             int64_t rows, int64_t columns, int bits, int64_t group, void* out, int out_dtype,
                             hipStream_t stream) {
  const int per_word = 32 / bits;
  const int64_t total_words = rows * (columns / per_word);
  const int64_t wpg = group % per_word == 0 ? group / per_word : 0;
  const bool pow2 = wpg > 0 && (wpg & (wpg - 1)) == 0;
  if (wpg > 0 && (pow2 || (total_words <= 0xffffffffll && wpg <= 0xffffffffll)) &&
      reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    int shift = -1;
    if (pow2)
      for (shift = 0; (int64_t{1} << shift) < wpg;) ++shift;
    const uint32_t w32 = static_cast<uint32_t>(wpg);
    const bool pbf = param_dtype == AFFON_ROCM_BF16, obf = out_dtype == AFFON_ROCM_BF16;
    if (pbf && obf)
      return launch_dequantize_words_bits<BF16, BF16>(bits, packed, scales, biases, total_words, shift, w32, out,
                                                      stream);
    if (pbf)
      return launch_dequantize_words_bits<BF16, F32>(bits, packed, scales, biases, total_words, shift, w32, out, stream);
    if (obf)
      return launch_dequantize_words_bits<F32, BF16>(bits, packed, scales, biases, total_words, shift, w32, out, stream);
    return launch_dequantize_words_bits<F32, F32>(bits, packed, scales, biases, total_words, shift, w32, out, stream);
  }
  const dim3 grid(blocks_for(total_words));
  if (param_dtype == AFFON_ROCM_BF16) {
    if (out_dtype == AFFON_ROCM_BF16)
      hipLaunchKernelGGL((dequantize_kernel<BF16, BF16>), grid, dim3(256), 0, stream, packed, scales, biases,
                         total_words, group, bits, out);
    else
      hipLaunchKernelGGL((dequantize_kernel<BF16, F32>), grid, dim3(256), 0, stream, packed, scales, biases,
                         total_words, group, bits, out);
  } else {
    if (out_dtype == AFFON_ROCM_BF16)
      hipLaunchKernelGGL((dequantize_kernel<F32, BF16>), grid, dim3(256), 0, stream, packed, scales, biases,
                         total_words, group, bits, out);
    else
      hipLaunchKernelGGL((dequantize_kernel<F32, F32>), grid, dim3(256), 0, stream, packed, scales, biases,
                         total_words, group, bits, out);
  }
  return hipGetLastError();
}

}  // namespace affon
