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

__device__ __forceinline__ uint32_t code(float w, float s, float b, float max_q) {
  if (s == 0.0f) return 0u;
  float r = rintf((w - b) / s);
  if (!(r >= 0.0f)) r = 0.0f;
  if (r > max_q) r = max_q;
  return static_cast<uint32_t>(r);
}

// One thread per packed word; the g/P threads of a group sit in one aligned
// lane group of size WPG (a power of two <= 64) and combine min/max with
// butterfly shuffles. Reads are contiguous per thread and across lanes.
template <int BITS, typename WT>
__global__ __launch_bounds__(256) void quantize_words_kernel(const uint8_t* weights, int64_t total_words, int wpg,
                                                             uint32_t* packed, void* scales, void* biases,
                                                             bool bf16_params) {
  constexpr int P = 32 / BITS;
  constexpr float kMaxQ = static_cast<float>((1u << BITS) - 1u);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool active = t < total_words;
  // Threads past the end belong to lane groups that hold no real word
  // (total_words is a multiple of wpg), so they may read any valid word.
  const int64_t tt = active ? t : total_words - 1;
  float v[P];
#pragma unroll
  for (int i = 0; i < P; ++i) v[i] = load_weight<WT>(weights, tt * P + i);
  float mn = v[0], mx = v[0];
#pragma unroll
  for (int i = 1; i < P; ++i) {
    mn = v[i] < mn ? v[i] : mn;
    mx = v[i] > mx ? v[i] : mx;
  }
  for (int offset = 1; offset < wpg; offset <<= 1) {
    const float omn = __shfl_xor(mn, offset);
    const float omx = __shfl_xor(mx, offset);
    mn = omn < mn ? omn : mn;
    mx = omx > mx ? omx : mx;
  }
  const float scale = (mx - mn) / kMaxQ + 0.0f;
  const float bias = mn + 0.0f;
  const float s = stored_param(scale, bf16_params);
  const float b = stored_param(bias, bf16_params);
  if (!active) return;
  if ((t & (wpg - 1)) == 0) {
    store_param(scales, t / wpg, scale, bf16_params);
    store_param(biases, t / wpg, bias, bf16_params);
  }
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < P; ++i) word |= code(v[i], s, b, kMaxQ) << (i * BITS);
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

unsigned blocks_for(int64_t threads) { return static_cast<unsigned>((threads + 255) / 256); }

template <int BITS, typename WT>
hipError_t launch_words(const void* weights, int64_t total_words, int wpg, uint32_t* packed, void* scales,
                        void* biases, bool bf16, hipStream_t stream) {
  hipLaunchKernelGGL((quantize_words_kernel<BITS, WT>), dim3(blocks_for(total_words)), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(weights), total_words, wpg, packed, scales, biases, bf16);
  return hipGetLastError();
}

template <typename WT>
hipError_t launch_words_bits(int bits, const void* weights, int64_t total_words, int wpg, uint32_t* packed,
                             void* scales, void* biases, bool bf16, hipStream_t stream) {
  switch (bits) {
    case 2: return launch_words<2, WT>(weights, total_words, wpg, packed, scales, biases, bf16, stream);
    case 4: return launch_words<4, WT>(weights, total_words, wpg, packed, scales, biases, bf16, stream);
    default: return launch_words<8, WT>(weights, total_words, wpg, packed, scales, biases, bf16, stream);
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
  const int64_t total_words = rows * (columns / (32 / bits));
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
