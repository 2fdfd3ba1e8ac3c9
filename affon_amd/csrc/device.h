// Device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace affon {

// bf16 -> f32 widening is exact: the bf16 bits are the top half of the f32.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// f32 -> bf16 round to nearest even on the bit pattern; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Element loads for the two floating dtypes the path accepts.
struct F32 {
  using storage = float;
  static constexpr int bytes = 4;
  __device__ __forceinline__ static float load(const uint8_t* base, int64_t index) {
    return reinterpret_cast<const float*>(base)[index];
  }
};
struct BF16 {
  using storage = uint16_t;
  static constexpr int bytes = 2;
  __device__ __forceinline__ static float load(const uint8_t* base, int64_t index) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[index]);
  }
};

__device__ __forceinline__ unsigned lane_id() { return __lane_id(); }

}  // namespace affon
