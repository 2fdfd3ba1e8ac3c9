// Output epilogues of quantized_matmul kernels.
//
// The reference authors a linear layer's output bias and the SiLU-gated
// feed-forward product as separate element-wise ops after quantized_matmul
// (docs/core/quantized-inference.md:37-42: `add(projected, output_bias)`;
// packages/@affon/models/src/llama/model.ts:82:
// `mul(silu(matmul(h, gate)), matmul(h, up))`). Here the kernel that produces
// an output element applies them as it stores it:
//   kBias     out[m,n] = y + bias[n]              (one f32 add, as `add`);
//   kGateMul  out[m,n] = silu(out[m,n]) * y       (out already holds the gate
//                                                   projection; the same
//                                                   thread reads and writes
//                                                   the element);
//   kSiluPair out[m,n] = silu(y_gate) * y_up      (both projections computed
//                                                   by the same wave; only
//                                                   kernels that pair rows
//                                                   accept it).
// silu(g) = g / (1 + e^-g), in f32 like the reference's f32 `silu`.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <type_traits>

namespace affon {

enum EpilogueKind : int { kEpiNone = 0, kEpiBias = 1, kEpiGateMul = 2, kEpiSiluPair = 3 };

struct Epilogue {
  int kind = kEpiNone;
  int bias_bf16 = 0;              // bias element type: 1 bf16, 0 f32
  const uint8_t* bias = nullptr;  // kBias: N contiguous elements
  // kSiluPair: the second (up) projection, with the strides of the first.
  const uint32_t* w2 = nullptr;
  const uint8_t* s2 = nullptr;
  const uint8_t* b2 = nullptr;
};

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float bias_at(const Epilogue& e, int64_t n) {
  if (e.bias_bf16) return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(e.bias)[n]) << 16);
  return reinterpret_cast<const float*>(e.bias)[n];
}

// Stores the finished value y of output element idx (column n).
__device__ __forceinline__ void store_output(const Epilogue& e, float* out, int64_t idx, int64_t n, float y) {
  if (e.kind == kEpiBias) {
    y = y + bias_at(e, n);
  } else if (e.kind == kEpiGateMul) {
    y = silu(out[idx]) * y;
  }
  out[idx] = y;
}

// The same for a kind known at compile time (kEpiNone, kEpiBias or
// kEpiGateMul), p pointing at the element.
template <int KIND>
__device__ __forceinline__ void store_as(const Epilogue& e, float* p, int64_t n, float y) {
  if constexpr (KIND == kEpiBias) {
    y = y + bias_at(e, n);
  } else if constexpr (KIND == kEpiGateMul) {
    y = silu(*p) * y;
  }
  *p = y;
}

// Calls f(std::integral_constant<int, KIND>) for the stored kind, branching
// once: kernels that store many elements per thread emit one straight-line
// store sequence per kind instead of a branch per element.
template <class F>
__device__ __forceinline__ void with_store_kind(int kind, F&& f) {
  if (kind == kEpiBias)
    f(std::integral_constant<int, kEpiBias>{});
  else if (kind == kEpiGateMul)
    f(std::integral_constant<int, kEpiGateMul>{});
  else
    f(std::integral_constant<int, kEpiNone>{});
}

}  // namespace affon
