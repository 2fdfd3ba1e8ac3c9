// The other ops of one decode step on the rocm device: rms_norm and softmax
// along the last axis and index_select along either axis of a contiguous
// rank-two tensor (test/parity/catalogs/cuda-apertus-decode-ops.json:1-26;
// ops src/js/ops.ts:97,99,119).
//
// rms_norm(x)[r, c] = x[r, c] / sqrt(mean_c(x[r, :]^2) + epsilon) and
// softmax(x)[r, c] = exp(x[r, c] - max_r) / sum_c exp(x[r, c] - max_r), both
// computed in f32 (bf16 inputs widened exactly, bf16 outputs rounded to
// nearest even), one wave per row. index_select copies whole rows (axis 0)
// or gathers columns (axis 1); an index outside [0, size) selects zeros
// (the reference's and PyTorch's behaviour,
// test/parity/reference/probe-capabilities.py:150-153). All of them are
// HBM-bound; rows are read once.

#include <type_traits>

#include "device.h"
#include "internal.h"

namespace affon {
namespace {

constexpr int kRowThreads = 256;  // four rows per workgroup, one per wave

template <typename T>
__device__ __forceinline__ float load_value(const uint8_t* base, int64_t i) {
  return T::load(base, i);
}

template <typename T>
__device__ __forceinline__ void store_value(uint8_t* base, int64_t i, float v) {
  if constexpr (T::bytes == 2) {
    reinterpret_cast<uint16_t*>(base)[i] = f32_to_bf16_bits(v);
  } else {
    reinterpret_cast<float*>(base)[i] = v;
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset));
  return v;
}

template <typename T>
__global__ __launch_bounds__(kRowThreads) void rms_norm_kernel(const uint8_t* x, uint8_t* out, int64_t rows,
                                                               int64_t cols, float epsilon) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kRowThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t base = row * cols;
  float ss = 0.0f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float v = load_value<T>(x, base + c);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float denominator = sqrtf(ss / static_cast<float>(cols) + epsilon);
  for (int64_t c = lane; c < cols; c += 64) store_value<T>(out, base + c, load_value<T>(x, base + c) / denominator);
}

template <typename T>
__global__ __launch_bounds__(kRowThreads) void softmax_kernel(const uint8_t* x, uint8_t* out, int64_t rows,
                                                              int64_t cols) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kRowThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t base = row * cols;
  float peak = -INFINITY;
  for (int64_t c = lane; c < cols; c += 64) peak = fmaxf(peak, load_value<T>(x, base + c));
  peak = wave_max(peak);
  float sum = 0.0f;
  for (int64_t c = lane; c < cols; c += 64) sum += expf(load_value<T>(x, base + c) - peak);
  sum = wave_sum(sum);
  for (int64_t c = lane; c < cols; c += 64) store_value<T>(out, base + c, expf(load_value<T>(x, base + c) - peak) / sum);
}

// out[i, c] = x[index[i], c] (axis 0) or out[r, i] = x[r, index[i]] (axis 1),
// one thread per output element; raw element copies (no arithmetic).
template <int BYTES>
__global__ __launch_bounds__(256) void index_select_kernel(const uint8_t* x, uint8_t* out, int64_t rows, int64_t cols,
                                                           int axis, const int64_t* index, int64_t count) {
  const int64_t out_cols = axis == 0 ? cols : count;
  const int64_t total = (axis == 0 ? count : rows) * out_cols;
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= total) return;
  const int64_t r = o / out_cols, c = o - r * out_cols;
  const int64_t sel = index[axis == 0 ? r : c];
  const int64_t size = axis == 0 ? rows : cols;
  using U = typename std::conditional<BYTES == 2, uint16_t, uint32_t>::type;
  U v = 0;
  if (sel >= 0 && sel < size) v = reinterpret_cast<const U*>(x)[axis == 0 ? sel * cols + c : r * cols + sel];
  reinterpret_cast<U*>(out)[o] = v;
}

}  // namespace

hipError_t rms_norm_launch(const void* x, int dtype, int64_t rows, int64_t cols, float epsilon, void* out,
                           hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const auto* xi = static_cast<const uint8_t*>(x);
  auto* o = static_cast<uint8_t*>(out);
  if (dtype == AFFON_ROCM_BF16)
    hipLaunchKernelGGL(rms_norm_kernel<BF16>, grid, dim3(kRowThreads), 0, stream, xi, o, rows, cols, epsilon);
  else
    hipLaunchKernelGGL(rms_norm_kernel<F32>, grid, dim3(kRowThreads), 0, stream, xi, o, rows, cols, epsilon);
  return hipGetLastError();
}

hipError_t softmax_launch(const void* x, int dtype, int64_t rows, int64_t cols, void* out, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const auto* xi = static_cast<const uint8_t*>(x);
  auto* o = static_cast<uint8_t*>(out);
  if (dtype == AFFON_ROCM_BF16)
    hipLaunchKernelGGL(softmax_kernel<BF16>, grid, dim3(kRowThreads), 0, stream, xi, o, rows, cols);
  else
    hipLaunchKernelGGL(softmax_kernel<F32>, grid, dim3(kRowThreads), 0, stream, xi, o, rows, cols);
  return hipGetLastError();
}

hipError_t index_select_launch(const void* x, int dtype, int64_t rows, int64_t cols, int axis, const int64_t* index,
                               int64_t count, void* out, hipStream_t stream) {
  const int64_t total = (axis == 0 ? count : rows) * (axis == 0 ? cols : count);
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  const auto* xi = static_cast<const uint8_t*>(x);
  auto* o = static_cast<uint8_t*>(out);
  if (dtype == AFFON_ROCM_BF16)
    hipLaunchKernelGGL(index_select_kernel<2>, grid, dim3(256), 0, stream, xi, o, rows, cols, axis, index, count);
  else
    hipLaunchKernelGGL(index_select_kernel<4>, grid, dim3(256), 0, stream, xi, o, rows, cols, axis, index, count);
  return hipGetLastError();
}

}  // namespace affon
