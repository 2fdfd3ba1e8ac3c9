// rocm_quantized_matmul.generic — the correctness path for every view and
// group layout the operation accepts, including groups that cross word
// boundaries and strided / transposed / offset operands
// (docs/core/quantized-inference.md:47-49,140,177-181).
//
// One thread owns one output element and walks k = 0..K-1 in order with an
// f32 accumulator; each product and sum is rounded separately (no fused
// multiply-add), so its results are bit-identical to the ordered scalar CPU
// loop (docs/core/quantized-inference.md:123-126). That makes it the one
// "exact" candidate, the only one an exact_only policy accepts.

#include "device.h"
#include "internal.h"

// Products and sums must stay separately rounded (this file is also built
// with -ffp-contract=off).
#pragma clang fp contract(off)

namespace affon {
namespace {

template <typename XT, typename PT>
__global__ __launch_bounds__(256) void qmm_generic_kernel(QmmProblem p) {
  const int64_t index = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index >= p.M * p.N) return;
  const int64_t n = index % p.N;
  const int64_t m = index / p.N;
  const int bits = p.bits;
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const uint32_t* row = p.w + n * p.ws0;
  const uint8_t* xrow = p.x + m * p.xs0 * XT::bytes;
  float acc = 0.0f;
  for (int64_t k = 0; k < p.K; ++k) {
    const int64_t word = k / per_word;
    const int lane = static_cast<int>(k - word * per_word);
    const uint32_t q = (row[word * p.ws1] >> (lane * bits)) & mask;
    const int64_t g = k / p.group;
    const float s = PT::load(p.s, n * p.ss0 + g * p.ss1);
    const float b = PT::load(p.b, n * p.bs0 + g * p.bs1);
    const float w = s * static_cast<float>(q) + b;
    acc = acc + XT::load(xrow, k * p.xs1) * w;
  }
  store_output(p.epi, p.out, m * p.N + n, n, acc);
}

template <typename XT>
hipError_t launch_x(const QmmProblem& p, dim3 grid, dim3 block, hipStream_t stream) {
  if (p.p_dtype == AFFON_ROCM_BF16)
    hipLaunchKernelGGL((qmm_generic_kernel<XT, BF16>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((qmm_generic_kernel<XT, F32>), grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace

bool generic_supports(const QmmProblem& p) {
  // The grid covers M*N threads in one dimension of at most 2^31 blocks.
  return p.M * p.N <= (int64_t(1) << 38);
}

hipError_t generic_launch(const QmmProblem& p, const Launch& l) {
  hipStream_t stream = l.stream;
  const int64_t total = p.M * p.N;
  const dim3 block(256);
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  if (p.x_dtype == AFFON_ROCM_BF16) return launch_x<BF16>(p, grid, block, stream);
  return launch_x<F32>(p, grid, block, stream);
}

}  // namespace affon
