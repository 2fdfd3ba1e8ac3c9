// rocm_quantized_matmul.gemv — HBM-bound decode kernel for small M.
//
// Counterpart of the reference's SIMD decode paths (metal simd1/simd4,
// docs/core/quantized-inference.md:136-149): fused unpack, affine decode and
// dot product, f32 accumulation, no floating weight matrix.
//
// Work mapping (wave64, gfx950):
//   * a wave owns R = 8 consecutive output rows n and one K-part; the 64 lanes
//     read consecutive 16-byte chunks of packed words of each row, so every
//     load instruction fetches 1 KiB of contiguous packed weights;
//   * the activation chunk a lane needs is loaded once into registers and
//     reused for all R rows (and for up to MR activation rows);
//   * per chunk (which lies inside one group) the lane accumulates the exact
//     integer codes: acc = sum x*q, then applies the group's parameters once:
//     y += s*acc + b*sum(x) — reassociated, f32 throughout;
//   * the R x MR partial sums are reduced across the wave with butterfly
//     shuffles, and across K-parts (waves of one block) through LDS.

#include "device.h"
#include "gemv1_dispatch.h"
#include "internal.h"

namespace affon {
namespace {

constexpr int kRows = 8;  // output rows per wave

template <int BITS>
__device__ __forceinline__ void decode_word(uint32_t w, float* q) {
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = static_cast<float>((w >> (8 * i)) & 0xffu);
  } else if constexpr (BITS == 4) {
    const uint32_t lo = w & 0x0f0f0f0fu;
    const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q[2 * j] = static_cast<float>((lo >> (8 * j)) & 0xffu);
      q[2 * j + 1] = static_cast<float>((hi >> (8 * j)) & 0xffu);
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t v = (w >> (2 * t)) & 0x03030303u;
#pragma unroll
      for (int j = 0; j < 4; ++j) q[4 * j + t] = static_cast<float>((v >> (8 * j)) & 0xffu);
    }
  }
}

// Loads CV activation values starting at element k0 of row xrow as f32.
template <typename XT, int CV>
__device__ __forceinline__ void load_x(const uint8_t* xrow, int64_t k0, float* out) {
  if constexpr (XT::bytes == 4) {
    const float4* src = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(xrow) + k0);
#pragma unroll
    for (int i = 0; i < CV / 4; ++i) {
      const float4 v = src[i];
      out[4 * i] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  } else {
    const uint2* src = reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(xrow) + k0);
#pragma unroll
    for (int i = 0; i < CV / 4; ++i) {
      const uint2 v = src[i];
      out[4 * i] = __uint_as_float(v.x << 16);
      out[4 * i + 1] = __uint_as_float(v.x & 0xffff0000u);
      out[4 * i + 2] = __uint_as_float(v.y << 16);
      out[4 * i + 3] = __uint_as_float(v.y & 0xffff0000u);
    }
  }
}

template <int CW>
__device__ __forceinline__ void load_words(const uint32_t* src, uint32_t* out) {
  if constexpr (CW == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(src);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  } else {
    out[0] = src[0];
  }
}

// CB: bytes of packed weights per lane per chunk (16 or 4). MR: activation
// rows handled per block row (grid.y covers M in steps of MR).
template <int BITS, int CB, int MR, typename XT, typename PT>
__global__ __launch_bounds__(256) void qgemv_kernel(QmmProblem p, int ksplit) {
  constexpr int P = 32 / BITS;
  constexpr int CW = CB / 4;
  constexpr int CV = CW * P;
  __shared__ float partial[4][kRows][MR];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int kp = wave % ksplit;
  const int64_t rb = static_cast<int64_t>(blockIdx.x) * (4 / ksplit) + wave / ksplit;
  const int64_t n0 = rb * kRows;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MR;
  const int64_t chunks = p.K / CV;

  float y[kRows][MR];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) y[r][m] = 0.0f;

  if (n0 < p.N) {
    for (int64_t c = static_cast<int64_t>(kp) * 64 + lane; c < chunks; c += 64 * ksplit) {
      const int64_t k0 = c * CV;
      // Packed words of the R rows (issued first so they are in flight
      // while the activations arrive).
      uint32_t wv[kRows][CW];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const int64_t n = n0 + r;
        if (n < p.N)
          load_words<CW>(p.w + n * p.ws0 + c * CW, wv[r]);
        else
#pragma unroll
          for (int i = 0; i < CW; ++i) wv[r][i] = 0u;
      }
      const int64_t gi = k0 / p.group;
      float sv[kRows], bv[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const int64_t n = n0 + r < p.N ? n0 + r : p.N - 1;
        sv[r] = PT::load(p.s, n * p.ss0 + gi);
        bv[r] = PT::load(p.b, n * p.bs0 + gi);
      }
      float xv[MR][CV];
      float xsum[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m0 + m < p.M) {
          load_x<XT, CV>(p.x + (m0 + m) * p.xs0 * XT::bytes, k0, xv[m]);
        } else {
#pragma unroll
          for (int i = 0; i < CV; ++i) xv[m][i] = 0.0f;
        }
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < CV; ++i) sum += xv[m][i];
        xsum[m] = sum;
      }
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < CW; ++i) {
          float q[P];
          decode_word<BITS>(wv[r][i], q);
#pragma unroll
          for (int j = 0; j < P; ++j)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[m] = fmaf(xv[m][i * P + j], q[j], acc[m]);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) y[r][m] += sv[r] * acc[m] + bv[r] * xsum[m];
      }
    }
  }

  // Wave reduction: every lane ends with the full sums.
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = y[r][m];
#pragma unroll
      for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset);
      y[r][m] = v;
    }

  if (ksplit == 1) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m)
          if (n0 + r < p.N && m0 + m < p.M) store_output(p.epi, p.out, (m0 + m) * p.N + n0 + r, n0 + r, y[r][m]);
    }
    return;
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m) partial[wave][r][m] = y[r][m];
  }
  __syncthreads();
  if (kp == 0 && lane < kRows * MR) {
    const int r = lane / MR;
    const int m = lane % MR;
    float v = 0.0f;
    for (int j = 0; j < ksplit; ++j) v += partial[wave + j][r][m];
    if (n0 + r < p.N && m0 + m < p.M) store_output(p.epi, p.out, (m0 + m) * p.N + n0 + r, n0 + r, v);
  }
}

template <int BITS, int CB, int MR, typename XT, typename PT>
hipError_t launch_typed(const QmmProblem& p, hipStream_t stream) {
  const int64_t row_blocks = (p.N + kRows - 1) / kRows;
  int ksplit = 1;
  if (row_blocks < 1024) ksplit = 4;
  else if (row_blocks < 2048) ksplit = 2;
  const int64_t blocks_x = (row_blocks + (4 / ksplit) - 1) / (4 / ksplit);
  const int64_t blocks_y = (p.M + MR - 1) / MR;
  hipLaunchKernelGGL((qgemv_kernel<BITS, CB, MR, XT, PT>), dim3(static_cast<unsigned>(blocks_x),
                     static_cast<unsigned>(blocks_y)), dim3(256), 0, stream, p, ksplit);
  return hipGetLastError();
}

template <int BITS, int CB, int MR>
hipError_t launch_mr(const QmmProblem& p, hipStream_t stream) {
  if (p.x_dtype == AFFON_ROCM_BF16) {
    if (p.p_dtype == AFFON_ROCM_BF16) return launch_typed<BITS, CB, MR, BF16, BF16>(p, stream);
    return launch_typed<BITS, CB, MR, BF16, F32>(p, stream);
  }
  if (p.p_dtype == AFFON_ROCM_BF16) return launch_typed<BITS, CB, MR, F32, BF16>(p, stream);
  return launch_typed<BITS, CB, MR, F32, F32>(p, stream);
}

template <int BITS, int CB>
hipError_t launch_cb(const QmmProblem& p, hipStream_t stream) {
  if (p.M == 1) return launch_mr<BITS, CB, 1>(p, stream);
  return launch_mr<BITS, CB, 4>(p, stream);
}

template <int BITS>
hipError_t launch_bits(const QmmProblem& p, hipStream_t stream) {
  constexpr int P = 32 / BITS;
  if (p.group % (4 * P) == 0 && (p.K / P) % 4 == 0 && p.ws0 % 4 == 0 &&
      reinterpret_cast<uintptr_t>(p.w) % 16 == 0)
    return launch_cb<BITS, 16>(p, stream);
  return launch_cb<BITS, 4>(p, stream);
}

}  // namespace

bool gemv_supports(const QmmProblem& p) {
  const int P = 32 / p.bits;
  const int xbytes = p.x_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  const uintptr_t x_align = xbytes == 4 ? 16 : 8;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  if (p.group % P != 0) return false;  // groups must be whole words
  if (reinterpret_cast<uintptr_t>(p.x) % x_align != 0 || (p.xs0 * xbytes) % static_cast<int64_t>(x_align) != 0)
    return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 4 != 0) return false;
  if (p.M > 65535 * 4) return false;
  return true;
}

bool gemv1_supports(const QmmProblem& p) {
  // One activation row, dense rows, 16-byte aligned packed rows and
  // activations, every 16-byte chunk inside one group, LDS for the row (the
  // one-row variant), parameters aligned to their element size.
  const int64_t cv = 128 / p.bits;
  const int xbytes = p.x_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  if (p.M != 1 || p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  if (p.K % cv != 0 || p.group % cv != 0) return false;
  const int64_t chunks_per_group = p.group / cv;
  if ((chunks_per_group & (chunks_per_group - 1)) != 0) return false;  // group index by shift
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || p.ws0 % 4 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return false;
  const int64_t chunks = p.K / cv;
  const int pbytes = p.p_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  if (reinterpret_cast<uintptr_t>(p.s) % pbytes != 0 || reinterpret_cast<uintptr_t>(p.b) % pbytes != 0) return false;
  if (chunks > gemv1::kMaxChunks) return false;
  const size_t lds = gemv1::lds_size_for(static_cast<int>(cv * xbytes / 16), static_cast<int>(chunks), 1);
  return lds <= static_cast<size_t>(gemv1::kMaxLdsBytes);
}

bool gemv_pair_supports(const QmmProblem& p) {
  // The second projection has the first one's shapes and strides (checked
  // by the caller); its pointers need the same alignment.
  const int pbytes = p.p_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  return gemv1_supports(p) && reinterpret_cast<uintptr_t>(p.epi.w2) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.epi.s2) % pbytes == 0 && reinterpret_cast<uintptr_t>(p.epi.b2) % pbytes == 0;
}

bool gemv_group_supports(const QmmProblem* group, int count) {
  if (count < 1 || count > kMaxGroup || count > gemv1::kMaxSegments) return false;
  const QmmProblem& p = group[0];
  for (int i = 0; i < count; ++i) {
    const QmmProblem& q = group[i];
    if (!gemv1_supports(q) || q.epi.kind == kEpiSiluPair || q.epi.kind == kEpiGateMul) return false;
    if (q.x != p.x || q.K != p.K || q.bits != p.bits || q.group != p.group || q.x_dtype != p.x_dtype ||
        q.p_dtype != p.p_dtype || q.ws0 != p.ws0 || q.ss0 != p.ss0 || q.bs0 != p.bs0)
      return false;
    if (q.epi.kind == kEpiBias) {
      for (int j = 0; j < count; ++j)
        if (group[j].epi.kind == kEpiBias && group[j].epi.bias_bf16 != q.epi.bias_bf16) return false;
    }
  }
  return true;
}

hipError_t gemv_group_launch(const QmmProblem* group, int count, const Launch& l) {
  if (!gemv_group_supports(group, count)) return hipErrorInvalidValue;
  switch (group[0].bits) {
    case 2: return gemv1_group_launch_b2(group, count, l.stream);
    case 4: return gemv1_group_launch_b4(group, count, l.stream);
    default: return gemv1_group_launch_b8(group, count, l.stream);
  }
}

hipError_t gemv_launch(const QmmProblem& p, const Launch& l) {
  hipStream_t stream = l.stream;
  if (p.epi.kind == kEpiSiluPair && !gemv_pair_supports(p)) return hipErrorInvalidValue;
  if (gemv1_supports(p)) {
    switch (p.bits) {
      case 2: return gemv1_launch_b2(p, stream);
      case 4: return gemv1_launch_b4(p, stream);
      default: return gemv1_launch_b8(p, stream);
    }
  }
  switch (p.bits) {
    case 2: return launch_bits<2>(p, stream);
    case 4: return launch_bits<4>(p, stream);
    default: return launch_bits<8>(p, stream);
  }
}

}  // namespace affon
