// Skinny decode (bf16 activations) on the matrix cores, with packed words
// loaded straight into the MFMA B operand: the 8-row layout. The kernel
// handles M <= 8 and 2/4/8-bit codes; the host uses it where it measured
// fastest (vrow_dispatch.h) and the 16-row layout (vrow16.h) elsewhere.
//
// One wave owns 8 weight rows and a K-part of them. The 16 columns of
// v_mfma_f32_16x16x32_bf16 are (row r, half h): lane l holds r = l % 8,
// h = (l / 8) % 2 and quarter q = l / 16. For every "set" of eight 16-byte
// chunks of a row, lane (r, h, q) loads chunk 4h + q, so one load
// instruction reads 128 contiguous bytes (one cache line) of each of 8 rows,
// and the codes go from the load registers through an exact bf16 conversion
// into the B operand without touching LDS.
//
// Columns of one MFMA thus hold different k ranges (the two halves of a
// set), and one MFMA's 32 k can span several quantization groups. Both are
// handled by the A operand's 16 rows, used as "virtual rows": row vr carries
// activation row m for half h(vr), masked to group ge of that half, for the
// sd-th set of a run of SPD sets (MP * SPD * GH = 8, GH groups per half-set).
// A lane whose virtual row does not match the set, half and group of the
// data it would supply reads zeros from a zero block in LDS, so masking
// costs one address select per set. Accumulator entry (vr, column) is used
// only when the column's half equals h(vr); after SPD sets each used entry
// holds the sum of x*q over exactly one group of one activation row, and the
// group parameters are applied once: y += s * D + b * sum(x over the group).
//
// Codes are exact in bf16 (FP8-read nibbles for 2/4-bit codes, n * 2^-9, with
// the unit divided out of the scale; v_cvt_f32_ubyte for 8-bit codes), the
// products are exact in the f32 accumulators, and only the order of the sums
// differs from the ordered loop: the reassociated class, like the other
// decode kernels.
#pragma once

#include <atomic>

#include "gemv1.h"
#include "lds_pipeline.h"

namespace affon {
namespace vrow {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
using gemv1::bf16x2_t;
using gemv1::u32x4_t;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = 8;        // weight rows per wave
constexpr int kZeroBytes = 128; // zero block (up to 8 MFMAs of 16 bytes per chunk)
// LDS per workgroup at most (8 activation rows of 4096 bf16 need 65.7 KB;
// two workgroups still fit a CU's 160 KB).
constexpr size_t kMaxLdsBytes = 80 * 1024;

struct Args {
  const uint8_t* x;  // bf16 [M, K]
  int64_t xs0;       // activation row stride in elements
  const uint32_t* w;
  int64_t ws0;       // packed row stride in words
  const uint8_t* s;
  int64_t ss0;
  const uint8_t* b;
  int64_t bs0;
  float* out;        // f32 [M, N], contiguous
  int M, N, K;
  int part;          // sets per K-part (the variant's CPL)
  int ks;            // K-parts per row block (waves per row block)
  int groups;        // groups per row
  Epilogue epi;
};

template <int BITS>
constexpr int chunk_codes() { return 128 / BITS; }
template <int BITS>
constexpr int set_codes() { return 8 * chunk_codes<BITS>(); }

// Bytes of one wave's group parameters in LDS: scales then biases, each
// [8 rows][CPL sets * 2 halves * GH groups].
__host__ __device__ constexpr int wave_param_bytes(int CPL, int GH, int pbytes) {
  return 2 * kRows * CPL * 2 * GH * pbytes;
}

// LDS (bytes): activation rows [MP][K*2 + 16] (the 16-byte pad moves
// consecutive rows to other banks), the zero block, group sums
// [MP][groups] f32, K-part partials [kWaves][MP*8] f32, then each wave's
// group parameters.
__host__ __device__ constexpr size_t lds_bytes(int MP, int K, int groups, int param_bytes) {
  return static_cast<size_t>(MP) * (static_cast<size_t>(K) * 2 + 16) + kZeroBytes +
         static_cast<size_t>(MP) * groups * 4 + static_cast<size_t>(kWaves) * MP * kRows * 4 +
         static_cast<size_t>(kWaves) * param_bytes;
}

template <bool HIGH>
__device__ __forceinline__ uint32_t fp8_pair(uint32_t m) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(m, 1.0f, HIGH));
}

__device__ __forceinline__ uint32_t bytes_bf16(uint32_t w, int lo) {
  const float a = static_cast<float>((w >> (8 * lo)) & 0xffu);
  const float b = static_cast<float>((w >> (8 * lo + 8)) & 0xffu);
  return __builtin_bit_cast(uint32_t, gemv1::pack2(a, b));
}

// B operand of MFMA u of a chunk (words wv[0..3]): 8 codes as bf16, in the
// pair order of the staged activations (gemv1::permute_bf16_piece).
template <int BITS, int U>
__device__ __forceinline__ bf16x8_t code_fragment(const uint32_t* wv) {
  u32x4_t d;
  if constexpr (BITS == 4) {
    const uint32_t w = wv[U];
    const uint32_t m0 = w & 0x0f0f0f0fu, m1 = (w >> 4) & 0x0f0f0f0fu;
    d = u32x4_t{fp8_pair<false>(m0), fp8_pair<true>(m0), fp8_pair<false>(m1), fp8_pair<true>(m1)};
  } else if constexpr (BITS == 8) {
    const uint32_t w0 = gemv1::opaque(wv[2 * U]), w1 = gemv1::opaque(wv[2 * U + 1]);
    d = u32x4_t{bytes_bf16(w0, 0), bytes_bf16(w0, 2), bytes_bf16(w1, 0), bytes_bf16(w1, 2)};
  } else {
    const uint32_t w = wv[U / 2];
    constexpr bool H = (U % 2) == 1;
    d = u32x4_t{fp8_pair<H>(w & 0x03030303u), fp8_pair<H>((w >> 2) & 0x03030303u),
                fp8_pair<H>((w >> 4) & 0x03030303u), fp8_pair<H>((w >> 6) & 0x03030303u)};
  }
  return __builtin_bit_cast(bf16x8_t, d);
}

__device__ __forceinline__ float dpp_ror8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));  // row_ror:8
}

// v summed with its partner lane across the 16-lane (bit 4) or 32-lane
// (bit 5) halves of the wave.
__device__ __forceinline__ float swap16_sum(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float swap32_sum(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Stages the 64 pieces (8 codes, 16 bytes of bf16) base .. base+63 of
// activation row m; pieces >= count are absent. The whole wave calls it.
template <int BITS, int PPG>
__device__ __forceinline__ void stage_pieces(u32x4_t v, int p, int count, uint8_t* xrow_lds, float* xsum_row) {
  const bool valid = p < count;
  const u32x4_t o = gemv1::permute_bf16_piece<BITS>(v);
  const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
  const uint32_t o0 = o.x, o1 = o.y, o2 = o.z, o3 = o.w;  // bit casts read whole scalars
  float sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o0), ones, 0.0f, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o1), ones, sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o2), ones, sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o3), ones, sum, false);
  sum = gemv1::group_sum<PPG>(valid ? sum : 0.0f);
  if (valid) {
    *reinterpret_cast<u32x4_t*>(xrow_lds + static_cast<uint32_t>(p) * 16u) = o;
    if (p % PPG == 0) xsum_row[p / PPG] = sum;
  }
}

// Virtual row vr (A-operand row, accumulator row): bit 2 is the half h;
// bits 0, 1, 3 form t = (m * SPD + sd) * GH + ge (activation row, set within
// the run, group within the half).
__device__ __forceinline__ int vrow_half(int vr) { return (vr >> 2) & 1; }
__device__ __forceinline__ int vrow_t(int vr) { return (vr & 3) | ((vr >> 3) << 2); }

// MP: activation rows rounded up to a power of two (M <= MP <= 8); GH: groups
// per half-set; CPL: sets per wave.
template <int BITS, typename PT, int MP, int GH, int CPL>
__global__ __launch_bounds__(kThreads) void kernel(Args a) {
  constexpr int CV = chunk_codes<BITS>();
  constexpr int SK = set_codes<BITS>();
  constexpr int U = CV / 8;              // MFMAs per chunk
  constexpr int SPD = 8 / (MP * GH);     // sets per accumulator run
  constexpr int E = SPD * GH;            // virtual rows per activation row and half
  constexpr int LGH = GH == 1 ? 0 : GH == 2 ? 1 : 2;
  constexpr int LE = E == 1 ? 0 : E == 2 ? 1 : E == 4 ? 2 : 3;
  constexpr int PPG = CV / (2 * GH);     // 16-byte activation pieces per group
  constexpr int kEarly = 2;              // activation pieces per thread and row loaded before the packed words
  constexpr int RG = CPL * 2 * GH;       // groups of one row in the wave's K-part
  constexpr int PR = RG * PT::bytes / 16;  // 16-byte parameter pieces per row and tensor
  constexpr int PW = 2 * kRows * PR;     // parameter pieces per wave
  constexpr int PL = (PW + 63) / 64;     // ... per lane
  static_assert(MP * SPD * GH == 8 && CPL % SPD == 0, "virtual row layout");
  static_assert(PPG >= 2 && PPG <= 16, "group size");

  extern __shared__ __align__(16) uint8_t smem[];
  const int xrow = a.K * 2 + 16;
  const int zero_off = MP * xrow;
  float* xsum = reinterpret_cast<float*>(smem + zero_off + kZeroBytes);
  float* red = xsum + MP * a.groups;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* prm = reinterpret_cast<uint8_t*>(red + kWaves * MP * kRows) + wave * (PW * 16);
  const int lane = threadIdx.x & 63;
  const int kp = wave % a.ks;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * (kWaves / a.ks) + wave / a.ks) * kRows;
  const int s_begin = kp * CPL;
  const int r = lane & 7, h = (lane >> 3) & 1, q = lane >> 4;
  const int64_t row = n0 + r < a.N ? n0 + r : a.N - 1;

  // 1. Loads in the order their data is needed (the load counter drains in
  //    order): activation pieces, group parameters, packed words.
  const int rp = a.K / 8;  // pieces per activation row
  // Unconditional loads from clamped positions (rows >= M and pieces past
  // the row read valid data that staging then ignores): no control flow, so
  // the loads stay in flight together.
  u32x4_t xp[MP][kEarly];
#pragma unroll
  for (int m = 0; m < MP; ++m)
#pragma unroll
    for (int e = 0; e < kEarly; ++e) {
      const int p = min(static_cast<int>(threadIdx.x) + e * kThreads, rp - 1);
      const int mm = min(m, a.M - 1);
      xp[m][e] = *reinterpret_cast<const u32x4_t*>(a.x + (static_cast<int64_t>(mm) * a.xs0 + p * 8) * 2);
    }
  __builtin_amdgcn_sched_barrier(0);

  // Group parameters of the wave's 8 rows over its K-part, as 16-byte
  // pieces (piece p: tensor p / (8 PR), row (p / PR) % 8, part p % PR).
  u32x4_t pp[PL];
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int p = min(lane + 64 * j, PW - 1);
    const int tensor = p / (kRows * PR), pr = (p / PR) % kRows, part = p % PR;
    const int64_t prow = n0 + pr < a.N ? n0 + pr : a.N - 1;
    const uint8_t* src = tensor == 0 ? a.s + (prow * a.ss0 + s_begin * 2 * GH) * PT::bytes
                                     : a.b + (prow * a.bs0 + s_begin * 2 * GH) * PT::bytes;
    pp[j] = *reinterpret_cast<const u32x4_t*>(src + part * 16);
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t wv[CPL][4];
  {
    const u32x4_t* wrow = reinterpret_cast<const u32x4_t*>(a.w + row * a.ws0) + 8 * s_begin + 4 * h + q;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const u32x4_t v = __builtin_nontemporal_load(wrow + 8 * c);
      wv[c][0] = v.x;
      wv[c][1] = v.y;
      wv[c][2] = v.z;
      wv[c][3] = v.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. Stage the activation rows (pair order of the code fragments), the
  //    group sums, and the zero block.
  if (threadIdx.x < kZeroBytes / 16)
    *reinterpret_cast<u32x4_t*>(smem + zero_off + threadIdx.x * 16) = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < PL; ++j)
    if (lane + 64 * j < PW) *reinterpret_cast<u32x4_t*>(prm + (lane + 64 * j) * 16) = pp[j];
#pragma unroll
  for (int m = 0; m < MP; ++m) {
    if (m < a.M) {
#pragma unroll
      for (int e = 0; e < kEarly; ++e) {
        const int base = wave * 64 + e * kThreads;
        if (base < rp) stage_pieces<BITS, PPG>(xp[m][e], base + lane, rp, smem + m * xrow, xsum + m * a.groups);
      }
    }
  }
  for (int m = 0; m < a.M; ++m) {
    for (int base = wave * 64 + kEarly * kThreads; base < rp; base += kThreads) {
      const int p = base + lane;
      u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
      if (p < rp) v = *reinterpret_cast<const u32x4_t*>(a.x + (static_cast<int64_t>(m) * a.xs0 + p * 8) * 2);
      stage_pieces<BITS, PPG>(v, p, rp, smem + m * xrow, xsum + m * a.groups);
    }
  }
  __syncthreads();

  // 3. MFMAs. A-operand lane (virtual row vr = l % 16, quarter q) supplies
  //    activation row m_a at chunk 4*h(vr) + q of each set, where that chunk
  //    lies in group ge_a of its half and the set is the sd_a-th of its run.
  const int vr = lane & 15;
  const int hv = vrow_half(vr), ta = vrow_t(vr);
  const int m_a = ta >> LE, sd_a = (ta >> LGH) & (SPD - 1), ge_a = ta & (GH - 1);
  const bool base_valid = m_a < a.M && ge_a == (q >> (2 - LGH));
  const uint32_t lane_x = static_cast<uint32_t>(m_a * xrow + (4 * hv + q) * CV * 2 + s_begin * SK * 2);
  const float inv_unit = BITS == 8 ? 1.0f : gemv1::pow2_reciprocal(gemv1::fp8_unit<BF16>());
  // The lane's accumulator rows vr = 4q + i hold t = 4(q/2) + i of half
  // q % 2; they are used when that half is the lane's own (h).
  const bool used = (q & 1) == h;
  auto param = [&](int tensor, int local_group) {
    return PT::load(prm + (tensor * kRows + r) * RG * PT::bytes, local_group);
  };
  const f32x4_t zero = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t acc[2] = {zero, zero};
  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  pipeline::Unroll<0, CPL>::run([&](auto cc) {
    constexpr int c = decltype(cc)::value;
    constexpr int sd = c % SPD, d = c / SPD;
    const bool valid = base_valid && sd_a == sd;
    const uint32_t aoff = valid ? lane_x + c * SK * 2 : static_cast<uint32_t>(zero_off);
    f32x4_t& D = acc[d & 1];
    pipeline::Unroll<0, U>::run([&](auto uu) {
      constexpr int u = decltype(uu)::value;
      const bf16x8_t A = *reinterpret_cast<const bf16x8_t*>(smem + aoff + 16 * u);
      const bf16x8_t B = code_fragment<BITS, u>(wv[c]);
      D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, (sd == 0 && u == 0) ? zero : D, 0, 0, 0);
    });
    if constexpr (sd == SPD - 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = i + 4 * (q >> 1);
        const int m = t >> LE, tsd = (t >> LGH) & (SPD - 1), ge = t & (GH - 1);
        const int lgrp = (d * SPD + tsd) * 2 * GH + h * GH + ge;  // within the wave's K-part
        const float xs = xsum[m * a.groups + s_begin * 2 * GH + lgrp];
        const float v = fmaf(param(0, lgrp) * inv_unit, D[i], fmaf(param(1, lgrp), xs, y[i]));
        y[i] = used && m < a.M ? v : y[i];
      }
    }
  });

  // 4. Sum each activation row's entries over the lane, then over the lanes
  //    holding the same weight row (bit 3: half, bit 4: quarter parity, and
  //    bit 5 when one activation row spans all quarters), then over the
  //    K-parts of the workgroup. Entry i of the lane belongs to activation
  //    row (i + 4(q/2)) >> LE.
  constexpr int NV = MP <= 2 ? 1 : MP == 4 ? 2 : 4;  // activation rows per lane
  float v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    float t = 0.0f;
#pragma unroll
    for (int i = j * (4 / NV); i < (j + 1) * (4 / NV); ++i) t += y[i];
    t += dpp_ror8(t);
    t = swap16_sum(t);
    if constexpr (MP == 1) t = swap32_sum(t);
    v[j] = t;
  }
  const bool writer = (lane & (MP == 1 ? 56 : 24)) == 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int m = (j * (4 / NV) + 4 * (q >> 1)) >> LE;
    if (a.ks == 1) {
      if (writer && m < a.M && n0 + r < a.N)
        store_output(a.epi, a.out, static_cast<int64_t>(m) * a.N + n0 + r, n0 + r, v[j]);
    } else if (writer && m < a.M) {
      red[(wave * MP + m) * kRows + r] = v[j];
    }
  }
  if (a.ks == 1) return;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int m = (j * (4 / NV) + 4 * (q >> 1)) >> LE;
    if (kp == 0 && writer && m < a.M && n0 + r < a.N) {
      float t = 0.0f;
      for (int k = 0; k < a.ks; ++k) t += red[((wave + k) * MP + m) * kRows + r];
      store_output(a.epi, a.out, static_cast<int64_t>(m) * a.N + n0 + r, n0 + r, t);
    }
  }
}

template <int BITS, typename PT, int MP, int GH, int CPL>
hipError_t launch(const Args& a, hipStream_t stream) {
  const size_t lds = lds_bytes(MP, a.K, a.groups, wave_param_bytes(CPL, GH, PT::bytes));
  const int64_t row_blocks = (a.N + kRows - 1) / kRows;
  const int64_t per_block = kWaves / a.ks;
  const unsigned blocks = static_cast<unsigned>((row_blocks + per_block - 1) / per_block);
  if (lds > 64 * 1024) {
    // Dynamic LDS beyond 64 KB must be allowed per kernel and device (once
    // each; not a stream operation, so it is also safe under graph capture).
    static std::atomic<uint64_t> allowed_devices{0};
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    const uint64_t bit = device < 64 ? uint64_t(1) << device : 0;
    if (bit == 0 || (allowed_devices.load() & bit) == 0) {
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(&kernel<BITS, PT, MP, GH, CPL>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMaxLdsBytes));
      if (e != hipSuccess) return e;
      allowed_devices.fetch_or(bit);
    }
  }
  hipLaunchKernelGGL((kernel<BITS, PT, MP, GH, CPL>), dim3(blocks), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace vrow

// Launchers of the two virtual-row layouts (vrow.h: 8 rows per wave, 8-bit
// codes; vrow16.h: 16 rows per wave), one translation unit per bit width.
hipError_t vrow_launch_b8(const QmmProblem& p, hipStream_t stream);
hipError_t vrow16_launch_b2(const QmmProblem& p, hipStream_t stream);
hipError_t vrow16_launch_b4(const QmmProblem& p, hipStream_t stream);
hipError_t vrow16_launch_b8(const QmmProblem& p, hipStream_t stream);

}  // namespace affon
