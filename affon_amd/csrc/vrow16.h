// Skinny decode (M <= 4, bf16 activations) on the matrix cores, with packed
// words loaded straight into the MFMA B operand: the 16-row layout.
// (vrow.h holds the 8-row layout, whose loads read whole cache lines but
// which has half the virtual-row budget; the host picks per shape.)
//
// One wave owns 16 weight rows (the 16 columns of v_mfma_f32_16x16x32_bf16)
// and a K-part of them. Lane l holds column n = l % 16 and quarter q = l / 16;
// for every "set" of four 16-byte chunks of a row, quarter q loads chunk q,
// so one load instruction reads 64 contiguous bytes of each of 16 rows, and
// the codes go from the load registers through an exact bf16 conversion into
// the B operand without touching LDS.
//
// An MFMA sums over 32 k that can span several quantization groups (a set is
// 128 k at 4 bits). Instead of splitting the MFMA, the A operand's 16 rows are
// used as "virtual rows": row vr = (m * SPD + sd) * G + gq carries activation
// row m, masked to group gq of the set, for the sd-th set of a run of SPD
// sets (G groups per set, SPD = 16 / (MP * G)). A lane whose virtual row does
// not match the set and group of the data it would supply reads zeros from a
// zero block in LDS, so masking costs one address select per set. After SPD
// sets every accumulator element holds the sum of x*q over exactly one group
// of one activation row, and the group parameters are applied once:
// y += s * D + b * sum(x over the group).
//
// Codes are exact in bf16 (FP8-read nibbles for 2/4-bit codes, n * 2^-9, with
// the unit divided out of the scale; v_cvt_f32_ubyte for 8-bit codes), the
// products are exact in the f32 accumulators, and only the order of the sums
// differs from the ordered loop: the reassociated class, like the other
// decode kernels.
#pragma once

#include "gemv1.h"
#include "lds_pipeline.h"

namespace affon {
namespace vrow16 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
using gemv1::bf16x2_t;
using gemv1::u32x4_t;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = 16;       // weight rows per wave
constexpr int kEarly = 2;       // activation pieces per thread and row loaded before the packed words
constexpr int kZeroBytes = 128; // zero block (up to 8 MFMAs of 16 bytes per set)

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
constexpr int set_codes() { return 4 * chunk_codes<BITS>(); }

// LDS (bytes): activation rows [MP][K*2 + 16] (the 16-byte pad moves
// consecutive rows to other banks), the zero block, chunk sums
// [MP][groups] f32, K-part partials [kWaves][MP*16] f32.
__host__ __device__ constexpr size_t lds_bytes(int MP, int K, int groups) {
  return static_cast<size_t>(MP) * (static_cast<size_t>(K) * 2 + 16) + kZeroBytes +
         static_cast<size_t>(MP) * groups * 4 + static_cast<size_t>(kWaves) * MP * kRows * 4;
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

// Four consecutive group parameters as f32.
template <typename PT>
struct Params4;
template <>
struct Params4<BF16> {
  u32x2_t raw;
  __device__ __forceinline__ void load(const uint8_t* p) { raw = *reinterpret_cast<const u32x2_t*>(p); }
  __device__ __forceinline__ float get(int i) const {
    const uint32_t v = raw[i / 2];
    return __uint_as_float(i % 2 == 0 ? v << 16 : v & 0xffff0000u);
  }
};
template <>
struct Params4<F32> {
  u32x4_t raw;
  __device__ __forceinline__ void load(const uint8_t* p) { raw = *reinterpret_cast<const u32x4_t*>(p); }
  __device__ __forceinline__ float get(int i) const { return __uint_as_float(raw[i]); }
};

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

// MP: activation rows rounded up to a power of two (M <= MP <= 4); G: groups
// per set; CPL: sets per wave.
template <int BITS, typename PT, int MP, int G, int CPL>
__global__ __launch_bounds__(kThreads) void kernel(Args a) {
  constexpr int CV = chunk_codes<BITS>();
  constexpr int SK = set_codes<BITS>();
  constexpr int U = CV / 8;              // MFMAs per set
  constexpr int SPD = 16 / (MP * G);     // sets per accumulator run
  constexpr int LG = G == 1 ? 0 : G == 2 ? 1 : 2;
  constexpr int LSG = MP == 1 ? 4 : MP == 2 ? 3 : 2;  // log2(SPD * G)
  constexpr int PPG = CV / (2 * G);      // 16-byte activation pieces per group
  static_assert(MP <= 4 && (1 << LSG) == SPD * G && CPL % SPD == 0, "virtual row layout");
  static_assert(PPG >= 2 && PPG <= 16, "group size");

  extern __shared__ __align__(16) uint8_t smem[];
  const int xrow = a.K * 2 + 16;
  const int zero_off = MP * xrow;
  float* xsum = reinterpret_cast<float*>(smem + zero_off + kZeroBytes);
  float* red = xsum + MP * a.groups;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kp = wave % a.ks;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * (kWaves / a.ks) + wave / a.ks) * kRows;
  const int s_begin = kp * CPL;
  const int n = lane & 15, q = lane >> 4;
  const int64_t row = n0 + n < a.N ? n0 + n : a.N - 1;

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

  // Accumulator run d covers sets s_begin + d*SPD ..; the lane's four
  // accumulator rows vr = 4q + i are four consecutive groups of one
  // activation row m_d, starting at group grp0(d).
  constexpr int ND = CPL / SPD;
  const int m_d = (4 * q) >> LSG;
  const int sd0 = ((4 * q) >> LG) & (SPD - 1);
  Params4<PT> sp[ND], bp[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) {
    const int grp0 = (s_begin + d * SPD + sd0) * G;
    sp[d].load(a.s + (row * a.ss0 + grp0) * PT::bytes);
    bp[d].load(a.b + (row * a.bs0 + grp0) * PT::bytes);
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t wv[CPL][4];
  {
    const u32x4_t* wrow = reinterpret_cast<const u32x4_t*>(a.w + row * a.ws0) + 4 * s_begin + q;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const u32x4_t v = __builtin_nontemporal_load(wrow + 4 * c);
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
  for (int m = 0; m < MP; ++m) {
    if (m < a.M) {
      uint8_t* xr = smem + m * xrow;
      float* xs = xsum + m * a.groups;
#pragma unroll
      for (int e = 0; e < kEarly; ++e) {
        const int base = wave * 64 + e * kThreads;
        if (base < rp) stage_pieces<BITS, PPG>(xp[m][e], base + lane, rp, xr, xs);
      }
      for (int base = wave * 64 + kEarly * kThreads; base < rp; base += kThreads) {
        const int p = base + lane;
        u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
        if (p < rp) v = *reinterpret_cast<const u32x4_t*>(a.x + (static_cast<int64_t>(m) * a.xs0 + p * 8) * 2);
        stage_pieces<BITS, PPG>(v, p, rp, xr, xs);
      }
    }
  }
  __syncthreads();

  // 3. MFMAs. A-operand lane (virtual row vr = l % 16, quarter q) supplies
  //    activation row m_a restricted to group gq_a of set sd_a of each run.
  const int vr = lane & 15;
  const int m_a = vr >> LSG, sd_a = (vr >> LG) & (SPD - 1), gq_a = vr & (G - 1);
  const bool base_valid = m_a < a.M && gq_a == (q >> (2 - LG));
  const uint32_t lane_x = static_cast<uint32_t>(m_a * xrow + q * CV * 2 + s_begin * SK * 2);
  const float inv_unit = BITS == 8 ? 1.0f : gemv1::pow2_reciprocal(gemv1::fp8_unit<BF16>());
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
      const int grp0 = (s_begin + d * SPD + sd0) * G;
      const f32x4_t xs = *reinterpret_cast<const f32x4_t*>(xsum + m_d * a.groups + grp0);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = fmaf(sp[d].get(i) * inv_unit, D[i], fmaf(bp[d].get(i), xs[i], y[i]));
    }
  });

  // 4. Sum the lane's groups, then the quarters that hold the same
  //    activation row (lane swaps across 16- and 32-lane halves), then the
  //    K-parts of the workgroup.
  float v = (y[0] + y[1]) + (y[2] + y[3]);
  if constexpr (MP <= 2) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  if constexpr (MP == 1) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  const bool writer = (q % (4 / MP)) == 0 && m_d < a.M;
  if (a.ks == 1) {
    if (writer && n0 + n < a.N) store_output(a.epi, a.out, static_cast<int64_t>(m_d) * a.N + n0 + n, n0 + n, v);
    return;
  }
  if (writer) red[(wave * MP + m_d) * kRows + n] = v;
  __syncthreads();
  if (kp == 0 && writer && n0 + n < a.N) {
    float t = 0.0f;
    for (int j = 0; j < a.ks; ++j) t += red[((wave + j) * MP + m_d) * kRows + n];
    store_output(a.epi, a.out, static_cast<int64_t>(m_d) * a.N + n0 + n, n0 + n, t);
  }
}

template <int BITS, typename PT, int MP, int G, int CPL>
hipError_t launch(const Args& a, hipStream_t stream) {
  const size_t lds = lds_bytes(MP, a.K, a.groups);
  const int64_t row_blocks = (a.N + kRows - 1) / kRows;
  const int64_t per_block = kWaves / a.ks;
  const unsigned blocks = static_cast<unsigned>((row_blocks + per_block - 1) / per_block);
  hipLaunchKernelGGL((kernel<BITS, PT, MP, G, CPL>), dim3(blocks), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace vrow16

}  // namespace affon
