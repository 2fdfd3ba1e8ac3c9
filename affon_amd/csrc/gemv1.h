// Single-row decode kernel (M = 1) of rocm_quantized_matmul.gemv.
//
// The decode GEMV is a pure stream over the packed weights (0.5 or 1 byte
// per weight), so the kernel is organised to keep as many bytes in flight as
// possible and to spend as few VALU instructions per weight as the exact
// arithmetic allows:
//   * a wave owns R output rows and a K-part of every row; each lane owns
//     CPL 16-byte chunks (4 packed words) per row, chunk c = part_base + lane
//     + 64*i, so one load instruction reads 1 KiB of contiguous packed words
//     of one row; all R*CPL chunk loads (and the group parameters) are issued
//     before anything waits;
//   * the activation row is staged once per workgroup in LDS, 16 bytes per
//     thread at a time, together with the sum of every chunk's activations;
//     activation and parameter loads are issued before the packed words, so
//     staging waits only for them; each wave copies its chunks into
//     registers once and reuses them for its R rows;
//   * codes are converted exactly (FP8 conversions for 2/4-bit codes,
//     v_cvt_f32_ubyte for 8-bit codes) and multiplied with v_dot2_f32_bf16
//     (bf16 x) or v_fma_f32 (f32 x); each chunk lies inside one group, so its
//     parameters are applied once per chunk: y += s * sum(x*q) + b * sum(x);
//   * when a group spans LG > 1 chunks (8-bit and 4-bit codes at group size
//     64 and up), aligned groups of LG lanes load the parameters of LG
//     different groups at once and each chunk takes its value from its lane
//     group with a quad-permute DPP move: ceil(CPL / LG) loads per row and
//     parameter instead of CPL, and fewer live registers;
//   * rows are reduced across the wave with butterfly shuffles and across the
//     K-parts of a workgroup through LDS;
//   * in paired mode the wave's first R/2 rows are rows of a gate projection
//     and the last R/2 the same rows of an up projection (same activations,
//     same strides), and the wave stores silu(gate) * up: the SiLU-gated
//     feed-forward input in one pass over both weight matrices;
//   * in grouped mode one launch runs up to kMaxSegments projections that
//     share the activation row (a decoder block's query, key and value): the
//     launch's rows are the projections' rows one after another, each
//     projection starting on a multiple of 8, so every wave lies in one
//     projection and picks its pointers once.
#pragma once

#include "device.h"
#include "internal.h"

namespace affon {
namespace gemv1 {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSegments = 4;

// Kernel modes.
constexpr int kPlain = 0, kPaired = 1, kGrouped = 2;

struct Args {
  const uint32_t* w;
  int64_t ws0;  // packed row stride in words
  const uint8_t* s;
  int64_t ss0;
  const uint8_t* b;
  int64_t bs0;
  const uint8_t* x;
  float* out;
  int64_t N;
  int cpg_shift;  // log2(16-byte chunks per group)
  int chunks;  // 16-byte chunks per row
  int part;    // chunks per K-part (a multiple of the kernel's LG)
  int ks;      // K-parts per row (waves per row block): 1, 2 or 4
  int ks_shift;  // log2(ks)
  Epilogue epi;
  // Grouped mode: projection i owns launch rows [first[i], first[i] + n[i])
  // (first[0] = 0, each first a multiple of 8), with the strides above.
  int segments;
  int64_t seg_first[kMaxSegments];
  int64_t seg_n[kMaxSegments];
  const uint32_t* seg_w[kMaxSegments];
  const uint8_t* seg_s[kMaxSegments];
  const uint8_t* seg_b[kMaxSegments];
  float* seg_out[kMaxSegments];
  const uint8_t* seg_bias[kMaxSegments];  // output bias (element type epi.bias_bf16) or null
};

// a[seg] for a uniform seg < kMaxSegments, by selects with constant indices
// (no dynamic indexing of the kernel argument block).
static_assert(kMaxSegments == 4, "pick spells out four segments");
template <typename T>
__device__ __forceinline__ T pick(const T (&a)[kMaxSegments], int seg) {
  return seg == 0 ? a[0] : seg == 1 ? a[1] : seg == 2 ? a[2] : a[3];
}

template <int BITS>
constexpr int chunk_values() { return 128 / BITS; }

// Chunks per group at group size 64 (the common case): the width of the
// lane groups that share one parameter load in the shared layout, used when
// a group spans at least that many chunks.
template <int BITS>
constexpr int kShare = BITS == 8 ? 4 : BITS == 4 ? 2 : 1;

// Value of lane (lane & ~(S-1)) | j of each aligned group of S lanes (S = 1,
// 2, 4), in every lane of the group: a quad-permute DPP move.
template <int S, int j>
__device__ __forceinline__ uint32_t lane_group_bcast(uint32_t v) {
  if constexpr (S == 1) {
    return v;
  } else {
    constexpr int lo = j, hi = S == 4 ? j : 2 + j;  // quad lanes 0-1 / 2-3 read
    constexpr int ctrl = lo | (lo << 2) | (hi << 4) | (hi << 6);
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), ctrl, 0xf, 0xf, false));
  }
}

// Chunk i's group parameter, given the shared-layout loads v of one row
// (load i / LG, lane (lane & ~(LG-1)) | (i % LG)). i is a constant after
// unrolling, so the selects fold to one DPP move.
template <int LG, int N>
__device__ __forceinline__ uint32_t param_of(const uint32_t (&v)[N], int i) {
  const uint32_t x = v[i / LG];
  const int j = i % LG;
  return j == 0   ? lane_group_bcast<LG, 0>(x)
         : j == 1 ? lane_group_bcast<LG, 1 % LG>(x)
         : j == 2 ? lane_group_bcast<LG, 2 % LG>(x)
                  : lane_group_bcast<LG, 3 % LG>(x);
}

// Activations of one chunk as staged in LDS: kPieces 16-byte pieces (2..16).
// Piece j of chunk c sits in slot j at uint4 index j * stride + (c ^ swizzle
// (j)), stride = chunks rounded up to 16. The swizzle spreads the pieces that
// one 16-lane LDS phase writes (kPieces consecutive pieces of 16 / kPieces
// chunks) over all 64 banks, and keeps the compute phase's reads (one slot of
// 16 consecutive chunks) conflict-free.
template <int BITS, typename XT>
struct XStage {
  static constexpr int kDwords = chunk_values<BITS>() * XT::bytes / 4;  // per chunk
  static constexpr int kPieces = kDwords / 4;
  static constexpr int kPieceShift = kPieces == 2 ? 1 : kPieces == 4 ? 2 : kPieces == 8 ? 3 : 4;
  static_assert((1 << kPieceShift) == kPieces, "pieces per chunk");
  __host__ __device__ static constexpr int stride(int chunks) { return (chunks + 15) & ~15; }
  __device__ static int slot(int c, int j, int stride) { return j * stride + (c ^ ((j * (16 / kPieces)) & 15)); }
};

// LDS of one workgroup: the staged activations, one f32 sum per chunk, then
// kWaves * R K-part partials.
__host__ __device__ constexpr size_t lds_size_for(int pieces_per_chunk, int chunks, int R) {
  return static_cast<size_t>(pieces_per_chunk) * ((chunks + 15) & ~15) * 16 + (static_cast<size_t>(chunks) + kWaves * R) * 4;
}
template <int BITS, typename XT, int R>
__host__ __device__ constexpr size_t lds_size(int chunks) {
  return lds_size_for(XStage<BITS, XT>::kPieces, chunks, R);
}

__device__ __forceinline__ bf16x2_t pack2(float a, float b) { return bf16x2_t{static_cast<__bf16>(a), static_cast<__bf16>(b)}; }

// Exact decoding of packed codes.
//
// 4-bit and 2-bit codes: a byte holding a code n < 16 read as an FP8 E4M3
// value is exactly n * 2^-9 (the subnormal range and the first binade of E4M3
// are evenly spaced by 2^-9), so one v_cvt_scalef32_pk_bf16_fp8 (bf16) or
// v_cvt_scalef32_pk_f32_fp8 (f32) turns two codes into exact operands. The
// unit is measured in the kernel (fp8_unit) rather than assumed, and the
// conversions scale by its reciprocal (a power of two), so they return the
// codes themselves. 8-bit codes use v_cvt_f32_ubyteN (one exact conversion
// each).
//
// Operand order: bf16 activations are staged in LDS in the pair order the
// conversions produce (see stage_chunk), f32 activations in k order.

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// `scale` multiplies the converted values; a power of two keeps them exact
// (the kernel passes 1 / unit, so the codes come out as integers).
__device__ __forceinline__ bf16x2_t fp8_pair_bf16(uint32_t bytes, bool high, float scale = 1.0f) {
  return high ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(bytes, scale, true)
              : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(bytes, scale, false);
}

__device__ __forceinline__ f32x2_t fp8_pair_f32(uint32_t bytes, bool high, float scale = 1.0f) {
  return high ? __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(bytes, scale, true)
              : __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(bytes, scale, false);
}

// Value of one code step after the FP8 conversion (2^-9 for OCP E4M3).
template <typename XT>
__device__ __forceinline__ float fp8_unit() {
  if constexpr (XT::bytes == 2) {
    const bf16x2_t v = fp8_pair_bf16(0x08u, false);
    return static_cast<float>(v.x) * 0.125f;
  } else {
    return fp8_pair_f32(0x08u, false).x * 0.125f;
  }
}

// 1 / u for a power of two u, exactly: u = 0.5 * 2^e, so 1 / u = 2^(1 - e).
__device__ __forceinline__ float pow2_reciprocal(float u) {
  return __builtin_amdgcn_ldexpf(1.0f, 1 - __builtin_amdgcn_frexp_expf(u));
}

__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Bytes of one word holding codes in their low bits, and the k index (within
// the word) of the code in byte j of mask t.
//   4-bit: mask 0 = w & 0x0f0f0f0f (k = 2j), mask 1 = (w >> 4) & .. (k = 2j+1)
//   2-bit: mask t = (w >> 2t) & 0x03030303 (k = 4j + t)
template <int BITS>
__device__ __forceinline__ int code_k(int t, int j) {
  return BITS == 4 ? 2 * j + t : 4 * j + t;
}

// Staged bf16 dword (within a chunk) that holds the activations of the code
// pair (bytes 2h, 2h+1 of mask t) of word i. Each 16-byte piece of staged
// activations holds the pairs of 8 consecutive k, so staging is local to a
// piece: 4-bit pieces are words (pairs (0,2) (4,6) (1,3) (5,7)), 2-bit pieces
// are half words (pairs (0,4) (1,5) (2,6) (3,7)).
template <int BITS>
__device__ __forceinline__ int pair_slot(int i, int t, int h) {
  return BITS == 4 ? i * 4 + 2 * t + h : i * 8 + 4 * h + t;
}

// Sum over one 16-byte chunk (4 words) of x*q, exactly in the codes: the fp8
// conversions of 2/4-bit codes take `scale` = 1 / unit (a power of two, so
// the converted codes are the integers themselves); 8-bit codes convert
// directly. xr holds the chunk's activations as staged: bf16 pairs, or f32
// values in k order.
template <int BITS, typename XT>
__device__ __forceinline__ float chunk_dot(const uint32_t* words, const uint32_t* xr, float scale = 1.0f) {
  constexpr int P = 32 / BITS;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = words[i];
    if constexpr (BITS == 8) {
      const uint32_t v = opaque(w);
      float q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) q[j] = static_cast<float>((v >> (8 * j)) & 0xffu);
      if constexpr (XT::bytes == 2) {
        acc = __builtin_amdgcn_fdot2_f32_bf16(pack2(q[0], q[1]), __builtin_bit_cast(bf16x2_t, xr[2 * i]), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(pack2(q[2], q[3]), __builtin_bit_cast(bf16x2_t, xr[2 * i + 1]), acc,
                                              false);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = fmaf(__uint_as_float(xr[4 * i + j]), q[j], acc);
      }
    } else {
      constexpr int T = BITS == 4 ? 2 : 4;  // masks per word
      constexpr uint32_t kMask = BITS == 4 ? 0x0f0f0f0fu : 0x03030303u;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint32_t m = (w >> (BITS * t)) & kMask;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if constexpr (XT::bytes == 2) {
            acc = __builtin_amdgcn_fdot2_f32_bf16(fp8_pair_bf16(m, h == 1, scale),
                                                  __builtin_bit_cast(bf16x2_t, xr[pair_slot<BITS>(i, t, h)]), acc,
                                                  false);
          } else {
            const f32x2_t q = fp8_pair_f32(m, h == 1, scale);
            acc = fmaf(__uint_as_float(xr[i * P + code_k<BITS>(t, 2 * h)]), q.x, acc);
            acc = fmaf(__uint_as_float(xr[i * P + code_k<BITS>(t, 2 * h + 1)]), q.y, acc);
          }
        }
      }
    }
  }
  return acc;
}

// Low (high) bf16 halves of dwords a and b as one pair: a's in the low half.
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// One 16-byte piece of bf16 activations (8 consecutive k) in the pair order
// chunk_dot consumes (pair_slot).
template <int BITS>
__device__ __forceinline__ u32x4_t permute_bf16_piece(u32x4_t d) {
  if constexpr (BITS == 8) {
    return d;
  } else if constexpr (BITS == 4) {
    return u32x4_t{pair_lo(d.x, d.y), pair_lo(d.z, d.w), pair_hi(d.x, d.y), pair_hi(d.z, d.w)};
  } else {
    return u32x4_t{pair_lo(d.x, d.z), pair_hi(d.x, d.z), pair_lo(d.y, d.w), pair_hi(d.y, d.w)};
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum of v over the 64 lanes of the wave, returned in every lane: DPP adds
// within rows of 16 (quad swaps, then row rotations by 4 and 8), then the
// four row sums are read out of lanes 0, 16, 32 and 48.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x128>(v);  // row_ror:8
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Wave totals of R per-lane values (R = 1, 2, 4, 8), uniform. Rows are
// paired first so that the lane reductions run on fewer registers:
// permlane32_swap turns rows (2k, 2k+1) into one register holding row 2k's
// 32-lane partials in lanes 0-31 and row 2k+1's in lanes 32-63;
// permlane16_swap turns two such registers into one whose 16-lane groups hold
// rows (4m, 4m+2, 4m+1, 4m+3). The 16-lane groups are then summed with DPP
// and read out of lanes 0, 16, 32 and 48.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
template <int R>
__device__ __forceinline__ void wave_totals(const float (&y)[R], float (&tot)[R]) {
  if constexpr (R == 1) {
    tot[0] = wave_sum(y[0]);
  } else {
    float h[R / 2];
#pragma unroll
    for (int k = 0; k < R / 2; ++k) {
      const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(y[2 * k]), __float_as_uint(y[2 * k + 1]), false,
                                                      false);
      h[k] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    if constexpr (R == 2) {
      const float v = row_sum16(h[0]);
      tot[0] = lane_value(v, 0) + lane_value(v, 16);
      tot[1] = lane_value(v, 32) + lane_value(v, 48);
    } else {
#pragma unroll
      for (int m = 0; m < R / 4; ++m) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(h[2 * m]), __float_as_uint(h[2 * m + 1]), false,
                                                        false);
        const float v = row_sum16(__uint_as_float(p[0]) + __uint_as_float(p[1]));
        tot[4 * m] = lane_value(v, 0);
        tot[4 * m + 2] = lane_value(v, 16);
        tot[4 * m + 1] = lane_value(v, 32);
        tot[4 * m + 3] = lane_value(v, 48);
      }
    }
  }
}

// Sum of v over aligned groups of G consecutive lanes (G = 2..16), in every
// lane of the group: quad swaps, then the half-row mirror (lane i of 8 reads
// lane 7-i, so each quad adds the other) and the row mirror (i of 16 reads
// 15-i).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp<0xb1>(v);   // quad_perm [1,0,3,2]
  if constexpr (G >= 4) v += dpp<0x4e>(v);   // quad_perm [2,3,0,1]
  if constexpr (G >= 8) v += dpp<0x141>(v);  // row_half_mirror
  if constexpr (G >= 16) v += dpp<0x140>(v); // row_mirror
  return v;
}

// Stages the 64 pieces base .. base+63 of the activation row (lane order;
// pieces >= count are absent) into LDS: the permuted piece into its slot and
// the chunk's sum into xsum. The whole wave calls it (the group sums read
// neighbouring lanes).
template <int BITS, typename XT>
__device__ __forceinline__ void stage_pieces(u32x4_t v, int p, int count, uint4* xs, float* xsum, int stride) {
  using XS = XStage<BITS, XT>;
  const bool valid = p < count;
  u32x4_t o;
  float sum;
  if constexpr (XT::bytes == 2) {
    o = permute_bf16_piece<BITS>(v);
    // (Elements are copied to scalars first: a bit cast applied directly to a
    // vector element reads element 0 with this compiler.)
    const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
    const uint32_t o0 = o.x, o1 = o.y, o2 = o.z, o3 = o.w;
    sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o0), ones, 0.0f, false);
    sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o1), ones, sum, false);
    sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o2), ones, sum, false);
    sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o3), ones, sum, false);
  } else {
    o = v;
    sum = (__uint_as_float(v.x) + __uint_as_float(v.y)) + (__uint_as_float(v.z) + __uint_as_float(v.w));
  }
  sum = group_sum<XS::kPieces>(valid ? sum : 0.0f);
  const int c = p >> XS::kPieceShift, j = p & (XS::kPieces - 1);
  if (valid) {
    xs[XS::slot(c, j, stride)] = make_uint4(o.x, o.y, o.z, o.w);
    if (j == 0) xsum[c] = sum;
  }
}

// LG: lanes per parameter-sharing lane group (1, or kShare<BITS> when every
// group spans at least LG chunks and K-parts start on multiples of LG).
template <int BITS, typename XT, typename PT, int R, int CPL, int MODE, int LG>
__global__ __launch_bounds__(kThreads) void kernel(Args a) {
  constexpr bool PAIR = MODE == kPaired;
  static_assert(!PAIR || R % 2 == 0, "paired rows");
  constexpr int RO = PAIR ? R / 2 : R;  // output rows per wave
  using XS = XStage<BITS, XT>;
  constexpr int XDW = XS::kDwords;
  extern __shared__ uint32_t smem[];
  const int stride = XS::stride(a.chunks);
  uint4* xs_lds = reinterpret_cast<uint4*>(smem);
  float* xsum_lds = reinterpret_cast<float*>(smem + XS::kPieces * stride * 4);
  float* red = xsum_lds + a.chunks;

  // The wave index is uniform; reading it into a scalar register keeps all
  // row addressing on the scalar unit.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kp = wave & (a.ks - 1);
  int64_t n0 = (static_cast<int64_t>(blockIdx.x) * (kWaves >> a.ks_shift) + (wave >> a.ks_shift)) * RO;
  const int c_begin = kp * a.part;
  const int c_end = min(a.chunks, c_begin + a.part);
  // The wave's projection: the launch's, or in grouped mode the one whose
  // rows hold n0 (all uniform).
  const uint32_t* W = a.w;
  const uint8_t* S = a.s;
  const uint8_t* B = a.b;
  float* out = a.out;
  int64_t N = a.N;
  Epilogue epi = a.epi;
  if constexpr (MODE == kGrouped) {
    int seg = 0;
    if (a.segments > 1 && n0 >= a.seg_first[1]) seg = 1;
    if (a.segments > 2 && n0 >= a.seg_first[2]) seg = 2;
    if (a.segments > 3 && n0 >= a.seg_first[3]) seg = 3;
    n0 -= pick(a.seg_first, seg);
    N = pick(a.seg_n, seg);
    W = pick(a.seg_w, seg);
    S = pick(a.seg_s, seg);
    B = pick(a.seg_b, seg);
    out = pick(a.seg_out, seg);
    epi.bias = pick(a.seg_bias, seg);
    epi.kind = epi.bias != nullptr ? kEpiBias : kEpiNone;
  }
  // Row r of the wave: output row n0 + r % RO of the first (r < RO) or the
  // second projection.
  auto row_of = [&](int r) {
    const int64_t n = n0 + (r % RO);
    return n < N ? n : N - 1;
  };
  auto second = [](int r) { return PAIR && r >= RO; };

  // 1. Loads, in the order their data is needed (the load counter drains in
  //    order): the activation pieces this thread stages, the group parameters
  //    of its chunks, then the packed words.
  constexpr int kEarly = 8;  // pieces per thread loaded before the packed words
  const int pieces = a.chunks * XS::kPieces;
  const int wave_piece = wave * 64;
  // A round of pieces is loaded when any of it exists (a uniform test, so
  // absent rounds cost no vector instructions); lanes past the row read its
  // last piece, which staging ignores.
  u32x4_t xp[kEarly];
  auto load_round = [&](int e) {
    const int base = wave_piece + e * kThreads;
    if (base < pieces)
      xp[e] = *reinterpret_cast<const u32x4_t*>(a.x + static_cast<uint32_t>(min(base + lane, pieces - 1)) * 16u);
  };
  load_round(0);
  load_round(1);
  if (wave_piece + 2 * kThreads < pieces) {  // rows of more than two rounds (one uniform test for the rest)
#pragma unroll
    for (int e = 2; e < kEarly; ++e) load_round(e);
  }
  __builtin_amdgcn_sched_barrier(0);

  // Group parameters; rows have uniform bases, lanes a 32-bit byte offset
  // shared by all rows.
  //   Per-lane layout: load i of a lane fetches the group of its chunk i.
  //   Shared layout (LG > 1 lanes per lane group): in load j, lane l
  //   fetches the group of chunk c_begin + (l & ~(LG-1)) + 64 (LG j + l % LG).
  //   Chunk i of every lane of that lane group lies in the same group when
  //   i = LG j + l % LG, because the LG-aligned run of chunks holding the
  //   lane group's chunks i lies inside one group. A row then needs
  //   ceil(CPL / LG) loads of each parameter instead of CPL, and chunk i reads
  //   its value from lane (l & ~(LG-1)) | (i % LG) of load i / LG, by a DPP
  //   move where it is used. (Aligned lane groups are wholly inside or
  //   outside the K-part, so the lane read from is active whenever the
  //   reading lane is.)
  static_assert(LG == 1 || LG == kShare<BITS>, "lane group width");
  constexpr int kLoads = (CPL + LG - 1) / LG;
  uint32_t sraw[R][kLoads], braw[R][kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int c = c_begin + (lane & ~(LG - 1)) + 64 * (LG * i + (lane & (LG - 1)));
    const uint32_t goff = static_cast<uint32_t>((c < c_end ? c : 0) >> a.cpg_shift) * PT::bytes;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = row_of(r);
      const uint8_t* srow = (second(r) ? a.epi.s2 : S) + n * a.ss0 * PT::bytes;
      const uint8_t* brow = (second(r) ? a.epi.b2 : B) + n * a.bs0 * PT::bytes;
      if constexpr (PT::bytes == 2) {  // widened to f32 bits once per load
        sraw[r][i] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(srow + goff)) << 16;
        braw[r][i] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(brow + goff)) << 16;
      } else {
        sraw[r][i] = *reinterpret_cast<const uint32_t*>(srow + goff);
        braw[r][i] = *reinterpret_cast<const uint32_t*>(brow + goff);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t wv[R][CPL][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = row_of(r);
    const u32x4_t* row = reinterpret_cast<const u32x4_t*>((second(r) ? a.epi.w2 : W) + n * a.ws0);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = c_begin + lane + 64 * i;
      const int cc = c < c_end ? c : 0;  // idle lanes read chunk 0 and discard it
      const u32x4_t v = __builtin_nontemporal_load(row + cc);
      wv[r][i][0] = v.x;
      wv[r][i][1] = v.y;
      wv[r][i][2] = v.z;
      wv[r][i][3] = v.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. Stage the activation row and the chunk sums (waits only for the
  //    activation loads). Rows longer than kEarly pieces per thread load the
  //    rest here.
#pragma unroll
  for (int e = 0; e < kEarly; ++e) {
    const int base = wave_piece + e * kThreads;
    if (base < pieces) stage_pieces<BITS, XT>(xp[e], base + lane, pieces, xs_lds, xsum_lds, stride);
  }
  for (int base = wave_piece + kEarly * kThreads; base < pieces; base += kThreads) {
    const int p = base + lane;
    u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
    if (p < pieces) v = *reinterpret_cast<const u32x4_t*>(a.x + static_cast<uint32_t>(p) * 16u);
    stage_pieces<BITS, XT>(v, p, pieces, xs_lds, xsum_lds, stride);
  }
  __syncthreads();

  // 3. Decode, multiply, apply group parameters per chunk. The fp8
  // conversions read a code n as n * unit; scaling them by 1 / unit (a power
  // of two, uniform across the wave) makes the converted codes exact integers.
  const float code_scale =
      BITS == 8 ? 1.0f : __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(pow2_reciprocal(fp8_unit<XT>()))));
  auto param = [](uint32_t bits) { return __uint_as_float(bits); };
  float y[R];
#pragma unroll
  for (int r = 0; r < R; ++r) y[r] = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = c_begin + lane + 64 * i;
    if (c < c_end) {
      uint32_t xr[XDW];
#pragma unroll
      for (int j = 0; j < XS::kPieces; ++j) {
        const uint4 v = xs_lds[XS::slot(c, j, stride)];
        xr[4 * j] = v.x;
        xr[4 * j + 1] = v.y;
        xr[4 * j + 2] = v.z;
        xr[4 * j + 3] = v.w;
      }
      const float xsum = xsum_lds[c];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float acc = chunk_dot<BITS, XT>(wv[r][i], xr, code_scale);
        y[r] = fmaf(param(param_of<LG>(sraw[r], i)), acc, fmaf(param(param_of<LG>(braw[r], i)), xsum, y[r]));
      }
    }
  }

  // 4. Reduce across the wave, then across K-parts.
  {
    float tot[R];
    wave_totals<R>(y, tot);
#pragma unroll
    for (int r = 0; r < R; ++r) y[r] = tot[r];
  }
  // Lane o < RO stores output row n0 + o.
  auto finish = [&](float v, float up) {
    if (n0 + lane >= N) return;
    if constexpr (PAIR)
      out[n0 + lane] = silu(v) * up;
    else
      store_output(epi, out, n0 + lane, n0 + lane, v);
  };
  if (a.ks == 1) {
    if (lane < RO) {
      float v = y[0], up = y[RO % R];
#pragma unroll
      for (int r = 1; r < RO; ++r) {
        v = lane == r ? y[r] : v;
        up = lane == r ? y[(r + RO) % R] : up;
      }
      finish(v, up);
    }
    return;
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) red[wave * R + r] = y[r];
  }
  __syncthreads();
  if (kp == 0 && lane < RO) {
    float v = 0.0f, up = 0.0f;
    for (int j = 0; j < a.ks; ++j) {
      v += red[(wave + j) * R + lane];
      if constexpr (PAIR) up += red[(wave + j) * R + RO + lane];
    }
    finish(v, up);
  }
}

template <int BITS, typename XT, typename PT, int R, int CPL, int MODE, int LG>
hipError_t launch(const Args& a, hipStream_t stream) {
  constexpr int RO = MODE == kPaired ? R / 2 : R;
  const size_t lds = lds_size<BITS, XT, R>(a.chunks);
  const int64_t row_blocks = (a.N + RO - 1) / RO;
  const int64_t per_block = kWaves / a.ks;
  const unsigned blocks = static_cast<unsigned>((row_blocks + per_block - 1) / per_block);
  hipLaunchKernelGGL((kernel<BITS, XT, PT, R, CPL, MODE, LG>), dim3(blocks), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace gemv1

// Per-bits entry points (one translation unit each).
bool gemv1_supports(const QmmProblem& p);
hipError_t gemv1_launch_b2(const QmmProblem& p, hipStream_t stream);
hipError_t gemv1_launch_b4(const QmmProblem& p, hipStream_t stream);
hipError_t gemv1_launch_b8(const QmmProblem& p, hipStream_t stream);
hipError_t gemv1_group_launch_b2(const QmmProblem* group, int count, hipStream_t stream);
hipError_t gemv1_group_launch_b4(const QmmProblem* group, int count, hipStream_t stream);
hipError_t gemv1_group_launch_b8(const QmmProblem* group, int count, hipStream_t stream);

}  // namespace affon
