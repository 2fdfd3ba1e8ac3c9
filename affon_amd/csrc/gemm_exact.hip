// Prefill GEMM of the reassociated class for 4-bit codes with bf16
// activations and bf16 group parameters, for any group size the packed
// format allows in whole 32-value units (32, 64, 128): the default policy's
// path for tall activations where the group-scaling GEMM (gemm_re.hip), which
// scales whole 64-value groups per K step, does not apply -- groups of 32.
//
// Counterpart of the reference's matrix paths, which decode weights to f32
// and are classified "reassociated" (docs/core/quantized-inference.md:
// 138-139,151-158,175-177). Arithmetic:
//
//   y = sum_k x_k * (s_g q_k)  +  sum_g b_g * X_g,     X_g = sum_{k in g} x_k.
//
// s_g q_k is split exactly into two bf16 planes through the scale: s = sh +
// sl with sh the top four significant bits of s (bf16 has eight) and sl the
// rest, so sh*q and sl*q have at most eight significant bits each (q < 16)
// and are exact in bf16. Both planes go into v_mfma_f32_32x32x16_bf16
// against the same activation fragment, so every product x * (sh q) and
// x * (sl q) is exact and the sums are f32 accumulations. No decoded weight
// is rounded. The bias term is a small matrix product over
// groups, as in gemm_re.hip: a pre-pass forms X for every activation row and
// group in f32 and splits it exactly into three bf16 planes (X = X1 + X2 +
// X3), and after the K loop each wave adds sum_t X_t * b^T from global memory,
// 16 groups per MFMA.
//
// Work mapping: workgroup tile 256 (rows) x 128 (columns), four waves in a
// 2 x 2 arrangement, one per SIMD; wave (mi, ni) computes rows 128 mi ..
// and columns 64 ni .. as 4 x 2 accumulator tiles of 32 x 32. K steps of 64;
// MFMA kk (0..3) of lane half h covers chunk 4h + kk of the step (8 k each),
// so a lane's codes of one column and step are 16 contiguous bytes. Each
// wave decodes the 64 columns it multiplies; the decode of chunk kk + 1 runs
// on the vector ALU beside chunk kk's sixteen MFMAs.
//
// Transfers, all direct global-to-LDS and counted: activations (256 rows x
// 128 bytes per step) into a 3-stage ring two steps ahead; packed words (64
// bytes per column and pair of steps) and 16-byte scale windows per column
// and pair of steps into two buffers, a pair of steps ahead. One barrier per
// step orders the shared tiles. Wave w moves the packed words and scale
// windows of columns 64 (w % 2) + 32 (w / 2) + (0..31).

#include "lds_pipeline.h"

namespace affon {
namespace {

using namespace pipeline;

constexpr int kRows = 256;                 // workgroup tile rows
constexpr int kCols = 128;                 // workgroup tile columns
constexpr int kAStage = kRows * 128;       // bytes: 256 rows x 64 k of bf16
constexpr int kAStages = 3;
constexpr int kAOps = kRows / 8 / kWaves;  // activation transfers per wave and step (1 KiB each)
constexpr int kWRun = 64;                  // packed bytes per column and pair of steps
constexpr int kWWave = 32 * kWRun;         // per wave and buffer: 32 columns
constexpr int kWOps = kWWave / 1024;       // packed-word transfers per wave and pair
constexpr int kPWin = 16;                  // bytes of a scale window (per column, pair)
constexpr int kPWave = 32 * kPWin;         // per wave and buffer
constexpr int kPOps = 32 * 4 / 64;         // dword transfers per wave and pair (scales)
constexpr int kPairOps = kWOps + kPOps;
constexpr int kXChunk = 16;                // groups per bias-term MFMA

static_assert(kAOps == 8 && kWOps == 2 && kPOps == 2, "transfer counts assumed by the waits below");

// Physical 16-byte slot of logical slot q in local activation row r: the
// fragment reads (consecutive rows, one slot) are bank-conflict free.
__device__ __forceinline__ int a_slot(int r, int q) { return q ^ (r & 7) ^ ((r >> 3) & 1); }

// Physical slot of logical slot q (0..3) in column c's 64-byte packed run.
__device__ __forceinline__ int w_slot(int c, int q) { return q ^ ((c >> 2) & 3); }

// Groups of one K range, padded to whole bias-term chunks (the planes' row length).
__host__ __device__ constexpr int padded_groups(int groups) { return (groups + kXChunk - 1) / kXChunk * kXChunk; }

// X = sum of the `group` activations of one row and group in f32, as three
// bf16 planes whose sum is X exactly. Layout [range][plane][row][gr]: group g
// of K range g / range_groups at entry g % range_groups of a row of gr
// entries; entries from range_groups to gr are zero. One thread per (row,
// entry).
__global__ __launch_bounds__(256) void exact_group_sums_kernel(const uint16_t* x, int64_t xs0, int M, int group,
                                                               int range_groups, int gr, int ranges,
                                                               uint16_t* planes) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t entries = static_cast<int64_t>(ranges) * gr;
  if (i >= static_cast<int64_t>(M) * entries) return;
  const int row = static_cast<int>(i / entries);
  const int e = static_cast<int>(i % entries);
  const int range = e / gr, gl = e % gr;
  uint16_t h1 = 0, h2 = 0, h3 = 0;
  if (gl < range_groups) {
    const uint16_t* src = x + row * xs0 + static_cast<int64_t>(range * range_groups + gl) * group;
    float sum = 0.0f;
    for (int c = 0; c < group; c += 8) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sum += __uint_as_float(v[q] << 16);
        sum += __uint_as_float(v[q] & 0xffff0000u);
      }
    }
    h1 = f32_to_bf16_bits(sum);
    if (__builtin_isfinite(sum)) {
      const float r1 = sum - bf16_bits_to_f32(h1);  // exact
      h2 = f32_to_bf16_bits(r1);
      h3 = f32_to_bf16_bits(r1 - bf16_bits_to_f32(h2));  // exact: the remaining bits fit bf16
    }
  }
  const int64_t plane = static_cast<int64_t>(M) * gr;
  const int64_t at = static_cast<int64_t>(range) * 3 * plane + static_cast<int64_t>(row) * gr + gl;
  planes[at] = h1;
  planes[plane + at] = h2;
  planes[2 * plane + at] = h3;
}

// Decode of one packed word (codes 0..7 of a column) into the two exact bf16
// planes of s*q, in k order, as seven pieces that the main loop spreads over
// the MFMA slots of a chunk. The group's scale arrives split in two, s = sh +
// sl, sh keeping the sign, the exponent and the top three stored mantissa
// bits of s's f32 pattern and sl = s - sh (exact): each half has at most four
// significant bits, so with a code q < 16 (4 bits) each product sh*q, sl*q has
// at most eight, is exact in f32, and its f32 pattern's high half is exactly
// its bf16 value. Both halves carry the 2^9 of the FP8 reading of a code (a
// byte n < 16 reads as n * 2^-9 in E4M3).
struct ExactTmp {
  uint32_t lo, hi;
  f32x2_t l, h;
  uint32_t ph[4], pl[4];  // f32 patterns of sh*q and sl*q of four codes
};

__device__ __forceinline__ uint32_t high_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);  // a's high 16 bits low, b's high
}

// Splits a scale (f32) into the halves above, each times 2^9.
__device__ __forceinline__ void split_scale(float s, float* sh, float* sl) {
  const float h = __uint_as_float(__float_as_uint(s) & 0xfff00000u);
  *sh = h * 512.0f;
  *sl = (s - h) * 512.0f;  // s - h is exact
}

template <int J>
__device__ __forceinline__ void exact_piece(uint32_t w, float sh, float sl, ExactTmp& d, u32x4_t& hi, u32x4_t& lo) {
  if constexpr (J == 0) {
    d.lo = w & 0x0f0f0f0fu;         // codes 0, 2, 4, 6
    d.hi = (w >> 4) & 0x0f0f0f0fu;  // codes 1, 3, 5, 7
  } else if constexpr (J == 1 || J == 4) {
    constexpr bool kHigh = J == 4;  // codes 4..7
    d.l = __builtin_amdgcn_cvt_pk_f32_fp8(d.lo, kHigh);
    d.h = __builtin_amdgcn_cvt_pk_f32_fp8(d.hi, kHigh);
    d.ph[0] = __float_as_uint(d.l.x * sh);
    d.ph[1] = __float_as_uint(d.h.x * sh);
    d.ph[2] = __float_as_uint(d.l.y * sh);
    d.ph[3] = __float_as_uint(d.h.y * sh);
  } else if constexpr (J == 2 || J == 5) {
    constexpr int o = J == 2 ? 0 : 2;
    d.pl[0] = __float_as_uint(d.l.x * sl);
    d.pl[1] = __float_as_uint(d.h.x * sl);
    d.pl[2] = __float_as_uint(d.l.y * sl);
    d.pl[3] = __float_as_uint(d.h.y * sl);
    hi[o] = high_halves(d.ph[0], d.ph[1]);
    hi[o + 1] = high_halves(d.ph[2], d.ph[3]);
  } else {
    constexpr int o = J == 3 ? 0 : 2;
    lo[o] = high_halves(d.pl[0], d.pl[1]);
    lo[o + 1] = high_halves(d.pl[2], d.pl[3]);
  }
}

__device__ __forceinline__ void exact_word(uint32_t w, float sh, float sl, u32x4_t& hi, u32x4_t& lo) {
  ExactTmp d;
  exact_piece<0>(w, sh, sl, d, hi, lo);
  exact_piece<1>(w, sh, sl, d, hi, lo);
  exact_piece<2>(w, sh, sl, d, hi, lo);
  exact_piece<3>(w, sh, sl, d, hi, lo);
  exact_piece<4>(w, sh, sl, d, hi, lo);
  exact_piece<5>(w, sh, sl, d, hi, lo);
  exact_piece<6>(w, sh, sl, d, hi, lo);
}

struct ExactArgs {
  TileArgs t;
  const uint16_t* planes;  // [range][3][M][gr] bf16
  int gr;                  // entries per plane row (the range's groups, padded)
  int groups;              // groups per parameter row (K / group)
};

template <int MI>
__device__ __forceinline__ void exact_tile(const ExactArgs& ea, uint8_t* lds_a, uint8_t* lds_w, uint8_t* lds_p, int m0,
                                           int n0, int split) {
  const TileArgs& a = ea.t;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ni = wave & 1;  // wave = 2*mi + ni
  const int li = lane & 31;
  const int lh = lane >> 5;
  const int steps = a.split_steps;  // even
  const int s0 = split * steps;     // even: pairs of local and global steps agree

  // ---- transfer offsets (constant over the loop) ----
  // Activations: wave w fills local rows 64w .. 64w+63, instruction i rows
  // 8(8w+i) .. +7; lane L -> row +L/8, physical slot L%8.
  uint32_t a_off[kAOps];
#pragma unroll
  for (int i = 0; i < kAOps; ++i) {
    const int r = 64 * wave + 8 * i + (lane >> 3);
    const int q = a_slot(r, lane & 7);  // logical slot (the swizzle is an involution)
    const int row = min(m0 + r, a.M - 1);  // rows past M repeat the last row
    a_off[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(a.xs0 * 2) + 16 * q;
  }
  // Packed words: this wave moves columns 64*ni + 32*MI + (0..31);
  // instruction j covers 16 of them, lane L -> column 16j + L/4, physical slot L%4.
  uint32_t w_off[kWOps];
#pragma unroll
  for (int j = 0; j < kWOps; ++j) {
    const int c = 16 * j + (lane >> 2);
    const int col = min(n0 + 64 * ni + 32 * MI + c, a.N - 1);  // columns past N feed unstored outputs
    w_off[j] = static_cast<uint32_t>(col) * static_cast<uint32_t>(a.ws0 * 4) + 16 * w_slot(c, lane & 3);
  }
  // Scale windows: instruction i (0, 1) lane L -> column 16i + L/4, dword L%4 of the window.
  uint32_t s_off[kPOps];
  const int row_dwords = ea.groups / 2;  // bf16 scales per row, in dwords
  auto window = [&](int pair) { return (pair * 128) >> (6 + a.group_shift); };  // first dword of a pair's groups
#pragma unroll
  for (int i = 0; i < kPOps; ++i) {
    const int col = min(n0 + 64 * ni + 32 * MI + 16 * i + (lane >> 2), a.N - 1);
    s_off[i] = static_cast<uint32_t>(col) * static_cast<uint32_t>(a.ss0 * 2);
  }

  const uint32_t a_lds = lds_address(lds_a);
  const uint32_t w_lds = lds_address(lds_w) + kWWave * wave;  // + buffer * 4 * kWWave
  const uint32_t p_lds = lds_address(lds_p) + kPWave * wave;  // + buffer * 4 * kPWave

  auto issue_a = [&](int t) {  // local step t (clamped to the range)
    const int g = s0 + min(t, steps - 1);
    const uint8_t* base = sadd(a.x, 128 * g);
    const uint32_t dst = a_lds + kAStage * (t % kAStages) + 1024 * kAOps * wave;
#pragma unroll
    for (int i = 0; i < kAOps; ++i) dma16(base, a_off[i], dst + 1024 * i);
  };
  auto issue_pair = [&](int pr) {  // local pair pr (clamped)
    const int gp = (s0 >> 1) + min(pr, (steps >> 1) - 1);
    const uint8_t* wb = sadd(a.w, static_cast<int64_t>(kWRun) * gp);
    const uint32_t buf = pr & 1;
#pragma unroll
    for (int j = 0; j < kWOps; ++j) dma16(wb, w_off[j], w_lds + buf * kWaves * kWWave + 1024 * j);
    const int d = min(window(gp) + (lane & 3), row_dwords - 1);
#pragma unroll
    for (int i = 0; i < kPOps; ++i) dma4(a.s, s_off[i] + 4 * d, p_lds + buf * kWaves * kPWave + 256 * i);
  };

  // ---- decode inputs of local step t: the lane's four words and scale
  // (times 2^9) for each of its two column tiles (column 64 ni + 32 c + li,
  // moved by wave 2c + ni) ----
  struct StepWords {
    u32x4_t w[2];
    float sh[2], sl[2];  // the group scale's halves (times 2^9), per column tile
  };
  auto load_words = [&](int t, StepWords& d) {
    const int tt = min(t, steps - 1);
    const int pr = tt >> 1, sp = tt & 1;
    const int gp = (s0 >> 1) + pr;
    const int grp = (gp * 128 + 64 * sp + 32 * lh) >> (5 + a.group_shift);
    const int off = 2 * grp - 4 * window(gp);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int src_wave = 2 * c + ni;
      const uint8_t* wbuf = lds_w + (pr & 1) * kWaves * kWWave + kWWave * src_wave;
      d.w[c] = *reinterpret_cast<const u32x4_t*>(wbuf + kWRun * li + 16 * w_slot(li, 2 * sp + lh));
      const uint8_t* pbuf = lds_p + (pr & 1) * kWaves * kPWave + kPWave * src_wave + kPWin * li + off;
      split_scale(bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(pbuf)), &d.sh[c], &d.sl[c]);
    }
  };

  // A fragment (mt, kk): local row 128*MI + 32*mt + li, logical slot 4*lh + kk.
  uint32_t a_frag[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a_frag[kk] = (128 * MI + li) * 128 + 16 * a_slot(li, 4 * lh + kk);

  f32x16_t acc[2][4];  // [column tile][row tile]
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[c][mt][v] = 0.0f;

  // ---- prologue: transfers as if issued by steps -3 .. -1 ----
  issue_pair(0);
  issue_a(0);
  issue_a(1);
  issue_pair(1);
  wait_vmcnt<2 * kAOps + kPairOps>();  // pair 0 landed
  __syncthreads();
  StepWords cur;
  load_words(0, cur);
  u32x4_t bq[2][2][2];  // [chunk parity][column tile][plane]: B operands of one chunk
#pragma unroll
  for (int c = 0; c < 2; ++c) exact_word(cur.w[c][0], cur.sh[c], cur.sl[c], bq[0][c][0], bq[0][c][1]);
  bf16x8_t af[2][4];  // activation fragments of a chunk, by chunk parity

  // One step: after the barrier the next step's words and scales and chunk
  // 0's activation fragments are read; then 64 slots of one MFMA each, chunk
  // kk in slots 16kk .. 16kk+15 (column tile, row tile, plane), beside them
  // the decode of chunk kk+1 (the next step's chunk 0 during chunk 3) in
  // slots 16kk+1 .. 16kk+14 (two words, seven pieces each), the activation
  // reads of chunk kk+1 at slot 16kk, and the transfers: activation
  // instruction i at slot 2i+1, and on odd steps the next pair's words and
  // scale windows at slot 17. Scheduling barriers keep the order.
  for (int t = 0; t < steps; ++t) {
    const bool odd = (t & 1) != 0;
    if (odd)
      wait_vmcnt<kAOps>();
    else
      wait_vmcnt<kAOps + kPairOps>();
    __syncthreads();
    StepWords nxt;
    load_words(t + 1, nxt);
    const uint8_t* stage = lds_a + kAStage * (t % kAStages);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) af[0][mt] = *reinterpret_cast<const bf16x8_t*>(stage + a_frag[0] + 4096 * mt);
    __builtin_amdgcn_sched_barrier(0);
    ExactTmp dt;
    Unroll<0, 64>::run([&](auto ic) {
      constexpr int p = decltype(ic)::value;
      constexpr int kk = p / 16, c = (p % 16) / 8, mt = (p % 8) / 2, plane = p % 2;
      acc[c][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk & 1][mt],
                                                           __builtin_bit_cast(bf16x8_t, bq[kk & 1][c][plane]),
                                                           acc[c][mt], 0, 0, 0);
      if constexpr (p % 16 == 0 && kk < 3) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
          af[(kk + 1) & 1][m] = *reinterpret_cast<const bf16x8_t*>(stage + a_frag[kk + 1] + 4096 * m);
      }
      // Decode of chunk kk + 1: word (column tile) dc, piece dj.
      constexpr int q = p % 16;
      if constexpr (q >= 1 && q <= 14) {
        constexpr int dc = (q - 1) / 7, dj = (q - 1) % 7;
        if constexpr (kk < 3)
          exact_piece<dj>(cur.w[dc][kk + 1], cur.sh[dc], cur.sl[dc], dt, bq[(kk + 1) & 1][dc][0],
                          bq[(kk + 1) & 1][dc][1]);
        else
          exact_piece<dj>(nxt.w[dc][0], nxt.sh[dc], nxt.sl[dc], dt, bq[0][dc][0], bq[0][dc][1]);
      }
      if constexpr (p % 2 == 1 && p / 2 < kAOps) {
        constexpr int i = p / 2;
        const int g = s0 + min(t + 2, steps - 1);
        dma16(sadd(a.x, 128 * g), a_off[i], a_lds + kAStage * ((t + 2) % kAStages) + 1024 * kAOps * wave + 1024 * i);
      }
      if constexpr (p == 17) {
        if (odd) issue_pair((t + 3) >> 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    cur = nxt;
  }
  wait_vmcnt<0>();  // no transfer in flight past the loop

  // ---- bias term: y += sum_t X_t[row][g] * b[col][g] over the range's
  // groups, 16 per MFMA: lane half h takes groups 16 cb + 8h .. +7 (X from
  // the planes, b from global memory; groups past the range are zero in the
  // planes and masked to zero in b). ----
  {
    const int rg = a.split_steps * kBK / (32 << a.group_shift);  // groups of the range
    const int g0 = split * rg;
    const int64_t plane_elems = static_cast<int64_t>(a.M) * ea.gr;
    const uint16_t* planes = ea.planes + static_cast<int64_t>(split) * 3 * plane_elems;
    const uint8_t* brow[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
      brow[c] = a.b + static_cast<int64_t>(min(n0 + 64 * ni + 32 * c + li, a.N - 1)) * a.bs0 * 2;
    const uint16_t* xrow[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      xrow[mt] = planes + static_cast<int64_t>(min(m0 + 128 * MI + 32 * mt + li, a.M - 1)) * ea.gr + 8 * lh;
    // Operands of chunk cb: plane fragments and the biases of both column
    // tiles; the next chunk's are loaded before this one's MFMAs.
    struct Chunk {
      u32x4_t x[3][4];
      u32x4_t b[2];
    };
    auto load_chunk = [&](int cb, Chunk& k) {
      const int gl = kXChunk * cb + 8 * lh;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int g = gl + 2 * e;  // local group of the dword's low half
          const int gg = min(g0 + g, ea.groups - 2);
          const uint32_t v = *reinterpret_cast<const uint32_t*>(brow[c] + 2 * (gg & ~1));
          k.b[c][e] = g < rg ? v : 0u;  // rg and g are even
        }
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          k.x[pl][mt] = *reinterpret_cast<const u32x4_t*>(xrow[mt] + pl * plane_elems + kXChunk * cb);
    };
    const int chunks = ea.gr / kXChunk;
    Chunk k0, k1;
    load_chunk(0, k0);
    for (int cb = 0; cb < chunks; cb += 2) {
      if (cb + 1 < chunks) load_chunk(cb + 1, k1);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int mt = 0; mt < 4; ++mt)
            acc[c][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, k0.x[pl][mt]),
                                                                 __builtin_bit_cast(bf16x8_t, k0.b[c]), acc[c][mt], 0,
                                                                 0, 0);
      if (cb + 1 >= chunks) break;
      if (cb + 2 < chunks) load_chunk(cb + 2, k0);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int mt = 0; mt < 4; ++mt)
            acc[c][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, k1.x[pl][mt]),
                                                                 __builtin_bit_cast(bf16x8_t, k1.b[c]), acc[c][mt], 0,
                                                                 0, 0);
    }
  }

  // Accumulator element v of lane l: row 8*(v/4) + 4*(l/32) + v%4, column l%32 of its 32 x 32 tile.
  // Offsets are 32-bit from the wave's first output row (rows * N * 4 < 2^31).
  const int row0 = m0 + 128 * MI;
  const bool full = row0 + 128 <= a.M;
  float* base = (a.splits == 1 ? a.out : a.partial + split * static_cast<int64_t>(a.M) * a.N) +
                static_cast<int64_t>(row0) * a.N;
  with_store_kind(a.splits == 1 ? a.epi.kind : kEpiNone, [&](auto kind) {
    constexpr int KIND = decltype(kind)::value;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int col = n0 + 64 * ni + 32 * c + li;
      if (col >= a.N) continue;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = 32 * mt + 8 * (v / 4) + 4 * lh + (v % 4);
          if (full || row0 + r < a.M) {
            const uint32_t off = static_cast<uint32_t>(r * a.N + col) * 4u;
            store_as<KIND>(a.epi, reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(base) + off), col, acc[c][mt][v]);
          }
        }
    }
  });
}

__global__ __launch_bounds__(kThreads, 1) void qgemm_exact_kernel(ExactArgs ea) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kAStages * kAStage];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2 * kWaves * kWWave];
  __shared__ __attribute__((aligned(16))) uint8_t lds_p[2 * kWaves * kPWave];
  const TileArgs& a = ea.t;
  const int nb_n = (a.N + kCols - 1) / kCols;
  int tile, split;
  work_unit(nb_n * ((a.M + kRows - 1) / kRows), a.splits, &tile, &split);
  const int m0 = (tile / nb_n) * kRows;
  const int n0 = (tile % nb_n) * kCols;
  const int mi = __builtin_amdgcn_readfirstlane(threadIdx.x >> 7);
  if (mi == 0)
    exact_tile<0>(ea, lds_a, lds_w, lds_p, m0, n0, split);
  else
    exact_tile<1>(ea, lds_a, lds_w, lds_p, m0, n0, split);
}

}  // namespace

// Shapes the exact-plane GEMM takes: 4-bit codes, bf16 activations and
// parameters (bf16 scales keep s * q within two bf16 planes), unit inner
// strides, K a whole number of step pairs (128), groups of 32, parameter
// rows of whole dwords, and every byte offset the transfers form within 31
// bits.
bool exact_supports(const QmmProblem& p) {
  if (p.bits != 4 || p.x_dtype != AFFON_ROCM_BF16 || p.p_dtype != AFFON_ROCM_BF16) return false;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  // Groups of 32: the group size neither the group-scaling GEMM nor the
  // LDS-tiled kernel takes (the kernel's arithmetic holds for any whole
  // number of 32-value units; only groups of 32 are routed here and tested).
  if (p.K % 128 != 0 || p.group != 32) return false;
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || (p.xs0 * 2) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || (p.ws0 * 4) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.s) % 4 != 0 || reinterpret_cast<uintptr_t>(p.b) % 4 != 0) return false;
  if (p.ss0 % 2 != 0 || p.bs0 % 2 != 0 || (p.K / p.group) % 2 != 0) return false;
  const int64_t limit = int64_t(1) << 31;
  if (p.M * p.xs0 * 2 >= limit || p.N * p.ws0 * 4 >= limit) return false;
  if (p.N * p.ss0 * 2 >= limit || p.N * p.bs0 * 2 >= limit) return false;
  if (p.M > (int64_t(1) << 24) || p.N > (int64_t(1) << 22) || p.K > (int64_t(1) << 24)) return false;
  if (((p.N + kCols - 1) / kCols) * ((p.M + kRows - 1) / kRows) > (int64_t(1) << 27)) return false;
  return true;
}

hipError_t exact_launch(const QmmProblem& p, const Launch& l) {
  ExactArgs ea;
  TileArgs& a = ea.t;
  a.x = reinterpret_cast<const uint16_t*>(p.x);
  a.xs0 = p.xs0;
  a.w = p.w;
  a.ws0 = p.ws0;
  a.s = p.s;
  a.ss0 = p.ss0;
  a.b = p.b;
  a.bs0 = p.bs0;
  a.out = p.out;
  a.epi = p.epi;
  a.M = static_cast<int>(p.M);
  a.N = static_cast<int>(p.N);
  a.K = static_cast<int>(p.K);
  a.group_shift = p.group == 32 ? 0 : p.group == 64 ? 1 : 2;
  const int tiles = static_cast<int>(((p.N + kCols - 1) / kCols) * ((p.M + kRows - 1) / kRows));
  const int steps = static_cast<int>(p.K / kBK);
  int splits = l.can_split() ? choose_splits(tiles, steps) : 1;
  // Whole step pairs and an even number of whole groups per K range (the
  // bias term reads biases in dwords of two groups).
  while (splits > 1 && ((steps / splits) % 2 != 0 || (steps / splits) * kBK % (2 * p.group) != 0)) --splits;
  a.splits = splits;
  a.split_steps = steps / splits;
  ea.groups = static_cast<int>(p.K / p.group);
  const int range_groups = a.split_steps * kBK / static_cast<int>(p.group);
  ea.gr = padded_groups(range_groups);
  const size_t partial_bytes = splits > 1 ? static_cast<size_t>(splits) * p.M * p.N * 4 : 0;
  const size_t plane_bytes = static_cast<size_t>(splits) * 3 * p.M * ea.gr * 2;
  const size_t total = ((partial_bytes + 255) & ~size_t(255)) + plane_bytes;
  uint8_t* scratch = static_cast<uint8_t*>(l.scratch(total));
  if (scratch == nullptr) return hipErrorOutOfMemory;  // nothing launched (l.fixed_short says why, if fixed)
  a.partial = splits > 1 ? reinterpret_cast<float*>(scratch) : nullptr;
  ea.planes = reinterpret_cast<const uint16_t*>(scratch + ((partial_bytes + 255) & ~size_t(255)));

  const int64_t entries = static_cast<int64_t>(p.M) * splits * ea.gr;
  hipLaunchKernelGGL(exact_group_sums_kernel, dim3(static_cast<unsigned>((entries + 255) / 256)), dim3(256), 0,
                     l.stream, a.x, a.xs0, a.M, static_cast<int>(p.group), range_groups, ea.gr, splits,
                     const_cast<uint16_t*>(ea.planes));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(qgemm_exact_kernel, dim3(tiles * splits), dim3(kThreads), 0, l.stream, ea);
  e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  return launch_reduce(a, l.stream);
}

}  // namespace affon
