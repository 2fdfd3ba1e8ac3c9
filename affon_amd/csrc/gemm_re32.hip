// Prefill GEMM of the reassociated class for 4-bit codes with bf16
// activations and bf16 group parameters, groups of 32: the default policy's
// path for tall activations at the group size the group-scaling GEMM
// (gemm_re.hip, whole 64-value groups per K step) and the LDS-tiled decode
// kernel do not take.
//
// Counterpart of the reference's matrix paths, which decode weights to f32
// and are classified "reassociated" (docs/core/quantized-inference.md:
// 138-139,151-158,175-177). Arithmetic, as in gemm_re.hip:
//
//   y = sum_g s_g * sum_{k in g} x_k q_k  +  sum_g b_g * X_g,   X_g = sum_{k in g} x_k.
//
// The packed codes q are exact integers in bf16 MFMA operands; each group's
// sums sum(x*q) come out of v_mfma_f32_32x32x16_bf16 (two per group) with f32
// accumulation, and y += s_g * sums is one f32 multiply-add per output and
// group on the vector ALU. No decoded weight is rounded. The bias term is a
// small matrix product over groups: a pre-pass forms X for every activation
// row and group in f32 and splits it exactly into three bf16 planes (X = X1 +
// X2 + X3), and after the K loop each tile adds sum_t X_t * b^T, 16 groups per
// MFMA, with the planes staged through LDS 64 groups at a time.
//
// Work mapping: workgroup tile 256 (rows) x 128 (columns), eight waves in a
// 2 x 4 arrangement, two per SIMD, so that one wave's scaling and decode run
// on the vector ALU while the other's MFMAs run; wave (mi, ni) computes rows
// 128 mi .. +127 and columns 32 ni .. +31 as four 32 x 32 accumulator tiles T
// on the same B operands. K steps of 64 = two groups. Each MFMA covers 16 k
// of one group: MFMA kk (0..3) of lane half h takes chunk
// 4 (kk / 2) + 2 h + kk % 2 (8 k each), so MFMAs 0, 1 hold the step's first
// group and 2, 3 its second. A lane's codes of one column and step are then
// two 8-byte pieces, one per group.
//
// Transfers, all direct global-to-LDS and counted: activations (256 rows x
// 128 bytes per step) into a 3-stage ring, two steps ahead; packed words of
// four steps at a time (128 bytes per column) and the matching 16-byte scale
// windows (eight groups per column) into two buffers, four steps ahead. One
// barrier per step orders the shared tiles.
//
// With ROUNDED the same frame runs the approximate class (the mfma
// candidate's path for these shapes past 128 rows): decoded weights
// bf16(s*q + b) in the B operands, MFMAs accumulating into y, no group sums
// or bias term; bias windows stream beside the scale windows.

#include "lds_pipeline.h"

namespace affon {
namespace {

using namespace pipeline;

constexpr int kRows = 256;                        // workgroup tile rows
constexpr int kCols = 128;                        // workgroup tile columns
constexpr int kWaves32 = 8;                       // 2 (rows) x 4 (columns)
constexpr int kThreads32 = 64 * kWaves32;
constexpr int kAStage = kRows * 128;              // bytes per step: 256 rows x 64 bf16
constexpr int kAStages = 3;
constexpr int kAOps = kRows / 8 / kWaves32;       // activation transfers per wave and step (1 KiB each)
constexpr int kWRun = 128;                        // packed bytes per column and four steps
constexpr int kWBuf = kCols * kWRun;
constexpr int kWOps = kWBuf / 1024 / kWaves32;    // packed-word transfers per wave and four steps
constexpr int kSRun = 16;                         // scale bytes per column and four steps (8 groups)
constexpr int kSBuf = kCols * kSRun;
constexpr int kSOps = kSBuf / 256 / kWaves32;     // 4-byte scale transfers per wave and four steps
constexpr int kPlaneRound = 64;                   // plane entries per row staged per bias-term round

static_assert(kAOps == 4 && kWOps == 2 && kSOps == 1, "transfer counts assumed by the issue slots and waits");
static_assert(3 * kRows * kPlaneRound * 2 <= kAStages * kAStage, "a round of the three planes fits the ring");

// vmcnt bound before the barrier of step t (j = t % 4), which sits between
// the step's third and fourth phase (ROUNDED: between its two groups'
// MFMAs). Before it, step t issues the activations of step t+2 and, when
// t % 4 == 0, then the packed words and scale windows (ROUNDED: and bias
// windows) of steps t+4 .. t+7; the prologue issues the words and windows
// of steps 0..3, then the activations of steps 0 and 1. At the
// barrier of step t the activations of step t+1 (issued by step t-1) must
// have landed, for the fragment reads of step t+1 that follow it, and with
// them everything issued before: the words and windows that the next steps
// read at their start. In flight may stay the words and windows issued by
// step t-1 (when t-1 = 0 mod 4) and every transfer of step t.
template <bool ROUNDED>
constexpr int mid_wait(int j) { return kAOps + (j == 0 || j == 1 ? kWOps + (ROUNDED ? 2 : 1) * kSOps : 0); }

// Slot (16-byte unit) of part `part` (0..7) in local column c's 128-byte
// packed run.
__device__ __forceinline__ int w_slot(int c, int part) { return part ^ (c & 7) ^ ((c >> 3) & 1); }

// Physical 16-byte slot of logical chunk q of local activation row r: the
// fragment reads (consecutive rows, one chunk) are bank-conflict free.
__device__ __forceinline__ int a_slot(int r, int q) { return q ^ (r & 7) ^ ((r >> 3) & 1); }

// Dword holding logical dword d of local column c's scale window: the
// per-step reads (32 consecutive columns, one dword) hit 32 distinct banks.
__device__ __forceinline__ int s_dword(int c, int d) { return d ^ ((c >> 3) & 3); }

// Groups of one K range, padded to whole bias-term rounds (the planes' row length).
__host__ __device__ constexpr int padded_groups(int groups) {
  return (groups + kPlaneRound - 1) / kPlaneRound * kPlaneRound;
}

// X = sum of the 32 activations of one row and group in f32, as three bf16
// planes whose sum is X exactly. Layout [range][plane][row][gr]: group g of K
// range g / range_groups at entry g % range_groups of a row of gr entries;
// entries from range_groups to gr are zero. One thread per (row, entry).
__global__ __launch_bounds__(256) void re32_group_sums_kernel(const uint16_t* x, int64_t xs0, int M,
                                                              int range_groups, int gr, int ranges, uint16_t* planes) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t entries = static_cast<int64_t>(ranges) * gr;
  if (i >= static_cast<int64_t>(M) * entries) return;
  const int row = static_cast<int>(i / entries);
  const int e = static_cast<int>(i % entries);
  const int range = e / gr, gl = e % gr;
  uint16_t h1 = 0, h2 = 0, h3 = 0;
  if (gl < range_groups) {
    const uint16_t* src = x + row * xs0 + static_cast<int64_t>(range * range_groups + gl) * 32;
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; c += 8) {
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

// Decode of one packed word into an MFMA B operand (its eight codes in k
// order as exact bf16 integers) in three pieces, so that a step's decode can
// be spread over its MFMAs: nibble masks, byte ordering, conversion. A byte
// holding n < 16 reads as n * 2^-9 in FP8 E4M3; the conversion's scale 2^9
// makes the operand the exact integer codes.
struct CodeTmp {
  uint32_t even, odd, lo, hi;
};
template <int PH>
__device__ __forceinline__ void code_piece(uint32_t w, CodeTmp& d, bf16x8_t& out) {
  if constexpr (PH == 0) {
    d.even = w & 0x0f0f0f0fu;         // byte j = code 2j
    d.odd = (w >> 4) & 0x0f0f0f0fu;   // byte j = code 2j+1
  } else if constexpr (PH == 1) {
    d.lo = __builtin_amdgcn_perm(d.odd, d.even, 0x05010400u);  // codes 0,1,2,3
    d.hi = __builtin_amdgcn_perm(d.odd, d.even, 0x07030602u);  // codes 4,5,6,7
  } else {
    const u32x4_t v{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d.lo, 512.0f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d.lo, 512.0f, true)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d.hi, 512.0f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d.hi, 512.0f, true))};
    out = __builtin_bit_cast(bf16x8_t, v);
  }
}

// ROUNDED: the B operand bf16(s*q + b) of one packed word's eight codes in k
// order (s carries the 2^9 of the FP8 reading of a code), the approximate
// class's decoded weights.
__device__ __forceinline__ bf16x8_t weights_rounded(uint32_t w, float s, float b) {
  const uint32_t even = w & 0x0f0f0f0fu, odd = (w >> 4) & 0x0f0f0f0fu;
  const f32x2_t e0 = __builtin_amdgcn_cvt_pk_f32_fp8(even, false), e1 = __builtin_amdgcn_cvt_pk_f32_fp8(even, true);
  const f32x2_t o0 = __builtin_amdgcn_cvt_pk_f32_fp8(odd, false), o1 = __builtin_amdgcn_cvt_pk_f32_fp8(odd, true);
  return __builtin_bit_cast(bf16x8_t, u32x4_t{pack_bf16(fmaf(e0.x, s, b), fmaf(o0.x, s, b)),
                                              pack_bf16(fmaf(e0.y, s, b), fmaf(o0.y, s, b)),
                                              pack_bf16(fmaf(e1.x, s, b), fmaf(o1.x, s, b)),
                                              pack_bf16(fmaf(e1.y, s, b), fmaf(o1.y, s, b))});
}

struct Re32Args {
  TileArgs t;
  const uint16_t* planes;  // [range][3][M][gr] bf16: X1, X2, X3 of every row and group
  int gr;                  // entries per plane row (the range's groups, padded)
  int groups;              // groups per parameter row (K / 32)
};

// Steps: a multiple of 4 per K range, or (a single range) 2 mod 4, whose
// last run of packed words holds two steps.
//
// Schedule. A step is four phases; an MFMA phase is one group's eight MFMAs
// (kk = 2G, 2G+1 of tiles 0..3; the first of each tile starts from zero), a
// vector phase the 64 multiply-adds y += s * sums of one group, the decode
// of two of the next step's packed words, the LDS reads of the next MFMA
// phase's fragments and the step's transfers. The two waves of a SIMD (mi =
// 0, 1) run them in opposite order, so that one wave's MFMAs run while the
// other wave's vector instructions issue:
//   mi = 0:  MFMA group 1 | vector group 1 | MFMA group 2 | barrier | vector group 2
//   mi = 1:  vector group 2 of the previous step | MFMA group 1 | vector group 1 | barrier | MFMA group 2
// Every read of step t's activation stage comes before the barrier of step
// t (mi = 0 reads its first-group fragments after the barrier of step t-1),
// and the next write of that stage (the activations of step t+3) is issued
// by step t+1, after it. The packed words and scales a step reads at its
// start are ordered against their transfers by earlier barriers the same way.
//
// ROUNDED: the approximate class instead. The B operands are the decoded
// weights bf16(s*q + b) (each MFMA's 16 k lie in one group), the MFMAs
// accumulate straight into y, and there is no group-sum pre-pass or bias
// term. Both waves of a SIMD run the same software pipeline (at its loop
// below) instead of the opposite phases. The biases stream in windows
// beside the scales, and each step reads the next step's parameters with
// its words.
template <int MI, bool ROUNDED>
__device__ __forceinline__ void re32_tile(const Re32Args& r, uint8_t* lds_a, uint8_t* lds_w, uint8_t* lds_s,
                                          uint8_t* lds_b) {
  const TileArgs& a = r.t;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31;
  const int lh = lane >> 5;
  constexpr int mi = MI;    // rows 128*mi ..
  const int ni = wave & 3;  // columns 32*ni ..

  const int nb_n = (a.N + kCols - 1) / kCols;
  int tile, split;
  work_unit(nb_n * ((a.M + kRows - 1) / kRows), a.splits, &tile, &split);
  const int m0 = (tile / nb_n) * kRows;
  const int n0 = (tile % nb_n) * kCols;
  // Steps are local to the K range; s0 (a multiple of 4) is its first global step.
  const int steps = a.split_steps;
  const int s0 = split * steps;
  const int last = steps - 1;
  const int last_run = last & ~3;           // first step of the last run of packed words
  const bool short_run = (steps & 3) != 0;  // the last run holds two steps

  // Activation transfers: this wave fills 8-row groups g8 = kAOps*wave + i of
  // a stage; lane L writes slot L%8 of local row 8*g8 + L/8, so it loads chunk
  // (L%8) ^ (L/8) ^ (g8%2). Rows past M repeat row M-1 (unstored outputs).
  uint32_t a_off[kAOps];
#pragma unroll
  for (int i = 0; i < kAOps; ++i) {
    const int g8 = kAOps * wave + i;
    const int row = min(m0 + 8 * g8 + (lane >> 3), a.M - 1);
    a_off[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(a.xs0 * 2) + 16 * ((lane & 7) ^ (lane >> 3) ^ (g8 & 1));
  }
  auto issue_a1 = [&](int step, int stage, int i) {
    dma16(sadd(a.x, static_cast<int64_t>(s0 + step) * 128), a_off[i],
          lds_address(lds_a) + stage * kAStage + 1024 * (kAOps * wave + i));
  };
  // Packed-word transfers: instruction j = kWOps*wave + i, lane L writes byte
  // 1024j + 16L of a buffer = physical slot L%8 of local column 8j + L/8,
  // holding part w_slot(c, L%8). In a run of two steps, parts 4..7 lie past
  // the row's end: those lanes load parts 0..3 again (never read).
  uint32_t w_off[kWOps];
  uint32_t w_back[kWOps];  // 64 for a lane holding a part 4..7, else 0
#pragma unroll
  for (int i = 0; i < kWOps; ++i) {
    const int c = 8 * (kWOps * wave + i) + (lane >> 3);
    const int col = min(n0 + c, a.N - 1);  // columns past N feed unstored outputs
    const int part = w_slot(c, lane & 7);
    w_off[i] = static_cast<uint32_t>(col) * static_cast<uint32_t>(a.ws0 * 4) + 16 * part;
    w_back[i] = part >= 4 ? 64u : 0u;
  }
  auto issue_w = [&](int step4, int buf) {
    const bool two = short_run && step4 == last_run;
#pragma unroll
    for (int i = 0; i < kWOps; ++i)
      dma16(sadd(a.w, static_cast<int64_t>(s0 + step4) * 32), w_off[i] - (two ? w_back[i] : 0u),
            lds_address(lds_w) + buf * kWBuf + 1024 * (kWOps * wave + i));
  };
  // Scale windows: lane L of this wave writes dword L%4 of local column
  // 16*wave + L/4's window, holding logical dword s_dword(c, L%4) = groups
  // 2d, 2d+1 of the run. Dwords past the row end repeat the row's last dword.
  const int sc = 16 * wave + (lane >> 2);
  const uint32_t s_off =
      static_cast<uint32_t>(min(n0 + sc, a.N - 1)) * static_cast<uint32_t>(a.ss0 * 2);
  const int s_d = s_dword(sc, lane & 3);
  const int row_dwords = r.groups / 2;
  auto issue_s = [&](int step4, int buf) {
    const int d = min((s0 + step4) + s_d, row_dwords - 1);  // run (s0+step4)/4 starts at dword s0+step4
    dma4(a.s, s_off + 4 * d, lds_address(lds_s) + buf * kSBuf + 256 * wave);
  };
  const uint32_t b_off =
      static_cast<uint32_t>(min(n0 + sc, a.N - 1)) * static_cast<uint32_t>(a.bs0 * 2);
  auto issue_b = [&](int step4, int buf) {  // ROUNDED: the bias windows, as the scale windows
    const int d = min((s0 + step4) + s_d, row_dwords - 1);
    dma4(a.b, b_off + 4 * d, lds_address(lds_b) + buf * kSBuf + 256 * wave);
  };

  // A fragment (T, kk): local row 128*mi + 32*T + li, chunk 4*(kk/2) + 2*lh + kk%2.
  // The swizzle depends on the row only through li, so T adds 4096 bytes.
  int a_rd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int row = 128 * mi + li;
    a_rd[kk] = row * 128 + 16 * a_slot(row, 4 * (kk / 2) + 2 * lh + kk % 2);
  }
  auto read_a = [&](int stage, int T, int kk) -> bf16x8_t {
    return *reinterpret_cast<const bf16x8_t*>(lds_a + stage * kAStage + a_rd[kk] + 4096 * T);
  };
  // The lane's packed words of step sub (0..3) of a run: words 2*lh, 2*lh+1
  // of part 2*sub (first group) and of part 2*sub+1 (second group).
  const int wc = 32 * ni + li;
  auto read_w = [&](int buf, int sub) -> u32x4_t {
    const uint8_t* run = lds_w + buf * kWBuf + kWRun * wc + 8 * lh;
    const uint64_t g0w = *reinterpret_cast<const uint64_t*>(run + 16 * w_slot(wc, 2 * sub));
    const uint64_t g1w = *reinterpret_cast<const uint64_t*>(run + 16 * w_slot(wc, 2 * sub + 1));
    return u32x4_t{static_cast<uint32_t>(g0w), static_cast<uint32_t>(g0w >> 32), static_cast<uint32_t>(g1w),
                   static_cast<uint32_t>(g1w >> 32)};
  };
  // The dword of both scales (bf16, groups of step sub) of this lane's column.
  auto read_s = [&](int buf, int sub) -> uint32_t {
    return *reinterpret_cast<const uint32_t*>(lds_s + buf * kSBuf + kSRun * wc + 4 * s_dword(wc, sub));
  };
  auto read_b = [&](int buf, int sub) -> uint32_t {  // ROUNDED: both biases, as read_s
    return *reinterpret_cast<const uint32_t*>(lds_b + buf * kSBuf + kSRun * wc + 4 * s_dword(wc, sub));
  };

  // Prologue, in the issue order the waits count: packed words and scale
  // windows of steps 0..3; activations of steps 0 and 1. Then the B operands
  // of step 0 (the loop decodes them one step ahead).
  issue_w(0, 0);
  issue_s(0, 0);
  if constexpr (ROUNDED) issue_b(0, 0);
#pragma unroll
  for (int i = 0; i < kAOps; ++i) issue_a1(0, 0, i);
#pragma unroll
  for (int i = 0; i < kAOps; ++i) issue_a1(min(1, last), 1, i);
  wait_vmcnt<kAOps>();  // the words and windows of steps 0..3, the activations of step 0
  __syncthreads();

  f32x16_t y[4];
#pragma unroll
  for (int T = 0; T < 4; ++T)
#pragma unroll
    for (int v = 0; v < 16; ++v) y[T][v] = 0.0f;
  bf16x8_t bq[4];  // B operands of the step, by kk
  // The fragments of one MFMA phase: MFMA i is tile i % 4, kk 2G + i / 4.
  auto read_group = [&](bf16x8_t (&af)[8], int stage, int G) {
#pragma unroll
    for (int i = 0; i < 8; ++i) af[i] = read_a(stage, i % 4, 2 * G + i / 4);
  };

  if constexpr (ROUNDED) {
    // Software pipeline, the same for both waves of a SIMD: a step is its
    // first group's eight MFMAs (accumulating into y), the barrier, its
    // second group's eight. Each phase's fragments are read at the start of
    // the phase before (the first group's of step t+1 right after the
    // barrier of step t), and each phase decodes, one piece per MFMA, the two
    // words the next phase but one needs: during the first group of step t
    // the second group's words of step t, during the second group the first
    // group's words of step t+1. The step's transfers are issued during its
    // first group, before the barrier.
    struct Params {
      float s[2], b[2];  // per group of the step: scale (times 2^9), bias
    };
    auto params = [&](uint32_t sdw, uint32_t bdw) {
      return Params{{__uint_as_float(sdw << 16) * 512.0f, __uint_as_float(sdw & 0xffff0000u) * 512.0f},
                    {__uint_as_float(bdw << 16), __uint_as_float(bdw & 0xffff0000u)}};
    };
    // Piece PC (0..3) of the rounded decode of word w into B operand k.
    struct Piece {
      uint32_t even, odd;
      f32x2_t e, o;
      u32x4_t out;
    };
    auto piece = [&](auto pc, uint32_t w, float sc, float bi, Piece& d, int k) {
      constexpr int PC = decltype(pc)::value;
      if constexpr (PC == 0 || PC == 2) {
        if constexpr (PC == 0) {
          d.even = w & 0x0f0f0f0fu;
          d.odd = (w >> 4) & 0x0f0f0f0fu;
        }
        d.e = __builtin_amdgcn_cvt_pk_f32_fp8(d.even, PC == 2);  // codes 0, 2 (4, 6)
        d.o = __builtin_amdgcn_cvt_pk_f32_fp8(d.odd, PC == 2);   // codes 1, 3 (5, 7)
      } else {
        constexpr int o = PC == 1 ? 0 : 2;
        d.out[o] = pack_bf16(fmaf(d.e.x, sc, bi), fmaf(d.o.x, sc, bi));
        d.out[o + 1] = pack_bf16(fmaf(d.e.y, sc, bi), fmaf(d.o.y, sc, bi));
        if constexpr (PC == 3) bq[k] = __builtin_bit_cast(bf16x8_t, d.out);
      }
    };
    bf16x8_t afa[8], afb[8];  // fragments of the first and second group's phase
    u32x4_t wcur = read_w(0, 0);
    Params pc = params(read_s(0, 0), read_b(0, 0));
#pragma unroll
    for (int k = 0; k < 2; ++k) bq[k] = weights_rounded(wcur[k], pc.s[0], pc.b[0]);
    read_group(afa, 0, 0);

    int stage = 0;  // t % 3
    for (int t = 0; t < steps; t += 4) {
      Unroll<0, 4>::run([&](auto jc) {
        constexpr int J = decltype(jc)::value;
        const int tt = t + J;
        if (J >= 2 && tt > last) return;  // a last run of two steps
        const int a_step = min(tt + 2, last), a_stage = stage == 0 ? 2 : stage - 1;
        const int w_step = min(tt + 4, last_run);
        const int buf = (tt >> 2) & 1;
        const int next_stage = stage == 2 ? 0 : stage + 1;
        // The next step's packed words and parameters (the last step reads its own again).
        const bool more = tt + 1 <= last;
        const int nb = J == 3 && more ? buf ^ 1 : buf, ns = J == 3 ? (more ? 0 : 3) : J + 1;
        const u32x4_t wvn = read_w(nb, ns);
        const Params pn = params(read_s(nb, ns), read_b(nb, ns));
        read_group(afb, stage, 1);
        Piece d;
        Unroll<0, 8>::run([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          y[i % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afa[i], bq[i / 4], y[i % 4], 0, 0, 0);
          // The activations first, then the words and windows: the counted
          // waits assume this order.
          if constexpr (i < kAOps) issue_a1(a_step, a_stage, i);
          if constexpr (J == 0 && i == 4) issue_w(w_step, buf ^ 1);
          if constexpr (J == 0 && i == 5) issue_s(w_step, buf ^ 1);
          if constexpr (J == 0 && i == 6) issue_b(w_step, buf ^ 1);
          piece(std::integral_constant<int, i % 4>{}, wcur[2 + i / 4], pc.s[1], pc.b[1], d, 2 + i / 4);
          __builtin_amdgcn_sched_barrier(0);
        });
        wait_vmcnt<mid_wait<true>(J)>();
        __syncthreads();
        read_group(afa, next_stage, 0);
        Unroll<0, 8>::run([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          y[i % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afb[i], bq[2 + i / 4], y[i % 4], 0, 0, 0);
          piece(std::integral_constant<int, i % 4>{}, wvn[i / 4], pn.s[0], pn.b[0], d, i / 4);
          __builtin_amdgcn_sched_barrier(0);
        });
        wcur = wvn;
        pc = pn;
        stage = next_stage;
      });
    }
    wait_vmcnt<0>();  // the loop's last transfers (re-fetches of the final step)
  } else {
    f32x16_t acc[4];
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[T][v] = 0.0f;  // mi = 1: the second group of "step -1" is scaled by 0
    const f32x16_t zero = {};
    float sb_prev = 0.0f;  // mi = 1: second-group scale of the previous step
    bf16x8_t af[8];
    u32x4_t wprev = read_w(0, 0);  // mi = 1: the words whose second group the next first phase decodes
    auto decode2 = [&](const u32x4_t& w, int kk0) {
#pragma unroll
      for (int k = kk0; k < kk0 + 2; ++k) {
        CodeTmp d;
        code_piece<0>(w[k], d, bq[k]);
        code_piece<1>(w[k], d, bq[k]);
        code_piece<2>(w[k], d, bq[k]);
      }
    };
    auto mfma_group = [&](int G) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int T = i % 4, kk = 2 * G + i / 4;
        acc[T] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bq[kk], i < 4 ? zero : acc[T], 0, 0, 0);
      }
    };
    auto scale_group = [&](float sc) {
#pragma unroll
      for (int T = 0; T < 4; ++T)
#pragma unroll
        for (int v = 0; v < 16; ++v) y[T][v] = fmaf(sc, acc[T][v], y[T][v]);
    };
    decode2(wprev, 0);
    if constexpr (MI == 0) {
      decode2(wprev, 2);
      read_group(af, 0, 0);
    }

    int stage = 0;  // t % 3
    for (int t = 0; t < steps; t += 4) {
      Unroll<0, 4>::run([&](auto jc) {
        constexpr int J = decltype(jc)::value;
        const int tt = t + J;
        if (J >= 2 && tt > last) return;  // a last run of two steps
        // Step tt issues the activations of step tt+2 (into the stage step
        // tt-1 used) and, at tt % 4 == 0, the packed words and scale windows
        // of steps tt+4 .. tt+7 (into the buffers steps tt-4 .. tt-1 used),
        // all before its barrier. Past the range end the last step (run) is
        // fetched again into the same free places, so that every step issues
        // the same transfers.
        const int a_step = min(tt + 2, last), a_stage = stage == 0 ? 2 : stage - 1;
        const int w_step = min(tt + 4, last_run);
        const int buf = (tt >> 2) & 1;
        const int next_stage = stage == 2 ? 0 : stage + 1;
        auto transfers = [&]() {
#pragma unroll
          for (int i = 0; i < kAOps; ++i) issue_a1(a_step, a_stage, i);
          if constexpr (J == 0) {
            issue_w(w_step, buf ^ 1);
            issue_s(w_step, buf ^ 1);
          }
        };
        // The next step's packed words (the last step reads its own again) and this step's scales.
        const bool more = tt + 1 <= last;
        const u32x4_t wvn = J == 3 ? read_w(more ? buf ^ 1 : buf, more ? 0 : 3) : read_w(buf, J + 1);
        const uint32_t sdw = read_s(buf, J);
        const float sa = __uint_as_float(sdw << 16), sb = __uint_as_float(sdw & 0xffff0000u);
        if constexpr (MI == 0) {
          mfma_group(0);
          __builtin_amdgcn_sched_barrier(0);
          read_group(af, stage, 1);
          transfers();
          decode2(wvn, 0);
          scale_group(sa);
          __builtin_amdgcn_sched_barrier(0);
          mfma_group(1);
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<mid_wait<false>(J)>();
          __syncthreads();
          read_group(af, next_stage, 0);
          decode2(wvn, 2);
          scale_group(sb);
          __builtin_amdgcn_sched_barrier(0);
        } else {
          read_group(af, stage, 0);
          decode2(wprev, 2);
          scale_group(sb_prev);
          __builtin_amdgcn_sched_barrier(0);
          mfma_group(0);
          __builtin_amdgcn_sched_barrier(0);
          read_group(af, stage, 1);
          transfers();
          decode2(wvn, 0);
          scale_group(sa);
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<mid_wait<false>(J)>();
          __syncthreads();
          mfma_group(1);
          __builtin_amdgcn_sched_barrier(0);
          wprev = wvn;
          sb_prev = sb;
        }
        stage = next_stage;
      });
    }
    if constexpr (MI == 1) scale_group(sb_prev);  // the second group of the last step

    // Bias term: y += sum over the range's groups of X_t[row][g] * b[col][g],
    // 16 groups per MFMA, in rounds of 64 groups: the tile's rows of the three
    // planes (plane t at 32 KiB * t of the activation ring, row r at 128 * r,
    // 16-byte slot q at a_slot(r, q)) arrive by whole-line transfers; the
    // lane's biases are read from global memory, zero past the range's groups
    // (where the planes are zero too).
    wait_vmcnt<0>();  // the loop's last transfers (re-fetches of the final step)
    __syncthreads();
    {
      const int rg = 2 * steps;  // groups of the range
      const int g0 = split * rg;
      const int rounds = r.gr / kPlaneRound;
      const uint16_t* planes = r.planes + static_cast<int64_t>(split) * 3 * a.M * r.gr;
      const uint8_t* brow = a.b + static_cast<int64_t>(min(n0 + wc, a.N - 1)) * a.bs0 * 2;
      constexpr int kXOps = 3 * kRows / 8 / kWaves32;
      for (int rd = 0; rd < rounds; ++rd) {
        if (rd > 0) __syncthreads();  // every wave is done with the previous round's planes
#pragma unroll
        for (int ii = 0; ii < kXOps; ++ii) {
          const int i = kXOps * wave + ii;  // plane i / 32, rows 8*(i%32) ..
          const int pl = i / (kRows / 8), rgi = i % (kRows / 8);
          const int row = min(m0 + 8 * rgi + (lane >> 3), a.M - 1);
          const int q = (lane & 7) ^ (lane >> 3) ^ (rgi & 1);
          load_lds<16>(planes + (static_cast<int64_t>(pl) * a.M + row) * r.gr + kPlaneRound * rd + 8 * q,
                       lds_address(lds_a) + pl * (kRows * 128) + 1024 * rgi);
        }
        u32x4_t bb[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int gl = kPlaneRound * rd + 16 * c + 8 * lh + 2 * e;  // even, as rg and g0
            bb[c][e] = gl < rg ? *reinterpret_cast<const uint32_t*>(brow + 2 * (g0 + gl)) : 0u;
          }
        wait_vmcnt<0>();
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u32x4_t xv[3][4];
#pragma unroll
          for (int pl = 0; pl < 3; ++pl)
#pragma unroll
            for (int T = 0; T < 4; ++T) {
              const int row = 128 * mi + 32 * T + li;
              xv[pl][T] = *reinterpret_cast<const u32x4_t*>(lds_a + pl * (kRows * 128) + row * 128 +
                                                            16 * a_slot(row, 2 * c + lh));
            }
#pragma unroll
          for (int pl = 0; pl < 3; ++pl)
#pragma unroll
            for (int T = 0; T < 4; ++T)
              y[T] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, xv[pl][T]),
                                                             __builtin_bit_cast(bf16x8_t, bb[c]), y[T], 0, 0, 0);
        }
      }
    }
  }

  // Accumulator tile T, element v of lane l is row 8*(v/4) + 4*(l/32) + v%4
  // and column l%32 of its 32x32 tile. Offsets are 32-bit from the tile's
  // first row (256 rows * N * 4 < 2^31).
  const bool full = m0 + kRows <= a.M;
  float* base = (a.splits == 1 ? a.out : a.partial + split * static_cast<int64_t>(a.M) * a.N) +
                static_cast<int64_t>(m0) * a.N;
  const int col = n0 + wc;
  with_store_kind(a.splits == 1 ? a.epi.kind : kEpiNone, [&](auto kind) {
    constexpr int KIND = decltype(kind)::value;
    if (col < a.N) {
#pragma unroll
      for (int T = 0; T < 4; ++T)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rr = 128 * mi + 32 * T + 8 * (v / 4) + 4 * lh + (v % 4);
          if (full || m0 + rr < a.M) {
            const uint32_t off = static_cast<uint32_t>(rr * a.N + col) * 4u;
            store_as<KIND>(a.epi, reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(base) + off), col, y[T][v]);
          }
        }
    }
  });
}

template <bool ROUNDED>
__global__ __launch_bounds__(kThreads32) void qgemm_re32_kernel(Re32Args r) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kAStages * kAStage];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2 * kWBuf];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s[2 * kSBuf];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[ROUNDED ? 2 * kSBuf : 16];  // ROUNDED: bias windows
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 8) == 0)
    re32_tile<0, ROUNDED>(r, lds_a, lds_w, lds_s, lds_b);
  else
    re32_tile<1, ROUNDED>(r, lds_a, lds_w, lds_s, lds_b);
}

}  // namespace

// Shapes the group-32 GEMM takes: 4-bit codes, bf16 activations and
// parameters, unit inner strides, groups of 32, K a whole number of step
// pairs (128), 16-byte aligned activation and packed-word rows, dword-aligned
// parameter rows, and every byte offset the transfers form within 31 bits.
bool re32_supports(const QmmProblem& p) {
  if (p.bits != 4 || p.x_dtype != AFFON_ROCM_BF16 || p.p_dtype != AFFON_ROCM_BF16) return false;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  if (p.K % 128 != 0 || p.group != 32) return false;
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || (p.xs0 * 2) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || (p.ws0 * 4) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.s) % 4 != 0 || reinterpret_cast<uintptr_t>(p.b) % 4 != 0) return false;
  if (p.ss0 % 2 != 0 || p.bs0 % 2 != 0) return false;
  const int64_t limit = int64_t(1) << 31;
  if (p.M * p.xs0 * 2 >= limit || p.N * p.ws0 * 4 >= limit) return false;
  if (p.N * p.ss0 * 2 >= limit || p.N * p.bs0 * 2 >= limit) return false;
  if (p.M > (int64_t(1) << 24) || p.N > (int64_t(1) << 22) || p.K > (int64_t(1) << 24)) return false;
  if (((p.N + kCols - 1) / kCols) * ((p.M + kRows - 1) / kRows) > (int64_t(1) << 27)) return false;
  return true;
}

hipError_t re32_launch(const QmmProblem& p, const Launch& l, bool rounded) {
  Re32Args r;
  TileArgs& a = r.t;
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
  a.group_shift = 0;
  const int tiles = static_cast<int>(((p.N + kCols - 1) / kCols) * ((p.M + kRows - 1) / kRows));
  const int steps = static_cast<int>(p.K / kBK);
  // K ranges of whole 4-step runs; a K with a last run of two steps is one range.
  const int splits = l.can_split() && steps % 4 == 0 ? choose_splits(tiles, steps) : 1;
  a.splits = splits;
  a.split_steps = steps / splits;
  r.groups = static_cast<int>(p.K / 32);
  const int range_groups = 2 * a.split_steps;
  r.gr = padded_groups(range_groups);
  const size_t partial_bytes = splits > 1 ? static_cast<size_t>(splits) * p.M * p.N * 4 : 0;
  // ROUNDED: no group-sum planes.
  const size_t plane_bytes = rounded ? 0 : static_cast<size_t>(splits) * 3 * p.M * r.gr * 2;
  const size_t total = ((partial_bytes + 255) & ~size_t(255)) + plane_bytes;
  uint8_t* scratch = nullptr;
  if (total > 0) {
    scratch = static_cast<uint8_t*>(l.scratch(total));
    if (scratch == nullptr) return hipErrorOutOfMemory;  // nothing launched (l.fixed_short says why, if fixed)
  }
  a.partial = splits > 1 ? reinterpret_cast<float*>(scratch) : nullptr;
  r.planes = rounded ? nullptr : reinterpret_cast<const uint16_t*>(scratch + ((partial_bytes + 255) & ~size_t(255)));

  hipError_t e = hipSuccess;
  if (!rounded) {
    const int64_t entries = static_cast<int64_t>(p.M) * splits * r.gr;
    hipLaunchKernelGGL(re32_group_sums_kernel, dim3(static_cast<unsigned>((entries + 255) / 256)), dim3(256), 0,
                       l.stream, a.x, a.xs0, a.M, range_groups, r.gr, splits, const_cast<uint16_t*>(r.planes));
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (rounded)
    hipLaunchKernelGGL(qgemm_re32_kernel<true>, dim3(tiles * splits), dim3(kThreads32), 0, l.stream, r);
  else
    hipLaunchKernelGGL(qgemm_re32_kernel<false>, dim3(tiles * splits), dim3(kThreads32), 0, l.stream, r);
  e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  return launch_reduce(a, l.stream);
}

}  // namespace affon
