// rocm_quantized_matmul.gemv_mfma — decode batches (M <= 32) with bf16
// activations on the matrix cores.
//
// Counterpart of the reference's small-M decode variants (metal simd4 /
// matrix32 by M, docs/core/quantized-inference.md:132-140,151-170). Numerical
// class "reassociated": the packed codes q are exact integers in bf16, so
// v_mfma_f32_16x16x32_bf16 forms each K step's sums sum(x*q) with f32
// accumulation and no rounding of decoded weights; every K step (64 k) lies
// in one group, and the group's scale and bias are applied in f32 to the
// step sums: y += s * sum(x*q) + b * sum(x) -- the arithmetic of the VALU
// decode kernel, with sum(x) from one more MFMA against a bf16 ones operand.
//
// Work mapping: an (8, 16 or 32) x 64 tile per workgroup (rows past M repeat
// row M-1 and are not stored; at 8 rows the MFMA's other 8 rows carry a
// second column tile), its four waves each on a quarter of the K range, K
// split further over workgroups when the tiles alone cannot fill the GPU.
// Operands reach LDS by the same direct transfers, ring and counted waits as
// the prefill GEMM (lds_pipeline.h).

#include "lds_pipeline.h"
#include "vrow16_dispatch.h"
#include "vrow_dispatch.h"

namespace affon {
namespace {

using namespace pipeline;

constexpr int kMaxRows = 32;  // activation rows per tile: up to two blocks of 16 MFMA rows; more
                              // rows run as row tiles of 32 (grid dimension y)
constexpr int kCols = 64;     // weight columns per workgroup (4 MFMA column tiles)
constexpr int kReMinRows = 128;  // from here on the reassociated GEMM (gemm_re.hip) takes the problem
// Each iteration of the decode-batch kernel issues its activation transfer
// before its packed words (Plan, AFIRST), so the words stay in flight until
// the step that needs them.
constexpr bool kActsFirst = true;

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Bytes 0,1 (HIGH false) or 2,3 (HIGH true) of `bytes` read as FP8 E4M3,
// converted to a bf16 pair.
template <bool HIGH>
__device__ __forceinline__ uint32_t bf16_pair_fp8(uint32_t bytes) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(bytes, 1.0f, HIGH));
}

// B operands of MFMA t = 0, 1 for one lane and column: the lane's 16 codes of
// the step (k = 16h .. 16h+15, h = lane / 16) in `words`, codes 8t .. 8t+7
// into operand t as bf16. 2/4-bit codes go through the FP8 conversion (a
// byte holding n < 16 reads as n * 2^-9, exactly; the scale carries 2^9),
// 8-bit codes through v_cvt_f32_ubyteN (exact in bf16 up to 255).
template <int BITS>
__device__ __forceinline__ void codes_bf16(const uint32_t* words, u32x4_t* op) {
  if constexpr (BITS == 4) {  // word t = codes 8t .. 8t+7, code i in nibble i
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t w = words[t];
      const uint32_t even = w & 0x0f0f0f0fu;         // byte j = code 2j
      const uint32_t odd = (w >> 4) & 0x0f0f0f0fu;   // byte j = code 2j+1
      const uint32_t lo = __builtin_amdgcn_perm(odd, even, 0x05010400u);  // codes 0,1,2,3
      const uint32_t hi = __builtin_amdgcn_perm(odd, even, 0x07030602u);  // codes 4,5,6,7
      op[t] = u32x4_t{bf16_pair_fp8<false>(lo), bf16_pair_fp8<true>(lo), bf16_pair_fp8<false>(hi),
                      bf16_pair_fp8<true>(hi)};
    }
  } else if constexpr (BITS == 2) {  // one word, code i at bits 2i
    const uint32_t w = words[0];
    uint32_t m[4];  // byte j of m[u] = code 4j + u
#pragma unroll
    for (int u = 0; u < 4; ++u) m[u] = (w >> (2 * u)) & 0x03030303u;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      // bytes 2t, 2t+1 of m[u] hold codes 8t+u and 8t+4+u.
      const uint32_t sel = (2 * t) | ((4 + 2 * t) << 8) | ((2 * t + 1) << 16) | ((5 + 2 * t) << 24);
      const uint32_t q01 = __builtin_amdgcn_perm(m[1], m[0], sel);  // codes 8t, 8t+1, 8t+4, 8t+5
      const uint32_t q23 = __builtin_amdgcn_perm(m[3], m[2], sel);  // codes 8t+2, 8t+3, 8t+6, 8t+7
      const uint32_t lo = __builtin_amdgcn_perm(q23, q01, 0x05040100u);  // codes 8t .. 8t+3
      const uint32_t hi = __builtin_amdgcn_perm(q23, q01, 0x07060302u);  // codes 8t+4 .. 8t+7
      op[t] = u32x4_t{bf16_pair_fp8<false>(lo), bf16_pair_fp8<true>(lo), bf16_pair_fp8<false>(hi),
                      bf16_pair_fp8<true>(hi)};
    }
  } else {  // words 2t, 2t+1 = codes 8t .. 8t+7, one byte each
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      uint32_t pairs[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t v = opaque(words[2 * t + i]);
        pairs[2 * i] = pack_bf16(static_cast<float>(v & 0xffu), static_cast<float>((v >> 8) & 0xffu));
        pairs[2 * i + 1] = pack_bf16(static_cast<float>((v >> 16) & 0xffu), static_cast<float>(v >> 24));
      }
      op[t] = u32x4_t{pairs[0], pairs[1], pairs[2], pairs[3]};
    }
  }
}

// Workgroup: 64 weight columns (4 MFMA column tiles of 16) x up to 32
// activation rows (XROWS = 8, 16 or 32 staged; 32 rows run as two blocks of
// 16 MFMA rows sharing the decoded codes); its four waves split the
// workgroup's K range into four contiguous parts of whole 4-step chunks and
// run independently (no barrier inside the K loop), each with its own
// activation transfers. At the end the four partial sums are added in wave
// order through LDS (each wave's activation ring, free by then).
//
// K order inside a step: MFMA t of lane quarter h (lanes 16h .. 16h+15)
// covers k = 16h + 8t .. 16h + 8t + 7, for both operands, so a lane's codes
// for the step are one contiguous run of 16 and every MFMA stays inside the
// step. A wave's XROWS activation rows of a step sit in LDS as 16-byte
// chunks, chunk c of row r at slot c ^ (r%8) ^ ((r/8)%2) (conflict-free
// fragment reads).
//
// Twin column tiles (XROWS = 8): each stage holds 16 rows, rows 8..15 zero
// (written once). Fragment "lo" reads rows 0..15 (live rows 0..7), "hi"
// reads row r ^ 8 (live rows 8..15, holding activation rows 0..7). One
// MFMA chain then forms column tile 2p against lo and tile 2p+1 against hi,
// so output rows 0..7 belong to tile 2p and rows 8..15 to tile 2p+1: every
// output lane carries a live result, and the per-group scaling runs on two
// accumulators instead of four half-used ones.
template <int XROWS>
struct RowBlocks {
  static constexpr int kBlocks = XROWS > 16 ? 2 : 1;  // blocks of 16 MFMA rows
  static constexpr int kRows = 16 * kBlocks;           // rows with results
};
//
// PWHOLE: the scales and biases of a wave's whole K range arrive once, in
// the prologue (issued before any other transfer, so every later wait covers
// them), when they fit 32 bytes per column (e.g. 16 groups of bf16); this
// cuts their memory requests by the number of 4-step windows.
//
// WS: K steps per packed-word transfer (Plan): 8-bit words move two steps at
// a time (whole 128-byte lines per column) where LDS has room for that ring
// (up to 16 activation rows), one step at a time otherwise.
template <int BITS, typename PT, int XROWS, bool PWHOLE, int WS = (BITS == 8 ? (XROWS <= 16 ? 2 : 1) : 4)>
__global__ __launch_bounds__(kThreads, 1) void qskinny_kernel(TileArgs args) {
  TileArgs a = args;
  constexpr int kXLoads = XROWS / 8;  // activation DMA instructions per step
  using P = Plan<BITS, PT, kXLoads, PWHOLE, WS, kActsFirst, 16>;
  constexpr int RB = RowBlocks<XROWS>::kBlocks;
  constexpr int kRows = RowBlocks<XROWS>::kRows;
  constexpr bool kTwin = XROWS == 8;             // twin column tiles
  constexpr int kLdsRows = kTwin ? 16 : XROWS;   // rows per stage in LDS
  constexpr int kAcc = kTwin ? 2 : 4;            // accumulators per row block
  constexpr int kOutRows = kTwin ? 8 : kRows;    // rows with results
  __shared__ __attribute__((aligned(16))) uint8_t lds_x[kWaves][kStages][kLdsRows * 128];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[P::kWBufs][kWaves][P::kWBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_p[2][kWaves][P::kPBytes];
  static_assert(kRows * kCols * 4 <= kStages * kLdsRows * 128, "partial sums fit in a wave's activation ring");

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15;   // row of the A operand, column of the B operand and output
  const int h = lane >> 4;   // lane quarter

  const int nb_n = a.seg.count > 0 ? a.seg.total_tiles : (a.N + kCols - 1) / kCols;
  int tile, split;
  work_unit(nb_n, a.splits, &tile, &split);
  // A grouped launch: the workgroup's projection (all uniform), and where
  // its columns sit in the partial planes.
  int col_base = 0;
  int64_t pstride = a.N;
  if (a.seg.count > 0) {
    const int k = seg_of(a.seg, a.seg.first_tile, tile);
    tile -= seg_pick(a.seg.first_tile, k);
    col_base = seg_pick(a.seg.col_base, k);
    pstride = a.seg.total_n;
    a.w = seg_pick(a.seg.w, k);
    a.s = seg_pick(a.seg.s, k);
    a.b = seg_pick(a.seg.b, k);
    a.out = seg_pick(a.seg.out, k);
    a.N = seg_pick(a.seg.n, k);
    a.epi.bias = seg_pick(a.seg.bias, k);
    a.epi.kind = a.epi.bias != nullptr ? kEpiBias : kEpiNone;
  }
  const int n0 = tile * kCols;
  const int m0 = static_cast<int>(blockIdx.y) * kMaxRows;  // this row tile's first activation row
  // K range of this wave, in whole 4-step chunks: chunks [c0, c1) of the
  // workgroup's range, itself chunks [split*C/S, (split+1)*C/S) of K.
  const int chunks = a.K / (4 * kBK);
  const int g0 = split * chunks / a.splits, g1 = (split + 1) * chunks / a.splits;
  const int c0 = g0 + wave * (g1 - g0) / kWaves, c1 = g0 + (wave + 1) * (g1 - g0) / kWaves;
  const int steps = 4 * (c1 - c0);
  const int s0 = 4 * c0;
  const int last = steps - 1;

  // Activation transfer i: lane L writes slot L%8 of row 8i + L/8.
  const uint16_t* x_src[kXLoads];
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    const int row = 8 * i + (lane >> 3);
    x_src[i] = a.x + static_cast<int64_t>(min(m0 + row, a.M - 1)) * a.xs0 + 8 * ((lane & 7) ^ (row & 7) ^ ((row >> 3) & 1));
  }
  auto issue_a = [&](int step) {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      load_lds<16>(x_src[i] + (s0 + step) * kBK, lds_address(lds_x[wave][step & 3]) + 1024 * i);
  };
  WeightStream<BITS, PT, kXLoads, PWHOLE, WS, kActsFirst, 16> ws;
  // PWHOLE keeps one window per wave: both window buffers of the wave, which
  // are adjacent when indexed [wave][buffer].
  uint8_t* p_base = PWHOLE ? lds_p[0][0] + wave * 2 * P::kPBytes : lds_p[0][wave];
  ws.init(a, n0, s0, lane, lds_w[0][wave], kWaves * P::kWBytes, p_base, kWaves * P::kPBytes);
  auto issue_all = [&](int j, int pstep, int wstep, int astep) {
    if (j == 0 && !PWHOLE)
      for (int i = 0; i < P::kPLoads; ++i) ws.issue_p(pstep, i);
    if (kActsFirst) issue_a(astep);
    if (P::w_issue(j))
      for (int i = 0; i < P::kWLoads; ++i) ws.issue_w(wstep, i);
    if (!kActsFirst) issue_a(astep);
  };
  // A operand of MFMA t from LDS row `row`, chunk 2h + t.
  auto read_row = [&](int stage, int row, int t) -> bf16x8_t {
    const int slot = (2 * h + t) ^ (row & 7) ^ ((row >> 3) & 1);
    return *reinterpret_cast<const bf16x8_t*>(&lds_x[wave][stage][(row >> 3) * 1024 + (8 * (row & 7) + slot) * 16]);
  };
  // Row block rb: row 16rb + r; twin tiles: side 0 ("lo") row r, side 1 ("hi") row r ^ 8.
  auto read_x = [&](int stage, int rb, int t) -> bf16x8_t {
    return read_row(stage, kTwin ? (r ^ (8 * rb)) : 16 * rb + r, t);
  };
  // The lane's 16 codes of column c (local) for `step`.
  auto read_codes = [&](int step, int c, uint32_t* words) {
    if constexpr (BITS == 2) {
      words[0] = *reinterpret_cast<const uint32_t*>(ws.w_part(step, c, 0) + 4 * h);
    } else if constexpr (BITS == 4) {
      const u32x2_t v = *reinterpret_cast<const u32x2_t*>(ws.w_part(step, c, h >> 1) + 8 * (h & 1));
      words[0] = v.x;
      words[1] = v.y;
    } else {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ws.w_part(step, c, h));
      words[0] = v.x;
      words[1] = v.y;
      words[2] = v.z;
      words[3] = v.w;
    }
  };

  const float code_scale = BITS == 8 ? 1.0f : 512.0f;
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
  f32x4_t y[RB][kAcc];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int ct = 0; ct < kAcc; ++ct) y[rb][ct] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (kTwin) {  // the zero rows 8..15 of every stage (no transfer writes them)
#pragma unroll
    for (int s = 0; s < kStages; ++s)
      *reinterpret_cast<u32x4_t*>(&lds_x[wave][s][1024 + 16 * lane]) = u32x4_t{0u, 0u, 0u, 0u};
  }
  constexpr int kSides = kTwin ? 2 : RB;  // activation fragment sets per step

  // Transfers in the order of the transfer plan (Plan<..., kXLoads, PWHOLE,
  // WS>), each wave for itself: iterations -4 .. -1 issue the prologue,
  // iteration t issues the parameter window at t%4 == 0 (unless PWHOLE),
  // the words of steps t+4 .. t+7 at t%4 == 0 (four-step transfers), of step
  // t+4 every step (one-step transfers) or of steps t+3, t+4 at odd t
  // (two-step transfers), then the activations of step t+3. Step t is
  // decoded in iteration t from LDS reads that complete before that
  // iteration's transfers are issued, and the wait at its start covers
  // exactly step t's transfers (Plan::wait_own): a transfer that reuses a
  // buffer reuses the one of the step(s) just read.
#define AFFON_QSKINNY_STEP(J)                                                                            \
  {                                                                                                      \
    wait_vmcnt<P::wait_own(J)>();                                                                        \
    bf16x8_t xf[kSides][2];                                                                              \
    _Pragma("unroll") for (int sd = 0; sd < kSides; ++sd) {                                              \
      xf[sd][0] = read_x((J), sd, 0);                                                                    \
      xf[sd][1] = read_x((J), sd, 1);                                                                    \
    }                                                                                                    \
    uint32_t words[4][BITS];                                                                             \
    uint32_t s_raw[kAcc], b_raw[kAcc];                                                                   \
    _Pragma("unroll") for (int ct = 0; ct < 4; ++ct) read_codes(t, 16 * ct + r, words[ct]);              \
    _Pragma("unroll") for (int ca = 0; ca < kAcc; ++ca)                                                  \
      ws.params(t, 16 * (kTwin ? 2 * ca + (h >> 1) : ca) + r, 0, &s_raw[ca], &b_raw[ca]);               \
    wait_lds_reads();                                                                                    \
    issue_all((J), min(t + 4, last & ~3), min(t + P::kWAhead, last & ~(WS - 1)),                         \
              min(t + 3, last));                                                                         \
    f32x4_t xs[RB];                                                                                      \
    _Pragma("unroll") for (int rb = 0; rb < RB; ++rb) {                                                  \
      xs[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[rb][0], ones, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0); \
      xs[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[rb][1], ones, xs[rb], 0, 0, 0);                \
      if constexpr (kTwin) {                                                                             \
        xs[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[1][0], ones, xs[rb], 0, 0, 0);               \
        xs[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[1][1], ones, xs[rb], 0, 0, 0);               \
      }                                                                                                  \
    }                                                                                                    \
    _Pragma("unroll") for (int ca = 0; ca < kAcc; ++ca) {                                                \
      const float sv = widen_param<PT>(s_raw[ca]) * code_scale, bv = widen_param<PT>(b_raw[ca]);         \
      u32x4_t op[2], oq[2];                                                                              \
      codes_bf16<BITS>(words[kTwin ? 2 * ca : ca], op);                                                  \
      if constexpr (kTwin) codes_bf16<BITS>(words[2 * ca + 1], oq);                                      \
      _Pragma("unroll") for (int rb = 0; rb < RB; ++rb) {                                                \
        f32x4_t q;                                                                                       \
        if constexpr (kTwin) {                                                                           \
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[0][0], __builtin_bit_cast(bf16x8_t, op[0]),     \
                                                      f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);         \
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[0][1], __builtin_bit_cast(bf16x8_t, op[1]), q, 0, 0, 0); \
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[1][0], __builtin_bit_cast(bf16x8_t, oq[0]), q, 0, 0, 0); \
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[1][1], __builtin_bit_cast(bf16x8_t, oq[1]), q, 0, 0, 0); \
        } else {                                                                                         \
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[rb][0], __builtin_bit_cast(bf16x8_t, op[0]),    \
                                                      f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);         \
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[rb][1], __builtin_bit_cast(bf16x8_t, op[1]), q, 0, 0, 0); \
        }                                                                                                \
        _Pragma("unroll") for (int i = 0; i < 4; ++i)                                                    \
            y[rb][ca][i] = fmaf(sv, q[i], fmaf(bv, xs[rb][i], y[rb][ca][i]));                            \
      }                                                                                                  \
    }                                                                                                    \
    ++t;                                                                                                 \
  }

  if (steps > 0) {
    if constexpr (PWHOLE) {
#pragma unroll
      for (int i = 0; i < P::kPWholeLoads; ++i) ws.issue_p_whole(i);
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      issue_all(rr, 0, min(rr - 4 + P::kWAhead, last & ~(WS - 1)), min(max(rr - 1, 0), last));
    for (int t = 0; t < steps;) {
      AFFON_QSKINNY_STEP(0)
      AFFON_QSKINNY_STEP(1)
      AFFON_QSKINNY_STEP(2)
      AFFON_QSKINNY_STEP(3)
    }
    wait_vmcnt<0>();  // no transfer in flight past this point
  }
#undef AFFON_QSKINNY_STEP

  // Partial sums of the four K parts, [kOutRows][kCols] f32 per wave in the
  // wave's own activation ring (no transfer into it is in flight any more):
  // output element i of row block rb and column tile ct is row 16rb + 4h + i,
  // column 16ct + r; with twin tiles, accumulator ca holds row 4(h%2) + i of
  // column tile 2ca + h/2. Added in wave order. Column col of row row sits at
  // col ^ (16 * (row/4 % 2)): the two lane quarters of a 32-lane LDS phase
  // write rows four apart, which then land on different banks.
  auto ysum = [&](int w) { return reinterpret_cast<float*>(&lds_x[w][0][0]); };
  auto ypos = [](int row, int col) { return row * kCols + (col ^ (16 * ((row >> 2) & 1))); };
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int ca = 0; ca < kAcc; ++ca)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = kTwin ? 4 * (h & 1) + i : 16 * rb + 4 * h + i;
        const int ct = kTwin ? 2 * ca + (h >> 1) : ca;
        ysum(wave)[ypos(row, 16 * ct + r)] = y[rb][ca][i];
      }
  __syncthreads();
  float* dst = a.partial + split * static_cast<int64_t>(a.M) * pstride;
  if (a.splits == 1) {
    with_store_kind(a.epi.kind, [&](auto kind) {
      constexpr int KIND = decltype(kind)::value;
#pragma unroll
      for (int e = 0; e < kOutRows * kCols / kThreads; ++e) {
        const int o = e * kThreads + tid;
        const int row = m0 + o / kCols, col = n0 + o % kCols;
        if (row < a.M && col < a.N) {
          const int q = ypos(o / kCols, o % kCols);
          const float v = ((ysum(0)[q] + ysum(1)[q]) + ysum(2)[q]) + ysum(3)[q];
          store_as<KIND>(a.epi, a.out + static_cast<int64_t>(row) * a.N + col, col, v);
        }
      }
    });
  } else {
#pragma unroll
    for (int e = 0; e < kOutRows * kCols / kThreads; ++e) {
      const int o = e * kThreads + tid;
      const int row = m0 + o / kCols, col = n0 + o % kCols;
      const int q = ypos(o / kCols, o % kCols);
      if (row < a.M && col < a.N)
        dst[static_cast<int64_t>(row) * pstride + col_base + col] = ((ysum(0)[q] + ysum(1)[q]) + ysum(2)[q]) + ysum(3)[q];
    }
  }
}

// Whether every wave's scales and biases fit one whole-range window of 32
// bytes per column: the dwords from the one holding a wave's first group
// through the one holding its last, for every K range and wave.
template <typename PT>
bool whole_range_params(const TileArgs& a) {
  const int chunks = a.K / (4 * kBK);
  for (int split = 0; split < a.splits; ++split) {
    const int g0 = split * chunks / a.splits, g1 = (split + 1) * chunks / a.splits;
    for (int w = 0; w < kWaves; ++w) {
      const int c0 = g0 + w * (g1 - g0) / kWaves, c1 = g0 + (w + 1) * (g1 - g0) / kWaves;
      if (c1 <= c0) continue;
      const int64_t first = (int64_t(4 * c0) * kBK >> (5 + a.group_shift)) * PT::bytes / 4;
      const int64_t last = ((int64_t(4 * c1) * kBK - 1) >> (5 + a.group_shift)) * PT::bytes / 4;
      if (last - first + 1 > 8) return false;
    }
  }
  return true;
}

template <int BITS, typename PT, bool PWHOLE>
void launch_skinny(const TileArgs& args, dim3 grid, hipStream_t stream) {
  if (args.M <= 8)
    hipLaunchKernelGGL((qskinny_kernel<BITS, PT, 8, PWHOLE>), grid, dim3(kThreads), 0, stream, args);
  else if (args.M <= 16)
    hipLaunchKernelGGL((qskinny_kernel<BITS, PT, 16, PWHOLE>), grid, dim3(kThreads), 0, stream, args);
  else
    hipLaunchKernelGGL((qskinny_kernel<BITS, PT, 32, PWHOLE>), grid, dim3(kThreads), 0, stream, args);
}

template <int BITS, typename PT>
hipError_t launch_typed(const TileArgs& args, hipStream_t stream) {
  const int tiles = args.seg.count > 0 ? args.seg.total_tiles : (args.N + kCols - 1) / kCols;
  const dim3 grid(tiles * args.splits, (args.M + kMaxRows - 1) / kMaxRows);
  if (whole_range_params<PT>(args))
    launch_skinny<BITS, PT, true>(args, grid, stream);
  else
    launch_skinny<BITS, PT, false>(args, grid, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || args.splits == 1) return e;
  return launch_reduce(args, stream);
}

}  // namespace

// Which virtual-row layout runs a problem: 1 = 8 rows per wave, 2 = 16 rows
// per wave, 0 = neither (the LDS-tiled kernel below).
namespace {
// Whether the LDS-tiled kernel takes the problem.
bool tiled_supports(const QmmProblem& p) {
  if (p.x_dtype != AFFON_ROCM_BF16 || p.M > (int64_t(1) << 20)) return false;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  // Each K step inside one group, groups addressed by shift.
  if (p.K % (4 * kBK) != 0 || p.group % kBK != 0) return false;
  const int64_t gq = p.group / 32;
  if ((gq & (gq - 1)) != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || (p.xs0 * 2) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || p.ws0 % 4 != 0) return false;
  const int64_t pbytes = p.p_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  if (reinterpret_cast<uintptr_t>(p.s) % 4 != 0 || reinterpret_cast<uintptr_t>(p.b) % 4 != 0) return false;
  if ((p.ss0 * pbytes) % 4 != 0 || (p.bs0 * pbytes) % 4 != 0 || (p.K / p.group * pbytes) % 4 != 0) return false;
  if (p.N > (int64_t(1) << 30) || p.K > (int64_t(1) << 30)) return false;
  return true;
}
}  // namespace

int vrow_layout(const QmmProblem& p) {
  // The LDS-tiled kernel takes the batch whenever it can from two activation
  // rows on for 8-bit codes and from three rows on for 2- and 4-bit codes:
  // measured on 14336 x 4096 weights (graph periods, one box) it is as fast
  // or faster there than either virtual-row layout (8-bit M = 2: 14.0 against
  // 15.2 us, M = 4: 14.0 against 17.0 us; 4-bit M = 4: 10.9 against 11.6 us),
  // while at two rows 2- and 4-bit codes run 1 % faster on the 16-row layout.
  if (p.M >= (p.bits == 8 ? 2 : 3) && tiled_supports(p)) return 0;
  vrow::Plan eight;
  vrow16::Plan sixteen;
  if (vrow::plan(p, &eight)) return 1;
  if (vrow16::plan(p, &sixteen)) return 2;
  return 0;
}


bool gemv_mfma_supports(const QmmProblem& p) {
  if (vrow_layout(p) != 0 || tiled_supports(p)) return true;
  // Batches past the virtual-row kernels whose groups the tiled kernels do
  // not take (groups of 32): the group-32 GEMM.
  return p.M > 4 && re32_supports(p);
}

namespace {
hipError_t tiled_launch(const QmmProblem& p, const QmmProblem* group, int count, const Launch& l);
}  // namespace

hipError_t gemv_mfma_launch(const QmmProblem& p, const Launch& l) {
  // A virtual-row kernel (packed words straight into the B operand, no LDS
  // for weights) where vrow_layout picks one; otherwise the LDS-tiled kernel.
  switch (vrow_layout(p)) {
    case 1:
      return vrow_launch_b8(p, l.stream);
    case 2:
      switch (p.bits) {
        case 2: return vrow16_launch_b2(p, l.stream);
        case 4: return vrow16_launch_b4(p, l.stream);
        default: return vrow16_launch_b8(p, l.stream);
      }
    default:
      break;
  }
  // Tall activations: the large-tile reassociated GEMM, when its scratch
  // (per-group activation sums) can be had.
  if (p.M >= kReMinRows && re_gemm_supports(p)) {
    hipError_t e = hipSuccess;
    if (re_gemm_launch(p, l, &e, false)) return e;
  }
  if (!tiled_supports(p)) return re32_launch(p, l, false);
  return tiled_launch(p, nullptr, 0, l);
}

namespace {

// The LDS-tiled kernel on one problem, or (count > 0) on a group of
// problems that share the activations, as one grouped launch.
hipError_t tiled_launch(const QmmProblem& p, const QmmProblem* group, int count, const Launch& l) {
  TileArgs a;
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
  while ((int64_t(32) << a.group_shift) < p.group) ++a.group_shift;
  int tiles = static_cast<int>((p.N + kCols - 1) / kCols);
  int64_t columns = p.N;
  if (count > 0) {
    a.seg.count = count;
    tiles = 0;
    columns = 0;
    for (int k = 0; k < kMaxSegments; ++k) {
      const bool used = k < count;
      a.seg.first_tile[k] = tiles;
      a.seg.col_base[k] = static_cast<int>(columns);
      a.seg.n[k] = used ? static_cast<int>(group[k].N) : 0;
      a.seg.w[k] = used ? group[k].w : nullptr;
      a.seg.s[k] = used ? group[k].s : nullptr;
      a.seg.b[k] = used ? group[k].b : nullptr;
      a.seg.out[k] = used ? group[k].out : nullptr;
      a.seg.bias[k] = used && group[k].epi.kind == kEpiBias ? group[k].epi.bias : nullptr;
      if (used) {
        if (group[k].epi.kind == kEpiBias) a.epi.bias_bf16 = group[k].epi.bias_bf16;
        tiles += static_cast<int>((group[k].N + kCols - 1) / kCols);
        columns += group[k].N;
      }
    }
    a.seg.total_tiles = tiles;
    a.seg.total_n = static_cast<int>(columns);
  }
  const int chunks = static_cast<int>(p.K / (4 * kBK));
  a.splits = 1;
  a.split_steps = 0;  // ranges are computed per workgroup from K and splits
  a.partial = nullptr;
  // Further K ranges over workgroups while the tiles (over columns and row
  // tiles) fill less than three quarters of the CUs and every wave keeps at
  // least two chunks.
  const int row_tiles = static_cast<int>((p.M + kMaxRows - 1) / kMaxRows);
  int splits = 1;
  if (l.can_split())
    while (splits < 8 && tiles * row_tiles * splits < device_cus() * 3 / 4 && chunks >= 2 * kWaves * 2 * splits)
      splits *= 2;
  if (splits > 1) {
    if (auto* w = static_cast<float*>(l.scratch(static_cast<size_t>(splits) * p.M * columns * 4))) {
      a.splits = splits;
      a.partial = w;
    } else if (l.fixed != nullptr) {
      return hipErrorOutOfMemory;  // the fixed scratch buffer cannot hold this plan's partial sums
    }
  }
  const bool bf16p = p.p_dtype == AFFON_ROCM_BF16;
  switch (p.bits) {
    case 2: return bf16p ? launch_typed<2, BF16>(a, l.stream) : launch_typed<2, F32>(a, l.stream);
    case 4: return bf16p ? launch_typed<4, BF16>(a, l.stream) : launch_typed<4, F32>(a, l.stream);
    default: return bf16p ? launch_typed<8, BF16>(a, l.stream) : launch_typed<8, F32>(a, l.stream);
  }
}

}  // namespace

bool gemv_mfma_group_supports(const QmmProblem* group, int count) {
  if (count < 2 || count > kMaxGroup || count > kMaxSegments) return false;
  const QmmProblem& p = group[0];
  for (int i = 0; i < count; ++i) {
    const QmmProblem& q = group[i];
    if (!tiled_supports(q) || vrow_layout(q) != 0) return false;  // the LDS-tiled kernel only
    if (q.epi.kind != kEpiNone && q.epi.kind != kEpiBias) return false;
    if (q.x != p.x || q.xs0 != p.xs0 || q.M != p.M || q.K != p.K || q.bits != p.bits || q.group != p.group ||
        q.p_dtype != p.p_dtype || q.ws0 != p.ws0 || q.ss0 != p.ss0 || q.bs0 != p.bs0)
      return false;
    for (int j = 0; j < count; ++j)
      if (q.epi.kind == kEpiBias && group[j].epi.kind == kEpiBias && group[j].epi.bias_bf16 != q.epi.bias_bf16)
        return false;
  }
  return true;
}

hipError_t gemv_mfma_group_launch(const QmmProblem* group, int count, const Launch& l) {
  if (!gemv_mfma_group_supports(group, count)) return hipErrorInvalidValue;
  return tiled_launch(group[0], group, count, l);
}

}  // namespace affon
