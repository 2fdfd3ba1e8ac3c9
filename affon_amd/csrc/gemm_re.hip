// Prefill GEMM for 4-bit codes, bf16 activations and parameters, groups of 64
// or 128, in two modes: the reassociated class (rocm_quantized_matmul.
// gemv_mfma, the default policy's path for tall activations) and, with
// ROUNDED, the approximate class (rocm_quantized_matmul.mfma: decoded weights
// rounded to bf16 in the B operand, no group sums or bias term).
//
// Counterpart of the reference's matrix paths (metal matrix32 /
// matrix32_packed, docs/core/quantized-inference.md:138-139,151-170), which
// decode weights to f32 and are classified "reassociated". In that mode the
// arithmetic is the decode-batch kernels' (gemv_mfma.hip): the packed codes q
// are exact integers in bf16 MFMA operands, each group's sums sum(x*q) come
// out of v_mfma_f32_32x32x16_bf16 with f32 accumulation, and the group's scale
// and bias are applied in f32:
//
//   y = sum_g s_g * sum_{k in g} x_k q_k  +  sum_g b_g * X_g,   X_g = sum_{k in g} x_k.
//
// No decoded weight is rounded. The bias term is a small matrix product over
// groups: a pre-pass (group_sums_kernel) forms X for every activation row and
// group in f32 and splits it exactly into three bf16 planes, X = X1 + X2 + X3
// (X1 = bf16(X), X2 = bf16(X - X1), X3 = X - X1 - X2: 8 + 8 + 8 significant
// bits cover f32's 24). After the K loop each tile adds X_t * b^T, t = 1..3,
// with the same MFMA (bf16 biases: every product exact in f32), which costs
// 3 * 64 / group / 64 of the main loop's matrix work (4.7% at group 64).
//
// Work mapping: workgroup tile 256 (rows) x 128 (columns), eight waves in a
// 2 x 4 arrangement (see qgemm_re_kernel), two waves per SIMD so that one
// wave's decode and scaling run on the vector ALU while the other's MFMAs
// run. K steps of 64; MFMA kk (0..3) of lane half h covers chunk 4h + kk of
// the step (8 k each), so a lane's codes of one column and step are 16
// contiguous bytes.
//
// Transfers, all direct global-to-LDS and counted (no compiler-visible loads
// in the loop): the tile's scales (and, ROUNDED, biases) for the whole K
// range once, first; packed words of four steps at a time (128 bytes per
// column: whole lines) into two buffers, four steps ahead; activations (256
// rows x 128 bytes per step) into a 3-stage ring, two steps ahead. One
// barrier per step orders the shared tiles.

#include "lds_pipeline.h"

namespace affon {
namespace {

using namespace pipeline;

constexpr int kRows = 256;                 // workgroup tile rows
constexpr int kCols = 128;                 // workgroup tile columns
constexpr int kReWaves = RePlan::kWaves;   // 4 x 2
constexpr int kReThreads = 64 * kReWaves;
constexpr int kAStage = kRows * 128;       // bytes per step: 256 rows x 64 bf16
constexpr int kAStages = 3;
constexpr int kWRun = 128;                 // packed bytes per column and four steps
constexpr int kWBuf = kCols * kWRun;
constexpr int kSCol = 128;                 // scale bytes per column for the K range (32 dwords)
constexpr int kMaxGroups = kSCol / 2;      // bf16 scales per column and K range
constexpr int kMinRangeSteps = 16;         // shortest K range worth the kernel's fixed costs

static_assert(kRows / 8 / kReWaves == RePlan::kAOps, "8-row activation transfers per wave and step");
static_assert(kWBuf / 1024 / kReWaves == RePlan::kWOps, "packed-word transfers per wave and four steps");
static_assert(kCols * kSCol / 256 / kReWaves == RePlan::kSOps, "scale transfers per wave");

struct ReArgs {
  TileArgs t;
  const uint16_t* planes;  // [K range][3][M][kMaxGroups] bf16: X1, X2, X3 of every row and group
};

// Slot (16-byte unit) of part `part` (0..7) in local column c's 128-byte
// packed run: within 8 consecutive columns the slots differ, and columns c
// and c + 8 differ in slot bit 0, so the decode reads (lanes = consecutive
// columns, one part) are bank-conflict free.
__device__ __forceinline__ int w_slot(int c, int part) { return part ^ (c & 7) ^ ((c >> 3) & 1); }

// Physical 16-byte slot of logical chunk q of local activation row r: the
// fragment reads (consecutive rows, one chunk) are bank-conflict free.
__device__ __forceinline__ int a_slot(int r, int q) { return q ^ (r & 7) ^ ((r >> 3) & 1); }

// X = sum of the `group` activations of one row and group in f32, stored as
// three bf16 planes whose sum is X exactly. Layout [range][plane][row][64]:
// group g of K range g / range_groups at entry g % range_groups of a 128-byte
// row (entries past the range's groups are never used unmasked). Thread i
// reads 16-byte chunk i of the activations (row i / (K/8)); the group/8
// consecutive lanes of one group add their partial sums by lane exchange and
// the first stores.
__global__ __launch_bounds__(256) void group_sums_kernel(const uint16_t* x, int64_t xs0, int M, int K, int group,
                                                         int range_groups, uint16_t* planes) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int chunks = K / 8;
  if (i >= static_cast<int64_t>(M) * chunks) return;  // whole groups of lanes (chunks % 32 == 0)
  const int row = static_cast<int>(i / chunks);
  const int c = static_cast<int>(i % chunks);
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(x + row * xs0 + 8 * c);
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    sum += __uint_as_float(v[e] << 16);
    sum += __uint_as_float(v[e] & 0xffff0000u);
  }
  const int lanes = group / 8;
  for (int o = 1; o < lanes; o <<= 1) sum += __shfl_xor(sum, o);
  if (c % lanes != 0) return;
  const uint16_t h1 = f32_to_bf16_bits(sum);
  uint16_t h2 = 0, h3 = 0;
  if (__builtin_isfinite(sum)) {
    const float r1 = sum - bf16_bits_to_f32(h1);  // exact
    h2 = f32_to_bf16_bits(r1);
    h3 = f32_to_bf16_bits(r1 - bf16_bits_to_f32(h2));  // exact: the remaining bits fit bf16
  }
  const int g = c / lanes;
  const int64_t plane = static_cast<int64_t>(M) * kMaxGroups;
  const int64_t at = (g / range_groups) * 3 * plane + static_cast<int64_t>(row) * kMaxGroups + g % range_groups;
  planes[at] = h1;
  planes[plane + at] = h2;
  planes[2 * plane + at] = h3;
}

// Decode of one packed word into an MFMA B operand in two pieces, so that a
// step's decode can be spread over its MFMAs: piece 0 separates and orders
// the nibbles (codes 0..3 and 4..7, one per byte), piece 1 converts them. A
// byte holding n < 16 reads as n * 2^-9 in FP8 E4M3; the conversion's scale
// 2^9 makes the operand the exact integer codes.
struct CodePair {
  uint32_t lo, hi;
};
__device__ __forceinline__ CodePair codes_split(uint32_t w) {
  const uint32_t even = w & 0x0f0f0f0fu;        // byte j = code 2j
  const uint32_t odd = (w >> 4) & 0x0f0f0f0fu;  // byte j = code 2j+1
  return CodePair{__builtin_amdgcn_perm(odd, even, 0x05010400u),   // codes 0,1,2,3
                  __builtin_amdgcn_perm(odd, even, 0x07030602u)};  // codes 4,5,6,7
}
__device__ __forceinline__ bf16x8_t codes_convert(CodePair p) {
  const u32x4_t v{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(p.lo, 512.0f, false)),
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(p.lo, 512.0f, true)),
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(p.hi, 512.0f, false)),
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(p.hi, 512.0f, true))};
  return __builtin_bit_cast(bf16x8_t, v);
}

// B operand of the ROUNDED mode from one packed word: bf16(s * q + b) for its
// eight codes in k order (s carries the 2^9 of the FP8 reading of a code).
__device__ __forceinline__ bf16x8_t weights_rounded(uint32_t w, float s, float b) {
  const uint32_t even = w & 0x0f0f0f0fu, odd = (w >> 4) & 0x0f0f0f0fu;
  const f32x2_t e0 = __builtin_amdgcn_cvt_pk_f32_fp8(even, false), e1 = __builtin_amdgcn_cvt_pk_f32_fp8(even, true);
  const f32x2_t o0 = __builtin_amdgcn_cvt_pk_f32_fp8(odd, false), o1 = __builtin_amdgcn_cvt_pk_f32_fp8(odd, true);
  return __builtin_bit_cast(bf16x8_t, u32x4_t{pack_bf16(fmaf(e0.x, s, b), fmaf(o0.x, s, b)),
                                              pack_bf16(fmaf(e0.y, s, b), fmaf(o0.y, s, b)),
                                              pack_bf16(fmaf(e1.x, s, b), fmaf(o1.x, s, b)),
                                              pack_bf16(fmaf(e1.y, s, b), fmaf(o1.y, s, b))});
}

// GSTEPS: K steps per group (1: group 64, 2: group 128). ROUNDED: the
// approximate class instead -- decoded weights bf16(s*q + b) in the B
// operand, accumulated straight into y; no group sums, no bias term.
//
// Waves: 2 (rows) x 4 (columns); wave (mi, ni) computes rows 128*mi .. +127
// and columns 32*ni .. +31 of the tile as accumulator tiles T = 0..3 (rows
// 32*T .. of its 128), all four on the same B operands, so a wave decodes
// only its 32 columns. One step is 16 slots, each one MFMA plus about seven
// vector instructions, in this order (the scheduling barriers keep it):
//   slots 0..7   MFMAs of tiles 0, 1 (chunk kk = slot/2), beside them the
//                scaling of tiles 2, 3 of the previous step;
//   slots 8..15  MFMAs of tiles 2, 3, beside them the scaling of tiles 0, 1;
// and through slots 2..13 the decode of the next step's B operands, three
// slots per packed word. A tile is scaled (y += s * group sums) at least two
// slots after its last MFMA and before its next first one, so one set of
// group-sum accumulators suffices and the matrix core and the vector ALU
// work side by side within a wave. Each A fragment feeds one MFMA and is read
// from LDS three slots ahead of it.
template <int GSTEPS, bool ROUNDED>
__global__ __launch_bounds__(kReThreads) void qgemm_re_kernel(ReArgs r) {
  const TileArgs& a = r.t;
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kAStages][kAStage];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2][kWBuf];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s[kCols * kSCol];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[ROUNDED ? kCols * kSCol : 16];  // ROUNDED: biases

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31;
  const int lh = lane >> 5;
  const int mi = wave >> 2;  // rows 128*mi ..
  const int ni = wave & 3;   // columns 32*ni ..

  const int nb_n = (a.N + kCols - 1) / kCols;
  int tile, split;
  work_unit(nb_n * ((a.M + kRows - 1) / kRows), a.splits, &tile, &split);
  const int m0 = (tile / nb_n) * kRows;
  const int n0 = (tile % nb_n) * kCols;
  // Steps are local to the K range; s0 (a multiple of 4) is its first global step.
  const int steps = a.split_steps;
  const int s0 = split * steps;
  const int last = steps - 1;
  const int g0 = s0 / GSTEPS;  // first group of the range (even)
  const int g1 = g0 + steps / GSTEPS;

  // Activation transfers: this wave fills 8-row groups g8 = kAOps*wave + i of
  // a stage; lane L writes slot L%8 of local row 8*g8 + L/8, so it loads chunk
  // (L%8) ^ (L/8) ^ (g8%2). Rows past M repeat row M-1 (unstored outputs).
  // Lane offsets are 32-bit from the step's scalar base x + 128*(s0+step).
  uint32_t a_off[RePlan::kAOps];
#pragma unroll
  for (int i = 0; i < RePlan::kAOps; ++i) {
    const int g8 = RePlan::kAOps * wave + i;
    const int row = min(m0 + 8 * g8 + (lane >> 3), a.M - 1);
    a_off[i] = static_cast<uint32_t>(row * a.xs0 * 2) + 16 * ((lane & 7) ^ (lane >> 3) ^ (g8 & 1));
  }
  // Activation transfer instruction i of step `step` into ring stage `stage`.
  auto issue_a1 = [&](int step, int stage, int i) {
    dma16(sadd(a.x, static_cast<int64_t>(s0 + step) * 128), a_off[i],
          lds_address(lds_a[0]) + stage * kAStage + 1024 * (RePlan::kAOps * wave + i));
  };
  auto issue_a = [&](int step, int stage) {
#pragma unroll
    for (int i = 0; i < RePlan::kAOps; ++i) issue_a1(step, stage, i);
  };
  // Packed-word transfers: instruction j = kWOps*wave + i, lane L writes byte
  // 1024j + 16L of a buffer = physical slot L%8 of local column 8j + L/8.
  uint32_t w_off[RePlan::kWOps];
#pragma unroll
  for (int i = 0; i < RePlan::kWOps; ++i) {
    const int c = 8 * (RePlan::kWOps * wave + i) + (lane >> 3);
    const int col = min(n0 + c, a.N - 1);  // columns past N feed unstored outputs
    w_off[i] = static_cast<uint32_t>(col * a.ws0 * 4) + 16 * w_slot(c, lane & 7);
  }
  // Instruction i of the packed words of steps step4 .. step4+3 into buffer buf.
  auto issue_w1 = [&](int step4, int buf, int i) {
    dma16(sadd(a.w, static_cast<int64_t>(s0 + step4) * 32), w_off[i],
          lds_address(lds_w[0]) + buf * kWBuf + 1024 * (RePlan::kWOps * wave + i));
  };
  auto issue_w = [&](int step4, int buf) {
#pragma unroll
    for (int i = 0; i < RePlan::kWOps; ++i) issue_w1(step4, buf, i);
  };
  // Scales of the K range: column c holds 32 dwords (groups g0 .. g0+63),
  // dword d at physical dword d ^ (c%32), so the per-step reads (32
  // consecutive columns, one group) hit distinct banks. Instruction i, lane L
  // writes dword 64i + L: column 2i + L/32, physical dword L%32. Dwords past
  // the row end repeat the row's last dword.
  // (ROUNDED: the biases the same way into lds_b.)
  auto issue_p = [&](const uint8_t* src, int64_t row_stride, uint8_t* dst, int ii) {
    const int i = RePlan::kSOps * wave + ii;
    const int c = 2 * i + (lane >> 5);
    const int col = min(n0 + c, a.N - 1);
    const int row_dwords = (a.K >> (5 + a.group_shift)) / 2;
    const int d = min((g0 >> 1) + ((lane & 31) ^ (c & 31)), row_dwords - 1);
    load_lds<4>(src + static_cast<int64_t>(col) * row_stride * 2 + 4 * d, lds_address(dst) + 256 * i);
  };
  auto issue_s = [&](int ii) { issue_p(a.s, a.ss0, lds_s, ii); };
  // Scale of this wave's column (local 32*ni + li) for global group g of the range.
  const int s_lane = kSCol * (32 * ni + li);
  auto param = [&](const uint8_t* lds, int g) -> float {
    const int gl = g - g0;
    const uint32_t bits = *reinterpret_cast<const uint16_t*>(lds + s_lane + 4 * ((gl >> 1) ^ li) + 2 * (gl & 1));
    return bf16_bits_to_f32(bits);
  };
  auto scale = [&](int g) -> float { return param(lds_s, g); };
  // A fragment (mt, kk): local row 128*mi + 32*mt + li, chunk 4*lh + kk. The
  // swizzle depends on the row only through li, so mt adds 4096 bytes.
  int a_rd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int row = 128 * mi + li;
    a_rd[kk] = (row >> 3) * 1024 + (8 * (row & 7) + a_slot(row, 4 * lh + kk)) * 16;
  }
  auto read_a = [&](int stage, int mt, int kk) -> bf16x8_t {
    return *reinterpret_cast<const bf16x8_t*>(&lds_a[0][0] + stage * kAStage + a_rd[kk] + 4096 * mt);
  };
  // The lane's four packed words (local column 32*ni + li, part 2*sub + lh)
  // of a step with t % 4 = sub, in buffer buf.
  int w_rd[4];
#pragma unroll
  for (int sub = 0; sub < 4; ++sub) {
    const int c = 32 * ni + li;
    w_rd[sub] = kWRun * c + 16 * w_slot(c, 2 * sub + lh);
  }
  auto read_w = [&](int buf, int sub) -> u32x4_t {
    return *reinterpret_cast<const u32x4_t*>(&lds_w[0][0] + buf * kWBuf + w_rd[sub]);
  };

  // Prologue, as the issue order the waits count (RePlan): scales; packed
  // words of steps 0..3; activations of steps 0 and 1. Then the B operands of
  // column block 0 for step 0 (the loop decodes them one step ahead).
#pragma unroll
  for (int ii = 0; ii < RePlan::kSOps; ++ii) issue_s(ii);
  if constexpr (ROUNDED) {
#pragma unroll
    for (int ii = 0; ii < RePlan::kSOps; ++ii) issue_p(a.b, a.bs0, lds_b, ii);
  }
  issue_w(0, 0);
  issue_a(0, 0);
  issue_a(min(1, last), 1);
  wait_vmcnt<2 * RePlan::kAOps>();  // the scales and the packed words of steps 0..3
  __syncthreads();
  bf16x8_t bq[4];  // B operands of the step, by chunk
  {
    const u32x4_t w = read_w(0, 0);
    if constexpr (ROUNDED) {
      const float s_0 = scale(s0 / GSTEPS) * 512.0f, b_0 = param(lds_b, s0 / GSTEPS);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) bq[kk] = weights_rounded(w[kk], s_0, b_0);
    } else {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) bq[kk] = codes_convert(codes_split(w[kk]));
    }
  }

  f32x16_t y[4], acc[4];
#pragma unroll
  for (int T = 0; T < 4; ++T)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      y[T][v] = 0.0f;
      acc[T][v] = 0.0f;  // tiles 2, 3 of "step -1" are scaled by 0 in the first step
    }
  const f32x16_t zero = {};
  float sc_prev = 0.0f;  // scale of the previous step

  int stage = 0;  // t % 3
  for (int t = 0; t < steps; t += 4) {
    Unroll<0, 4>::run([&](auto jc) {
      constexpr int J = decltype(jc)::value;
      const int tt = t + J;
      wait_vmcnt<RePlan::wait(J)>();
      __syncthreads();
      // Iteration tt issues the activations of step tt+2 (into the stage
      // step tt-1 used), then at tt % 4 == 0 the packed words of steps tt+4 ..
      // tt+7 (into the buffer steps tt-4 .. tt-1 used), one instruction every
      // other slot (slots 0, 2, 4, 6, then 8, 10) so that the workgroup's
      // transfers do not queue up at the start of the step. Past the range
      // end the last step is fetched again into the same free places, so
      // every iteration issues the same transfers.
      const int a_step = min(tt + 2, last), a_stage = stage == 0 ? 2 : stage - 1;
      const int w_step = min(tt + 4, last & ~3), w_buf = ((tt >> 2) + 1) & 1;
      static_assert(RePlan::kAOps == 4 && RePlan::kWOps == 2, "transfer slots below");
      // The next step's packed words (the last step reads its own again),
      // decoded during this step; the fragments of slots 0..2.
      const int buf = (tt >> 2) & 1;
      const u32x4_t wvn = J == 3 ? read_w(tt + 1 <= last ? buf ^ 1 : buf, tt + 1 <= last ? 0 : 3) : read_w(buf, J + 1);
      bf16x8_t af[16];  // by slot
      af[0] = read_a(stage, 0, 0);
      af[1] = read_a(stage, 1, 0);
      af[2] = read_a(stage, 0, 1);
      constexpr bool kFirst = GSTEPS == 1 || (J & 1) == 0;     // first step of its group
      constexpr bool kLast = GSTEPS == 1 || (J & 1) == 1;      // last step of its group
      constexpr bool kPrevLast = GSTEPS == 1 || (J & 1) == 0;  // the previous step ended a group
      bf16x8_t bqn[4];
      uint32_t m_even = 0, m_odd = 0;
      CodePair cp;
      f32x2_t ce[2], co[2];  // ROUNDED: converted codes (even, odd) of one word
      float sc = 0.0f;
      float sn = 0.0f, bn = 0.0f;  // ROUNDED: scale (times 2^9) and bias of the next step's group
      Unroll<0, 16>::run([&](auto sc_) {
        constexpr int s = decltype(sc_)::value;
        constexpr int half = s / 8, rr = s % 8, kk = rr / 2, mt = 2 * half + rr % 2;
        if constexpr (s % 2 == 0 && s < 8) issue_a1(a_step, a_stage, s / 2);
        if constexpr (J == 0 && (s == 8 || s == 10)) issue_w1(w_step, w_buf, (s - 8) / 2);
        if constexpr (s + 3 < 16) {
          constexpr int s3 = s + 3, r3 = s3 % 8;
          af[s3] = read_a(stage, 2 * (s3 / 8) + r3 % 2, r3 / 2);
        }
        if constexpr (!ROUNDED && s == 4) sc = scale((s0 + tt) / GSTEPS);
        if constexpr (ROUNDED && s == 0) {
          const int gn = (s0 + min(tt + 1, last)) / GSTEPS;
          sn = scale(gn) * 512.0f;
          bn = param(lds_b, gn);
        }
        if constexpr (ROUNDED)
          y[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s], bq[kk], y[mt], 0, 0, 0);
        else
          acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s], bq[kk], (kFirst && kk == 0) ? zero : acc[mt], 0,
                                                            0, 0);
        // Scaling: four elements of tile 2 + rr/4 (previous step) or rr/4.
        constexpr int ST = half == 0 ? 2 + rr / 4 : rr / 4, v0 = 4 * (rr % 4);
        if constexpr (!ROUNDED && (half == 0 ? kPrevLast : kLast)) {
          const float s_t = half == 0 ? sc_prev : sc;
#pragma unroll
          for (int v = v0; v < v0 + 4; ++v) y[ST][v] = fmaf(s_t, acc[ST][v], y[ST][v]);
        }
        // Decode of the next step's word w in slots 2+3w (nibble masks),
        // 3+3w (ordering), 4+3w (conversion).
        if constexpr (ROUNDED && s >= 2 && s < 14) {
          // ROUNDED: nibble masks and the even codes' conversion; the odd
          // codes' conversion and dwords 0, 1; dwords 2, 3 of bf16(s*q + b).
          constexpr int w = (s - 2) / 3, ph = (s - 2) % 3;
          if constexpr (ph == 0) {
            m_even = wvn[w] & 0x0f0f0f0fu;
            m_odd = (wvn[w] >> 4) & 0x0f0f0f0fu;
            ce[0] = __builtin_amdgcn_cvt_pk_f32_fp8(m_even, false);  // codes 0, 2
            ce[1] = __builtin_amdgcn_cvt_pk_f32_fp8(m_even, true);   // codes 4, 6
          } else if constexpr (ph == 1) {
            co[0] = __builtin_amdgcn_cvt_pk_f32_fp8(m_odd, false);  // codes 1, 3
            co[1] = __builtin_amdgcn_cvt_pk_f32_fp8(m_odd, true);   // codes 5, 7
            bqn[w] = __builtin_bit_cast(bf16x8_t, u32x4_t{pack_bf16(fmaf(ce[0].x, sn, bn), fmaf(co[0].x, sn, bn)),
                                                          pack_bf16(fmaf(ce[0].y, sn, bn), fmaf(co[0].y, sn, bn)), 0u,
                                                          0u});
          } else {
            u32x4_t v = __builtin_bit_cast(u32x4_t, bqn[w]);
            v[2] = pack_bf16(fmaf(ce[1].x, sn, bn), fmaf(co[1].x, sn, bn));
            v[3] = pack_bf16(fmaf(ce[1].y, sn, bn), fmaf(co[1].y, sn, bn));
            bqn[w] = __builtin_bit_cast(bf16x8_t, v);
          }
        } else if constexpr (!ROUNDED && s >= 2 && s < 14) {
          constexpr int w = (s - 2) / 3, ph = (s - 2) % 3;
          if constexpr (ph == 0) {
            m_even = wvn[w] & 0x0f0f0f0fu;
            m_odd = (wvn[w] >> 4) & 0x0f0f0f0fu;
          } else if constexpr (ph == 1) {
            cp = CodePair{__builtin_amdgcn_perm(m_odd, m_even, 0x05010400u),
                          __builtin_amdgcn_perm(m_odd, m_even, 0x07030602u)};
          } else {
            bqn[w] = codes_convert(cp);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      });
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) bq[kk] = bqn[kk];
      sc_prev = sc;
      stage = stage == 2 ? 0 : stage + 1;
    });
  }
  if constexpr (ROUNDED) {
    wait_vmcnt<0>();  // the loop's last transfers (re-fetches of the final step)
  } else {
    // Bias term: y += sum over the range's groups of X_t[row][g] * b[col][g],
    // 16 groups per MFMA. Its operands go through LDS, brought by whole-line
    // transfers once every wave is done with the loop's buffers: the tile's
    // rows of the three planes (this range's 128-byte rows, groups g0 ..
    // g0+63) into the activation ring, plane t at 32 KiB * t, row r at 128 * r,
    // 16-byte slot q at a_slot(r, q); the tile's biases into the scale area
    // with the scales' layout.
    wait_vmcnt<0>();  // the loop's last transfers (re-fetches of the final step)
    __syncthreads();
    {
      static_assert(3 * kRows * 128 <= kAStages * kAStage, "three plane tiles fit the activation ring");
      static_assert(3 * kRows / 8 % kReWaves == 0, "whole plane transfers per wave");
      constexpr int kXOps = 3 * kRows / 8 / kReWaves;
      const uint16_t* planes = r.planes + static_cast<int64_t>(split) * 3 * a.M * kMaxGroups;
  #pragma unroll
      for (int ii = 0; ii < kXOps; ++ii) {
        const int i = kXOps * wave + ii;  // plane i / 32, rows 8*(i%32) ..
        const int pl = i / (kRows / 8), rg = i % (kRows / 8);
        const int row = min(m0 + 8 * rg + (lane >> 3), a.M - 1);
        const int q = (lane & 7) ^ (lane >> 3) ^ (rg & 1);
        load_lds<16>(planes + (static_cast<int64_t>(pl) * a.M + row) * kMaxGroups + 8 * q,
                     lds_address(lds_a[0]) + pl * (kRows * 128) + 1024 * rg);
      }
      const int row_dwords = (a.K >> (5 + a.group_shift)) / 2;
  #pragma unroll
      for (int ii = 0; ii < RePlan::kSOps; ++ii) {
        const int i = RePlan::kSOps * wave + ii;
        const int c = 2 * i + (lane >> 5);
        const int col = min(n0 + c, a.N - 1);
        const int d = min((g0 >> 1) + ((lane & 31) ^ (c & 31)), row_dwords - 1);
        load_lds<4>(a.b + static_cast<int64_t>(col) * a.bs0 * 2 + 4 * d, lds_address(lds_s) + 256 * i);
      }
    }
    // Tiles 2, 3 of the last step (the range ends a group), while the transfers fly.
  #pragma unroll
    for (int T = 2; T < 4; ++T)
  #pragma unroll
      for (int v = 0; v < 16; ++v) y[T][v] = fmaf(sc_prev, acc[T][v], y[T][v]);
    wait_vmcnt<0>();
    __syncthreads();
    // Chunk c: lane half h takes local groups 16c + 8h .. +7; entries of groups
    // past the range are replaced by zeros on both sides.
    const int gcount = g1 - g0;
  #pragma unroll
    for (int c = 0; c < kMaxGroups / 16; ++c) {
      const int gl = 16 * c + 8 * lh;
      u32x4_t bb, xv[3][4];
  #pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(lds_s + s_lane + 4 * (((gl >> 1) + e) ^ li));
        bb[e] = gl + 2 * e < gcount ? v : 0u;
      }
  #pragma unroll
      for (int pl = 0; pl < 3; ++pl)
  #pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const int row = 128 * mi + 32 * mt + li;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&lds_a[0][0] + pl * (kRows * 128) + row * 128 +
                                                              16 * a_slot(row, 2 * c + lh));
  #pragma unroll
          for (int e = 0; e < 4; ++e) xv[pl][mt][e] = gl + 2 * e < gcount ? v[e] : 0u;
        }
  #pragma unroll
      for (int pl = 0; pl < 3; ++pl)
  #pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          y[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, xv[pl][mt]),
                                                          __builtin_bit_cast(bf16x8_t, bb), y[mt], 0, 0, 0);
    }
  }

  // Accumulator tile mt, element v of lane l is row 8*(v/4) + 4*(l/32) + v%4
  // and column l%32 of its 32x32 tile. Offsets are 32-bit from the tile's
  // first row (256 rows * N * 4 < 2^31).
  const bool full = m0 + kRows <= a.M;
  float* base = (a.splits == 1 ? a.out : a.partial + split * static_cast<int64_t>(a.M) * a.N) +
                static_cast<int64_t>(m0) * a.N;
  const int col = n0 + 32 * ni + li;
  with_store_kind(a.splits == 1 ? a.epi.kind : kEpiNone, [&](auto kind) {
    constexpr int KIND = decltype(kind)::value;
    if (col < a.N) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rr = 128 * mi + 32 * mt + 8 * (v / 4) + 4 * lh + (v % 4);
          if (full || m0 + rr < a.M) {
            const uint32_t off = static_cast<uint32_t>(rr * a.N + col) * 4u;
            store_as<KIND>(a.epi, reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(base) + off), col, y[mt][v]);
          }
        }
    }
  });
}

// K ranges for the reassociated GEMM: as the other tiled kernels, raised until
// each range holds at most kMaxGroups groups; 0 when no count up to 8 does.
int re_splits(int tiles, int steps, int gsteps) {
  for (int s = choose_splits(tiles, steps); s <= 8; ++s) {
    if ((steps / 4) % s != 0) continue;
    if (steps / s / gsteps <= kMaxGroups) return s;
  }
  return 0;
}

}  // namespace

bool re_gemm_supports(const QmmProblem& p) {
  if (p.bits != 4 || p.x_dtype != AFFON_ROCM_BF16 || p.p_dtype != AFFON_ROCM_BF16) return false;
  if (p.group != 64 && p.group != 128) return false;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  if (p.K % (4 * kBK) != 0) return false;  // whole 4-step packed-word runs
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || (p.xs0 * 2) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || p.ws0 % 4 != 0) return false;
  // Scales and biases are read in dwords: dword-aligned rows.
  if (reinterpret_cast<uintptr_t>(p.s) % 4 != 0 || reinterpret_cast<uintptr_t>(p.b) % 4 != 0) return false;
  if (p.ss0 % 2 != 0 || p.bs0 % 2 != 0) return false;
  if (p.M > (int64_t(1) << 24) || p.N > (int64_t(1) << 20) || p.K > (int64_t(1) << 24)) return false;
  // The transfers take 32-bit lane offsets from a scalar base: the row of
  // the last activation row and the column of the last weight column, in
  // bytes, stay below 2^31 (as the parameter rows, read with 64-bit offsets,
  // do for symmetry); the grid (tiles x at most 8 K ranges) stays an int.
  const int64_t limit = int64_t(1) << 31;
  if (p.M * p.xs0 * 2 >= limit || p.N * p.ws0 * 4 >= limit) return false;
  if (p.N * p.ss0 * 2 >= limit || p.N * p.bs0 * 2 >= limit) return false;
  if (((p.N + kCols - 1) / kCols) * ((p.M + kRows - 1) / kRows) > (int64_t(1) << 27)) return false;
  return true;
}

bool re_gemm_launch(const QmmProblem& p, const Launch& l, hipError_t* status, bool rounded) {
  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  const int steps = K / kBK;
  const int gsteps = static_cast<int>(p.group / kBK);
  const int tiles = ((N + kCols - 1) / kCols) * ((M + kRows - 1) / kRows);
  const int splits = l.can_split() ? re_splits(tiles, steps, gsteps) : (steps / gsteps <= kMaxGroups ? 1 : 0);
  // A K range of fewer than 16 steps leaves too little loop for the kernel's
  // fixed costs (prologue, partial sums; for the reassociated class also the
  // group-sum pre-pass and the bias term): the other kernels of the class
  // are faster there (e.g. 128 x 4096 x 4096 on the row-tiled decode kernel:
  // 15.7 against 31.4 us).
  if (splits == 0 || steps / splits < kMinRangeSteps) return false;
  const int range_groups = steps / splits / gsteps;
  const size_t partial_bytes = splits > 1 ? static_cast<size_t>(splits) * M * N * 4 : 0;
  const size_t plane_bytes = rounded ? 0 : static_cast<size_t>(splits) * 3 * M * kMaxGroups * 2;
  const size_t total = ((partial_bytes + 255) & ~size_t(255)) + plane_bytes;
  uint8_t* scratch = nullptr;
  if (total > 0) {
    if (l.fixed != nullptr && total > l.fixed_bytes) {
      // A fixed buffer too small for this plan: nothing is launched and the
      // caller rejects the shape (running another kernel would change the
      // plan the allocating entry point runs).
      l.fixed_short = total;
      *status = hipErrorOutOfMemory;
      return true;
    }
    if (!l.can_split() || (scratch = static_cast<uint8_t*>(l.scratch(total))) == nullptr) return false;
  }

  ReArgs r;
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
  a.M = M;
  a.N = N;
  a.K = K;
  a.group_shift = p.group == 64 ? 1 : 2;
  a.splits = splits;
  a.split_steps = steps / splits;
  a.partial = splits > 1 ? reinterpret_cast<float*>(scratch) : nullptr;
  r.planes = rounded ? nullptr : reinterpret_cast<const uint16_t*>(scratch + ((partial_bytes + 255) & ~size_t(255)));

  hipError_t e = hipSuccess;
  if (!rounded) {
    const int64_t chunks = static_cast<int64_t>(M) * (K / 8);
    hipLaunchKernelGGL(group_sums_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0, l.stream,
                       a.x, a.xs0, M, K, static_cast<int>(p.group), range_groups, const_cast<uint16_t*>(r.planes));
    e = hipGetLastError();
  }
  if (e == hipSuccess) {
    const dim3 grid(tiles * splits), block(kReThreads);
    if (rounded)
      hipLaunchKernelGGL((gsteps == 1 ? qgemm_re_kernel<1, true> : qgemm_re_kernel<2, true>), grid, block, 0,
                         l.stream, r);
    else
      hipLaunchKernelGGL((gsteps == 1 ? qgemm_re_kernel<1, false> : qgemm_re_kernel<2, false>), grid, block, 0,
                         l.stream, r);
    e = hipGetLastError();
  }
  if (e == hipSuccess && splits > 1) e = launch_reduce(a, l.stream);
  *status = e;
  return true;
}

}  // namespace affon
