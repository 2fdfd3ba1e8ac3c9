// rocm_quantized_matmul.gemv_mfma for prefill: the reassociated class on a
// large-tile GEMM (4-bit codes, bf16 activations and parameters, groups of 64
// or 128).
//
// Counterpart of the reference's matrix paths (metal matrix32 /
// matrix32_packed, docs/core/quantized-inference.md:138-139,151-170), which
// decode weights to f32 and are classified "reassociated". Same arithmetic
// as the decode-batch kernels (gemv_mfma.hip): the packed codes q are exact
// integers in bf16 MFMA operands, each group's sums sum(x*q) come out of
// v_mfma_f32_32x32x16_bf16 with f32 accumulation, and the group's scale and
// bias are applied in f32:
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
// 4 x 2 arrangement; wave (mi, ni) computes rows 64*mi.. x columns 64*ni..
// (2 x 2 accumulators of 32 x 32 for y, as many for the current group's
// sums), two waves per SIMD so that one wave's decode and scaling run on the
// vector ALU while the other's MFMAs run. K steps of 64; MFMA kk (0..3) of
// lane half h covers chunk 4h + kk of the step (8 k each), so a lane's codes
// of one column and step are 16 contiguous bytes.
//
// Transfers, all direct global-to-LDS and counted (no compiler-visible loads
// in the loop): the tile's scales for the whole K range once, first; packed
// words of four steps at a time (128 bytes per column: whole lines) into two
// buffers, four steps ahead; activations (256 rows x 128 bytes per step) into
// a 3-stage ring, two steps ahead. One barrier per step orders the shared
// tiles.

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

static_assert(kRows / 8 / kReWaves == RePlan::kAOps, "8-row activation transfers per wave and step");
static_assert(kWBuf / 1024 / kReWaves == RePlan::kWOps, "packed-word transfers per wave and four steps");
static_assert(kCols * kSCol / 256 / kReWaves == RePlan::kSOps, "scale transfers per wave");

struct ReArgs {
  TileArgs t;
  const uint16_t* planes;  // [3][M][gp] bf16: X1, X2, X3 of every row and group
  int gp;                  // plane row stride (groups, a multiple of 8)
};

// Slot (16-byte unit) of part `part` (0..7) in local column c's 128-byte
// packed run: within 8 consecutive columns the slots differ, and columns c
// and c + 8 differ in slot bit 0, so the decode reads (lanes = consecutive
// columns, one part) are bank-conflict free.
__device__ __forceinline__ int w_slot(int c, int part) { return part ^ (c & 7) ^ ((c >> 3) & 1); }

// Physical 16-byte slot of logical chunk q of local activation row r: the
// fragment reads (consecutive rows, one chunk) are bank-conflict free.
__device__ __forceinline__ int a_slot(int r, int q) { return q ^ (r & 7) ^ ((r >> 3) & 1); }

// B operand of MFMA kk from the lane's packed word kk (codes 8 per word, code
// i in nibble i): the codes as exact bf16 integers times 2^-9 (a byte holding
// n < 16 reads as n * 2^-9 in FP8 E4M3; the scale carries 2^9).
__device__ __forceinline__ bf16x8_t codes_op(uint32_t w) {
  const uint32_t even = w & 0x0f0f0f0fu;         // byte j = code 2j
  const uint32_t odd = (w >> 4) & 0x0f0f0f0fu;   // byte j = code 2j+1
  const uint32_t lo = __builtin_amdgcn_perm(odd, even, 0x05010400u);  // codes 0,1,2,3
  const uint32_t hi = __builtin_amdgcn_perm(odd, even, 0x07030602u);  // codes 4,5,6,7
  const u32x4_t v{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false)),
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true)),
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false)),
                  __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true))};
  return __builtin_bit_cast(bf16x8_t, v);
}

// X = sum of the `group` activations of one row and group in f32 (k order),
// stored as three bf16 planes whose sum is X exactly; plane entries past the
// last group are zero.
__global__ __launch_bounds__(256) void group_sums_kernel(const uint16_t* x, int64_t xs0, int M, int G, int gp,
                                                         int group, uint16_t* planes) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(M) * gp) return;
  const int row = static_cast<int>(i / gp);
  const int g = static_cast<int>(i % gp);
  float sum = 0.0f;
  if (g < G) {
    const uint16_t* p = x + row * xs0 + static_cast<int64_t>(g) * group;
    for (int k = 0; k < group; k += 8) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p + k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sum += __uint_as_float(v[e] << 16);
        sum += __uint_as_float(v[e] & 0xffff0000u);
      }
    }
  }
  const uint16_t h1 = f32_to_bf16_bits(sum);
  uint16_t h2 = 0, h3 = 0;
  if (__builtin_isfinite(sum)) {
    const float r1 = sum - bf16_bits_to_f32(h1);  // exact
    h2 = f32_to_bf16_bits(r1);
    h3 = f32_to_bf16_bits(r1 - bf16_bits_to_f32(h2));  // exact: the remaining bits fit bf16
  }
  planes[i] = h1;
  planes[static_cast<int64_t>(M) * gp + i] = h2;
  planes[2 * static_cast<int64_t>(M) * gp + i] = h3;
}

// GSTEPS: K steps per group (1: group 64, 2: group 128).
template <int GSTEPS>
__global__ __launch_bounds__(kReThreads) void qgemm_re_kernel(ReArgs r) {
  const TileArgs& a = r.t;
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kAStages][kAStage];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2][kWBuf];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s[kCols * kSCol];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31;
  const int lh = lane >> 5;
  const int mi = wave >> 1;  // rows 64*mi ..
  const int ni = wave & 1;   // columns 64*ni ..

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
  const uint16_t* a_src[RePlan::kAOps];
#pragma unroll
  for (int i = 0; i < RePlan::kAOps; ++i) {
    const int g8 = RePlan::kAOps * wave + i;
    const int row = min(m0 + 8 * g8 + (lane >> 3), a.M - 1);
    a_src[i] = a.x + static_cast<int64_t>(row) * a.xs0 + 8 * ((lane & 7) ^ (lane >> 3) ^ (g8 & 1));
  }
  auto issue_a = [&](int step, int stage) {
#pragma unroll
    for (int i = 0; i < RePlan::kAOps; ++i)
      load_lds<16>(a_src[i] + static_cast<int64_t>(s0 + step) * kBK,
                   lds_address(lds_a[0]) + stage * kAStage + 1024 * (RePlan::kAOps * wave + i));
  };
  // Packed-word transfers: instruction j = kWOps*wave + i, lane L writes byte
  // 1024j + 16L of a buffer = physical slot L%8 of local column 8j + L/8.
  const uint8_t* w_src[RePlan::kWOps];
#pragma unroll
  for (int i = 0; i < RePlan::kWOps; ++i) {
    const int c = 8 * (RePlan::kWOps * wave + i) + (lane >> 3);
    const int col = min(n0 + c, a.N - 1);  // columns past N feed unstored outputs
    w_src[i] = reinterpret_cast<const uint8_t*>(a.w + static_cast<int64_t>(col) * a.ws0) + 16 * w_slot(c, lane & 7);
  }
  // The packed words of steps step4 .. step4+3 into buffer buf.
  auto issue_w = [&](int step4, int buf) {
#pragma unroll
    for (int i = 0; i < RePlan::kWOps; ++i)
      load_lds<16>(w_src[i] + static_cast<int64_t>(s0 + step4) * 32,
                   lds_address(lds_w[0]) + buf * kWBuf + 1024 * (RePlan::kWOps * wave + i));
  };
  // Scales of the K range: column c holds 32 dwords (groups g0 .. g0+63),
  // dword d at physical dword d ^ (c%32), so the per-step reads (32
  // consecutive columns, one group) hit distinct banks. Instruction i, lane L
  // writes dword 64i + L: column 2i + L/32, physical dword L%32. Dwords past
  // the row end repeat the row's last dword.
  auto issue_s = [&](int ii) {
    const int i = RePlan::kSOps * wave + ii;
    const int c = 2 * i + (lane >> 5);
    const int col = min(n0 + c, a.N - 1);
    const int row_dwords = (a.K >> (5 + a.group_shift)) / 2;
    const int d = min((g0 >> 1) + ((lane & 31) ^ (c & 31)), row_dwords - 1);
    load_lds<4>(a.s + static_cast<int64_t>(col) * a.ss0 * 2 + 4 * d, lds_address(lds_s) + 256 * i);
  };
  // Scale (times 2^9) of local column c for global group g of the range.
  auto scale = [&](int c, int g) -> float {
    const int gl = g - g0;
    const int d = (gl >> 1) ^ (c & 31);
    const uint32_t bits = *reinterpret_cast<const uint16_t*>(lds_s + kSCol * c + 4 * d + 2 * (gl & 1));
    return bf16_bits_to_f32(bits) * 512.0f;
  };
  // A fragment (mt, kk): local row 64*mi + 32*mt + li, chunk 4*lh + kk.
  auto read_a = [&](int stage, int mt, int kk) -> bf16x8_t {
    const int row = 64 * mi + 32 * mt + li;
    return *reinterpret_cast<const bf16x8_t*>(&lds_a[0][0] + stage * kAStage + (row >> 3) * 1024 +
                                              (8 * (row & 7) + a_slot(row, 4 * lh + kk)) * 16);
  };
  // The lane's four packed words of column 64*ni + 32*nt + li for step t.
  auto read_w = [&](int t, int nt) -> u32x4_t {
    const int c = 64 * ni + 32 * nt + li;
    return *reinterpret_cast<const u32x4_t*>(&lds_w[0][0] + ((t >> 2) & 1) * kWBuf + kWRun * c +
                                             16 * w_slot(c, 2 * (t & 3) + lh));
  };

  // Prologue, as the issue order the waits count (RePlan): scales; packed
  // words of steps 0..3; activations of steps 0 and 1.
#pragma unroll
  for (int ii = 0; ii < RePlan::kSOps; ++ii) issue_s(ii);
  issue_w(0, 0);
  issue_a(0, 0);
  issue_a(min(1, last), 1);

  f32x16_t y[2][2], acc[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int v = 0; v < 16; ++v) y[mt][nt][v] = 0.0f;
  const f32x16_t zero = {};

  int stage = 0;  // t % 3
  for (int t = 0; t < steps; t += 4) {
    Unroll<0, 4>::run([&](auto jc) {
      constexpr int J = decltype(jc)::value;
      const int tt = t + J;
      wait_vmcnt<RePlan::wait(J)>();
      __syncthreads();
      // Iteration tt issues the activations of step tt+2 (into the stage
      // step tt-1 used), then at tt % 4 == 0 the packed words of steps tt+4 ..
      // tt+7 (into the buffer steps tt-4 .. tt-1 used). Past the range end
      // the last step is fetched again into the same free places, so every
      // iteration issues the same transfers.
      issue_a(min(tt + 2, last), stage == 0 ? 2 : stage - 1);
      if constexpr (J == 0) issue_w(min(tt + 4, last & ~3), ((tt >> 2) + 1) & 1);

      const u32x4_t wv[2] = {read_w(tt, 0), read_w(tt, 1)};
      constexpr bool kFirst = GSTEPS == 1 || (J & 1) == 0;  // first step of its group
      constexpr bool kLast = GSTEPS == 1 || (J & 1) == 1;   // last step of its group
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8_t af[2] = {read_a(stage, 0, kk), read_a(stage, 1, kk)};
        const bf16x8_t bq[2] = {codes_op(wv[0][kk]), codes_op(wv[1][kk])};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bq[nt],
                                                                  (kFirst && kk == 0) ? zero : acc[mt][nt], 0, 0, 0);
      }
      if constexpr (kLast) {
        const int g = (s0 + tt) / GSTEPS;
        const float sc[2] = {scale(64 * ni + li, g), scale(64 * ni + 32 + li, g)};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) y[mt][nt][v] = fmaf(sc[nt], acc[mt][nt][v], y[mt][nt][v]);
      }
      stage = stage == 2 ? 0 : stage + 1;
    });
  }
  // Leave no transfer in flight (the last iterations re-fetch the final step).
  wait_vmcnt<0>();

  // Bias term: y += sum over the range's groups of X_t[row][g] * b[col][g],
  // 16 groups per MFMA; lane half h takes groups gb .. gb+7, gb = c0 + 8h.
  // Groups past the range end enter as zeros on both sides.
  for (int c0 = g0; c0 < g1; c0 += 16) {
    const int gb = c0 + 8 * lh;
    u32x4_t bb[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = min(n0 + 64 * ni + 32 * nt + li, a.N - 1);
      const uint32_t* bp = reinterpret_cast<const uint32_t*>(a.b + (static_cast<int64_t>(col) * a.bs0 + gb) * 2);
#pragma unroll
      for (int e = 0; e < 4; ++e) bb[nt][e] = gb + 2 * e < g1 ? bp[e] : 0u;
    }
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
      u32x4_t xv[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int row = min(m0 + 64 * mi + 32 * mt + li, a.M - 1);
        const uint32_t* xp =
            reinterpret_cast<const uint32_t*>(r.planes + (static_cast<int64_t>(pl) * a.M + row) * r.gp + gb);
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[mt][e] = gb + 2 * e < g1 ? xp[e] : 0u;
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          y[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, xv[mt]),
                                                              __builtin_bit_cast(bf16x8_t, bb[nt]), y[mt][nt], 0, 0, 0);
    }
  }

  // Accumulator (mt, nt) element v of lane l is row 8*(v/4) + 4*(l/32) + v%4
  // and column l%32 of its 32x32 tile. Offsets are 32-bit from the tile's
  // first row (256 rows * N * 4 < 2^31).
  const bool full = m0 + kRows <= a.M;
  float* base = (a.splits == 1 ? a.out : a.partial + split * static_cast<int64_t>(a.M) * a.N) +
                static_cast<int64_t>(m0) * a.N;
  with_store_kind(a.splits == 1 ? a.epi.kind : kEpiNone, [&](auto kind) {
    constexpr int KIND = decltype(kind)::value;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = n0 + 64 * ni + 32 * nt + li;
      if (col < a.N) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int rr = 64 * mi + 32 * mt + 8 * (v / 4) + 4 * lh + (v % 4);
            if (full || m0 + rr < a.M) {
              const uint32_t off = static_cast<uint32_t>(rr * a.N + col) * 4u;
              store_as<KIND>(a.epi, reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(base) + off), col,
                             y[mt][nt][v]);
            }
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
  return true;
}

bool re_gemm_launch(const QmmProblem& p, const Launch& l, hipError_t* status) {
  if (!l.can_split()) return false;
  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  const int steps = K / kBK;
  const int gsteps = static_cast<int>(p.group / kBK);
  const int tiles = ((N + kCols - 1) / kCols) * ((M + kRows - 1) / kRows);
  const int splits = re_splits(tiles, steps, gsteps);
  if (splits == 0) return false;
  const int G = static_cast<int>(K / p.group);
  const int gp = (G + 7) & ~7;
  const size_t partial_bytes = splits > 1 ? static_cast<size_t>(splits) * M * N * 4 : 0;
  const size_t plane_bytes = static_cast<size_t>(3) * M * gp * 2;
  const size_t total = ((partial_bytes + 255) & ~size_t(255)) + plane_bytes;
  if (l.fixed != nullptr && total > l.fixed_bytes) return false;  // the caller's other path runs instead
  uint8_t* scratch = static_cast<uint8_t*>(l.scratch(total));
  if (scratch == nullptr) return false;

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
  r.planes = reinterpret_cast<const uint16_t*>(scratch + ((partial_bytes + 255) & ~size_t(255)));
  r.gp = gp;

  const int64_t sums = static_cast<int64_t>(M) * gp;
  hipLaunchKernelGGL(group_sums_kernel, dim3(static_cast<unsigned>((sums + 255) / 256)), dim3(256), 0, l.stream,
                     a.x, a.xs0, M, G, gp, static_cast<int>(p.group), const_cast<uint16_t*>(r.planes));
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    if (gsteps == 1)
      hipLaunchKernelGGL(qgemm_re_kernel<1>, dim3(tiles * splits), dim3(kReThreads), 0, l.stream, r);
    else
      hipLaunchKernelGGL(qgemm_re_kernel<2>, dim3(tiles * splits), dim3(kReThreads), 0, l.stream, r);
    e = hipGetLastError();
  }
  if (e == hipSuccess && splits > 1) e = launch_reduce(a, l.stream);
  *status = e;
  return true;
}

}  // namespace affon
