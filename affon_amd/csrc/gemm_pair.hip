// rocm_quantized_matmul.mfma for 4-bit weights and tall activations: a
// prefill GEMM in which the two waves that share a column block each decode
// half of its weights and hand the decoded fragments to each other through
// LDS.
//
// Same arithmetic as qgemm_kernel (gemm.hip): packed codes are decoded in
// registers to s*q + b, rounded to bf16 and fed to v_mfma_f32_32x32x16_bf16
// with f32 accumulation (the "approximate" class); no floating weight matrix
// exists in memory. What changes is the work split:
//
//   * Workgroup tile 256 (rows) x 128 (columns), four waves in a 2 x 2
//     arrangement; wave (mi, ni) computes rows 128*mi.. x columns 64*ni.. of
//     the tile (4 x 2 accumulators of 32 x 32).
//   * The waves (0, ni) and (1, ni) need the same decoded weights. Wave
//     (mi, ni) decodes only the 32 columns 64*ni + 32*mi + (0..31), keeps
//     them in registers for its own MFMAs and writes them to LDS, where its
//     partner reads them. Each decoded weight then feeds 256 rows of MFMA
//     work instead of 128, halving the decode instructions per MFMA.
//   * All global reads are direct-to-LDS transfers issued as inline asm
//     (global_load_lds with an SGPR base and a constant 32-bit lane offset,
//     so the per-step address advance is scalar work), counted by hand:
//     activations into a 3-stage ring two steps ahead, packed words and
//     group-parameter windows per pair of steps, two pairs ahead.
//
// K order: K is walked in steps of 64 (8 chunks of 8 k); MFMA kk (0..3) of
// lane half h covers chunk 4h + kk of the step. So a lane's weights for one
// step are 16 contiguous bytes of its column (4 words) and each activation
// row of a step is one whole 128-byte line. Both operands use this order.
// Packed words travel per pair of steps: 64 bytes per column.

#include "lds_pipeline.h"

namespace affon {
namespace {

using namespace pipeline;

constexpr int kRows = 256;         // workgroup tile rows
constexpr int kCols = 128;         // workgroup tile columns
constexpr int kAStage = kRows * 128;   // bytes: 256 rows x 64 k of bf16
constexpr int kAStages = 3;
constexpr int kAOps = kRows / 8 / kWaves;  // activation transfers per wave and step (1 KiB each)
constexpr int kWRun = 64;          // packed bytes per column and pair of steps (4-bit)
constexpr int kWWave = 32 * kWRun; // per wave and buffer: 32 columns
constexpr int kWOps = kWWave / 1024;   // packed-word transfers per wave and pair
constexpr int kPWin = 16;          // bytes of a parameter window (per column, pair)
constexpr int kPWave = 32 * kPWin; // per wave, buffer and parameter (scales or biases)
constexpr int kPOps = 2 * (32 * 4) / 64;  // dword transfers per wave and pair: scales, biases
constexpr int kPairOps = kWOps + kPOps;

static_assert(kAOps == 8 && kWOps == 2 && kPOps == 4, "transfer counts assumed by the waits below");

// Physical 16-byte slot of logical slot q in local activation row r: XOR
// swizzle that makes the fragment reads (16 consecutive rows, one slot)
// bank-conflict free for 16-lane (256-byte) LDS phases.
__device__ __forceinline__ int a_slot(int r, int q) { return q ^ (r & 7) ^ ((r >> 3) & 1); }

// Physical slot of logical slot q (0..3) in column c's 64-byte packed run:
// the decode reads (16 consecutive columns, one slot) hit 16 distinct 16-byte
// units of a 256-byte window.
__device__ __forceinline__ int w_slot(int c, int q) { return q ^ ((c >> 2) & 3); }

// Inputs of a step's decode for one lane: its four packed words (8 codes
// each, fragments kk = 0..3) and its group's scale (times 2^9) and bias.
struct Decode {
  uint32_t words[4];
  float s, b;
};

// Intermediate values of one word's decode while it is spread over slots.
struct DecodeTmp {
  uint32_t lo, hi;
  f32x2_t l, h;
};

// Piece j (0..6) of word w's decode into the four bf16 pairs of its
// fragment, in k order. Codes n < 16 held in a byte read as n * 2^-9 in FP8
// (E4M3); the scale carries the 2^9. Pieces: masks; low conversions; pairs
// 0, 1; high conversions; pairs 2, 3.
template <int J>
__device__ __forceinline__ void decode_piece(uint32_t w, float s, float b, DecodeTmp& d, u32x4_t& out) {
  if constexpr (J == 0) {
    d.lo = w & 0x0f0f0f0fu;         // codes 0, 2, 4, 6
    d.hi = (w >> 4) & 0x0f0f0f0fu;  // codes 1, 3, 5, 7
  } else if constexpr (J == 1 || J == 4) {
    d.l = __builtin_amdgcn_cvt_pk_f32_fp8(d.lo, J == 4);
    d.h = __builtin_amdgcn_cvt_pk_f32_fp8(d.hi, J == 4);
  } else if constexpr (J == 2 || J == 5) {
    out[J == 2 ? 0 : 2] = pack_bf16(fmaf(d.l.x, s, b), fmaf(d.h.x, s, b));
  } else {
    out[J == 3 ? 1 : 3] = pack_bf16(fmaf(d.l.y, s, b), fmaf(d.h.y, s, b));
  }
}

__device__ __forceinline__ void decode_word(uint32_t w, float s, float b, u32x4_t& out) {
  DecodeTmp d;
  decode_piece<0>(w, s, b, d, out);
  decode_piece<1>(w, s, b, d, out);
  decode_piece<2>(w, s, b, d, out);
  decode_piece<3>(w, s, b, d, out);
  decode_piece<4>(w, s, b, d, out);
  decode_piece<5>(w, s, b, d, out);
  decode_piece<6>(w, s, b, d, out);
}

template <typename PT, int MI>
__device__ __forceinline__ void pair_tile(const TileArgs& a, uint8_t* lds_a, uint8_t* lds_bx, uint8_t* lds_w,
                                          uint8_t* lds_p, int m0, int n0, int split) {
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
    const int q = a_slot(r, lane & 7);  // logical slot (involution)
    const int row = min(m0 + r, a.M - 1);  // rows past M repeat the last row
    a_off[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(a.xs0 * 2) + 16 * q;
  }
  // Packed words: this wave decodes columns c = 64*ni + 32*MI + (0..31);
  // instruction j covers 16 of them, lane L -> column 16j + L/4, physical slot L%4.
  uint32_t w_off[kWOps];
#pragma unroll
  for (int j = 0; j < kWOps; ++j) {
    const int c = 16 * j + (lane >> 2);
    const int col = min(n0 + 64 * ni + 32 * MI + c, a.N - 1);  // columns past N feed unstored outputs
    w_off[j] = static_cast<uint32_t>(col) * static_cast<uint32_t>(a.ws0 * 4) + 16 * w_slot(c, lane & 3);
  }
  // Parameter windows: instruction i (0, 1 scales; 2, 3 biases) lane L ->
  // column 16(i%2) + L/4, dword L%4 of the window.
  uint32_t p_col[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int col = min(n0 + 64 * ni + 32 * MI + 16 * i + (lane >> 2), a.N - 1);
    p_col[i] = static_cast<uint32_t>(col);
  }
  const int row_dwords = (a.K >> (5 + a.group_shift)) * PT::bytes / 4;
  auto window = [&](int pair) { return ((pair * 128) >> (5 + a.group_shift)) * PT::bytes / 4; };

  const uint32_t a_lds = lds_address(lds_a);
  const uint32_t w_lds = lds_address(lds_w) + kWWave * wave;  // + buffer * 4 * kWWave
  const uint32_t p_lds = lds_address(lds_p) + 2 * kPWave * wave;  // + buffer * 8 * kPWave

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
    for (int i = 0; i < 4; ++i) {
      const uint8_t* pbase = i < 2 ? a.s : a.b;
      const int64_t ps0 = i < 2 ? a.ss0 : a.bs0;
      const uint32_t off = static_cast<uint32_t>(p_col[i & 1] * ps0 * PT::bytes) + 4 * d;
      dma4(pbase, off, p_lds + buf * kWaves * 2 * kPWave + (i >> 1) * kPWave + 256 * (i & 1));
    }
  };

  // ---- decode inputs of local step t for this lane ----
  const int wq_lane = 64 * li;  // column li's run in the wave's buffer
  const float code_scale = 512.0f;
  auto load_decode = [&](int t, Decode& d) {
    const int tt = min(t, steps - 1);
    const int pr = tt >> 1, s = tt & 1;
    const uint8_t* wbuf = lds_w + (pr & 1) * kWaves * kWWave + kWWave * wave;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wbuf + wq_lane + 16 * w_slot(li, 2 * s + lh));
    d.words[0] = v.x;
    d.words[1] = v.y;
    d.words[2] = v.z;
    d.words[3] = v.w;
    const int gp = (s0 >> 1) + pr;
    const int grp = (gp * 128 + 64 * s + 32 * lh) >> (5 + a.group_shift);
    const int off = grp * PT::bytes - 4 * window(gp);
    const uint8_t* pbuf = lds_p + (pr & 1) * kWaves * 2 * kPWave + 2 * kPWave * wave + kPWin * li + off;
    uint32_t sr, br;
    if constexpr (PT::bytes == 2) {
      sr = *reinterpret_cast<const uint16_t*>(pbuf);
      br = *reinterpret_cast<const uint16_t*>(pbuf + kPWave);
    } else {
      sr = *reinterpret_cast<const uint32_t*>(pbuf);
      br = *reinterpret_cast<const uint32_t*>(pbuf + kPWave);
    }
    d.s = widen_param<PT>(sr) * code_scale;
    d.b = widen_param<PT>(br);
  };

  // ---- LDS addresses of the fragment reads ----
  // A fragment (mt, kk): local row 128*MI + 32*mt + li, logical slot 4*lh + kk.
  uint32_t a_frag[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    a_frag[kk] = (128 * MI + li) * 128 + 16 * a_slot(li, 4 * lh + kk);
  // Exchanged fragments: [buf][ni][mi][kk] x 1 KiB, lane-major.
  auto bx_at = [&](int buf, int mi, int kk) -> uint8_t* {
    return lds_bx + (((buf * 2 + ni) * 2 + mi) * 4 + kk) * 1024 + 16 * lane;
  };

  f32x16_t acc_own[4], acc_par[4];  // columns 32*MI + li and 32*(1-MI) + li of the wave's 64
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc_own[mt][v] = acc_par[mt][v] = 0.0f;
  u32x4_t bo[2][4];  // own decoded fragments by step parity
  u32x4_t bp[4];     // the partner's fragments of the current step
  bf16x8_t af[2][4]; // activation fragments of chunks kk by parity
  // The four partner MFMAs of chunk 3 run after the next step's barrier,
  // from af[1] and bp[3] (zero before the first step).
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) af[1][mt] = __builtin_bit_cast(bf16x8_t, u32x4_t{0, 0, 0, 0});
  bp[3] = u32x4_t{0, 0, 0, 0};

  // ---- prologue: transfers as if issued by steps -3 .. -1 ----
  issue_pair(0);
  issue_a(0);
  issue_a(1);
  issue_pair(1);
  wait_vmcnt<2 * kAOps + kPairOps>();  // pair 0 landed
  {
    Decode d;
    load_decode(0, d);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      decode_word(d.words[kk], d.s, d.b, bo[0][kk]);
      *reinterpret_cast<u32x4_t*>(bx_at(0, MI, kk)) = bo[0][kk];
    }
  }

  // One step, hand-ordered. At entry the activations of step t and the words
  // of step t+1 were requested at least two steps earlier, and the own
  // fragments of step t are in bo[P] and in LDS buffer P. After the barrier:
  // the reads of chunk 0's activation fragments and of the partner's
  // fragments, then the four partner MFMAs left over from the previous step
  // (their operands are in registers) while those reads land, then 28 slots
  // of one MFMA each. Slot p carries one piece of the decode of the next
  // step's fragments (word p/7, piece p%7; the fragment goes to LDS after its
  // last piece), transfer p/2 on odd p, and at the start of each chunk the
  // activation reads of the following chunk. Scheduling barriers keep the
  // order, so the vector ALU and the memory pipelines work while the matrix
  // core does.
#define AFFON_PAIR_STEP(P)                                                                                   \
  {                                                                                                          \
    wait_vmcnt<(P) ? kAOps : kAOps + kPairOps>();                                                           \
    Decode d;                                                                                                \
    load_decode(t + 1, d);                                                                                   \
    __syncthreads();                                                                                         \
    const uint8_t* stage = lds_a + kAStage * (t % kAStages);                                                 \
    _Pragma("unroll") for (int mt = 0; mt < 4; ++mt)                                                         \
      af[0][mt] = *reinterpret_cast<const bf16x8_t*>(stage + a_frag[0] + 4096 * mt);                         \
    _Pragma("unroll") for (int kk = 0; kk < 3; ++kk)                                                         \
      bp[kk] = *reinterpret_cast<const u32x4_t*>(bx_at(P, 1 - MI, kk));                                      \
    __builtin_amdgcn_sched_barrier(0);                                                                       \
    _Pragma("unroll") for (int mt = 0; mt < 4; ++mt) {                                                       \
      acc_par[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][mt], __builtin_bit_cast(bf16x8_t, bp[3]),   \
                                                            acc_par[mt], 0, 0, 0);                           \
      __builtin_amdgcn_sched_barrier(0);                                                                     \
    }                                                                                                        \
    DecodeTmp dt;                                                                                            \
    Unroll<0, 28>::run([&](auto ic) {                                                                        \
      constexpr int p = decltype(ic)::value;                                                                 \
      /* MFMA order: own chunk 0 (4), then for chunk kk = 0..2 partner kk (4) and own kk+1 (4); partner */   \
      /* chunk 3 runs after the next barrier. */                                                            \
      constexpr int q = p < 4 ? 0 : (p - 4) / 8;        /* chunk of a partner MFMA slot group */             \
      constexpr int r = p < 4 ? p : (p - 4) % 8;                                                             \
      constexpr bool own = p < 4 || r >= 4;                                                                  \
      constexpr int ck = p < 4 ? 0 : (own ? q + 1 : q); /* chunk of this MFMA */                             \
      constexpr int mt = p < 4 ? p : r % 4;                                                                  \
      if constexpr (own)                                                                                     \
        acc_own[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ck & 1][mt],                                \
                          __builtin_bit_cast(bf16x8_t, bo[P][ck]), acc_own[mt], 0, 0, 0);                    \
      else                                                                                                   \
        acc_par[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ck & 1][mt],                                \
                          __builtin_bit_cast(bf16x8_t, bp[ck]), acc_par[mt], 0, 0, 0);                       \
      /* Activation fragments of chunk p/8 + 1, read at the first MFMA of chunk p/8 (8 slots ahead of */   \
      /* their use); the partner's chunk-3 fragment once the deferred MFMAs have read the old one. */         \
      if constexpr (p == 0 || p == 8 || p == 16) {                                                           \
        constexpr int nk = p / 8 + 1;                                                                        \
        _Pragma("unroll") for (int m = 0; m < 4; ++m)                                                        \
          af[nk & 1][m] = *reinterpret_cast<const bf16x8_t*>(stage + a_frag[nk] + 4096 * m);                 \
      }                                                                                                      \
      if constexpr (p == 1) bp[3] = *reinterpret_cast<const u32x4_t*>(bx_at(P, 1 - MI, 3));                  \
      /* Decode piece of the next step's fragments. */                                                       \
      constexpr int dw = p / 7, dj = p % 7;                                                                  \
      decode_piece<dj>(d.words[dw], d.s, d.b, dt, bo[(P) ^ 1][dw]);                                          \
      if constexpr (dj == 6)                                                                                 \
        *reinterpret_cast<u32x4_t*>(bx_at((P) ^ 1, MI, dw)) = bo[(P) ^ 1][dw];                               \
      /* Transfers: activations of step t+2, then (odd steps) the words and parameters of pair (t+3)/2. */   \
      if constexpr (p % 2 == 1 && p / 2 < kAOps) {                                                           \
        constexpr int i = p / 2;                                                                             \
        const int g = s0 + min(t + 2, steps - 1);                                                            \
        dma16(sadd(a.x, 128 * g), a_off[i],                                           \
              a_lds + kAStage * ((t + 2) % kAStages) + 1024 * kAOps * wave + 1024 * i);                     \
      }                                                                                                      \
      if constexpr ((P) == 1 && p == 17) issue_pair((t + 3) >> 1);                                           \
      __builtin_amdgcn_sched_barrier(0);                                                                     \
    });                                                                                                      \
    ++t;                                                                                                     \
  }

  for (int t = 0; t < steps;) {
    AFFON_PAIR_STEP(0)
    AFFON_PAIR_STEP(1)
  }
#undef AFFON_PAIR_STEP
  // The partner MFMAs of the last step's chunk 3.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
    acc_par[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][mt], __builtin_bit_cast(bf16x8_t, bp[3]),
                                                          acc_par[mt], 0, 0, 0);
  wait_vmcnt<0>();  // no transfer in flight at exit

  // Accumulator element v of lane l: row 8*(v/4) + 4*(l/32) + v%4, column l%32 of its 32 x 32 tile.
  // Offsets are 32-bit from the wave's first output row (rows * N * 4 < 2^31).
  const int row0 = m0 + 128 * MI;
  const bool full = row0 + 128 <= a.M;  // no row checks for whole tiles
  float* base = (a.splits == 1 ? a.out : a.partial + split * static_cast<int64_t>(a.M) * a.N) +
                static_cast<int64_t>(row0) * a.N;
  const int col_own = n0 + 64 * ni + 32 * MI + li;
  const int col_par = n0 + 64 * ni + 32 * (1 - MI) + li;
  with_store_kind(a.splits == 1 ? a.epi.kind : kEpiNone, [&](auto kind) {
    constexpr int KIND = decltype(kind)::value;
    auto emit = [&](const f32x16_t (&acc)[4], int col) {
      if (col >= a.N) return;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = 32 * mt + 8 * (v / 4) + 4 * lh + (v % 4);
          if (full || row0 + r < a.M) {
            const uint32_t off = static_cast<uint32_t>(r * a.N + col) * 4u;
            store_as<KIND>(a.epi, reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(base) + off), col,
                           acc[mt][v]);
          }
        }
    };
    emit(acc_own, col_own);
    emit(acc_par, col_par);
  });
}

template <typename PT>
__global__ __launch_bounds__(kThreads, 1) void qgemm_pair_kernel(TileArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kAStages * kAStage];
  __shared__ __attribute__((aligned(16))) uint8_t lds_bx[2 * 2 * 2 * 4 * 1024];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2 * kWaves * kWWave];
  __shared__ __attribute__((aligned(16))) uint8_t lds_p[2 * kWaves * 2 * kPWave];
  const int nb_n = (a.N + kCols - 1) / kCols;
  int tile, split;
  work_unit(nb_n * ((a.M + kRows - 1) / kRows), a.splits, &tile, &split);
  const int m0 = (tile / nb_n) * kRows;
  const int n0 = (tile % nb_n) * kCols;
  const int mi = __builtin_amdgcn_readfirstlane(threadIdx.x >> 7);
  if (mi == 0)
    pair_tile<PT, 0>(a, lds_a, lds_bx, lds_w, lds_p, m0, n0, split);
  else
    pair_tile<PT, 1>(a, lds_a, lds_bx, lds_w, lds_p, m0, n0, split);
}

template <typename PT>
hipError_t launch_pair(const TileArgs& args, hipStream_t stream) {
  const int tiles = ((args.N + kCols - 1) / kCols) * ((args.M + kRows - 1) / kRows);
  hipLaunchKernelGGL((qgemm_pair_kernel<PT>), dim3(tiles * args.splits), dim3(kThreads), 0, stream, args);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || args.splits == 1) return e;
  return launch_reduce(args, stream);
}

}  // namespace

// Shapes the pair kernel takes: 4-bit bf16 activations with unit inner
// strides, K a whole number of step pairs (128), groups of 32, 64 or 128,
// parameter rows of whole dwords, and every byte offset the transfers form
// within 32 bits.
bool pair_supports(const QmmProblem& p) {
  if (p.bits != 4 || p.x_dtype != AFFON_ROCM_BF16) return false;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  if (p.K % 128 != 0 || (p.group != 32 && p.group != 64 && p.group != 128)) return false;
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || (p.xs0 * 2) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || (p.ws0 * 4) % 16 != 0) return false;
  const int64_t pbytes = p.p_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  if (reinterpret_cast<uintptr_t>(p.s) % 4 != 0 || reinterpret_cast<uintptr_t>(p.b) % 4 != 0) return false;
  if ((p.ss0 * pbytes) % 4 != 0 || (p.bs0 * pbytes) % 4 != 0 || (p.K / p.group * pbytes) % 4 != 0) return false;
  const int64_t limit = int64_t(1) << 31;
  if (p.M * p.xs0 * 2 >= limit || p.N * p.ws0 * 4 >= limit) return false;
  if (p.N * p.ss0 * pbytes >= limit || p.N * p.bs0 * pbytes >= limit) return false;
  if (p.M > (int64_t(1) << 30) || p.N > (int64_t(1) << 22)) return false;  // 256 rows * N * 4 < 2^31
  if (((p.N + kCols - 1) / kCols) * ((p.M + kRows - 1) / kRows) > (int64_t(1) << 28)) return false;
  return true;
}

hipError_t pair_launch(const QmmProblem& p, const Launch& l) {
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
  const int tiles = static_cast<int>(((p.N + kCols - 1) / kCols) * ((p.M + kRows - 1) / kRows));
  const int steps = static_cast<int>(p.K / kBK);
  a.splits = 1;
  a.split_steps = steps;
  a.partial = nullptr;
  const int splits = l.can_split() ? choose_splits(tiles, steps) : 1;
  if (splits > 1 && (steps / splits) % 2 == 0) {
    if (auto* ws = static_cast<float*>(l.scratch(static_cast<size_t>(splits) * p.M * p.N * 4))) {
      a.splits = splits;
      a.split_steps = steps / splits;
      a.partial = ws;
    } else if (l.fixed != nullptr) {
      return hipErrorOutOfMemory;  // the fixed scratch buffer cannot hold this plan's partial sums
    }
  }
  return p.p_dtype == AFFON_ROCM_BF16 ? launch_pair<BF16>(a, l.stream) : launch_pair<F32>(a, l.stream);
}

}  // namespace affon
