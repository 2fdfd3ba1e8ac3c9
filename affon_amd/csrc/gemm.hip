// rocm_quantized_matmul.mfma — prefill GEMM for bf16 activations (M >= 64).
//
// Counterpart of the reference's matrix paths (metal matrix32 / matrix32_packed,
// docs/core/quantized-inference.md:138-139,151-170): packed weights are
// decoded in registers straight into matrix-core operands and multiplied with
// f32 accumulation; no floating weight matrix exists in memory.
// Unlike the reference (which keeps decoded weights in f32), decoded weights
// are rounded to bf16 to feed v_mfma_f32_32x32x16_bf16, so this candidate is
// classified "approximate".
//
// Work mapping (gfx950, wave64): see qgemm_kernel. In short, a 128 x 256
// workgroup tile, four waves of 128 x 64, every operand brought into a 4-stage
// LDS ring by direct global-to-LDS transfers, weights decoded per wave into
// MFMA B fragments in registers (codes -> f32 via FP8 conversion for 2/4-bit
// or v_cvt_f32_ubyte for 8-bit -> s*q + b -> bf16).

#include "lds_pipeline.h"

namespace affon {
namespace {

using namespace pipeline;

constexpr int kBM = 128;                       // tile rows (activations)
constexpr int kBN = 256;                       // tile columns (weights), 64 per wave
constexpr int kAStageBytes = kBM * kBK * 2;    // 16 KiB: 128 rows x 128 bytes
constexpr int kAGroupsPerWave = kBM / 8 / kWaves;  // 8-row DMA groups per wave

// Inputs of one step's decode for one lane: BITS packed words (32 weights)
// and the raw parameter bits of each of the lane's two columns.
template <int BITS>
struct DecodeIn {
  uint32_t words[2][BITS];
  uint32_t s_raw[2], b_raw[2];
};

// Intermediate values of the decode while its pieces are spread over a
// step's MFMAs.
struct DecodeTmp {
  float s[2], b[2];
  f32x2_t lo[4], hi[4];
};

// Piece p (0..31) of a step's decode: the 64 weights of a lane (2 columns x
// 32 k) split into 32 pieces of 5-6 VALU instructions, one per MFMA. Words
// are decoded in order; a word takes 16/BITS pieces: for 2/4-bit first one
// piece per code mask (FP8 conversion of the masked bytes: codes n < 16 read
// as n * 2^-9, the scale carries the 2^9), then pieces that apply s*q + b and
// pack bf16 pairs; for 8-bit two pieces of two bytes each. Pair q of column
// nt (weights 2q, 2q+1 of the lane's run) goes to out[nt][q/4][q%4].
template <int BITS, typename PT, int p>
__device__ __forceinline__ void decode_piece(const DecodeIn<BITS>& in, DecodeTmp& d, u32x4_t (&out)[2][4],
                                             float code_scale) {
  constexpr int kPieces = 16 / BITS;  // pieces per word
  constexpr int wi = p / kPieces, st = p % kPieces;
  constexpr int nt = wi / BITS, w = wi % BITS;
  if constexpr (st == 0 && w == 0) {
    d.s[nt] = widen_param<PT>(in.s_raw[nt]) * code_scale;
    d.b[nt] = widen_param<PT>(in.b_raw[nt]);
  }
  const float s = d.s[nt], b = d.b[nt];
  const uint32_t word = in.words[nt][w];
  if constexpr (BITS == 4) {  // code 2j + t sits in byte j of mask t
    if constexpr (st < 2) {
      const uint32_t m = (word >> (4 * st)) & 0x0f0f0f0fu;
      d.lo[st] = __builtin_amdgcn_cvt_pk_f32_fp8(m, false);
      d.hi[st] = __builtin_amdgcn_cvt_pk_f32_fp8(m, true);
    } else {
      const f32x2_t* v = st == 2 ? d.lo : d.hi;  // codes 0..3 or 4..7
      constexpr int q = 4 * w + 2 * (st - 2);
      out[nt][q / 4][q % 4] = pack_bf16(fmaf(v[0].x, s, b), fmaf(v[1].x, s, b));
      out[nt][(q + 1) / 4][(q + 1) % 4] = pack_bf16(fmaf(v[0].y, s, b), fmaf(v[1].y, s, b));
    }
  } else if constexpr (BITS == 2) {  // code 4j + t sits in byte j of mask t
    if constexpr (st < 4) {
      const uint32_t m = (word >> (2 * st)) & 0x03030303u;
      d.lo[st] = __builtin_amdgcn_cvt_pk_f32_fp8(m, false);
      d.hi[st] = __builtin_amdgcn_cvt_pk_f32_fp8(m, true);
    } else {
      constexpr int j = st - 4;  // codes 4j .. 4j+3
      float v[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] = j == 0 ? d.lo[t].x : j == 1 ? d.lo[t].y : j == 2 ? d.hi[t].x : d.hi[t].y;
      constexpr int q = 8 * w + 2 * j;
      out[nt][q / 4][q % 4] = pack_bf16(fmaf(v[0], s, b), fmaf(v[1], s, b));
      out[nt][(q + 1) / 4][(q + 1) % 4] = pack_bf16(fmaf(v[2], s, b), fmaf(v[3], s, b));
    }
  } else {  // bytes 2*st and 2*st+1 of the word
    const uint32_t v = opaque(word);
    const float q0 = static_cast<float>((v >> (16 * st)) & 0xffu);
    const float q1 = static_cast<float>((v >> (16 * st + 8)) & 0xffu);
    constexpr int q = 2 * w + st;
    out[nt][q / 4][q % 4] = pack_bf16(fmaf(q0, s, b), fmaf(q1, s, b));
  }
}

// Workgroup tile 128 x 256, K step 64, four waves side by side along N (each
// all 128 rows x 64 columns = 4 x 2 tiles of 32x32 accumulators). Blocks are
// ordered so that the blocks one XCD runs share one row panel of activations
// (one L2 per XCD).
//
// K order inside a step: MFMA kk of lane half h covers the 8 k values of
// chunk c = 4h + kk (k = 8c .. 8c+7). Both operands use this order, so each
// lane's B operand for a step is one contiguous run of 32 weights.
//
// All global reads are direct-to-LDS transfers: activations into a 4-stage
// ring three steps ahead (four 1 KiB transfers per wave and step, 8 rows x
// 128 bytes each; 16-byte chunk c of row r stored at slot
// c ^ (r%8) ^ ((r/8)%2), so the A-fragment reads -- consecutive rows, one
// chunk -- are bank-conflict free for 8- and 16-lane LDS phases); packed words, scales and biases
// of the wave's own 64 columns per Plan. A wave decodes B fragments only from
// its own transfers (no barrier needed for them); the barrier orders the
// shared activation tile. Step t+1 is decoded while step t's MFMAs run.
template <int BITS, typename PT>
__global__ __launch_bounds__(kThreads, 1) void qgemm_kernel(TileArgs a) {
  using P = Plan<BITS, PT, kAGroupsPerWave>;
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kStages][kAStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[P::kWBufs][kWaves][P::kWBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_p[2][kWaves][P::kPBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31;
  const int lh = lane >> 5;

  const int nb_n = (a.N + kBN - 1) / kBN;
  int tile, split;
  work_unit(nb_n * ((a.M + kBM - 1) / kBM), a.splits, &tile, &split);
  const int m0 = (tile / nb_n) * kBM;
  const int n0 = (tile % nb_n) * kBN + 64 * wave;  // this wave's first column
  // Steps below are local to the K range; s0 is its first global step
  // (a multiple of 4, so local and global steps agree mod 4).
  const int steps = a.split_steps;
  const int s0 = split * steps;
  const int last = steps - 1;

  // Activation transfers: this wave fills 8-row groups g = kAGroupsPerWave*wave + i.
  // Lane L writes slot L%8 of local row 8g + L/8, so it loads chunk
  // (L%8) ^ (L/8) ^ (g%2) (rows past M repeat row M-1 and feed only unstored
  // outputs).
  static_assert(kAGroupsPerWave % 2 == 0, "group parity is i % 2");
  const uint16_t* a_src[P::kALoads];
#pragma unroll
  for (int i = 0; i < P::kALoads; ++i) {
    const int row = min(m0 + 8 * (kAGroupsPerWave * wave + i) + (lane >> 3), a.M - 1);
    a_src[i] = a.x + static_cast<int64_t>(row) * a.xs0 + 8 * ((lane & 7) ^ (lane >> 3) ^ (i & 1));
  }
  WeightStream<BITS, PT, kAGroupsPerWave> ws;
  ws.init(a, n0, s0, lane, lds_w[0][wave], kWaves * P::kWBytes, lds_p[0][wave], kWaves * P::kPBytes);
  auto issue_p = [&](int step, int i) { ws.issue_p(step, i); };
  auto issue_w = [&](int step, int j) { ws.issue_w(step, j); };
  auto issue_a = [&](int step, int i) {
    load_lds<16>(a_src[i] + (s0 + step) * kBK, lds_address(lds_a[step & 3]) + 1024 * (kAGroupsPerWave * wave + i));
  };
  // All transfers of the iteration with index j, in the order the waits count them.
  auto issue_all = [&](int j, int pstep, int wstep, int astep) {
    if (j == 0)
      for (int i = 0; i < P::kPLoads; ++i) issue_p(pstep, i);
    if (P::kStepsPerW == 1 || j == 0)
      for (int i = 0; i < P::kWLoads; ++i) issue_w(wstep, i);
    for (int i = 0; i < P::kALoads; ++i) issue_a(astep, i);
  };

  // Decode inputs of one step for this lane: local columns 32*nt + li, k
  // 32*lh .. 32*lh+31 of the step.
  const float code_scale = BITS == 8 ? 1.0f : 512.0f;
  auto load_decode = [&](int step, DecodeIn<BITS>& in) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int c = 32 * nt + li;
      if constexpr (BITS == 2) {  // 8 bytes: half of the step's 16-byte part
        const uint2 v = *reinterpret_cast<const uint2*>(ws.w_part(step, c, 0) + 8 * lh);
        in.words[nt][0] = v.x;
        in.words[nt][1] = v.y;
      } else {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {  // 4-bit: part lh; 8-bit: parts 2*lh, 2*lh + 1
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ws.w_part(step, c, BITS == 4 ? lh : 2 * lh + i));
          in.words[nt][4 * i] = v.x;
          in.words[nt][4 * i + 1] = v.y;
          in.words[nt][4 * i + 2] = v.z;
          in.words[nt][4 * i + 3] = v.w;
        }
      }
      ws.params(step, c, 32 * lh, &in.s_raw[nt], &in.b_raw[nt]);
    }
  };

  // A fragment (mt, kk) of this lane: row 32*mt + li, chunk 4*lh + kk.
  auto read_a = [&](int stage, int mt, int kk) -> bf16x8_t {
    const int row = 32 * mt + li;
    const int slot = (4 * lh + kk) ^ (row & 7) ^ ((row >> 3) & 1);
    return *reinterpret_cast<const bf16x8_t*>(&lds_a[stage][(row >> 3) * 1024 + (8 * (row & 7) + slot) * 16]);
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][nt][v] = 0.0f;
  u32x4_t bf[2][2][4];  // B fragments (bf16 pairs) of two steps: [step parity][nt][kk]
  DecodeTmp dtmp;

  // Iteration t (j = t % 4) issues, in this order: at j == 0 the parameter
  // windows and (2/4-bit) the packed words of steps t+4 .. t+7; (8-bit) the
  // packed words of step t+4; the activations of step t+3. The transfers
  // before iteration 0 are issued as if by iterations -4 .. -1 (the
  // activations of "step -1" repeat step 0), so every wait below counts the
  // same transfers in the prologue as in the loop.
#pragma unroll
  for (int r = 0; r < 4; ++r) issue_all(r, 0, min(r, last), min(max(r - 1, 0), last));
  wait_vmcnt<P::ops_after(0, 4, 1)>();  // words (issued after the parameters) of step 0
  {
    DecodeIn<BITS> din;
    load_decode(0, din);
    Unroll<0, 32>::run([&](auto ic) { decode_piece<BITS, PT, decltype(ic)::value>(din, dtmp, bf[0], code_scale); });
  }

  // One K step, hand-ordered: decode inputs of step t+1 and the activation
  // fragments of chunks 0 and 1 are read first; then each of the 32 MFMAs is
  // followed by one decode piece and, spread evenly, the iteration's transfer
  // instructions (the scheduling barriers keep this order, so the vector ALU
  // and the memory pipeline work while the matrix core does); chunk kk+1's
  // fragments are read when chunk kk starts.
#define AFFON_QGEMM_STEP(J)                                                                                     \
  {                                                                                                             \
    constexpr int RB = (J)&1;                                                                                   \
    wait_vmcnt<P::wait(J)>();                                                                                   \
    __syncthreads();                                                                                            \
    DecodeIn<BITS> din;                                                                                         \
    load_decode(min(t + 1, last), din);                                                                         \
    bf16x8_t af[2][4];                                                                                          \
    _Pragma("unroll") for (int mt = 0; mt < 4; ++mt) af[0][mt] = read_a(J, mt, 0);                              \
    _Pragma("unroll") for (int mt = 0; mt < 4; ++mt) af[1][mt] = read_a(J, mt, 1);                              \
    const int pstep = min(t + 4, last & ~3);                                                                    \
    const int wstep = min(t + 4, P::kStepsPerW == 1 ? last : (last & ~3));                                      \
    const int astep = min(t + 3, last);                                                                         \
    Unroll<0, 32>::run([&](auto ic) {                                                                           \
      constexpr int p = decltype(ic)::value;                                                                    \
      constexpr int kk = p / 8, mt = (p % 8) / 2, nt = p % 2;                                                   \
      if constexpr (p % 8 == 0 && kk >= 1 && kk < 3) {                                                          \
        _Pragma("unroll") for (int m = 0; m < 4; ++m) af[(kk + 1) & 1][m] = read_a(J, m, kk + 1);              \
      }                                                                                                         \
      acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk & 1][mt], __builtin_bit_cast(bf16x8_t, bf[RB][nt][kk]), \
                                                            acc[mt][nt], 0, 0, 0);                              \
      decode_piece<BITS, PT, p>(din, dtmp, bf[RB ^ 1], code_scale);                                            \
      constexpr int nP = P::group_ops(J, 0), nW = P::group_ops(J, 1), nX = nP + nW + P::group_ops(J, 2);        \
      Unroll<0, nX>::run([&](auto kc) {                                                                         \
        constexpr int k = decltype(kc)::value;                                                                  \
        if constexpr (k * 32 / nX == p) {                                                                       \
          if constexpr (k < nP) issue_p(pstep, k);                                                              \
          else if constexpr (k < nP + nW) issue_w(wstep, k - nP);                                               \
          else issue_a(astep, k - nP - nW);                                                                     \
        }                                                                                                       \
      });                                                                                                       \
      __builtin_amdgcn_sched_barrier(0);                                                                        \
    });                                                                                                         \
    ++t;                                                                                                        \
  }

  for (int t = 0; t < steps;) {
    AFFON_QGEMM_STEP(0)
    AFFON_QGEMM_STEP(1)
    AFFON_QGEMM_STEP(2)
    AFFON_QGEMM_STEP(3)
  }
#undef AFFON_QGEMM_STEP
  // Leave no transfer in flight at exit (the last iterations re-issue the
  // final step's data).
  wait_vmcnt<0>();

  // Accumulator (mt, nt) element v of lane l is row 8*(v/4) + 4*(l/32) + v%4
  // and column l%32 of its 32x32 tile. Offsets are 32-bit from the tile's
  // first output row (128 rows * N * 4 < 2^31), and the epilogue kind is
  // branched on once.
  const bool full = m0 + kBM <= a.M;  // no row checks for whole tiles
  float* base = (a.splits == 1 ? a.out : a.partial + split * static_cast<int64_t>(a.M) * a.N) +
                static_cast<int64_t>(m0) * a.N;
  with_store_kind(a.splits == 1 ? a.epi.kind : kEpiNone, [&](auto kind) {
    constexpr int KIND = decltype(kind)::value;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = n0 + 32 * nt + li;
      if (col < a.N) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int r = 32 * mt + 8 * (v / 4) + 4 * lh + (v % 4);
            if (full || m0 + r < a.M) {
              const uint32_t off = static_cast<uint32_t>(r * a.N + col) * 4u;
              store_as<KIND>(a.epi, reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(base) + off), col,
                             acc[mt][nt][v]);
            }
          }
      }
    }
  });
}

template <int BITS, typename PT>
hipError_t launch_typed(const TileArgs& args, hipStream_t stream) {
  const int tiles = ((args.N + kBN - 1) / kBN) * ((args.M + kBM - 1) / kBM);
  hipLaunchKernelGGL((qgemm_kernel<BITS, PT>), dim3(tiles * args.splits), dim3(kThreads), 0, stream, args);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || args.splits == 1) return e;
  return launch_reduce(args, stream);
}

}  // namespace

bool mfma_supports(const QmmProblem& p) {
  if (p.x_dtype != AFFON_ROCM_BF16) return false;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  if (p.K % (4 * kBK) != 0 || p.group % 32 != 0) return false;  // main loop unrolled by four K steps
  const int64_t gq = p.group / 32;
  if ((gq & (gq - 1)) != 0) return false;  // group index by shift
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || (p.xs0 * 2) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || p.ws0 % 4 != 0) return false;
  // Parameters travel in dwords (rows of whole dwords, dword-aligned) and a
  // 16-byte window must hold every group of four K steps (f32: groups of 64
  // or more).
  const int64_t pbytes = p.p_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  if (reinterpret_cast<uintptr_t>(p.s) % 4 != 0 || reinterpret_cast<uintptr_t>(p.b) % 4 != 0) return false;
  if ((p.ss0 * pbytes) % 4 != 0 || (p.bs0 * pbytes) % 4 != 0 || (p.K / p.group * pbytes) % 4 != 0) return false;
  if (4 * kBK / p.group > 16 / pbytes) return false;
  // 128 rows * N * 4 bytes of output offsets fit in 31 bits.
  if (p.M > (int64_t(1) << 30) || p.N > (int64_t(1) << 22) || p.K > (int64_t(1) << 30)) return false;
  if (((p.N + kBN - 1) / kBN) * ((p.M + kBM - 1) / kBM) > (int64_t(1) << 31) - 1) return false;
  return true;
}

hipError_t mfma_launch(const QmmProblem& p, const Launch& l) {
  // Above 128 rows (at 128 this kernel's 128-row tile wins: 38.1 against
  // 47.0 us for 128 x 14336 x 4096), 4-bit weights with bf16 parameters and
  // groups of 64 or 128 run the 8-wave GEMM of gemm_re.hip in its
  // rounded-weight form where its K ranges are long enough, groups of 32 the
  // 8-wave GEMM of gemm_re32.hip in its rounded-weight form; the pair kernel
  // takes the other 4-bit shapes.
  if (p.M > 128 && re_gemm_supports(p)) {
    hipError_t e = hipSuccess;
    if (re_gemm_launch(p, l, &e, true)) return e;
  }
  if (p.M > 128 && re32_supports(p)) return re32_launch(p, l, true);
  if (p.M > 128 && pair_supports(p)) return pair_launch(p, l);
  hipStream_t stream = l.stream;
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
  const int tiles = static_cast<int>(((p.N + kBN - 1) / kBN) * ((p.M + kBM - 1) / kBM));
  const int steps = static_cast<int>(p.K / kBK);
  a.splits = 1;
  a.split_steps = steps;
  a.partial = nullptr;
  const int splits = l.can_split() ? choose_splits(tiles, steps) : 1;
  if (splits > 1) {
    if (auto* ws = static_cast<float*>(l.scratch(static_cast<size_t>(splits) * p.M * p.N * 4))) {
      a.splits = splits;
      a.split_steps = steps / splits;
      a.partial = ws;
    } else if (l.fixed != nullptr) {
      return hipErrorOutOfMemory;  // the fixed scratch buffer cannot hold this plan's partial sums
    }
  }
  const bool bf16p = p.p_dtype == AFFON_ROCM_BF16;
  switch (p.bits) {
    case 2: return bf16p ? launch_typed<2, BF16>(a, stream) : launch_typed<2, F32>(a, stream);
    case 4: return bf16p ? launch_typed<4, BF16>(a, stream) : launch_typed<4, F32>(a, stream);
    default: return bf16p ? launch_typed<8, BF16>(a, stream) : launch_typed<8, F32>(a, stream);
  }
}


}  // namespace affon
