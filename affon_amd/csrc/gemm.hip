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

#include "device.h"
#include "internal.h"

namespace affon {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;                       // tile rows (activations)
constexpr int kBN = 256;                       // tile columns (weights), 64 per wave
constexpr int kBK = 64;                        // K step
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 4;                     // LDS ring depth (steps)
constexpr int kAStageBytes = kBM * kBK * 2;    // 16 KiB: 128 rows x 128 bytes
constexpr int kAGroupsPerWave = kBM / 8 / kWaves;  // 8-row DMA groups per wave

struct GemmArgs {
  const uint16_t* x;  // bf16 [M, K], row stride xs0 elements
  int64_t xs0;
  const uint32_t* w;  // packed [N, K/P], row stride ws0 words
  int64_t ws0;
  const uint8_t* s;
  int64_t ss0;
  const uint8_t* b;
  int64_t bs0;
  float* out;  // [M, N]
  int M, N, K;
  int group_shift;  // log2(group / 32): groups of 32, 64, 128, ...
};

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{static_cast<__bf16>(a), static_cast<__bf16>(b)});
}

__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Decodes 32 consecutive weights (words[] holds BITS words) with w = s*q + b
// into four bf16x8 fragments (weights 8f .. 8f+7 in fragment f).
template <int BITS>
__device__ __forceinline__ void decode32(const uint32_t* words, float s, float b, bf16x8_t* frag) {
  uint32_t pairs[16];
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = opaque(words[i]);
      float w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = fmaf(static_cast<float>((v >> (8 * j)) & 0xffu), s, b);
      pairs[2 * i] = pack_bf16(w[0], w[1]);
      pairs[2 * i + 1] = pack_bf16(w[2], w[3]);
    }
  } else {
    // FP8 conversion of bytes holding codes < 16: exactly n * 2^-9 (the
    // caller passes s already multiplied by 2^9).
    constexpr int P = 32 / BITS;
    constexpr int T = BITS == 4 ? 2 : 4;
    constexpr uint32_t kMask = BITS == 4 ? 0x0f0f0f0fu : 0x03030303u;
#pragma unroll
    for (int i = 0; i < BITS; ++i) {  // BITS words per 32 values
      const uint32_t word = words[i];
      float w[P];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint32_t m = (word >> (BITS * t)) & kMask;
        const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(m, false);  // bytes 0, 1
        const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(m, true);   // bytes 2, 3
        const float q[4] = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = BITS == 4 ? 2 * j + t : 4 * j + t;  // code position of byte j of mask t
          w[k] = fmaf(q[j], s, b);
        }
      }
#pragma unroll
      for (int j = 0; j < P / 2; ++j) pairs[i * (P / 2) + j] = pack_bf16(w[2 * j], w[2 * j + 1]);
    }
  }
#pragma unroll
  for (int f = 0; f < 4; ++f)
    frag[f] = __builtin_bit_cast(bf16x8_t, make_uint4(pairs[4 * f], pairs[4 * f + 1], pairs[4 * f + 2], pairs[4 * f + 3]));
}

// Waits until at most N vector-memory operations of this wave are in flight.
// Written as asm with a memory clobber so that no memory access moves across
// it (the compiler does not see the direct-to-LDS loads it stands guard for).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// size bytes per lane (4 or 16) from global memory straight into LDS: lane
// L's bytes land at lds_addr + size * L (lds_addr wave-uniform). Issued as
// asm: the compiler would otherwise drain the load counter before every LDS
// read it cannot prove disjoint from the transfer; here the caller orders them
// with wait_vmcnt and a barrier.
template <int SIZE>
__device__ __forceinline__ void load_lds(const void* src, uint32_t lds_addr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  if constexpr (SIZE == 16)
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds_addr) : "memory", "m0");
#pragma clang diagnostic pop
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Per-wave LDS traffic of one K step.
template <int BITS, typename PT>
struct StepShape {
  static constexpr int kWColBytes = 8 * BITS;             // packed bytes of one column per step
  static constexpr int kWBytes = 64 * kWColBytes;         // this wave's 64 columns
  static constexpr int kWLoads = kWBytes / 1024;          // 16-byte DMA instructions
  static constexpr int kPLoads = PT::bytes == 2 ? 2 : 4;  // 4-byte DMA instructions (scales, biases)
  static constexpr int kPBytes = kPLoads * 256;
  static constexpr int kALoads = kAGroupsPerWave;         // 16-byte DMA instructions (activations)
  static constexpr int kOps = kWLoads + kPLoads + kALoads;
  static_assert(kWBytes % 1024 == 0, "whole DMA instructions");
};

// Workgroup tile 128 x 256, K step 64, four waves side by side along N (each
// all 128 rows x 64 columns = 4 x 2 tiles of 32x32 accumulators). Blocks are
// ordered so that the blocks one XCD runs share one row panel of activations
// (one L2 per XCD).
//
// K order inside a step: MFMA kk of lane half h covers the 8 k values of
// chunk c = 4h + kk (k = 8c .. 8c+7). Both operands use this order, so each
// lane's B operand for a step is one contiguous run of 32 weights.
//
// All global reads are direct-to-LDS transfers into a 4-stage ring, issued
// three steps ahead: per step and wave, four 1 KiB activation transfers
// (8 rows x 128 bytes each; 16-byte chunk c of row r stored at slot c ^ (r%8)
// so the A-fragment reads are bank-conflict free), the packed words of the
// wave's own 64 columns and their scales and biases. A wave decodes B
// fragments only from its own transfers (no barrier needed for them); the
// barrier orders the shared activation tile. Step t+1 is decoded while step
// t's MFMAs run.
template <int BITS, typename PT>
__global__ __launch_bounds__(kThreads, 1) void qgemm_kernel(GemmArgs a) {
  using S = StepShape<BITS, PT>;
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kStages][kAStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[kStages][kWaves][S::kWBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_p[kStages][kWaves][S::kPBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31;
  const int lh = lane >> 5;

  // Tile of this block: consecutive blocks go to consecutive XCDs, so the
  // block index is remapped to give each XCD a contiguous run of tiles.
  const int nb_n = (a.N + kBN - 1) / kBN;
  const int total = nb_n * ((a.M + kBM - 1) / kBM);
  int tile = blockIdx.x;
  if ((total & 7) == 0) tile = (tile & 7) * (total >> 3) + (tile >> 3);
  const int m0 = (tile / nb_n) * kBM;
  const int n0 = (tile % nb_n) * kBN + 64 * wave;  // this wave's first column
  const int steps = a.K / kBK;
  const int last = steps - 1;

  // Activation transfers: this wave fills 8-row groups kAGroupsPerWave*wave + i.
  // Lane L loads row 8g + L/8, chunk (L%8) ^ (L/8) (rows past M repeat row
  // M-1 and feed only unstored outputs).
  const uint16_t* a_src[S::kALoads];
#pragma unroll
  for (int i = 0; i < S::kALoads; ++i) {
    const int row = min(m0 + 8 * (kAGroupsPerWave * wave + i) + (lane >> 3), a.M - 1);
    a_src[i] = a.x + static_cast<int64_t>(row) * a.xs0 + 8 * ((lane & 7) ^ (lane >> 3));
  }
  // Packed-word transfers: 16-byte chunk q = 1024j/16 + L of the wave's slice
  // is column q / (BITS/2), part q % (BITS/2); the slice is stored in column
  // order, kWColBytes per column.
  const uint8_t* w_src[S::kWLoads];
#pragma unroll
  for (int j = 0; j < S::kWLoads; ++j) {
    const int q = 64 * j + lane;
    const int col = min(n0 + q / (BITS / 2), a.N - 1);  // columns past N feed unstored outputs
    w_src[j] = reinterpret_cast<const uint8_t*>(a.w + static_cast<int64_t>(col) * a.ws0) + 16 * (q % (BITS / 2));
  }
  // Scale and bias transfers: lane L carries column n0 + L. bf16 parameters
  // travel as the 4-byte pair holding the step's group(s); f32 parameters as
  // one 4-byte value per lane half (the groups of k 0..31 and 32..63).
  const int pcol = min(n0 + lane, a.N - 1);
  const uint8_t* s_row = a.s + static_cast<int64_t>(pcol) * a.ss0 * PT::bytes;
  const uint8_t* b_row = a.b + static_cast<int64_t>(pcol) * a.bs0 * PT::bytes;

  auto issue = [&](int step, int stage) {
    const uint32_t wdst = lds_address(lds_w[stage][wave]);
#pragma unroll
    for (int j = 0; j < S::kWLoads; ++j) load_lds<16>(w_src[j] + step * S::kWColBytes, wdst + 1024 * j);
    const uint32_t pdst = lds_address(lds_p[stage][wave]);
    const int g0 = (step * kBK) >> (5 + a.group_shift);
    if constexpr (PT::bytes == 2) {
      load_lds<4>(s_row + 4 * (g0 >> 1), pdst);
      load_lds<4>(b_row + 4 * (g0 >> 1), pdst + 256);
    } else {
      const int g1 = (step * kBK + 32) >> (5 + a.group_shift);
      load_lds<4>(s_row + 4 * g0, pdst);
      load_lds<4>(s_row + 4 * g1, pdst + 256);
      load_lds<4>(b_row + 4 * g0, pdst + 512);
      load_lds<4>(b_row + 4 * g1, pdst + 768);
    }
    const uint32_t adst = lds_address(lds_a[stage]) + 1024 * kAGroupsPerWave * wave;
#pragma unroll
    for (int i = 0; i < S::kALoads; ++i) load_lds<16>(a_src[i] + step * kBK, adst + 1024 * i);
  };

  // B fragments of one step for this lane: columns 32*nt + li of the wave's
  // slice, k 32*lh .. 32*lh+31.
  const float code_scale = BITS == 8 ? 1.0f : 512.0f;
  auto decode_step = [&](int step, int stage, bf16x8_t (*frag)[4]) {
    const int g = (step * kBK + 32 * lh) >> (5 + a.group_shift);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int c = 32 * nt + li;
      const uint8_t* wp = lds_w[stage][wave] + c * S::kWColBytes + lh * (S::kWColBytes / 2);
      uint32_t words[BITS];
      if constexpr (BITS == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(wp);
        words[0] = v.x;
        words[1] = v.y;
      } else {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
          const u32x4_t v = reinterpret_cast<const u32x4_t*>(wp)[i];
          words[4 * i] = v.x;
          words[4 * i + 1] = v.y;
          words[4 * i + 2] = v.z;
          words[4 * i + 3] = v.w;
        }
      }
      const uint32_t* pp = reinterpret_cast<const uint32_t*>(lds_p[stage][wave]);
      float sv, bv;
      if constexpr (PT::bytes == 2) {
        const int sh = 16 * (1 - (g & 1));  // low half holds the even group
        sv = __uint_as_float((pp[c] << sh) & 0xffff0000u);
        bv = __uint_as_float((pp[64 + c] << sh) & 0xffff0000u);
      } else {
        sv = __uint_as_float(pp[64 * lh + c]);
        bv = __uint_as_float(pp[128 + 64 * lh + c]);
      }
      decode32<BITS>(words, sv * code_scale, bv, frag[nt]);
    }
  };

  // A fragment (mt, kk) of this lane: row 32*mt + li, chunk 4*lh + kk.
  auto read_a = [&](int stage, int mt, int kk) -> bf16x8_t {
    const int row = 32 * mt + li;
    const int slot = (4 * lh + kk) ^ (row & 7);
    return *reinterpret_cast<const bf16x8_t*>(&lds_a[stage][(row >> 3) * 1024 + (8 * (row & 7) + slot) * 16]);
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][nt][v] = 0.0f;
  bf16x8_t bf[2][2][4];

  // Every iteration issues S::kOps transfers per wave, packed words and
  // parameters first, activations last. Waits (this wave's own transfers):
  //   step t's activations (issued three iterations before t's):   vmcnt(2*kOps)
  //   step t+1's words and parameters (first of iteration t-2):   vmcnt(2*kOps + kALoads)
  issue(0, 0);
  issue(min(1, last), 1);
  issue(min(2, last), 2);
  wait_vmcnt<2 * S::kOps + S::kALoads>();
  decode_step(0, 0, bf[0]);

#define AFFON_QGEMM_STEP(J)                                                                                   \
  {                                                                                                           \
    constexpr int RB = (J)&1;                                                                                 \
    wait_vmcnt<2 * S::kOps>();                                                                                \
    __syncthreads();                                                                                          \
    issue(min(t + 3, last), ((J) + 3) & 3);                                                                   \
    _Pragma("unroll") for (int kk = 0; kk < 4; ++kk) {                                                        \
      bf16x8_t af[4];                                                                                         \
      _Pragma("unroll") for (int mt = 0; mt < 4; ++mt) af[mt] = read_a(J, mt, kk);                            \
      _Pragma("unroll") for (int mt = 0; mt < 4; ++mt) _Pragma("unroll") for (int nt = 0; nt < 2; ++nt)       \
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bf[RB][nt][kk], acc[mt][nt], 0, 0, 0); \
      if (kk == 1) {                                                                                          \
        wait_vmcnt<2 * S::kOps + S::kALoads>();                                                               \
        decode_step(min(t + 1, last), ((J) + 1) & 3, bf[RB ^ 1]);                                             \
      }                                                                                                       \
    }                                                                                                         \
    ++t;                                                                                                      \
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
  // and column l%32 of its 32x32 tile.
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int col = n0 + 32 * nt + li;
    if (col >= a.N) continue;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + 32 * mt + 8 * (v / 4) + 4 * lh + (v % 4);
        if (row < a.M) a.out[static_cast<int64_t>(row) * a.N + col] = acc[mt][nt][v];
      }
  }
}

template <int BITS, typename PT>
hipError_t launch_typed(const GemmArgs& args, hipStream_t stream) {
  const int tiles = ((args.N + kBN - 1) / kBN) * ((args.M + kBM - 1) / kBM);
  hipLaunchKernelGGL((qgemm_kernel<BITS, PT>), dim3(tiles), dim3(kThreads), 0, stream, args);
  return hipGetLastError();
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
  // Parameters travel in 4-byte units: bf16 pairs must not straddle a row end.
  if (reinterpret_cast<uintptr_t>(p.s) % 4 != 0 || reinterpret_cast<uintptr_t>(p.b) % 4 != 0) return false;
  if (p.p_dtype == AFFON_ROCM_BF16 && (p.ss0 % 2 != 0 || p.bs0 % 2 != 0 || (p.K / p.group) % 2 != 0)) return false;
  if (p.M > (int64_t(1) << 30) || p.N > (int64_t(1) << 30) || p.K > (int64_t(1) << 30)) return false;
  if (((p.N + kBN - 1) / kBN) * ((p.M + kBM - 1) / kBM) > (int64_t(1) << 31) - 1) return false;
  return true;
}

hipError_t mfma_launch(const QmmProblem& p, hipStream_t stream) {
  GemmArgs a;
  a.x = reinterpret_cast<const uint16_t*>(p.x);
  a.xs0 = p.xs0;
  a.w = p.w;
  a.ws0 = p.ws0;
  a.s = p.s;
  a.ss0 = p.ss0;
  a.b = p.b;
  a.bs0 = p.bs0;
  a.out = p.out;
  a.M = static_cast<int>(p.M);
  a.N = static_cast<int>(p.N);
  a.K = static_cast<int>(p.K);
  a.group_shift = 0;
  while ((int64_t(32) << a.group_shift) < p.group) ++a.group_shift;
  const bool bf16p = p.p_dtype == AFFON_ROCM_BF16;
  switch (p.bits) {
    case 2: return bf16p ? launch_typed<2, BF16>(a, stream) : launch_typed<2, F32>(a, stream);
    case 4: return bf16p ? launch_typed<4, BF16>(a, stream) : launch_typed<4, F32>(a, stream);
    default: return bf16p ? launch_typed<8, BF16>(a, stream) : launch_typed<8, F32>(a, stream);
  }
}

bool gemv_mfma_supports(const QmmProblem&) { return false; }
hipError_t gemv_mfma_launch(const QmmProblem&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace affon
