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

#include <mutex>
#include <type_traits>

#include "device.h"
#include "internal.h"

namespace affon {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

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
  // Split of K over workgroups: splits ranges of split_steps K steps each.
  // With splits > 1 each range writes its sums to partial [splits, M, N] f32
  // and reduce_partials_kernel forms the output.
  int splits, split_steps;
  float* partial;
};

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{static_cast<__bf16>(a), static_cast<__bf16>(b)});
}

__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
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

// Compile-time unrolled loop: f(std::integral_constant<int, I>) for I in [I0, N).
template <int I, int N>
struct Unroll {
  template <class F>
  __device__ __forceinline__ static void run(F&& f) {
    f(std::integral_constant<int, I>{});
    Unroll<I + 1, N>::run(f);
  }
};
template <int N>
struct Unroll<N, N> {
  template <class F>
  __device__ __forceinline__ static void run(F&&) {}
};

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

template <typename PT>
__device__ __forceinline__ float widen_param(uint32_t raw) {
  return PT::bytes == 2 ? __uint_as_float(raw << 16) : __uint_as_float(raw);
}

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

// Transfer plan of one wave (64 weight columns) for a weight format.
//
// Packed words reach LDS in runs of kColBytes per column: four K steps at a
// time for 2/4-bit (64 / 128 bytes, 4 / 8 lanes per column), one step at a
// time for 8-bit (64 bytes) -- so each transfer instruction covers whole
// half or full 128-byte lines. Inside a column run the 16-byte slots are
// XOR-swizzled with the column index so that the decode's fragment reads
// (lanes = consecutive columns) are bank-conflict free whether the LDS serves
// 8 lanes x 16 bytes (128 bytes) or 16 lanes x 16 bytes (256 bytes) per cycle. Scales and biases come as one 16-byte window per
// column every four steps (four lanes per column, one dword each; bf16: 8
// groups, f32: 4 groups), starting at the dword that holds the first group of
// those 256 k values, which covers all of their groups for the group sizes
// the kernel accepts; dwords past the row end repeat the row's last dword.
template <int BITS, typename PT>
struct Plan {
  static constexpr int kStepsPerW = BITS == 8 ? 1 : 4;           // steps per packed-word transfer
  static constexpr int kColBytes = 8 * BITS * kStepsPerW;         // bytes per column per transfer
  static constexpr int kSlots = kColBytes / 16;                   // 16-byte slots per column run
  static constexpr int kWLoads = 64 * kColBytes / 1024;           // 16-byte DMA instructions per transfer
  static constexpr int kWBytes = 64 * kColBytes;                  // per wave and buffer
  static constexpr int kWBufs = kStepsPerW == 1 ? kStages : 2;    // ring depth (buffers)
  static constexpr int kPLoads = 8;                               // 4-byte DMA: 4 for scales, 4 for biases
  static constexpr int kPBytes = 2 * 64 * 16;                     // per wave and buffer: 16-byte windows of scales, biases
  static constexpr int kALoads = kAGroupsPerWave;

  // Slot (16-byte unit) holding part `part` of column c's run. 128-byte runs:
  // within 8 consecutive columns the slots differ; columns c and c+8 (same
  // 128-byte bank phase in a 256-byte window) differ in slot bit 0. 64-byte
  // runs: even columns 0,2,4,6 (and odd 1,3,5,7) use different slots, and so
  // do columns c, c+4, c+8, c+12.
  static __device__ __forceinline__ int slot(int c, int part) {
    return kSlots == 8 ? part ^ (c & 7) ^ ((c >> 3) & 1) : part ^ (((c >> 1) ^ (c >> 3)) & 3);
  }

  // Transfers issued by iteration j (= step index mod 4), in issue order
  // parameters, words, activations; group 0 = parameters, 1 = words, 2 = activations.
  static constexpr int group_ops(int j, int g) {
    return g == 0 ? (j == 0 ? kPLoads : 0) : g == 1 ? (kStepsPerW == 1 || j == 0 ? kWLoads : 0) : kALoads;
  }
  static constexpr int ops(int j) { return group_ops(j, 0) + group_ops(j, 1) + group_ops(j, 2); }
  // Transfers issued after group g of the iteration r iterations before one
  // with index j, up to the start of that one.
  static constexpr int ops_after(int j, int r, int g) {
    const int jr = ((j - r) % 4 + 4) % 4;
    int n = 0;
    for (int h = g + 1; h < 3; ++h) n += group_ops(jr, h);
    for (int i = 1; i < r; ++i) n += ops(((j - i) % 4 + 4) % 4);
    return n;
  }
  // vmcnt bound at the start of iteration j: the activations of its step
  // (issued three iterations before) and the words and parameters of the
  // next step (decoded during it) must have landed.
  static constexpr int wait(int j) {
    int n = ops_after(j, 3, 2);
    const int rw = kStepsPerW == 1 ? 3 : (j == 3 ? 3 : j + 4);
    const int rp = j == 3 ? 3 : j + 4;
    const int nw = ops_after(j, rw, 1), np = ops_after(j, rp, 0);
    n = nw < n ? nw : n;
    n = np < n ? np : n;
    return n;
  }
  static_assert(kWLoads * 1024 == kWBytes, "whole DMA instructions");
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
// All global reads are direct-to-LDS transfers: activations into a 4-stage
// ring three steps ahead (four 1 KiB transfers per wave and step, 8 rows x
// 128 bytes each; 16-byte chunk c of row r stored at slot
// c ^ (r%8) ^ ((r/8)%2), so the A-fragment reads -- consecutive rows, one
// chunk -- are bank-conflict free for 8- and 16-lane LDS phases); packed words, scales and biases
// of the wave's own 64 columns per Plan. A wave decodes B fragments only from
// its own transfers (no barrier needed for them); the barrier orders the
// shared activation tile. Step t+1 is decoded while step t's MFMAs run.
template <int BITS, typename PT>
__global__ __launch_bounds__(kThreads, 1) void qgemm_kernel(GemmArgs a) {
  using P = Plan<BITS, PT>;
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kStages][kAStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[P::kWBufs][kWaves][P::kWBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_p[2][kWaves][P::kPBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31;
  const int lh = lane >> 5;

  // Work unit of this block (tile, K range): consecutive blocks go to
  // consecutive XCDs, so the block index is remapped to give each XCD a
  // contiguous run of units (same K range, neighbouring tiles).
  const int nb_n = (a.N + kBN - 1) / kBN;
  const int tiles = nb_n * ((a.M + kBM - 1) / kBM);
  const int units = tiles * a.splits;
  int unit = blockIdx.x;
  if ((units & 7) == 0) unit = (unit & 7) * (units >> 3) + (unit >> 3);
  const int split = unit / tiles;
  const int tile = unit % tiles;
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
  // Packed-word transfers: DMA lane L of instruction j writes LDS byte
  // 1024j + 16L of the wave's buffer = slot (16L % kColBytes) / 16 of local
  // column (1024j + 16L) / kColBytes, which holds part slot ^ swizzle.
  const uint8_t* w_src[P::kWLoads];
#pragma unroll
  for (int j = 0; j < P::kWLoads; ++j) {
    const int pos = 1024 * j + 16 * lane;
    const int c = pos / P::kColBytes;
    const int part = P::slot(c, (pos % P::kColBytes) / 16);  // the swizzle is an involution
    const int col = min(n0 + c, a.N - 1);  // columns past N feed unstored outputs
    w_src[j] = reinterpret_cast<const uint8_t*>(a.w + static_cast<int64_t>(col) * a.ws0) + 16 * part;
  }
  // Parameter windows: DMA lane L of instruction i carries dword L%4 of the
  // window of local column 16i + L/4, stored at byte 16*(16i + L/4) + 4*(L%4).
  const int row_dwords = (a.K >> (5 + a.group_shift)) * PT::bytes / 4;  // whole dwords per parameter row
  const uint8_t* s_col[4];
  const uint8_t* b_col[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int col = min(n0 + 16 * i + (lane >> 2), a.N - 1);
    s_col[i] = a.s + static_cast<int64_t>(col) * a.ss0 * PT::bytes;
    b_col[i] = a.b + static_cast<int64_t>(col) * a.bs0 * PT::bytes;
  }
  // First dword of the window for the four steps starting at `step`.
  auto window = [&](int step) { return (((step * kBK) >> (5 + a.group_shift)) * PT::bytes) >> 2; };

  // Single transfer instructions: parameter window i (0..3 scales, 4..7
  // biases) of the four steps starting at `step` (a multiple of 4); packed-word
  // instruction j of the transfer starting at `step`; activation group i of `step`.
  auto issue_p = [&](int step, int i) {
    const uint32_t dst = lds_address(lds_p[(step >> 2) & 1][wave]) + (i < 4 ? 256 * i : 1024 + 256 * (i - 4));
    const int off = 4 * min(window(s0 + step) + (lane & 3), row_dwords - 1);
    load_lds<4>((i < 4 ? s_col[i] : b_col[i - 4]) + off, dst);
  };
  auto issue_w = [&](int step, int j) {
    const int buf = P::kStepsPerW == 1 ? (step & 3) : ((step >> 2) & 1);
    load_lds<16>(w_src[j] + static_cast<int64_t>(s0 + step) * (8 * BITS), lds_address(lds_w[buf][wave]) + 1024 * j);
  };
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
    const int wbuf = P::kStepsPerW == 1 ? (step & 3) : ((step >> 2) & 1);
    const int sub = P::kStepsPerW == 1 ? 0 : (step & 3);  // step within the transfer
    // Position of this lane's group in the parameter window.
    const int g = (((s0 + step) * kBK + 32 * lh) >> (5 + a.group_shift)) - window(s0 + (step & ~3)) * (4 / PT::bytes);
    const uint8_t* pbuf = lds_p[(step >> 2) & 1][wave];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int c = 32 * nt + li;
      const uint8_t* col = lds_w[wbuf][wave] + c * P::kColBytes;
      if constexpr (BITS == 2) {  // 8 bytes: half of slot `sub`
        const uint2 v = *reinterpret_cast<const uint2*>(col + 16 * P::slot(c, sub) + 8 * lh);
        in.words[nt][0] = v.x;
        in.words[nt][1] = v.y;
      } else {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {  // 4-bit: part 2*sub + lh; 8-bit: parts 2*lh, 2*lh + 1
          const int part = BITS == 4 ? 2 * sub + lh : 2 * lh + i;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(col + 16 * P::slot(c, part));
          in.words[nt][4 * i] = v.x;
          in.words[nt][4 * i + 1] = v.y;
          in.words[nt][4 * i + 2] = v.z;
          in.words[nt][4 * i + 3] = v.w;
        }
      }
      if constexpr (PT::bytes == 2) {
        in.s_raw[nt] = *reinterpret_cast<const uint16_t*>(pbuf + 16 * c + 2 * g);
        in.b_raw[nt] = *reinterpret_cast<const uint16_t*>(pbuf + 1024 + 16 * c + 2 * g);
      } else {
        in.s_raw[nt] = *reinterpret_cast<const uint32_t*>(pbuf + 16 * c + 4 * g);
        in.b_raw[nt] = *reinterpret_cast<const uint32_t*>(pbuf + 1024 + 16 * c + 4 * g);
      }
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
  // and column l%32 of its 32x32 tile.
  auto for_each_output = [&](auto&& f) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = n0 + 32 * nt + li;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + 32 * mt + 8 * (v / 4) + 4 * lh + (v % 4);
          if (row < a.M && col < a.N) f(static_cast<int64_t>(row) * a.N + col, acc[mt][nt][v]);
        }
    }
  };
  float* dst = a.splits == 1 ? a.out : a.partial + split * static_cast<int64_t>(a.M) * a.N;
  for_each_output([&](int64_t i, float v) { dst[i] = v; });
}

// out[i] = sum of the K ranges' partial sums, added in range order (the same
// result on every run). Four outputs per thread; `count` = M*N; `vec` when
// count % 4 == 0 and out is 16-byte aligned (partial always is).
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* partial, float* out, int64_t count,
                                                              int splits, int vec) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= count) return;
  if (vec) {
    f32x4_t sum = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(partial + i));
    for (int r = 1; r < splits; ++r) sum += __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(partial + r * count + i));
    *reinterpret_cast<f32x4_t*>(out + i) = sum;
  } else {
    for (int64_t j = i; j < i + 4 && j < count; ++j) {
      float sum = partial[j];
      for (int r = 1; r < splits; ++r) sum += partial[r * count + j];
      out[j] = sum;
    }
  }
}

template <int BITS, typename PT>
hipError_t launch_typed(const GemmArgs& args, hipStream_t stream) {
  const int tiles = ((args.N + kBN - 1) / kBN) * ((args.M + kBM - 1) / kBM);
  hipLaunchKernelGGL((qgemm_kernel<BITS, PT>), dim3(tiles * args.splits), dim3(kThreads), 0, stream, args);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || args.splits == 1) return e;
  const int64_t count = static_cast<int64_t>(args.M) * args.N;
  const int64_t blocks = (count + 1023) / 1024;
  const int vec = count % 4 == 0 && reinterpret_cast<uintptr_t>(args.out) % 16 == 0;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     args.partial, args.out, count, args.splits, vec);
  return hipGetLastError();
}

int device_cus() {
  static std::mutex mutex;
  static int cached[64] = {0};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  std::lock_guard<std::mutex> lock(mutex);
  if (cached[device] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) cus = 256;
    cached[device] = cus;
  }
  return cached[device];
}

// Number of K ranges: 1 when the tiles alone fill three quarters of the CUs;
// otherwise the smallest count of equal 4-step-aligned ranges (at most 8, at
// least 8 steps each) that does, or the largest allowed.
int choose_splits(int tiles, int steps) {
  const int target = device_cus() * 3 / 4;
  int splits = 1;
  if (tiles >= target) return 1;
  for (int s = 2; s <= 8; ++s) {
    if ((steps / 4) % s != 0) continue;
    if (steps / s < 8) break;
    splits = s;
    if (tiles * s >= target) break;
  }
  return splits;
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
  if (p.M > (int64_t(1) << 30) || p.N > (int64_t(1) << 30) || p.K > (int64_t(1) << 30)) return false;
  if (((p.N + kBN - 1) / kBN) * ((p.M + kBM - 1) / kBM) > (int64_t(1) << 31) - 1) return false;
  return true;
}

hipError_t mfma_launch(const QmmProblem& p, const Launch& l) {
  hipStream_t stream = l.stream;
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
  const int tiles = static_cast<int>(((p.N + kBN - 1) / kBN) * ((p.M + kBM - 1) / kBM));
  const int steps = static_cast<int>(p.K / kBK);
  a.splits = 1;
  a.split_steps = steps;
  a.partial = nullptr;
  const int splits = l.workspace != nullptr ? choose_splits(tiles, steps) : 1;
  if (splits > 1) {
    if (auto* ws = static_cast<float*>(l.workspace->get(static_cast<size_t>(splits) * p.M * p.N * 4))) {
      a.splits = splits;
      a.split_steps = steps / splits;
      a.partial = ws;
    }
  }
  const bool bf16p = p.p_dtype == AFFON_ROCM_BF16;
  switch (p.bits) {
    case 2: return bf16p ? launch_typed<2, BF16>(a, stream) : launch_typed<2, F32>(a, stream);
    case 4: return bf16p ? launch_typed<4, BF16>(a, stream) : launch_typed<4, F32>(a, stream);
    default: return bf16p ? launch_typed<8, BF16>(a, stream) : launch_typed<8, F32>(a, stream);
  }
}

bool gemv_mfma_supports(const QmmProblem&) { return false; }
hipError_t gemv_mfma_launch(const QmmProblem&, const Launch&) { return hipErrorNotSupported; }

}  // namespace affon
