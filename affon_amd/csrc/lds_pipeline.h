// Shared pieces of the tiled quantized-matmul kernels (prefill GEMM and the
// small-M MFMA decode kernel) for gfx950: direct global-to-LDS transfers with
// counted waits, the packed-word / parameter transfer plan of one wave, the
// split of K over workgroups and the ordered reduction of its partial sums.
#pragma once

#include <mutex>
#include <type_traits>

#include "device.h"
#include "internal.h"

namespace affon {
namespace pipeline {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;        // K step
constexpr int kWaves = 4;      // waves per workgroup, side by side along N (64 columns each)
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 4;     // LDS ring depth (steps)

constexpr int kMaxSegments = 4;

// A grouped tiled launch: up to kMaxSegments projections of one activation
// tensor (same K, group size, dtypes and strides). Segment j owns the
// launch's tiles [first_tile[j], first_tile[j+1]) and columns [col_base[j],
// col_base[j] + n[j]) of the launch's column space, in which the split-K
// partial planes are laid out (row stride total_n).
struct Segments {
  int count = 0;  // 0: an ordinary launch (the operands in TileArgs)
  int total_tiles, total_n;
  int first_tile[kMaxSegments], col_base[kMaxSegments], n[kMaxSegments];
  const uint32_t* w[kMaxSegments];
  const uint8_t* s[kMaxSegments];
  const uint8_t* b[kMaxSegments];
  float* out[kMaxSegments];
  const uint8_t* bias[kMaxSegments];  // output bias (element type epi.bias_bf16) or null
};

// v[k] for a uniform k < kMaxSegments, by selects with constant indices (so
// that a copy of the arguments stays in scalar registers).
static_assert(kMaxSegments == 4, "seg_pick and seg_of spell out four segments");
template <typename T>
__device__ __forceinline__ T seg_pick(const T (&v)[kMaxSegments], int k) {
  return k == 0 ? v[0] : k == 1 ? v[1] : k == 2 ? v[2] : v[3];
}

// The segment holding launch tile (or column) t, given each segment's first.
__device__ __forceinline__ int seg_of(const Segments& g, const int (&first)[kMaxSegments], int t) {
  int k = 0;
  if (g.count > 1 && t >= first[1]) k = 1;
  if (g.count > 2 && t >= first[2]) k = 2;
  if (g.count > 3 && t >= first[3]) k = 3;
  return k;
}

// Operands of one tiled launch.
struct TileArgs {
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
  Epilogue epi;  // applied where the output is stored (the reduction when splits > 1)
  Segments seg;
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

// Waits until this wave's LDS reads have returned (memory clobber: no memory
// access moves across it), e.g. before a transfer may overwrite what they read.
__device__ __forceinline__ void wait_lds_reads() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

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

// 64-bit scalar pointer plus a byte offset, as an SGPR pair for the asm.
__device__ __forceinline__ const uint8_t* sadd(const void* p, int64_t off) {
  return static_cast<const uint8_t*>(p) + off;
}

// The transfers of load_lds with a scalar (wave-uniform) base address saddr
// and a 32-bit per-lane offset voff, so that per-step address advances stay
// scalar work. 16 bytes per lane from saddr + voff into LDS at
// lds_addr + 16 * lane.
__device__ __forceinline__ void dma16(const uint8_t* saddr, uint32_t voff, uint32_t lds_addr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(saddr), "s"(lds_addr)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// 4 bytes per lane from saddr + voff into LDS at lds_addr + 4 * lane.
__device__ __forceinline__ void dma4(const uint8_t* saddr, uint32_t voff, uint32_t lds_addr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(saddr), "s"(lds_addr)
               : "memory", "m0");
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

// Transfer plan of one wave (64 weight columns) for a weight format, with
// ALOADS activation transfer instructions per step and wave. With PWHOLE the
// scales and biases of the wave's whole K range arrive once, before the
// first step, instead of a window every four steps (WeightStream::
// issue_p_whole; the caller checks that the range fits kPWholeBytes).
//
// Packed words reach LDS in runs of kColBytes per column: WSTEPS K steps at
// a time, by default four for 2/4-bit (64 / 128 bytes, 4 / 8 lanes per
// column) and one for 8-bit (64 bytes) -- so each transfer instruction covers
// whole half or full 128-byte lines. WSTEPS = 2 (8-bit: 128-byte runs, whole
// lines) issues at odd iterations the two steps 3 and 4 ahead into a ring of
// two buffers: the buffer written is the one of the two steps just read.
//
// Issue order within an iteration: parameters, words, activations; with
// AFIRST parameters, activations, words. Transfers complete in issue order
// for the load counter, so waiting for a step's activations (issued three
// iterations before) also waits for every transfer issued before them:
// with AFIRST the words issued in that same iteration stay in flight one
// iteration longer. Scales and biases come as one 16-byte window per column
// every four steps (four lanes per column, one dword each; bf16: 8 groups,
// f32: 4 groups), starting at the dword that holds the first group of those
// 256 k values, which covers all of their groups for the group sizes the
// kernel accepts; dwords past the row end repeat the row's last dword.
//
// LDS banks. The swizzles below follow how gfx950 serves DS reads, as
// measured with SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE on access-pattern
// probes: 128-bit reads in four phases of 16 lanes (the lanes sharing lane
// bits 0 and 5) over 128 banks of 4 bytes; 64-bit reads in two phases of 32
// lanes (lanes 0-31, 32-63) over 64 banks; 32- and 16-bit reads in the same
// two phases over 32 banks. Within a phase, distinct dwords in one bank are
// served one per cycle. Inside a column run the 16-byte slots of the packed
// words, and inside a column's parameter window the dwords, are XOR-swizzled
// with the column index so that the decode's reads (lanes = consecutive
// columns) hit distinct banks. DMA writes fill LDS contiguously, 4 or 16 bytes
// per lane, whatever the swizzle: each lane fetches the source address whose
// data belongs in its LDS slot.
template <int BITS, typename PT, int ALOADS, bool PWHOLE = false, int WSTEPS = (BITS == 8 ? 1 : 4),
          bool AFIRST = false, int LANE_COLS = 32>
struct Plan {
  static constexpr int kStepsPerW = WSTEPS;                       // steps per packed-word transfer
  static_assert(WSTEPS == 1 || WSTEPS == 2 || WSTEPS == 4, "packed-word transfer length");
  static constexpr int kColBytes = 8 * BITS * kStepsPerW;         // bytes per column per transfer
  static constexpr int kSlots = kColBytes / 16;                   // 16-byte slots per column run
  static_assert(kSlots == 4 || kSlots == 8, "the slot swizzle covers runs of 64 or 128 bytes");
  static constexpr int kWLoads = 64 * kColBytes / 1024;           // 16-byte DMA instructions per transfer
  static constexpr int kWBytes = 64 * kColBytes;                  // per wave and buffer
  static constexpr int kWBufs = kStepsPerW == 1 ? kStages : 2;    // ring depth (buffers)
  static constexpr int kPLoads = 8;                               // 4-byte DMA: 4 for scales, 4 for biases
  static constexpr int kPBytes = 2 * 64 * 16;                     // per wave and buffer: 16-byte windows of scales, biases
  static constexpr int kALoads = ALOADS;                          // activation DMA instructions per step
  static constexpr int kPWholeBytes = 32;                         // per column and parameter (PWHOLE)
  static constexpr int kPWholeLoads = 2 * 64 * kPWholeBytes / 256;  // 4-byte DMA instructions (PWHOLE)
  static_assert(2 * 64 * kPWholeBytes <= 2 * kPBytes, "whole-range parameters fit the window buffers");

  // LANE_COLS: the consumer's lanes read LANE_COLS consecutive columns per
  // instruction (16: the decode-batch kernel, lanes 16q + r on column
  // 16t + r; 32: the 128-row GEMM, lanes 32h + r on column 32t + r).
  static_assert(LANE_COLS == 16 || LANE_COLS == 32, "lane layouts of the consumers");
  // Slot (16-byte unit) holding part `part` of column c's run (c_i = bit i
  // of c).
  //
  // 16 lane columns (the decode-batch kernel): 128-byte runs part XOR
  // (c1 ^ c4, c2 ^ c5, c3), 64-byte runs part XOR (c2, c3). Under the bank
  // model above its 4-bit (b64) and 8-bit (b128) reads are conflict-free, and
  // the counters agree; 2-bit runs of 64 bytes keep a 2-way conflict that no
  // XOR of column bits removes (16 columns x 2 lanes per phase over 8 bank
  // positions). The c4, c5 terms (constant within one read) give the four
  // column tiles different slot orders: reads whose addresses differ by a
  // multiple of 512 bytes would otherwise be merged into one ds_read2st64,
  // whose two halves share banks.
  //
  // 32 lane columns (the 128-row GEMM): part XOR (c0..c2) XOR c3 for
  // 128-byte runs and part XOR ((c1 ^ c3), (c2 ^ c4)) for 64-byte runs. Its
  // counters show 0.30 of LDS-active cycles in conflicts with these, and
  // 0.01 with the decode kernel's kind of layout, which made the GEMM 0.5 to
  // 1.6 % slower (more address arithmetic): these stay.
  static __device__ __forceinline__ int slot(int c, int part) {
    if constexpr (LANE_COLS == 16)
      return kSlots == 8 ? part ^ ((c >> 1) & 7) ^ ((c >> 4) & 3) : part ^ ((c >> 2) & 3);
    return kSlots == 8 ? part ^ (c & 7) ^ ((c >> 3) & 1) : part ^ (((c >> 1) ^ (c >> 3)) & 3);
  }
  // Dword holding logical dword d of column c's 16-byte parameter window, and
  // of its 32-byte whole-range window (PWHOLE): for the decode kernel the 16
  // columns of one read land on distinct banks; the GEMM's windows are not
  // swizzled (as for its slots).
  static __device__ __forceinline__ int p_dword(int c, int d) { return LANE_COLS == 16 ? d ^ ((c >> 3) & 1) : d; }
  static __device__ __forceinline__ int p_whole_dword(int c, int d) { return d ^ ((c >> 2) & 3); }

  // Whether iteration j issues a packed-word transfer, and how many steps
  // ahead of the iteration's own step that transfer starts.
  static constexpr bool w_issue(int j) { return kStepsPerW == 2 ? (j & 1) == 1 : (kStepsPerW == 1 || j == 0); }
  static constexpr int kWAhead = kStepsPerW == 2 ? 3 : 4;

  // Kinds of transfer and their position in an iteration's issue order.
  static constexpr int kParams = 0, kWords = 1, kActs = 2;
  static constexpr int pos(int kind) { return kind == kParams ? 0 : (kind == kWords) == !AFIRST ? 1 : 2; }
  static constexpr int kind_ops(int j, int kind) {
    return kind == kParams ? (j == 0 && !PWHOLE ? kPLoads : 0) : kind == kWords ? (w_issue(j) ? kWLoads : 0) : kALoads;
  }
  // Transfers issued by iteration j (= step index mod 4) in position g of
  // its issue order.
  static constexpr int group_ops(int j, int g) {
    return g == 0 ? kind_ops(j, kParams) : kind_ops(j, g == pos(kWords) ? kWords : kActs);
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
  // vmcnt bound at the start of iteration j when the iteration reads only
  // its own step: the activations, words and parameters of that step must
  // have landed (activations issued three iterations before; words by the
  // transfer holding the step; parameters by the window holding it).
  static constexpr int wait_own(int j) {
    int n = ops_after(j, 3, pos(kActs));
    const int rw = kStepsPerW == 1 ? 4 : kStepsPerW == 4 ? j + 4 : ((j & 1) ? 4 : 3);
    const int nw = ops_after(j, rw, pos(kWords));
    n = nw < n ? nw : n;
    if (!PWHOLE) {
      const int np = ops_after(j, j + 4, pos(kParams));
      n = np < n ? np : n;
    }
    return n;
  }
  // vmcnt bound at the start of iteration j: the activations of its step
  // (issued three iterations before) and the words and parameters of the
  // next step (decoded during it) must have landed. (Transfers of one or
  // four steps; the prefill GEMM's plan.)
  static constexpr int wait(int j) {
    int n = ops_after(j, 3, pos(kActs));
    const int rw = kStepsPerW == 1 ? 3 : (j == 3 ? 3 : j + 4);
    const int rp = j == 3 ? 3 : j + 4;
    const int nw = ops_after(j, rw, pos(kWords)), np = ops_after(j, rp, pos(kParams));
    n = nw < n ? nw : n;
    if (!PWHOLE) n = np < n ? np : n;  // whole-range parameters precede every transfer waited for
    return n;
  }
  static_assert(kWLoads * 1024 == kWBytes, "whole DMA instructions");
};

// Transfer plan of the reassociated prefill GEMM (gemm_re.hip), per wave of
// its eight: kSOps 4-byte scale transfers once (the tile's scales for the
// whole K range), then iteration t issues kAOps activation transfers (step
// t+2) and, when t % 4 == 0, kWOps packed-word transfers (steps t+4 .. t+7),
// in that order. The prologue issues the scales, the packed words of steps
// 0..3 and the activations of steps 0 and 1.
struct RePlan {
  static constexpr int kWaves = 8;
  static constexpr int kAOps = 4, kWOps = 2, kSOps = 8;
  // vmcnt bound at the start of iteration t (j = t % 4): the activations of
  // step t (issued by iteration t-2, before its packed words) must have
  // landed, which also covers step t's packed words and the scales (issued
  // earlier). In flight may stay the packed words issued by iteration t-2
  // (when t-2 = 0 mod 4) and every transfer of iteration t-1.
  static constexpr int wait(int j) { return kAOps + (j == 1 || j == 2 ? kWOps : 0); }
};

// The packed-word and parameter transfers of one wave's 64 columns
// [n0, n0 + 64) over one K range starting at global step s0, per Plan, into
// the wave's slices of a ring of LDS buffers: w_lds(buf) = w_base + buf *
// w_stride (Plan::kWBufs buffers of kWBytes), p_lds(buf) likewise (2 buffers
// of kPBytes). Steps passed to the methods are local to the K range.
template <int BITS, typename PT, int ALOADS, bool PWHOLE = false, int WSTEPS = (BITS == 8 ? 1 : 4),
          bool AFIRST = false, int LANE_COLS = 32>
struct WeightStream {
  using P = Plan<BITS, PT, ALOADS, PWHOLE, WSTEPS, AFIRST, LANE_COLS>;
  const uint8_t* w_src[P::kWLoads];
  const uint8_t* s_col[4];
  const uint8_t* b_col[4];
  const uint8_t* s_whole;  // PWHOLE: parameter tensors, their row strides in bytes, the columns
  const uint8_t* b_whole;
  int64_t s_row_bytes, b_row_bytes;
  int n0_, n_cols;
  uint8_t* w_base;
  uint8_t* p_base;
  int w_stride, p_stride;
  int s0, group_shift, row_dwords, lane;
  int p_whole_off[2];  // PWHOLE: source byte offset in a column's row, for even and odd instructions

  __device__ __forceinline__ void init(const TileArgs& a, int n0, int s0_, int lane_, uint8_t* w_base_, int w_stride_,
                                       uint8_t* p_base_, int p_stride_) {
    s0 = s0_;
    lane = lane_;
    group_shift = a.group_shift;
    w_base = w_base_;
    w_stride = w_stride_;
    p_base = p_base_;
    p_stride = p_stride_;
    // Packed-word transfers: DMA lane L of instruction j writes LDS byte
    // 1024j + 16L of the buffer = slot (16L % kColBytes) / 16 of local column
    // (1024j + 16L) / kColBytes, which holds part slot ^ swizzle.
#pragma unroll
    for (int j = 0; j < P::kWLoads; ++j) {
      const int pos = 1024 * j + 16 * lane;
      const int c = pos / P::kColBytes;
      const int part = P::slot(c, (pos % P::kColBytes) / 16);  // the swizzle is an involution
      const int col = min(n0 + c, a.N - 1);  // columns past N feed unstored outputs
      w_src[j] = reinterpret_cast<const uint8_t*>(a.w + static_cast<int64_t>(col) * a.ws0) + 16 * part;
    }
    // Parameter windows: DMA lane L of instruction i carries window dword
    // p_dword(c, L%4) of local column c = 16i + L/4, stored at byte 16c + 4*(L%4).
    row_dwords = (a.K >> (5 + a.group_shift)) * PT::bytes / 4;  // whole dwords per parameter row
    s_whole = a.s;
    b_whole = a.b;
    s_row_bytes = a.ss0 * PT::bytes;
    b_row_bytes = a.bs0 * PT::bytes;
    n0_ = n0;
    n_cols = a.N;
    // Instruction i carries columns whose swizzle term depends only on i % 2
    // and lane / 32 (columns 8i + L/8: bits 2, 3 are bit 0 of i and lane bit 5).
    if constexpr (PWHOLE) {
#pragma unroll
      for (int odd = 0; odd < 2; ++odd)
        p_whole_off[odd] = 4 * min(window(s0) + P::p_whole_dword(8 * odd + (lane >> 3), lane & 7), row_dwords - 1);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = min(n0 + 16 * i + (lane >> 2), a.N - 1);
      s_col[i] = a.s + static_cast<int64_t>(col) * a.ss0 * PT::bytes;
      b_col[i] = a.b + static_cast<int64_t>(col) * a.bs0 * PT::bytes;
    }
  }
  // First dword of the parameter window for the four global steps starting at gstep.
  __device__ __forceinline__ int window(int gstep) const {
    return (((gstep * kBK) >> (5 + group_shift)) * PT::bytes) >> 2;
  }
  // PWHOLE: the scales and biases of all steps of the K range (local steps
  // 0 .. steps-1) as one window per column and parameter of kPWholeBytes,
  // from the dword that holds the range's first group: instruction i, lane L
  // carries dword p_whole_dword(c, L%8) of column-parameter 8i + L/8 (scales
  // of columns c = 0..63, then their biases) to LDS byte 256i + 4L of p_base
  // (one buffer of 2 * 64 * kPWholeBytes).
  __device__ __forceinline__ void issue_p_whole(int i) const {
    const int cp = 8 * i + (lane >> 3);
    const int64_t col = min(n0_ + (cp & 63), n_cols - 1);  // columns past N feed unstored outputs
    const int off = p_whole_off[i & 1];
    const uint8_t* src = cp < 64 ? s_whole + col * s_row_bytes : b_whole + col * b_row_bytes;
    load_lds<4>(src + off, lds_address(p_base) + 256 * i);
  }
  __device__ __forceinline__ int w_buf(int step) const { return (step / P::kStepsPerW) % P::kWBufs; }
  __device__ __forceinline__ const uint8_t* w_lds(int step) const { return w_base + w_buf(step) * w_stride; }
  __device__ __forceinline__ const uint8_t* p_lds(int step) const { return p_base + ((step >> 2) & 1) * p_stride; }
  // Parameter window instruction i (0..3 scales, 4..7 biases) of the four
  // steps starting at `step` (a multiple of 4).
  __device__ __forceinline__ void issue_p(int step, int i) const {
    const uint32_t dst = lds_address(p_lds(step)) + (i < 4 ? 256 * i : 1024 + 256 * (i - 4));
    const int off = 4 * min(window(s0 + step) + P::p_dword(16 * (i & 3) + (lane >> 2), lane & 3), row_dwords - 1);
    load_lds<4>((i < 4 ? s_col[i] : b_col[i - 4]) + off, dst);
  }
  // Packed-word instruction j of the transfer starting at `step`.
  __device__ __forceinline__ void issue_w(int step, int j) const {
    load_lds<16>(w_src[j] + static_cast<int64_t>(s0 + step) * (8 * BITS), lds_address(w_lds(step)) + 1024 * j);
  }
  // Bytes [off, off + n) of local column c's packed run for `step`, as laid
  // out by the swizzle: 16-byte part q of the step's BITS*8 bytes.
  __device__ __forceinline__ const uint8_t* w_part(int step, int c, int q) const {
    const int sub = step % P::kStepsPerW;  // step within the transfer
    return w_lds(step) + c * P::kColBytes + 16 * P::slot(c, sub * (BITS / 2) + q);
  }
  // Raw scale and bias bits (bf16 in the low half, or f32) of local column c
  // for the group holding k offset `k` of `step`.
  __device__ __forceinline__ void params(int step, int c, int k, uint32_t* s_raw, uint32_t* b_raw) const {
    if constexpr (PWHOLE) {
      const int g = (((s0 + step) * kBK + k) >> (5 + group_shift)) - window(s0) * (4 / PT::bytes);
      const int byte = PT::bytes == 2 ? 4 * P::p_whole_dword(c, g >> 1) + 2 * (g & 1) : 4 * P::p_whole_dword(c, g);
      const uint8_t* sp = p_base + c * P::kPWholeBytes + byte;
      const uint8_t* bp = sp + 64 * P::kPWholeBytes;
      if constexpr (PT::bytes == 2) {
        *s_raw = *reinterpret_cast<const uint16_t*>(sp);
        *b_raw = *reinterpret_cast<const uint16_t*>(bp);
      } else {
        *s_raw = *reinterpret_cast<const uint32_t*>(sp);
        *b_raw = *reinterpret_cast<const uint32_t*>(bp);
      }
      return;
    }
    const int g = (((s0 + step) * kBK + k) >> (5 + group_shift)) - window(s0 + (step & ~3)) * (4 / PT::bytes);
    const uint8_t* pbuf = p_lds(step);
    if constexpr (PT::bytes == 2) {
      const int byte = LANE_COLS == 16 ? 16 * c + 4 * P::p_dword(c, g >> 1) + 2 * (g & 1) : 16 * c + 2 * g;
      *s_raw = *reinterpret_cast<const uint16_t*>(pbuf + byte);
      *b_raw = *reinterpret_cast<const uint16_t*>(pbuf + 1024 + byte);
    } else {
      const int byte = 16 * c + 4 * P::p_dword(c, g);
      *s_raw = *reinterpret_cast<const uint32_t*>(pbuf + byte);
      *b_raw = *reinterpret_cast<const uint32_t*>(pbuf + 1024 + byte);
    }
  }
};

template <typename PT>
__device__ __forceinline__ float widen_param(uint32_t raw) {
  return PT::bytes == 2 ? __uint_as_float(raw << 16) : __uint_as_float(raw);
}

// Work unit (tile, K range) of this workgroup: consecutive blocks go to
// consecutive XCDs, so the block index is remapped to give each XCD a
// contiguous run of units (same K range, neighbouring tiles).
__device__ __forceinline__ void work_unit(int tiles, int splits, int* tile, int* split) {
  const int units = tiles * splits;
  int unit = blockIdx.x;
  if ((units & 7) == 0) unit = (unit & 7) * (units >> 3) + (unit >> 3);
  *split = unit / tiles;
  *tile = unit % tiles;
}

int device_cus();

// Number of K ranges: 1 when the tiles alone fill three quarters of the CUs;
// otherwise the smallest count of equal 4-step-aligned ranges (at most 8, at
// least 8 steps each) that does, or the largest allowed.
int choose_splits(int tiles, int steps);

// Enqueues the ordered sum of args.splits partial planes into args.out.
hipError_t launch_reduce(const TileArgs& args, hipStream_t stream);

}  // namespace pipeline
}  // namespace affon
