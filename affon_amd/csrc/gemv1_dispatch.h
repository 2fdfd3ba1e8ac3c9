// Host-side shape selection for the M = 1 decode kernel.
//
// For every (R rows, CPL chunks per lane) variant the number of K-parts is the
// smallest that gives each lane at most CPL chunks; the variant chosen is the
// one that runs in the fewest rounds of resident waves (occupancy from the
// compiled kernel), then with the fewest K-parts (no LDS reduction and
// barrier), then with the most waves (more latency hiding). On MI355X this
// picks the fastest variant, or one within 3% of it, on each of 8-bit
// 14336x4096 and 4096x14336, 4-bit 14336x4096, 4096x14336, 4096x4096,
// 1024x4096 and 128256x4096 (bf16), and 4-bit 4096x4096 with f32 operands.
// Paired gate/up problems choose among the even-R variants the same way,
// counting R/2 output rows per wave; grouped launches count the rows of all
// their projections (each padded to a multiple of 8).
#pragma once

#include <map>
#include <mutex>
#include <utility>

#include "gemv1.h"

namespace affon {
namespace gemv1 {

constexpr int64_t kMaxLdsBytes = 64 * 1024;
// Largest row the variants cover: 4 K-parts x 64 lanes x 4 chunks.
constexpr int64_t kMaxChunks = 4 * 64 * 4;

struct Variant {
  int R;
  int CPL;
  hipError_t (*launch)(const Args&, hipStream_t);
  const void* fn;
  size_t (*lds)(int chunks);
};

template <int BITS, typename XT, int R>
size_t lds_bytes(int chunks) {
  return lds_size<BITS, XT, R>(chunks);
}

#define AFFON_GEMV1_VARIANT(R, CPL)                                                     \
  {R, CPL, launch<BITS, XT, PT, R, CPL, MODE, LG>,                                       \
   reinterpret_cast<const void*>(&kernel<BITS, XT, PT, R, CPL, MODE, LG>), lds_bytes<BITS, XT, R>}

template <int BITS, typename XT, typename PT, int MODE, int LG>
const Variant* variants(int* count) {
  if constexpr (MODE == kPaired) {
    static const Variant table[] = {
        AFFON_GEMV1_VARIANT(2, 1), AFFON_GEMV1_VARIANT(4, 1), AFFON_GEMV1_VARIANT(8, 1), AFFON_GEMV1_VARIANT(2, 2),
        AFFON_GEMV1_VARIANT(4, 2), AFFON_GEMV1_VARIANT(2, 4), AFFON_GEMV1_VARIANT(4, 4),
    };
    *count = static_cast<int>(sizeof(table) / sizeof(table[0]));
    return table;
  } else {
    static const Variant table[] = {
        AFFON_GEMV1_VARIANT(1, 1), AFFON_GEMV1_VARIANT(2, 1), AFFON_GEMV1_VARIANT(4, 1), AFFON_GEMV1_VARIANT(8, 1),
        AFFON_GEMV1_VARIANT(1, 2), AFFON_GEMV1_VARIANT(2, 2), AFFON_GEMV1_VARIANT(4, 2), AFFON_GEMV1_VARIANT(1, 4),
        AFFON_GEMV1_VARIANT(2, 4), AFFON_GEMV1_VARIANT(4, 4),
    };
    *count = static_cast<int>(sizeof(table) / sizeof(table[0]));
    return table;
  }
}
#undef AFFON_GEMV1_VARIANT

inline int device_cus() {
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

// Resident blocks per CU of a compiled variant at a given LDS size (cached:
// the query costs more than a launch).
inline int blocks_per_cu(const void* fn, size_t lds) {
  static std::mutex mutex;
  static std::map<std::pair<const void*, size_t>, int> cache;
  std::lock_guard<std::mutex> lock(mutex);
  const auto key = std::make_pair(fn, lds);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kThreads, lds) != hipSuccess || blocks <= 0) blocks = 1;
  cache.emplace(key, blocks);
  return blocks;
}

// p: the problem (grouped mode: the first projection; group holds all
// `count` projections, which share everything but the weights and outputs).
template <int BITS, typename XT, typename PT, int MODE>
hipError_t dispatch(const QmmProblem& p, const QmmProblem* group, int count, hipStream_t stream) {
  constexpr bool PAIR = MODE == kPaired;
  Args a;
  a.w = p.w;
  a.ws0 = p.ws0;
  a.s = p.s;
  a.ss0 = p.ss0;
  a.b = p.b;
  a.bs0 = p.bs0;
  a.x = p.x;
  a.out = p.out;
  a.epi = p.epi;
  a.N = p.N;
  a.segments = 1;
  for (int i = 0; i < kMaxSegments; ++i) {
    a.seg_first[i] = 0;
    a.seg_n[i] = 0;
    a.seg_w[i] = nullptr;
    a.seg_s[i] = a.seg_b[i] = a.seg_bias[i] = nullptr;
    a.seg_out[i] = nullptr;
  }
  if constexpr (MODE == kGrouped) {
    if (count < 1 || count > kMaxSegments) return hipErrorInvalidValue;
    int64_t first = 0;
    for (int i = 0; i < count; ++i) {
      a.seg_first[i] = first;
      a.seg_n[i] = group[i].N;
      a.seg_w[i] = group[i].w;
      a.seg_s[i] = group[i].s;
      a.seg_b[i] = group[i].b;
      a.seg_out[i] = group[i].out;
      a.seg_bias[i] = group[i].epi.kind == kEpiBias ? group[i].epi.bias : nullptr;
      first += (group[i].N + 7) / 8 * 8;
    }
    a.segments = count;
    a.N = a.seg_first[count - 1] + a.seg_n[count - 1];
    a.epi.bias_bf16 = 0;
    for (int i = 0; i < count; ++i)
      if (group[i].epi.kind == kEpiBias) a.epi.bias_bf16 = group[i].epi.bias_bf16;
  }
  a.chunks = static_cast<int>(p.K * BITS / 128);
  a.cpg_shift = 0;
  while ((int64_t(1) << a.cpg_shift) * chunk_values<BITS>() < p.group) ++a.cpg_shift;
  // Parameter loads are shared by lane groups of kShare<BITS> lanes when a
  // group spans that many chunks (K-parts then start on multiples of it).
  const bool share = (1 << a.cpg_shift) >= kShare<BITS>;
  const int lg = share ? kShare<BITS> : 1;
  int nvariants = 0;
  const Variant* table =
      share ? variants<BITS, XT, PT, MODE, kShare<BITS>>(&nvariants) : variants<BITS, XT, PT, MODE, 1>(&nvariants);
  const int cus = device_cus();
  const Variant* best = nullptr;
  int best_ks = 0;
  int64_t best_rounds = 0, best_waves = 0;
  // Variants that would leave a chunk slot of every lane empty are passed
  // over, unless no other variant covers the row (the K-part count is 1, 2
  // or 4, so e.g. 688 chunks run as 4 parts of 172 on 4-chunk lanes).
  for (int pass = 0; pass < 2 && best == nullptr; ++pass) {
    for (int i = 0; i < nvariants; ++i) {
      const Variant& v = table[i];
      int ks = static_cast<int>((a.chunks + 64 * v.CPL - 1) / (64 * v.CPL));
      if (ks == 3) ks = 4;
      if (ks > 4) continue;
      const int part = ((a.chunks + ks - 1) / ks + lg - 1) / lg * lg;
      if (pass == 0 && v.CPL > 1 && 64 * (v.CPL - 1) >= part) continue;  // a chunk slot would stay empty
      const size_t lds = v.lds(a.chunks);
      if (lds > static_cast<size_t>(kMaxLdsBytes)) continue;
      const int64_t capacity = static_cast<int64_t>(blocks_per_cu(v.fn, lds)) * cus * kWaves;
      const int rows_out = PAIR ? v.R / 2 : v.R;
      const int64_t waves = (a.N + rows_out - 1) / rows_out * ks;
      const int64_t rounds = (waves + capacity - 1) / capacity;
      const bool better = best == nullptr || rounds < best_rounds ||
                          (rounds == best_rounds && (ks < best_ks || (ks == best_ks && waves > best_waves)));
      if (better) {
        best = &v;
        best_ks = ks;
        best_rounds = rounds;
        best_waves = waves;
      }
    }
  }
  if (best == nullptr) return hipErrorInvalidValue;
  a.ks = best_ks;
  a.part = ((a.chunks + best_ks - 1) / best_ks + lg - 1) / lg * lg;
  return best->launch(a, stream);
}

template <int BITS, int MODE>
hipError_t dispatch_mode(const QmmProblem& p, const QmmProblem* group, int count, hipStream_t stream) {
  if (p.x_dtype == AFFON_ROCM_BF16) {
    if (p.p_dtype == AFFON_ROCM_BF16) return dispatch<BITS, BF16, BF16, MODE>(p, group, count, stream);
    return dispatch<BITS, BF16, F32, MODE>(p, group, count, stream);
  }
  if (p.p_dtype == AFFON_ROCM_BF16) return dispatch<BITS, F32, BF16, MODE>(p, group, count, stream);
  return dispatch<BITS, F32, F32, MODE>(p, group, count, stream);
}

template <int BITS>
hipError_t dispatch_bits(const QmmProblem& p, hipStream_t stream) {
  if (p.epi.kind == kEpiSiluPair) return dispatch_mode<BITS, kPaired>(p, nullptr, 0, stream);
  return dispatch_mode<BITS, kPlain>(p, nullptr, 0, stream);
}

template <int BITS>
hipError_t dispatch_group_bits(const QmmProblem* group, int count, hipStream_t stream) {
  return dispatch_mode<BITS, kGrouped>(group[0], group, count, stream);
}

}  // namespace gemv1
}  // namespace affon
