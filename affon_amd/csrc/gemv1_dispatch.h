// Host-side shape selection for the M = 1 decode kernel.
//
// For every (R rows, CPL chunks per lane) variant the number of K-parts is the
// smallest that gives each lane at most CPL chunks (1, 2 or 4 parts). The
// choice, in order of precedence:
//   * no lane slot left empty by every K-part, and at least XT bytes * 8 /
//     BITS weight rows per workgroup (each workgroup stages the whole
//     activation row from L2; fewer rows make that staging outweigh the
//     packed words);
//   * the least work on the busiest SIMD -- waves per SIMD, rounded up, times
//     the chunk-rows of a wave -- within 5 % (an uneven last wave per SIMD is
//     a tail the whole launch waits for);
//   * the fewest rounds of resident waves (occupancy from the compiled
//     kernel), then the fewest K-parts, then the most waves.
// On MI355X (graph periods, random data) this picks the fastest variant, or
// one within 2 % of it, on each of 8-bit 14336x4096, 4096x14336, 4096x4096
// and 1024x4096, 4-bit 14336x4096, 4096x14336, 11008x4096, 4096x11008,
// 4096x4096, 2048x2048, 1024x4096 and 128256x4096, 2-bit 14336x4096 (bf16),
// and 4-bit 4096x4096 with f32 operands. Paired gate/up problems choose among the
// even-R variants the same way, counting R/2 output rows per wave; grouped
// launches count the rows of all their projections (each padded to a
// multiple of 8).
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
  // Candidates, each with the measures the choice uses.
  struct Candidate {
    const Variant* v;
    int ks, tier;
    int64_t waves, rounds, load;
  };
  Candidate cand[16];
  int ncand = 0;
  const int cus = device_cus();
  const int64_t simds = static_cast<int64_t>(cus) * 4;
  // Weight rows per workgroup that keep the activation staging (K * x bytes
  // per workgroup, from L2) at most the packed bytes of those rows.
  const int min_rows = XT::bytes * 8 / BITS;
  for (int i = 0; i < nvariants && ncand < 16; ++i) {
    const Variant& v = table[i];
    int ks = static_cast<int>((a.chunks + 64 * v.CPL - 1) / (64 * v.CPL));
    if (ks == 3) ks = 4;
    if (ks > 4) continue;
    const int part = ((a.chunks + ks - 1) / ks + lg - 1) / lg * lg;
    const size_t lds = v.lds(a.chunks);
    if (lds > static_cast<size_t>(kMaxLdsBytes)) continue;
    const bool empty_slot = v.CPL > 1 && 64 * (v.CPL - 1) >= part;
    const bool thin = kWaves * v.R / ks < min_rows;
    Candidate c;
    c.v = &v;
    c.ks = ks;
    c.tier = empty_slot ? 2 : thin ? 1 : 0;
    const int rows_out = PAIR ? v.R / 2 : v.R;
    c.waves = (a.N + rows_out - 1) / rows_out * ks;
    const int64_t capacity = static_cast<int64_t>(blocks_per_cu(v.fn, lds)) * cus * kWaves;
    c.rounds = (c.waves + capacity - 1) / capacity;
    // Chunk-rows on the busiest SIMD: waves per SIMD (rounded up) times the
    // chunk-rows of one wave.
    c.load = (c.waves + simds - 1) / simds * v.R * ((part + 63) / 64);
    cand[ncand++] = c;
  }
  // The lowest tier present (no empty lane slot and enough rows per
  // workgroup; then the thin ones; then those with an empty slot). Within
  // it, variants whose busiest-SIMD load is within 5 % of the least; among
  // those the fewest rounds of resident waves, then the fewest K-parts, then
  // the most waves.
  int tier = 3;
  for (int i = 0; i < ncand; ++i) tier = cand[i].tier < tier ? cand[i].tier : tier;
  int64_t least = -1;
  for (int i = 0; i < ncand; ++i)
    if (cand[i].tier == tier && (least < 0 || cand[i].load < least)) least = cand[i].load;
  const Candidate* pick = nullptr;
  for (int i = 0; i < ncand; ++i) {
    const Candidate& c = cand[i];
    if (c.tier != tier || c.load * 100 > least * 105) continue;
    const bool better = pick == nullptr || c.rounds < pick->rounds ||
                        (c.rounds == pick->rounds && (c.ks < pick->ks || (c.ks == pick->ks && c.waves > pick->waves)));
    if (better) pick = &c;
  }
  const Variant* best = pick != nullptr ? pick->v : nullptr;
  const int best_ks = pick != nullptr ? pick->ks : 0;
  if (best == nullptr) return hipErrorInvalidValue;
  a.ks = best_ks;
  a.ks_shift = best_ks == 1 ? 0 : best_ks == 2 ? 1 : 2;
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
