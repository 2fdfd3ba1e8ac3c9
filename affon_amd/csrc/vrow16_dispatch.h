// Host-side selection for the 16-row virtual-row decode kernel (vrow16.h).
#pragma once

#include "gemv1_dispatch.h"
#include "vrow16.h"

namespace affon {
namespace vrow16 {

// Shape rules shared by the guard and the launcher. Returns false when the
// kernel cannot run the problem; otherwise fills MP, G and the (CPL, ks)
// candidates (CPL * ks == sets, CPL a multiple of the accumulator run).
struct Plan {
  int MP = 0, G = 0, sets = 0;
};

inline bool plan(const QmmProblem& p, Plan* out) {
  if (p.x_dtype != AFFON_ROCM_BF16 || p.M < 1 || p.M > 4) return false;
  if (p.bits != 2 && p.bits != 4 && p.bits != 8) return false;
  if (p.xs1 != 1 || p.ws1 != 1 || p.ss1 != 1 || p.bs1 != 1) return false;
  const int64_t cv = 128 / p.bits, sk = 4 * cv;
  if (p.group < 16 || p.group > 128 || (p.group & (p.group - 1)) != 0 || p.group < cv || p.group > sk) return false;
  if (p.K % sk != 0 || p.K > (int64_t(1) << 20) || p.N > (int64_t(1) << 30)) return false;
  const int G = static_cast<int>(sk / p.group);
  const int MP = p.M <= 1 ? 1 : p.M <= 2 ? 2 : 4;
  const int pbytes = p.p_dtype == AFFON_ROCM_BF16 ? 2 : 4;
  const int64_t groups = p.K / p.group;
  if (groups % 4 != 0 || p.ss0 % 4 != 0 || p.bs0 % 4 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.s) % (4 * pbytes) != 0 || reinterpret_cast<uintptr_t>(p.b) % (4 * pbytes) != 0)
    return false;
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0 || (p.xs0 * 2) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || p.ws0 % 4 != 0) return false;
  if (lds_bytes(MP, static_cast<int>(p.K), static_cast<int>(groups)) > static_cast<size_t>(gemv1::kMaxLdsBytes))
    return false;
  const int sets = static_cast<int>(p.K / sk);
  const int spd = 16 / (MP * G);
  bool any = false;
  for (int cpl : {4, 8, 16})
    for (int ks : {1, 2, 4})
      if (cpl % spd == 0 && cpl * ks == sets) any = true;
  if (!any) return false;
  out->MP = MP;
  out->G = G;
  out->sets = sets;
  return true;
}

struct Variant {
  int CPL;
  hipError_t (*launch)(const Args&, hipStream_t);
  const void* fn;
};

template <int BITS, typename PT, int MP, int G>
hipError_t dispatch_mg(const QmmProblem& p, const Plan& pl, Args a, hipStream_t stream) {
  constexpr int PPG = chunk_codes<BITS>() / (2 * G);
  if constexpr (PPG < 2 || PPG > 16) {
    return hipErrorInvalidValue;  // group sizes plan() rejects for this width
  } else {
  constexpr int SPD = 16 / (MP * G);
  static const Variant table[] = {
      {4, SPD <= 4 ? launch<BITS, PT, MP, G, (SPD <= 4 ? 4 : SPD)> : nullptr,
       reinterpret_cast<const void*>(&kernel<BITS, PT, MP, G, (SPD <= 4 ? 4 : SPD)>)},
      {8, SPD <= 8 ? launch<BITS, PT, MP, G, (SPD <= 8 ? 8 : SPD)> : nullptr,
       reinterpret_cast<const void*>(&kernel<BITS, PT, MP, G, (SPD <= 8 ? 8 : SPD)>)},
      {16, launch<BITS, PT, MP, G, 16>, reinterpret_cast<const void*>(&kernel<BITS, PT, MP, G, 16>)},
  };
  const int cus = gemv1::device_cus();
  const size_t lds = lds_bytes(MP, a.K, a.groups);
  const Variant* best = nullptr;
  int best_ks = 0;
  int64_t best_rounds = 0, best_waves = 0;
  for (const Variant& v : table) {
    if (v.launch == nullptr || v.CPL % SPD != 0 || pl.sets % v.CPL != 0) continue;
    const int ks = pl.sets / v.CPL;
    if (ks != 1 && ks != 2 && ks != 4) continue;
    const int64_t capacity = static_cast<int64_t>(gemv1::blocks_per_cu(v.fn, lds)) * cus * kWaves;
    const int64_t waves = (p.N + kRows - 1) / kRows * ks;
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
  if (best == nullptr) return hipErrorInvalidValue;
  a.part = best->CPL;
  a.ks = best_ks;
  return best->launch(a, stream);
  }
}

template <int BITS, typename PT>
hipError_t dispatch_pt(const QmmProblem& p, hipStream_t stream) {
  Plan pl;
  if (!plan(p, &pl)) return hipErrorInvalidValue;
  Args a;
  a.x = p.x;
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
  a.groups = static_cast<int>(p.K / p.group);
  a.part = 0;
  a.ks = 0;
#define AFFON_VROW_CASE(MP_, G_) \
  if (pl.MP == MP_ && pl.G == G_) return dispatch_mg<BITS, PT, MP_, G_>(p, pl, a, stream);
  AFFON_VROW_CASE(1, 1) AFFON_VROW_CASE(1, 2) AFFON_VROW_CASE(1, 4)
  AFFON_VROW_CASE(2, 1) AFFON_VROW_CASE(2, 2) AFFON_VROW_CASE(2, 4)
  AFFON_VROW_CASE(4, 1) AFFON_VROW_CASE(4, 2) AFFON_VROW_CASE(4, 4)
#undef AFFON_VROW_CASE
  return hipErrorInvalidValue;
}

template <int BITS>
hipError_t dispatch_bits(const QmmProblem& p, hipStream_t stream) {
  return p.p_dtype == AFFON_ROCM_BF16 ? dispatch_pt<BITS, BF16>(p, stream) : dispatch_pt<BITS, F32>(p, stream);
}

}  // namespace vrow16
}  // namespace affon
