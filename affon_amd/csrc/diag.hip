// Measurement helper (no counterpart in the reference): one launch that reads
// every byte of up to four device buffers once, as a decode GEMV over the same
// weights must, and does nothing else. Its graph-replay period is the floor a
// decode launch of those bytes can reach on this GPU: HBM streaming plus the
// fixed cost of a launch that starts, ramps up and drains.
//
// Geometry of the M = 1 decode kernel: 256-thread workgroups, each lane issuing
// all its 16-byte non-temporal loads (kLoads of them, 1 KiB contiguous per wave
// and load) before it waits on any. A second kernel sweeps that geometry (KiB
// per wave, workgroup size) and adds the two costs a decode launch carries on
// top of its reads: vector arithmetic per wave and output stores; an empty
// kernel gives the launch period itself.

#include "internal.h"

namespace affon {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kLoads = 4;
constexpr int kMaxBuffers = 4;

struct ReadArgs {
  const u32x4_t* buf[kMaxBuffers];
  uint64_t chunks[kMaxBuffers];  // whole 16-byte chunks per buffer
  uint64_t first[kMaxBuffers];   // first global chunk index of each buffer
  uint64_t total;                // chunks of all buffers
  uint32_t* sink;                // written only if the data xor equals `never` (it cannot be relied on)
  uint32_t never;
};

__global__ __launch_bounds__(kThreads) void read_kernel(ReadArgs a) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
  u32x4_t v[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const uint64_t c = t + j * stride;
    v[j] = u32x4_t{0, 0, 0, 0};
    if (c < a.total) {
      int b = 0;
#pragma unroll
      for (int i = 1; i < kMaxBuffers; ++i)
        if (a.chunks[i] > 0 && c >= a.first[i]) b = i;
      const u32x4_t* p = b == 0 ? a.buf[0] : b == 1 ? a.buf[1] : b == 2 ? a.buf[2] : a.buf[3];
      const uint64_t f = b == 0 ? a.first[0] : b == 1 ? a.first[1] : b == 2 ? a.first[2] : a.first[3];
      v[j] = __builtin_nontemporal_load(p + (c - f));
    }
  }
  uint32_t x = 0;
#pragma unroll
  for (int j = 0; j < kLoads; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  if (x == a.never) a.sink[0] = x;
}

// Geometry sweep of the same floor: each wave reads KIB contiguous KiB (one
// 16-byte non-temporal load per lane per KiB, all issued before any wait),
// waves in workgroups of any size, optionally followed by `valu` dependent
// f32 multiply-adds on the loaded data (eight chains, so the work is the
// instruction count, not a latency chain) and by an 8-byte store from every
// `store_every`-th wave. Every loaded dword feeds the result, so no load is
// dead.
template <int KIB>
__global__ __launch_bounds__(1024) void geometry_kernel(const u32x4_t* __restrict__ p, uint64_t total, float* sink,
                                                        int valu_rounds, int store_every) {
  const uint64_t gw = (static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  u32x4_t v[KIB];
#pragma unroll
  for (int j = 0; j < KIB; ++j) {
    const uint64_t c = (gw * KIB + j) * 64 + lane;
    v[j] = u32x4_t{0, 0, 0, 0};
    if (c < total) v[j] = __builtin_nontemporal_load(p + c);
  }
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) a[k] = __uint_as_float((v[0][k % 4] ^ (k < 4 ? 0u : 0x5a5a5a5au)) & 0x3f7fffffu);
#pragma unroll
  for (int j = 1; j < KIB; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k + 4 * (j & 1)] += __uint_as_float(v[j][k] & 0x3f7fffffu);
  const float m = a[7] * 0x1p-40f;
  for (int r = 0; r < valu_rounds; ++r) {
#pragma unroll
    for (int k = 0; k < 8; ++k) a[k] = fmaf(m, a[(k + 1) & 7], a[k]);
  }
  const float s = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  if (store_every > 0) {
    if (gw % static_cast<uint64_t>(store_every) == 0 && lane < 2) sink[(gw / store_every) * 2 + lane] = s;
  } else if (s == -1.0f) {  // never: the loaded values are non-negative
    sink[0] = s;
  }
}

__global__ void empty_kernel() {}

}  // namespace

hipError_t read_geometry_launch(const void* buffer, uint64_t bytes, float* sink, int kib_per_wave, int threads,
                                int store_every, int valu_per_wave, hipStream_t stream) {
  const uint64_t total = bytes / 16;
  const uint64_t per_wave = 64ull * kib_per_wave;
  const uint64_t waves = (total + per_wave - 1) / per_wave;
  const uint64_t wpb = static_cast<uint64_t>(threads / 64);
  const uint64_t blocks = (waves + wpb - 1) / wpb;
  if (blocks == 0 || blocks > 0x7fffffffull) return hipErrorInvalidValue;
  const u32x4_t* p = static_cast<const u32x4_t*>(buffer);
  const int rounds = valu_per_wave / 8;
  const dim3 grid(static_cast<unsigned>(blocks)), block(static_cast<unsigned>(threads));
  switch (kib_per_wave) {
    case 1: hipLaunchKernelGGL(geometry_kernel<1>, grid, block, 0, stream, p, total, sink, rounds, store_every); break;
    case 2: hipLaunchKernelGGL(geometry_kernel<2>, grid, block, 0, stream, p, total, sink, rounds, store_every); break;
    case 4: hipLaunchKernelGGL(geometry_kernel<4>, grid, block, 0, stream, p, total, sink, rounds, store_every); break;
    case 8: hipLaunchKernelGGL(geometry_kernel<8>, grid, block, 0, stream, p, total, sink, rounds, store_every); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

uint64_t read_geometry_waves(uint64_t bytes, int kib_per_wave) {
  const uint64_t per_wave = 64ull * static_cast<uint64_t>(kib_per_wave);
  return (bytes / 16 + per_wave - 1) / per_wave;
}

hipError_t empty_launch(unsigned blocks, unsigned threads, hipStream_t stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(threads), 0, stream);
  return hipGetLastError();
}

hipError_t read_floor_launch(const void* const* buffers, const uint64_t* bytes, int count, uint32_t* sink,
                             hipStream_t stream) {
  ReadArgs a = {};
  uint64_t total = 0;
  for (int i = 0; i < count; ++i) {
    a.buf[i] = static_cast<const u32x4_t*>(buffers[i]);
    a.chunks[i] = bytes[i] / 16;
    a.first[i] = total;
    total += a.chunks[i];
  }
  a.total = total;
  a.sink = sink;
  a.never = 0x9e3779b9u;
  const uint64_t threads = (total + kLoads - 1) / kLoads;
  const uint64_t blocks = (threads + kThreads - 1) / kThreads;
  if (blocks == 0 || blocks > 0x7fffffffull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace affon
