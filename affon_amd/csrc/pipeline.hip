// Host-side pieces shared by the tiled kernels, and the ordered reduction of
// split-K partial sums.
#include "lds_pipeline.h"

namespace affon {
namespace pipeline {
namespace {

// out[i] = sum of the K ranges' partial sums, added in range order (the same
// result on every run), then the output epilogue. Four outputs per thread;
// `count` = M*N, `n` = N; `vec` when count % 4 == 0 and out is 16-byte
// aligned (partial always is). A grouped launch's partials span all its
// segments' columns (row stride n = total columns); each sum goes to its
// segment's output.
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* partial, float* out, int64_t count,
                                                              int64_t n, int splits, int vec, Epilogue epi,
                                                              Segments seg) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= count) return;
  if (seg.count > 0) {
    for (int64_t j = i; j < i + 4 && j < count; ++j) {
      float sum = partial[j];
      for (int r = 1; r < splits; ++r) sum += partial[r * count + j];
      const int64_t row = j / n;
      const int c = static_cast<int>(j - row * n);
      const int k = seg_of(seg, seg.col_base, c);
      const int col = c - seg_pick(seg.col_base, k);
      Epilogue e = epi;
      e.bias = seg_pick(seg.bias, k);
      e.kind = e.bias != nullptr ? kEpiBias : kEpiNone;
      store_output(e, seg_pick(seg.out, k), row * seg_pick(seg.n, k) + col, col, sum);
    }
    return;
  }
  if (vec) {
    f32x4_t sum = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(partial + i));
    for (int r = 1; r < splits; ++r) sum += __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(partial + r * count + i));
    if (epi.kind == kEpiNone) {
      *reinterpret_cast<f32x4_t*>(out + i) = sum;
    } else {
      const float v[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) store_output(epi, out, i + k, (i + k) % n, v[k]);
    }
  } else {
    for (int64_t j = i; j < i + 4 && j < count; ++j) {
      float sum = partial[j];
      for (int r = 1; r < splits; ++r) sum += partial[r * count + j];
      store_output(epi, out, j, j % n, sum);
    }
  }
}

}  // namespace

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


hipError_t launch_reduce(const TileArgs& args, hipStream_t stream) {
  const int64_t n = args.seg.count > 0 ? args.seg.total_n : args.N;
  const int64_t count = static_cast<int64_t>(args.M) * n;
  const int64_t blocks = (count + 1023) / 1024;
  const int vec = args.seg.count == 0 && count % 4 == 0 && reinterpret_cast<uintptr_t>(args.out) % 16 == 0;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     args.partial, args.out, count, n, args.splits, vec, args.epi, args.seg);
  return hipGetLastError();
}

}  // namespace pipeline
}  // namespace affon
