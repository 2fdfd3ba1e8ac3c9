// Internal interfaces between the C ABI (abi.cpp) and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <vector>

#include "affon_rocm.h"
#include "epilogue.h"

namespace affon {

// A validated quantized_matmul problem. Pointers already include the byte
// offset of logical element [0,0]; strides are in elements.
struct QmmProblem {
  int64_t M = 0, N = 0, K = 0;
  int bits = 0;
  int64_t group = 0;
  const uint8_t* x = nullptr;
  int64_t xs0 = 0, xs1 = 0;
  int x_dtype = AFFON_ROCM_F32;
  const uint32_t* w = nullptr;
  int64_t ws0 = 0, ws1 = 0;
  const uint8_t* s = nullptr;
  int64_t ss0 = 0, ss1 = 0;
  const uint8_t* b = nullptr;
  int64_t bs0 = 0, bs1 = 0;
  int p_dtype = AFFON_ROCM_F32;
  float* out = nullptr;
  Epilogue epi;  // applied by the kernel that stores each output element
};

// Device scratch memory owned by a session and ordered by its stream.
// Buffers it outgrows are retired, not freed, until the session ends: a
// graph captured earlier keeps the old address in its kernel arguments and
// may still be replayed.
class Workspace {
 public:
  Workspace(int device, hipStream_t stream) : device_(device), stream_(stream) {}
  ~Workspace();
  Workspace(const Workspace&) = delete;
  Workspace& operator=(const Workspace&) = delete;
  // At least `bytes` of device memory, or nullptr when it cannot grow now
  // (the stream is being captured into a graph, or the allocation failed).
  void* get(size_t bytes);
  size_t retired() const { return retired_.size(); }

 private:
  int device_;
  hipStream_t stream_;
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
  std::vector<void*> retired_;
  size_t retired_bytes_ = 0;  // size of the last retired buffer
};

// Where a launcher enqueues its work, and the scratch memory it may use for
// split-K partial sums: the session's workspace (grown on demand), or a
// fixed buffer of fixed_bytes (the no-allocation entry point), or none.
struct Launch {
  hipStream_t stream = nullptr;
  Workspace* workspace = nullptr;
  void* fixed = nullptr;
  size_t fixed_bytes = 0;
  // Set when a fixed buffer is too small for the launcher's plan; the
  // launcher then launches nothing and returns hipErrorOutOfMemory.
  mutable size_t fixed_short = 0;

  bool can_split() const { return workspace != nullptr || fixed != nullptr; }
  // At least `bytes` of scratch, or nullptr (workspace: it cannot grow now;
  // fixed buffer: too small, recorded in fixed_short).
  void* scratch(size_t bytes) const {
    if (workspace != nullptr) return workspace->get(bytes);
    if (fixed != nullptr && bytes <= fixed_bytes) return fixed;
    if (fixed != nullptr) fixed_short = bytes;
    return nullptr;
  }
};

// Per-candidate capability guards and launchers. A guard returns true when
// the candidate can run the problem (shape, layout, alignment); launchers
// enqueue on the given stream and return the launch status.
bool generic_supports(const QmmProblem& p);
hipError_t generic_launch(const QmmProblem& p, const Launch& l);

bool gemv_supports(const QmmProblem& p);
// The M = 1 kernel of the gemv candidate (gemv1.h).
bool gemv1_supports(const QmmProblem& p);
// Whether the gemv candidate computes a kSiluPair problem (both projections)
// in one launch.
bool gemv_pair_supports(const QmmProblem& p);
hipError_t gemv_launch(const QmmProblem& p, const Launch& l);
// Grouped launch of up to 4 M = 1 problems that share the activation row,
// bits, group size, dtypes and strides (each with no epilogue or an output
// bias of one element type).
constexpr int kMaxGroup = 4;
bool gemv_group_supports(const QmmProblem* group, int count);
hipError_t gemv_group_launch(const QmmProblem* group, int count, const Launch& l);

bool gemv_mfma_supports(const QmmProblem& p);
hipError_t gemv_mfma_launch(const QmmProblem& p, const Launch& l);
// Grouped launch of 2..4 problems on the LDS-tiled kernel (decode batches
// the virtual-row kernels do not take) that share the activations, bits,
// group size, dtypes and strides.
bool gemv_mfma_group_supports(const QmmProblem* group, int count);
hipError_t gemv_mfma_group_launch(const QmmProblem* group, int count, const Launch& l);

// The reassociated prefill GEMM (gemm_re.hip) that gemv_mfma_launch runs for
// tall activations: 4-bit codes as exact bf16 MFMA operands, each group's
// scale applied in f32, the bias term from per-group activation sums.
bool re_gemm_supports(const QmmProblem& p);
// Enqueues it and returns true (*status: the launch status), or returns
// false with nothing enqueued when the shape's K ranges are too short for it
// or its scratch memory cannot be had now. `rounded`: the same kernel in the
// approximate class (decoded weights rounded to bf16, no per-group scaling),
// which mfma_launch runs.
bool re_gemm_launch(const QmmProblem& p, const Launch& l, hipError_t* status, bool rounded);

// The reassociated prefill GEMM for groups of 32 (gemm_re32.hip), which
// gemv_mfma_launch runs for tall activations whose groups the group-scaling
// GEMM and the LDS-tiled kernel do not take. `rounded`: the same kernel in
// the approximate class (decoded weights rounded to bf16), which mfma_launch
// runs for such shapes past 128 rows.
bool re32_supports(const QmmProblem& p);
hipError_t re32_launch(const QmmProblem& p, const Launch& l, bool rounded);

bool mfma_supports(const QmmProblem& p);
hipError_t mfma_launch(const QmmProblem& p, const Launch& l);
// The 4-bit prefill kernel whose column-sharing waves split the decode
// (gemm_pair.hip); mfma_launch runs it for the shapes it takes with more
// than 128 rows.
bool pair_supports(const QmmProblem& p);
hipError_t pair_launch(const QmmProblem& p, const Launch& l);

hipError_t quantize_launch(const void* weights, int weight_dtype, int64_t rows, int64_t columns,
                           int bits, int64_t group, uint32_t* packed, void* scales, void* biases,
                           int param_dtype, hipStream_t stream);
hipError_t rms_norm_launch(const void* x, int dtype, int64_t rows, int64_t cols, float epsilon, void* out,
                           hipStream_t stream);
hipError_t softmax_launch(const void* x, int dtype, int64_t rows, int64_t cols, void* out, hipStream_t stream);
hipError_t index_select_launch(const void* x, int dtype, int64_t rows, int64_t cols, int axis, const int64_t* index,
                               int64_t count, void* out, hipStream_t stream);
// One launch that reads every whole 16-byte chunk of up to four buffers once
// (diag.hip); sink receives at most one word.
hipError_t read_floor_launch(const void* const* buffers, const uint64_t* bytes, int count, uint32_t* sink,
                             hipStream_t stream);
// Geometry sweep of the read floor and an empty launch (diag.hip).
hipError_t read_geometry_launch(const void* buffer, uint64_t bytes, float* sink, int kib_per_wave, int threads,
                                int store_every, int valu_per_wave, hipStream_t stream);
uint64_t read_geometry_waves(uint64_t bytes, int kib_per_wave);
hipError_t empty_launch(unsigned blocks, unsigned threads, hipStream_t stream);
hipError_t dequantize_launch(const uint32_t* packed, const void* scales, const void* biases,
                             int param_dtype, int64_t rows, int64_t columns, int bits, int64_t group,
                             void* out, int out_dtype, hipStream_t stream);

}  // namespace affon
