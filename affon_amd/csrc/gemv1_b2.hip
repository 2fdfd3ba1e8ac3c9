// M = 1 decode kernels for 2-bit packed weights (one translation unit per
// bit width so the variants compile in parallel).
#include "gemv1_dispatch.h"

namespace affon {

hipError_t gemv1_launch_b2(const QmmProblem& p, hipStream_t stream) { return gemv1::dispatch_bits<2>(p, stream); }
hipError_t gemv1_group_launch_b2(const QmmProblem* group, int count, hipStream_t stream) {
  return gemv1::dispatch_group_bits<2>(group, count, stream);
}

}  // namespace affon
