// M = 1 decode kernels for 2-bit packed weights (one translation unit per
// bit width so the variants compile in parallel).
#include "gemv1_dispatch.h"

namespace affon {

hipError_t gemv1_launch_b2(const QmmProblem& p, hipStream_t stream) { return gemv1::dispatch_bits<2>(p, stream); }

}  // namespace affon
