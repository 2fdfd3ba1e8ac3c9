// Virtual-row MFMA decode kernels for 2-bit packed weights, 16-row layout
// (one translation unit per bit width so the variants compile in parallel).
#include "vrow16_dispatch.h"

namespace affon {

hipError_t vrow16_launch_b2(const QmmProblem& p, hipStream_t stream) { return vrow16::dispatch_bits<2>(p, stream); }

}  // namespace affon
