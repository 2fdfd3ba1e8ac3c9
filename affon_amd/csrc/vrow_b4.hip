// Virtual-row MFMA decode kernels for 4-bit packed weights, 16-row layout
// (one translation unit per bit width so the variants compile in parallel).
#include "vrow16_dispatch.h"

namespace affon {

hipError_t vrow16_launch_b4(const QmmProblem& p, hipStream_t stream) { return vrow16::dispatch_bits<4>(p, stream); }

}  // namespace affon
