// Virtual-row MFMA decode kernels for 4-bit packed weights (one translation
// unit per bit width so the variants compile in parallel).
#include "vrow_dispatch.h"

namespace affon {

hipError_t vrow_launch_b4(const QmmProblem& p, hipStream_t stream) { return vrow::dispatch_bits<4>(p, stream); }

}  // namespace affon
