// Virtual-row MFMA decode kernels for 8-bit packed weights, both layouts
// (one translation unit per bit width so the variants compile in parallel).
#include "vrow16_dispatch.h"
#include "vrow_dispatch.h"

namespace affon {

hipError_t vrow_launch_b8(const QmmProblem& p, hipStream_t stream) { return vrow::dispatch_bits<8>(p, stream); }
hipError_t vrow16_launch_b8(const QmmProblem& p, hipStream_t stream) { return vrow16::dispatch_bits<8>(p, stream); }

}  // namespace affon
