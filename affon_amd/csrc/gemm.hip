// rocm_quantized_matmul.mfma and .gemv_mfma — MFMA kernels (not yet built).
#include "internal.h"

namespace affon {

bool gemv_mfma_supports(const QmmProblem&) { return false; }
hipError_t gemv_mfma_launch(const QmmProblem&, hipStream_t) { return hipErrorNotSupported; }
bool mfma_supports(const QmmProblem&) { return false; }
hipError_t mfma_launch(const QmmProblem&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace affon
