// LayerNorm over the last axis: geometry and launch entry points
// (layernorm.hip), used by the C ABI (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvm {

struct NormGeom {
  int64_t rows, cols;
  int64_t xs;  // row stride of x
  int64_t ys;  // row stride of y, dy, dres and dx
  float eps;
};

// workgroups of the backward's row pass (each writes one partial row)
int64_t norm_bwd_blocks(const NormGeom& g);
// float32 elements of the dgamma | dbeta partial buffer the backward needs
int64_t norm_partial_floats(const NormGeom& g);
hipError_t launch_norm_fwd(const NormGeom& g, const float* x, const float* gamma,
                           const float* beta, float* y, float* mean, float* rstd, hipStream_t s);
hipError_t launch_norm_bwd(const NormGeom& g, const float* x, const float* gamma,
                           const float* mean, const float* rstd, const float* dy,
                           const float* dres, float* dx, float* dgamma, float* dbeta,
                           float* part, hipStream_t s);

}  // namespace mvm
