// Causal depthwise conv1d (+ bias + SiLU) with direction remap: geometry and
// launch entry points (conv.hip), used by the C ABI (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvm {

struct ConvGeom {
  int64_t B, L, D, K;
  int64_t xsb, xsk, xst;   // input strides (channel stride 1)
  int64_t ysb, ysk, yst;   // output / dy strides (channel stride 1)
  int64_t dxsb, dxsk, dxst;  // dx strides (channel stride 1)
  const int32_t* tok;      // (K, L) scan position -> token row, or nullptr
};

// float32 elements of the dw | dbias partial buffer mvm_conv_bwd needs
int64_t conv_partial_floats(const ConvGeom& g, int kc);
hipError_t launch_conv_fwd(const ConvGeom& g, int kc, const float* x, const float* w,
                           const float* b, float* y, hipStream_t s);
hipError_t launch_conv_bwd(const ConvGeom& g, int kc, const float* x, const float* w,
                           const float* b, const float* dy, float* dx, float* dw, float* db,
                           float* part, hipStream_t s);

}  // namespace mvm
