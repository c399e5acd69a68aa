// Multi-tensor AdamW: launch description and entry point (optim.hip), used
// by the C ABI (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvm {

constexpr int kAdamPerLaunch = 64;      // tensors described in one launch's arguments
constexpr int kAdamThreads = 256;
constexpr int kAdamPerThread = 8;       // elements per thread, loaded before any is used
constexpr int kAdamElems = kAdamThreads * kAdamPerThread;  // elements per workgroup

struct AdamSlice {
  float* p;
  const float* g;
  int64_t n;       // elements
  int64_t soff;    // element offset of its m / v
  int32_t blk0;    // first workgroup of this tensor in the launch
  int32_t pad;
};

struct AdamLaunch {
  AdamSlice t[kAdamPerLaunch];
  int32_t nt;      // tensors in this launch (blk0 ascending)
  int32_t nblk;    // workgroups in this launch
  float lr, beta1, beta2, eps, wd;
  const float* step;
  float* m;
  float* v;
};

hipError_t launch_adamw(const AdamLaunch& a, hipStream_t s);

}  // namespace mvm
