// Multi-tensor AdamW for gfx950: every parameter tensor of a launch is cut
// into 2048-element pieces, one workgroup each, so a model's update is one
// grid that fills the chip.  A workgroup finds its tensor by a binary search
// over the launch's (ascending) first-workgroup table, which sits in the
// kernel arguments (scalar loads); each thread loads its 8 elements of p, g,
// m and v before any is used, so their latencies overlap, then updates and
// stores them.  Streaming: 28 bytes of HBM traffic per element.
#include "optim_kernels.h"

namespace mvm {

__global__ void __launch_bounds__(kAdamThreads) adamw_kernel(AdamLaunch a) {
  const int b = blockIdx.x;
  int lo = 0, hi = a.nt - 1;
  while (lo < hi) {  // last tensor whose first workgroup is <= b (block-uniform)
    const int mid = (lo + hi + 1) >> 1;
    if (a.t[mid].blk0 <= b) lo = mid;
    else hi = mid - 1;
  }
  float* __restrict__ p = a.t[lo].p;
  const float* __restrict__ g = a.t[lo].g;
  float* __restrict__ m = a.m + a.t[lo].soff;
  float* __restrict__ v = a.v + a.t[lo].soff;
  const int64_t n = a.t[lo].n;
  const int64_t e0 = static_cast<int64_t>(b - a.t[lo].blk0) * kAdamElems + threadIdx.x;

  const float t = *a.step;
  const float bc1 = 1.f - powf(a.beta1, t);
  const float bc2_sqrt = sqrtf(1.f - powf(a.beta2, t));
  const float step_size = a.lr / bc1;
  const float decay = 1.f - a.lr * a.wd;
  const float w1 = 1.f - a.beta1, w2 = 1.f - a.beta2;

  float pv[kAdamPerThread], gv[kAdamPerThread], mv[kAdamPerThread], vv[kAdamPerThread];
#pragma unroll
  for (int k = 0; k < kAdamPerThread; ++k) {
    const int64_t i = e0 + k * kAdamThreads;
    const int64_t ic = i < n ? i : n - 1;  // in bounds; not stored past n
    pv[k] = p[ic];
    gv[k] = g[ic];
    mv[k] = m[ic];
    vv[k] = v[ic];
  }
#pragma unroll
  for (int k = 0; k < kAdamPerThread; ++k) {
    const int64_t i = e0 + k * kAdamThreads;
    const float gk = gv[k];
    const float pk = pv[k] * decay;
    const float mk = mv[k] + w1 * (gk - mv[k]);
    const float vk = vv[k] * a.beta2 + w2 * (gk * gk);
    const float denom = sqrtf(vk) / bc2_sqrt + a.eps;
    if (i < n) {
      p[i] = pk - step_size * (mk / denom);
      m[i] = mk;
      v[i] = vk;
    }
  }
}

hipError_t launch_adamw(const AdamLaunch& a, hipStream_t s) {
  if (a.nblk <= 0) return hipSuccess;
  hipLaunchKernelGGL(adamw_kernel, dim3(static_cast<unsigned>(a.nblk)), dim3(kAdamThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace mvm
