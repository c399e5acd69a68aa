// Causal depthwise conv1d + bias + SiLU along each direction's scan order,
// forward and backward, for gfx950.
//
// Reference: MambaBlock's conv1d (mlx_vision_mamba/mamba_block.py:129-132,
// :170) is a depthwise Conv1d with kernel d_conv and symmetric padding
// d_conv - 1 whose first L outputs are kept, followed by SiLU (:171):
//   pre[s] = bias + sum_{j<kc} w[j] * x[s - (kc-1) + j]   (x[<0] = 0)
//   out[s] = pre[s] * sigmoid(pre[s])
// For direction k, position s reads and writes token row seq_to_tok[k, s],
// so the permuted copies of mamba_block.py:254-338 are never built.
//
// Work split: a 256-thread block covers 64 channels x 64 scan positions of
// one (batch, direction); lane = channel (coalesced rows), wave w owns
// positions 16w .. 16w+15 and keeps its input window (16 + kc - 1 values)
// in registers.  dw / dbias are summed per block in a fixed order and the
// per-block partials reduced by conv_reduce_kernel (deterministic).
#include "conv_kernels.h"
#include "scan_common.h"

namespace mvm {

constexpr int kCvPos = 16;        // positions per wave
constexpr int kCvBlockPos = 64;   // positions per block

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

// one position's pre-activation from a window w[0..kc) over x[s-kc+1 .. s]
template <int KC>
__device__ __forceinline__ float conv_at(const float* wv, const float* xw, float bias) {
  float acc = bias;
#pragma unroll
  for (int j = 0; j < KC; ++j) acc = fmaf(wv[j], xw[j], acc);
  return acc;
}

template <int KC>
__global__ void __launch_bounds__(kThreads)
conv_fwd_kernel(ConvGeom g, const float* __restrict__ x, const float* __restrict__ w,
                const float* __restrict__ bias, float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool dvalid = d < g.D;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / g.K, k = bk - (bk / g.K) * g.K;
  const int64_t s0 = static_cast<int64_t>(blockIdx.z) * kCvBlockPos + wave * kCvPos;
  if (s0 >= g.L) return;
  const int32_t* tok = g.tok ? g.tok + k * g.L : nullptr;
  const int64_t xb = b * g.xsb + k * g.xsk;
  const int64_t yb = b * g.ysb + k * g.ysk;
  float wv[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) wv[j] = dvalid ? w[(k * g.D + d) * KC + j] : 0.f;
  const float bs = dvalid ? bias[k * g.D + d] : 0.f;
  // window: xw[i] = x at position s0 - (KC-1) + i
  float xw[kCvPos + KC - 1];
#pragma unroll
  for (int i = 0; i < kCvPos + KC - 1; ++i) {
    const int64_t p = s0 - (KC - 1) + i;
    xw[i] = (dvalid && p >= 0 && p < g.L) ? x[xb + token_row(tok, p, g.L) * g.xst + d] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < kCvPos; ++i) {
    const int64_t p = s0 + i;
    if (p < g.L && dvalid) {
      const float pre = conv_at<KC>(wv, xw + i, bs);
      y[yb + token_row(tok, p, g.L) * g.yst + d] = pre * sigmoidf_(pre);
    }
  }
}

template <int KC>
__global__ void __launch_bounds__(kThreads)
conv_bwd_kernel(ConvGeom g, const float* __restrict__ x, const float* __restrict__ w,
                const float* __restrict__ bias, const float* __restrict__ dy,
                float* __restrict__ dx, float* __restrict__ part) {
  __shared__ float sPart[4][KC + 1][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool dvalid = d < g.D;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / g.K, k = bk - (bk / g.K) * g.K;
  const int64_t s0 = static_cast<int64_t>(blockIdx.z) * kCvBlockPos + wave * kCvPos;
  const int32_t* tok = g.tok ? g.tok + k * g.L : nullptr;
  const int64_t xb = b * g.xsb + k * g.xsk;
  const int64_t yb = b * g.ysb + k * g.ysk;
  const int64_t dxb = b * g.dxsb + k * g.dxsk;
  float wv[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) wv[j] = dvalid ? w[(k * g.D + d) * KC + j] : 0.f;
  const float bs = dvalid ? bias[k * g.D + d] : 0.f;
  // x at positions s0 - (KC-1) .. s0 + kCvPos - 1 + (KC-1)
  constexpr int kXW = kCvPos + 2 * (KC - 1);
  float xw[kXW];
#pragma unroll
  for (int i = 0; i < kXW; ++i) {
    const int64_t p = s0 - (KC - 1) + i;
    xw[i] = (dvalid && p >= 0 && p < g.L) ? x[xb + token_row(tok, p, g.L) * g.xst + d] : 0.f;
  }
  // dpre at positions s0 .. s0 + kCvPos - 1 + (KC-1)
  constexpr int kGW = kCvPos + KC - 1;
  float gp[kGW];
#pragma unroll
  for (int i = 0; i < kGW; ++i) {
    const int64_t p = s0 + i;
    float v = 0.f;
    if (dvalid && p < g.L) {
      const float pre = conv_at<KC>(wv, xw + i, bs);
      const float sg = sigmoidf_(pre);
      v = dy[yb + token_row(tok, p, g.L) * g.yst + d] * sg * (1.f + pre * (1.f - sg));
    }
    gp[i] = v;
  }
  float dwp[KC], dbp = 0.f;
#pragma unroll
  for (int j = 0; j < KC; ++j) dwp[j] = 0.f;
#pragma unroll
  for (int i = 0; i < kCvPos; ++i) {
    const int64_t p = s0 + i;
    // dx[p] = sum_j w[j] * dpre[p + (KC-1) - j]
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < KC; ++j) acc = fmaf(wv[j], gp[i + (KC - 1) - j], acc);
    if (dvalid && p < g.L) dx[dxb + token_row(tok, p, g.L) * g.dxst + d] = acc;
    // dw[j] += dpre[p] * x[p - (KC-1) + j]; db += dpre[p]
#pragma unroll
    for (int j = 0; j < KC; ++j) dwp[j] = fmaf(gp[i], xw[i + j], dwp[j]);
    dbp += gp[i];
  }
#pragma unroll
  for (int j = 0; j < KC; ++j) sPart[wave][j][lane] = dwp[j];
  sPart[wave][KC][lane] = dbp;
  __syncthreads();
  if (wave == 0 && dvalid) {
    const int64_t blk = b * gridDim.z + blockIdx.z;  // partial index over (b, position block)
    float* pp = part + ((blk * g.K + k) * g.D + d) * (KC + 1);
#pragma unroll
    for (int j = 0; j <= KC; ++j)
      pp[j] = (sPart[0][j][lane] + sPart[1][j][lane]) + (sPart[2][j][lane] + sPart[3][j][lane]);
  }
}

// dw (K, D, KC) and dbias (K, D): fixed-order float64 sum of the partials.
__global__ void __launch_bounds__(kThreads)
conv_reduce_kernel(ConvGeom g, int kc, int64_t nparts, const float* __restrict__ part,
                   float* __restrict__ dw, float* __restrict__ db) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t total = g.K * g.D * (kc + 1);
  if (idx >= total) return;
  const int j = static_cast<int>(idx % (kc + 1));
  const int64_t kd = idx / (kc + 1);
  double s = 0.0;
  for (int64_t q = 0; q < nparts; ++q) s += part[(q * g.K * g.D + kd) * (kc + 1) + j];
  if (j < kc)
    dw[kd * kc + j] = static_cast<float>(s);
  else
    db[kd] = static_cast<float>(s);
}

template <int KC>
static hipError_t conv_fwd_t(const ConvGeom& g, const float* x, const float* w, const float* b,
                             float* y, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((g.D + 63) / 64), static_cast<unsigned>(g.B * g.K),
                  static_cast<unsigned>((g.L + kCvBlockPos - 1) / kCvBlockPos));
  hipLaunchKernelGGL((conv_fwd_kernel<KC>), grid, dim3(kThreads), 0, s, g, x, w, b, y);
  return hipGetLastError();
}

template <int KC>
static hipError_t conv_bwd_t(const ConvGeom& g, const float* x, const float* w, const float* b,
                             const float* dy, float* dx, float* dw, float* db, float* part,
                             hipStream_t s) {
  const unsigned nz = static_cast<unsigned>((g.L + kCvBlockPos - 1) / kCvBlockPos);
  const dim3 grid(static_cast<unsigned>((g.D + 63) / 64), static_cast<unsigned>(g.B * g.K), nz);
  hipLaunchKernelGGL((conv_bwd_kernel<KC>), grid, dim3(kThreads), 0, s, g, x, w, b, dy, dx, part);
  const int64_t total = g.K * g.D * (KC + 1);
  hipLaunchKernelGGL(conv_reduce_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, s, g, KC, g.B * static_cast<int64_t>(nz), part, dw, db);
  return hipGetLastError();
}

int64_t conv_partial_floats(const ConvGeom& g, int kc) {
  return g.B * ((g.L + kCvBlockPos - 1) / kCvBlockPos) * g.K * g.D * (kc + 1);
}

hipError_t launch_conv_fwd(const ConvGeom& g, int kc, const float* x, const float* w,
                           const float* b, float* y, hipStream_t s) {
  switch (kc) {
    case 1: return conv_fwd_t<1>(g, x, w, b, y, s);
    case 2: return conv_fwd_t<2>(g, x, w, b, y, s);
    case 3: return conv_fwd_t<3>(g, x, w, b, y, s);
    case 4: return conv_fwd_t<4>(g, x, w, b, y, s);
    case 5: return conv_fwd_t<5>(g, x, w, b, y, s);
    case 6: return conv_fwd_t<6>(g, x, w, b, y, s);
    case 7: return conv_fwd_t<7>(g, x, w, b, y, s);
    case 8: return conv_fwd_t<8>(g, x, w, b, y, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_conv_bwd(const ConvGeom& g, int kc, const float* x, const float* w,
                           const float* b, const float* dy, float* dx, float* dw, float* db,
                           float* part, hipStream_t s) {
  switch (kc) {
    case 1: return conv_bwd_t<1>(g, x, w, b, dy, dx, dw, db, part, s);
    case 2: return conv_bwd_t<2>(g, x, w, b, dy, dx, dw, db, part, s);
    case 3: return conv_bwd_t<3>(g, x, w, b, dy, dx, dw, db, part, s);
    case 4: return conv_bwd_t<4>(g, x, w, b, dy, dx, dw, db, part, s);
    case 5: return conv_bwd_t<5>(g, x, w, b, dy, dx, dw, db, part, s);
    case 6: return conv_bwd_t<6>(g, x, w, b, dy, dx, dw, db, part, s);
    case 7: return conv_bwd_t<7>(g, x, w, b, dy, dx, dw, db, part, s);
    case 8: return conv_bwd_t<8>(g, x, w, b, dy, dx, dw, db, part, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mvm
