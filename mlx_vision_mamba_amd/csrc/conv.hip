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

// Every row load goes to an in-bounds, clamped address whose value is then
// selected away when the position or channel is out of range: no load sits
// behind a divergent branch, so the window's loads issue back to back
// instead of waiting one by one.  A row's address is a scalar base (the
// token row, read out of lane_rows) plus the lane's 32-bit byte offset, so
// each load needs one VGPR of address, not two.
//
// lane_rows: the token row of position p0 + step * lane (clamped into
// [0, L)) in each lane.  One vector load fetches the rows of up to 64
// wave-uniform positions, which row_at then reads out with readlane (into
// SGPRs), instead of one dependent scalar load per position.
template <bool TOK>
__device__ __forceinline__ int32_t lane_rows(const int32_t* tok, int64_t p0, int step, int lane,
                                             int64_t L) {
  const int64_t p = p0 + static_cast<int64_t>(step) * lane;
  const int64_t pc = p < 0 ? 0 : (p >= L ? L - 1 : p);
  if constexpr (TOK) {
    const int32_t r = tok[pc];
    return r < 0 ? 0 : (r >= L ? static_cast<int32_t>(L - 1) : r);
  } else {
    return static_cast<int32_t>(pc);
  }
}
__device__ __forceinline__ int64_t row_at(int32_t rows, int i) {
  return static_cast<int64_t>(__builtin_amdgcn_readlane(rows, i));
}

// v, or +0 when the (wave-uniform) position is outside [0, L): a bit mask
// rather than a select, so the load is not moved under a branch
__device__ __forceinline__ float keep_if(float v, bool in_range) {
  return __uint_as_float(__float_as_uint(v) & (in_range ? ~0u : 0u));
}

// one position's pre-activation from a window w[0..kc) over x[s-kc+1 .. s]
template <int KC>
__device__ __forceinline__ float conv_at(const float* wv, const float* xw, float bias) {
  float acc = bias;
#pragma unroll
  for (int j = 0; j < KC; ++j) acc = fmaf(wv[j], xw[j], acc);
  return acc;
}

template <int KC, bool TOK>
__global__ void __launch_bounds__(kThreads)
conv_fwd_kernel(ConvGeom g, const float* __restrict__ x, const float* __restrict__ w,
                const float* __restrict__ bias, float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool dvalid = d < g.D;
  const int64_t dc = dvalid ? d : 0;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / g.K, k = bk - (bk / g.K) * g.K;
  const int64_t s0 = static_cast<int64_t>(blockIdx.z) * kCvBlockPos +
                     __builtin_amdgcn_readfirstlane(wave) * kCvPos;
  if (s0 >= g.L) return;
  const int32_t* tok = g.tok ? g.tok + k * g.L : nullptr;
  const float* xs = x + b * g.xsb + k * g.xsk;
  float* ys = y + b * g.ysb + k * g.ysk;
  const uint32_t lo = static_cast<uint32_t>(dc) * 4u;  // lane byte offset
  float wv[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) wv[j] = w[(k * g.D + dc) * KC + j];
  const float bs = bias[k * g.D + dc];
  // window: xw[i] = x at position s0 - (KC-1) + i (token row: lane i of rx)
  const int32_t rx = lane_rows<TOK>(tok, s0 - (KC - 1), 1, lane, g.L);
  float xw[kCvPos + KC - 1];
#pragma unroll
  for (int i = 0; i < kCvPos + KC - 1; ++i) xw[i] = *at_bytes(xs + row_at(rx, i) * g.xst, lo);
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first use
#pragma unroll
  for (int i = 0; i < kCvPos + KC - 1; ++i) {
    const int64_t p = s0 - (KC - 1) + i;
    xw[i] = keep_if(xw[i], p >= 0 && p < g.L);
  }
#pragma unroll
  for (int i = 0; i < kCvPos; ++i) {
    const int64_t p = s0 + i;
    const float pre = conv_at<KC>(wv, xw + i, bs);
    if (p < g.L && dvalid) *at_bytes(ys + row_at(rx, i + KC - 1) * g.yst, lo) = pre * sigmoid_f(pre);
  }
}

template <int KC, bool TOK>
__global__ void __launch_bounds__(kThreads)
conv_bwd_kernel(ConvGeom g, const float* __restrict__ x, const float* __restrict__ w,
                const float* __restrict__ bias, const float* __restrict__ dy,
                float* __restrict__ dx, float* __restrict__ part) {
  __shared__ float sPart[4][KC + 1][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool dvalid = d < g.D;
  const int64_t dc = dvalid ? d : 0;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / g.K, k = bk - (bk / g.K) * g.K;
  const int64_t s0 = static_cast<int64_t>(blockIdx.z) * kCvBlockPos + wave * kCvPos;
  const int32_t* tok = g.tok ? g.tok + k * g.L : nullptr;
  const float* xs = x + b * g.xsb + k * g.xsk;
  const float* dys = dy + b * g.ysb + k * g.ysk;
  float* dxs = dx + b * g.dxsb + k * g.dxsk;
  const uint32_t lo = static_cast<uint32_t>(dc) * 4u;  // lane byte offset
  float wv[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) wv[j] = w[(k * g.D + dc) * KC + j];
  const float bs = bias[k * g.D + dc];
  // x at positions s0 - (KC-1) .. s0 + kCvPos - 1 + (KC-1) (token row of
  // position s0 - (KC-1) + i: lane i of rx)
  const int32_t rx = lane_rows<TOK>(tok, s0 - (KC - 1), 1, lane, g.L);
  constexpr int kXW = kCvPos + 2 * (KC - 1);
  float xw[kXW];
#pragma unroll
  for (int i = 0; i < kXW; ++i) xw[i] = *at_bytes(xs + row_at(rx, i) * g.xst, lo);
  // dpre at positions s0 .. s0 + kCvPos - 1 + (KC-1)
  constexpr int kGW = kCvPos + KC - 1;
  float gp[kGW];
#pragma unroll
  for (int i = 0; i < kGW; ++i) gp[i] = *at_bytes(dys + row_at(rx, i + KC - 1) * g.yst, lo);
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first use
#pragma unroll
  for (int i = 0; i < kXW; ++i) {
    const int64_t p = s0 - (KC - 1) + i;
    xw[i] = keep_if(xw[i], p >= 0 && p < g.L);
  }
#pragma unroll
  for (int i = 0; i < kGW; ++i) gp[i] = keep_if(gp[i], s0 + i < g.L);
#pragma unroll
  for (int i = 0; i < kGW; ++i) {
    const float pre = conv_at<KC>(wv, xw + i, bs);
    const float sg = sigmoid_f(pre);
    gp[i] = dvalid ? gp[i] * sg * fmaf(pre, 1.f - sg, 1.f) : 0.f;
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
    if (dvalid && p < g.L) *at_bytes(dxs + row_at(rx, i + KC - 1) * g.dxst, lo) = acc;
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
// A block covers 64 consecutive (k, d, j) columns; its 4 waves each sum a
// quarter of the partials, and the quarters are added in wave order.
__global__ void __launch_bounds__(kThreads)
conv_reduce_kernel(ConvGeom g, int kc, int64_t nparts, const float* __restrict__ part,
                   float* __restrict__ dw, float* __restrict__ db) {
  __shared__ double sq[4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t ncol = g.K * g.D * (kc + 1);
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const int64_t colc = col < ncol ? col : 0;
  const int64_t per = (nparts + 3) / 4;
  const int64_t q0 = wave * per, q1 = min(nparts, q0 + per);
  // the partials are added in order; each batch's loads are in flight
  // together (from in-bounds rows), not waited for one at a time
  constexpr int kBatch = 8;
  double s = 0.0;
  for (int64_t qb = q0; qb < q1; qb += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) v[u] = part[(qb + u < q1 ? qb + u : q0) * ncol + colc];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (qb + u < q1) s += v[u];
  }
  sq[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && col < ncol) {
    const double t = (sq[0][lane] + sq[1][lane]) + (sq[2][lane] + sq[3][lane]);
    const int j = static_cast<int>(col % (kc + 1));
    const int64_t kd = col / (kc + 1);
    if (j < kc)
      dw[kd * kc + j] = static_cast<float>(t);
    else
      db[kd] = static_cast<float>(t);
  }
}

template <int KC>
static hipError_t conv_fwd_t(const ConvGeom& g, const float* x, const float* w, const float* b,
                             float* y, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((g.D + 63) / 64), static_cast<unsigned>(g.B * g.K),
                  static_cast<unsigned>((g.L + kCvBlockPos - 1) / kCvBlockPos));
  if (g.tok)
    hipLaunchKernelGGL((conv_fwd_kernel<KC, true>), grid, dim3(kThreads), 0, s, g, x, w, b, y);
  else
    hipLaunchKernelGGL((conv_fwd_kernel<KC, false>), grid, dim3(kThreads), 0, s, g, x, w, b, y);
  return hipGetLastError();
}

template <int KC>
static hipError_t conv_bwd_t(const ConvGeom& g, const float* x, const float* w, const float* b,
                             const float* dy, float* dx, float* dw, float* db, float* part,
                             hipStream_t s) {
  const unsigned nz = static_cast<unsigned>((g.L + kCvBlockPos - 1) / kCvBlockPos);
  const dim3 grid(static_cast<unsigned>((g.D + 63) / 64), static_cast<unsigned>(g.B * g.K), nz);
  if (g.tok)
    hipLaunchKernelGGL((conv_bwd_kernel<KC, true>), grid, dim3(kThreads), 0, s, g, x, w, b, dy, dx, part);
  else
    hipLaunchKernelGGL((conv_bwd_kernel<KC, false>), grid, dim3(kThreads), 0, s, g, x, w, b, dy, dx, part);
  const int64_t total = g.K * g.D * (KC + 1);
  hipLaunchKernelGGL(conv_reduce_kernel, dim3(static_cast<unsigned>((total + 63) / 64)),
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
