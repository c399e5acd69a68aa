// LayerNorm over the last axis for gfx950 (MI355X): the pre-norm of every
// VisionMamba block and the encoder's final norm (mamba_block.py:201-205,
// :222-227, :401, :548; vision_mamba.py:192, :223).
//
// Memory-bound: one pass over x forward, one over (x, dy[, dres]) backward.
// A wave owns a row; lane l holds columns l, l + 64, ... (PER of them) in
// registers, so every load and store instruction moves 256 contiguous bytes
// and the row statistics are two butterfly sums over the wave.  Waves walk
// rows with a grid stride and issue the next row's loads before reducing
// and storing the current one.
//   forward   mean, then the variance from the registers (two passes over
//             registers, none over memory), y, and mean / rstd per row; one
//             row per wave up to 262,144 rows (measured fastest: the whole
//             6272 x 384 VisionMamba tensor in one round of waves);
//   backward  dx from the two row sums of g = dy * gamma and g * xh, plus
//             the residual branch's gradient (dres) in the same store;
//             dgamma / dbeta accumulate per lane over the rows a wave
//             visits, are summed over the workgroup's 8 waves in LDS and
//             written as one partial row per workgroup (at most 256); a
//             second kernel sums the partial rows in a fixed order (no
//             atomics: deterministic).  At 6272 x 384: 5.7 us forward,
//             11.6 us backward + reduce on MI355X.
#include "norm_kernels.h"

namespace mvm {
namespace {

constexpr int kNormThreads = 256;  // forward: 4 rows per workgroup pass
constexpr int kNormWaves = kNormThreads / 64;
constexpr int kNormBwdThreads = 512;
constexpr int kNormBwdWaves = kNormBwdThreads / 64;
constexpr int64_t kNormFwdMaxBlocks = 65536;
constexpr int64_t kNormBwdMaxBlocks = 256;
constexpr int kReduceWaves = 16;

// Butterfly sum over the 64 lanes; every lane ends with the same value
// (each step adds the same two operands in both lanes of a pair).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Row loads of one wave: PER columns per lane, 0 beyond cols.
template <int PER>
__device__ __forceinline__ void load_row(float (&v)[PER], const float* p, int64_t cols, int lane) {
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < cols ? p[c] : 0.f;
  }
}

// Each wave walks rows blockIdx.x * 4 + wave + k * (4 * gridDim.x); the
// next row's loads are issued before the current row is reduced and
// stored, so a wave's reads and writes overlap.
template <int PER>
__global__ void __launch_bounds__(kNormThreads)
norm_fwd_kernel(NormGeom g, const float* __restrict__ x, const float* __restrict__ gamma,
                const float* __restrict__ beta, float* __restrict__ y, float* __restrict__ mean,
                float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kNormWaves;
  int64_t row = static_cast<int64_t>(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  const float n = static_cast<float>(g.cols);
  float v[PER];
  if (row < g.rows) load_row(v, x + row * g.xs, g.cols, lane);
  for (; row < g.rows; row += step) {  // wave-uniform; no barrier in the loop
    float nv[PER];
    const int64_t nrow = row + step;
    if (nrow < g.rows) load_row(nv, x + nrow * g.xs, g.cols, lane);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) s += v[i];
    const float mu = wave_sum(s) / n;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + 64 * i;
      const float d = c < g.cols ? v[i] - mu : 0.f;
      q = fmaf(d, d, q);
    }
    const float r = rsqrtf(wave_sum(q) / n + g.eps);
    float* yr = y + row * g.ys;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + 64 * i;
      if (c < g.cols) yr[c] = fmaf((v[i] - mu) * r, gamma[c], beta[c]);
    }
    if (lane == 0) {
      mean[row] = mu;
      rstd[row] = r;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = nv[i];
  }
}

template <int PER, bool RES>
__global__ void __launch_bounds__(kNormBwdThreads)
norm_bwd_kernel(NormGeom g, const float* __restrict__ x, const float* __restrict__ gamma,
                const float* __restrict__ mean, const float* __restrict__ rstd,
                const float* __restrict__ dy, const float* dres, float* dx,
                float* __restrict__ part) {
  __shared__ float red[kNormBwdWaves][2][PER * 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const float n = static_cast<float>(g.cols);
  float gm[PER], ag[PER], ab[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane + 64 * i;
    gm[i] = c < g.cols ? gamma[c] : 0.f;
    ag[i] = 0.f;
    ab[i] = 0.f;
  }
  const int64_t step = static_cast<int64_t>(gridDim.x) * kNormBwdWaves;
  int64_t row = static_cast<int64_t>(blockIdx.x) * kNormBwdWaves + wave;
  // the row in registers (padding columns load 0: xh = 0 there, since the
  // centring below is masked too) and the next row's loads in flight
  float xv[PER], dv[PER], rv[PER];
  float mu = 0.f, r = 0.f;
  auto load = [&](int64_t rw, float (&a)[PER], float (&b)[PER], float (&c)[PER], float& m,
                  float& rs) {
    load_row(a, x + rw * g.xs, g.cols, lane);
    load_row(b, dy + rw * g.ys, g.cols, lane);
    if (RES) load_row(c, dres + rw * g.ys, g.cols, lane);
    m = mean[rw];
    rs = rstd[rw];
  };
  if (row < g.rows) load(row, xv, dv, rv, mu, r);
  for (; row < g.rows; row += step) {  // wave-uniform; the barrier is after the loop
    float nx[PER], nd[PER], nr[PER];
    float nmu = 0.f, nrs = 0.f;
    const int64_t nrow = row + step;
    if (nrow < g.rows) load(nrow, nx, nd, nr, nmu, nrs);
    float xh[PER], gg[PER];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + 64 * i;
      xh[i] = c < g.cols ? (xv[i] - mu) * r : 0.f;
      gg[i] = dv[i] * gm[i];
      s1 += gg[i];
      s2 = fmaf(gg[i], xh[i], s2);
      ag[i] = fmaf(dv[i], xh[i], ag[i]);
      ab[i] += dv[i];
    }
    const float m1 = wave_sum(s1) / n;
    const float m2 = wave_sum(s2) / n;
    float* dxr = dx + row * g.ys;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + 64 * i;
      const float v = r * (gg[i] - m1 - xh[i] * m2);
      if (c < g.cols) dxr[c] = RES ? v + rv[i] : v;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      xv[i] = nx[i];
      dv[i] = nd[i];
      if (RES) rv[i] = nr[i];
    }
    mu = nmu;
    r = nrs;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    red[wave][0][lane + 64 * i] = ag[i];
    red[wave][1][lane + 64 * i] = ab[i];
  }
  __syncthreads();
  float* pr = part + static_cast<int64_t>(blockIdx.x) * 2 * g.cols;
  for (int64_t j = threadIdx.x; j < 2 * g.cols; j += kNormBwdThreads) {
    const int t = j < g.cols ? 0 : 1;
    const int c = static_cast<int>(j - t * g.cols);
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kNormBwdWaves; ++w) v += red[w][t][c];
    pr[j] = v;
  }
}

// dgamma | dbeta column j of 2 * cols: the sum over the nblk partial rows,
// strided over 16 waves (16 independent loads in flight per wave, added in
// row order), then over the waves in order.
__global__ void __launch_bounds__(64 * kReduceWaves)
norm_reduce_kernel(const float* __restrict__ part, int64_t nblk, int64_t cols,
                   float* __restrict__ dgamma, float* __restrict__ dbeta) {
  constexpr int kBatch = 16;
  __shared__ float red[kReduceWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t n2 = 2 * cols;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  float s = 0.f;
  if (j < n2) {
    for (int64_t b0 = wave; b0 < nblk; b0 += kReduceWaves * kBatch) {
      float v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t b = b0 + static_cast<int64_t>(u) * kReduceWaves;
        v[u] = b < nblk ? part[b * n2 + j] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) s += v[u];
    }
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && j < n2) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kReduceWaves; ++w) t += red[w][lane];
    if (j < cols)
      dgamma[j] = t;
    else
      dbeta[j - cols] = t;
  }
}

// columns per lane: the smallest instantiated PER with 64 * PER >= cols
int pick_per(int64_t cols) {
  const int need = static_cast<int>((cols + 63) / 64);
  for (int p : {1, 2, 4, 6, 8, 12, 16})
    if (p >= need) return p;
  return 0;
}

template <int PER>
void fwd_per(const NormGeom& g, const float* x, const float* gamma, const float* beta, float* y,
             float* mean, float* rstd, hipStream_t s) {
  const int64_t want = (g.rows + kNormWaves - 1) / kNormWaves;
  const unsigned blocks = static_cast<unsigned>(want < kNormFwdMaxBlocks ? want : kNormFwdMaxBlocks);
  hipLaunchKernelGGL(norm_fwd_kernel<PER>, dim3(blocks), dim3(kNormThreads), 0, s, g, x, gamma,
                     beta, y, mean, rstd);
}

template <int PER>
void bwd_per(const NormGeom& g, const float* x, const float* gamma, const float* mean,
             const float* rstd, const float* dy, const float* dres, float* dx, float* part,
             hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>(norm_bwd_blocks(g));
  if (dres != nullptr)
    hipLaunchKernelGGL((norm_bwd_kernel<PER, true>), dim3(blocks), dim3(kNormBwdThreads), 0, s, g, x,
                       gamma, mean, rstd, dy, dres, dx, part);
  else
    hipLaunchKernelGGL((norm_bwd_kernel<PER, false>), dim3(blocks), dim3(kNormBwdThreads), 0, s, g,
                       x, gamma, mean, rstd, dy, dres, dx, part);
}

}  // namespace

int64_t norm_bwd_blocks(const NormGeom& g) {
  const int64_t want = (g.rows + kNormBwdWaves - 1) / kNormBwdWaves;
  return want < 1 ? 1 : (want > kNormBwdMaxBlocks ? kNormBwdMaxBlocks : want);
}

int64_t norm_partial_floats(const NormGeom& g) { return norm_bwd_blocks(g) * 2 * g.cols; }

hipError_t launch_norm_fwd(const NormGeom& g, const float* x, const float* gamma,
                           const float* beta, float* y, float* mean, float* rstd, hipStream_t s) {
  if (g.rows <= 0) return hipSuccess;
  switch (pick_per(g.cols)) {
    case 1: fwd_per<1>(g, x, gamma, beta, y, mean, rstd, s); break;
    case 2: fwd_per<2>(g, x, gamma, beta, y, mean, rstd, s); break;
    case 4: fwd_per<4>(g, x, gamma, beta, y, mean, rstd, s); break;
    case 6: fwd_per<6>(g, x, gamma, beta, y, mean, rstd, s); break;
    case 8: fwd_per<8>(g, x, gamma, beta, y, mean, rstd, s); break;
    case 12: fwd_per<12>(g, x, gamma, beta, y, mean, rstd, s); break;
    case 16: fwd_per<16>(g, x, gamma, beta, y, mean, rstd, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_norm_bwd(const NormGeom& g, const float* x, const float* gamma,
                           const float* mean, const float* rstd, const float* dy,
                           const float* dres, float* dx, float* dgamma, float* dbeta,
                           float* part, hipStream_t s) {
  // with no rows the backward kernel writes zero partials: dgamma = dbeta = 0
  switch (pick_per(g.cols)) {
    case 1: bwd_per<1>(g, x, gamma, mean, rstd, dy, dres, dx, part, s); break;
    case 2: bwd_per<2>(g, x, gamma, mean, rstd, dy, dres, dx, part, s); break;
    case 4: bwd_per<4>(g, x, gamma, mean, rstd, dy, dres, dx, part, s); break;
    case 6: bwd_per<6>(g, x, gamma, mean, rstd, dy, dres, dx, part, s); break;
    case 8: bwd_per<8>(g, x, gamma, mean, rstd, dy, dres, dx, part, s); break;
    case 12: bwd_per<12>(g, x, gamma, mean, rstd, dy, dres, dx, part, s); break;
    case 16: bwd_per<16>(g, x, gamma, mean, rstd, dy, dres, dx, part, s); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t nblk = norm_bwd_blocks(g);
  const unsigned rblocks = static_cast<unsigned>((2 * g.cols + 63) / 64);
  hipLaunchKernelGGL(norm_reduce_kernel, dim3(rblocks), dim3(64 * kReduceWaves), 0, s, part, nblk,
                     g.cols, dgamma, dbeta);
  return hipGetLastError();
}

}  // namespace mvm
