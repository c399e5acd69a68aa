// Backward (VJP) of the selective scan for gfx950 (MI355X).
//
// Adjoint recurrence (mamba_metal_fused.py:66-145): going backwards in time
// with mu = the adjoint carried in from step t+1 (mu = 0 after the last step)
//   lam_t   = mu + C_t * g_t                         (:92-94)
//   w_t     = lam_t * exp(delta_t A) * h_{t-1}
//   ddelta_t = sum_n (w_t * A + lam_t * B_t * u_t)     (:116-117)
//   dA     += delta_t * w_t                          (:122, reduced :218)
//   dB_t    = sum_d lam_t * delta_t * u_t            (:130, reduced :221)
//   du_t    = D g_t + delta_t * sum_n lam_t * B_t    (:87, :133)
//   dC_t    = sum_d g_t * h_t                        (:224)
//   dD     += g_t * u_t                              (:89, :214)
//   mu      = exp(delta_t A) * lam_t                 (:136)
//
// Work split as in the forward: lane (c, g) owns 4 states of one channel, a
// workgroup owns 64 channels x one time chunk.  Each 16-step tile is
// processed in reverse: the states h_{t-1}, h_t of the tile are recomputed
// from the forward's checkpoint into VGPRs together with exp(delta A)
// (one transcendental per element for the whole backward), then the adjoint
// sweep runs over the registers.
//
// Reductions are atomic-free and in a fixed order (bitwise deterministic):
//   dB, dC   sum over 16 channels per wave with cross-lane ops, over the 4
//            waves in LDS, then over channel blocks in reduce_bc_kernel;
//   dA, dD   per-lane float32 sums over each 16-step tile, folded into
//            float64 running sums (a long chunk of unit-size terms can
//            cancel to ~1e-3, far below float32 running-sum error), float64
//            partials per (b, chunk), summed in float64 by reduce_ad_kernel.
// Long sequences: the adjoint carry between time chunks uses the same
// two-pass idea as the forward, run right to left (bwd_agg + bwd_carry).
#include "scan_common.h"
#include "scan_kernels.h"

namespace mvm {

// Pass 1: adjoint aggregate of chunks 1..nchunk-1: the mu that leaves the
// chunk's first position when mu = 0 enters its last, and sum(delta).
template <typename XT>
__global__ void __launch_bounds__(kThreads)
scan_bwd_agg_kernel(Geom gm, BwdBufs bf) {
  __shared__ float sC[kSub][kStatePad];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = lane & 3;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kChPerBlock + wave * kChPerWave + (lane >> 2);
  const bool dvalid = d < gm.D;
  const int64_t dc = dvalid ? d : 0;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / gm.K;
  const int64_t k = bk - b * gm.K;
  const int64_t chunk = blockIdx.z + 1;
  const int64_t t0 = chunk * gm.chunk_len;
  const int64_t t1 = min(gm.L, t0 + gm.chunk_len);
  const int32_t* tok = gm.tok ? gm.tok + k * gm.L : nullptr;
  const int64_t xbase = b * gm.xsb + k * gm.xsk + dc;
  const int64_t bcbase = b * gm.bsb + k * gm.bsk;
  const XT* __restrict__ Cm = static_cast<const XT*>(bf.Cm);
  const XT* __restrict__ dy = static_cast<const XT*>(bf.dy);

  float a2[4], mu[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = 4 * grp + j;
    a2[j] = (dvalid && n < gm.N) ? bf.A[(k * gm.D + d) * gm.N + n] * kLog2e : 0.f;
    mu[j] = 0.f;
  }
  float dsum = 0.f;
  const int64_t ntile = (t1 - t0 + kSub - 1) / kSub;
  for (int64_t it = ntile - 1; it >= 0; --it) {
    const int64_t ts = t0 + it * kSub;
    const int nt = static_cast<int>(min<int64_t>(kSub, t1 - ts));
    __syncthreads();
    for (int i = tid; i < kSub * kStatePad; i += kThreads) {
      const int tt = i / kStatePad, n = i % kStatePad;
      float v = 0.f;
      if (tt < nt && n < gm.N) {
        const int64_t row = token_row(tok, ts + tt, gm.L);
        v = ld(Cm, bcbase + row * gm.bst + n);
      }
      sC[tt][n] = v;
    }
    __syncthreads();
    float dl[kSub], gg[kSub];
#pragma unroll
    for (int tt = 0; tt < kSub; ++tt) {
      dl[tt] = 0.f;
      gg[tt] = 0.f;
      if (tt < nt && dvalid) {
        const int64_t row = token_row(tok, ts + tt, gm.L);
        const int64_t off = xbase + row * gm.xst;
        dl[tt] = bf.delta[off];
        gg[tt] = ld(dy, off);
      }
    }
#pragma unroll
    for (int tt = kSub - 1; tt >= 0; --tt) {
      if (tt < nt) {
        const float4 c4 = *reinterpret_cast<const float4*>(&sC[tt][4 * grp]);
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lam = fmaf(cv[j], gg[tt], mu[j]);
          mu[j] = fast_exp2(dl[tt] * a2[j]) * lam;
        }
        dsum += dl[tt];
      }
    }
  }
  if (dvalid) {
    const int64_t slot = (bk * gm.nchunk + chunk) * gm.D + d;
    *reinterpret_cast<float4*>(bf.agg_mu + slot * kStatePad + 4 * grp) =
        make_float4(mu[0], mu[1], mu[2], mu[3]);
    if (grp == 0) bf.agg_s[slot] = dsum;
  }
}

// Pass 2: fold adjoint aggregates right to left; agg_mu[c] becomes the mu
// entering chunk c's last position.
__global__ void __launch_bounds__(kThreads)
scan_bwd_carry_kernel(Geom gm, BwdBufs bf) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t total = gm.B * gm.K * gm.D * kStatePad;
  if (idx >= total) return;
  const int n = static_cast<int>(idx % kStatePad);
  const int64_t d = (idx / kStatePad) % gm.D;
  const int64_t bk = idx / (kStatePad * gm.D);
  const int64_t k = bk % gm.K;
  const float a2 = n < gm.N ? bf.A[(k * gm.D + d) * gm.N + n] * kLog2e : 0.f;
  float carry = 0.f;
  for (int64_t c = gm.nchunk - 1; c >= 0; --c) {
    const int64_t slot = (bk * gm.nchunk + c) * gm.D + d;
    float a = 0.f, s = 0.f;
    if (c >= 1) {
      a = bf.agg_mu[slot * kStatePad + n];
      s = bf.agg_s[slot];
    }
    bf.agg_mu[slot * kStatePad + n] = carry;
    carry = fmaf(fast_exp2(a2 * s), carry, a);
  }
}

// Pass 3: the reverse sweep.
template <typename XT, typename OT>
__global__ void __launch_bounds__(kThreads)
scan_bwd_kernel(Geom gm, BwdBufs bf) {
  __shared__ float sBC[2][kSub][kStatePad];
  __shared__ float sRed[4][kSub][2][kStatePad];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = lane & 3;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kChPerBlock + wave * kChPerWave + (lane >> 2);
  const bool dvalid = d < gm.D;
  const int64_t dc = dvalid ? d : 0;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / gm.K;
  const int64_t k = bk - b * gm.K;
  const int64_t chunk = blockIdx.z;
  const int64_t t0 = chunk * gm.chunk_len;
  const int64_t t1 = min(gm.L, t0 + gm.chunk_len);
  const int32_t* tok = gm.tok ? gm.tok + k * gm.L : nullptr;
  const int64_t xbase = b * gm.xsb + k * gm.xsk + dc;
  const int64_t bcbase = b * gm.bsb + k * gm.bsk;

  const XT* __restrict__ u = static_cast<const XT*>(bf.u);
  const XT* __restrict__ Bm = static_cast<const XT*>(bf.Bm);
  const XT* __restrict__ Cm = static_cast<const XT*>(bf.Cm);
  const XT* __restrict__ dy = static_cast<const XT*>(bf.dy);
  OT* __restrict__ du_out = static_cast<OT*>(bf.du);

  float a2[4], an[4], mu[4];
  double dacc[4];
  const int64_t slot = (bk * gm.nchunk + chunk) * gm.D + dc;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = 4 * grp + j;
    an[j] = (dvalid && n < gm.N) ? bf.A[(k * gm.D + d) * gm.N + n] : 0.f;
    a2[j] = an[j] * kLog2e;
    mu[j] = 0.f;
    dacc[j] = 0.0;
  }
  if (chunk + 1 < gm.nchunk && dvalid) {
    const float4 m4 = *reinterpret_cast<const float4*>(bf.agg_mu + slot * kStatePad + 4 * grp);
    mu[0] = m4.x; mu[1] = m4.y; mu[2] = m4.z; mu[3] = m4.w;
  }
  const float dskip = dvalid ? bf.Dv[k * gm.D + d] : 0.f;
  double dDacc = 0.0;
  // lanes whose (channel-sum) result they publish: one per (g, j)
  const int red_j = (lane >> 4) & 3;
  const bool red_writer = ((lane >> 2) & 3) == 0;

  const int64_t ntile = (t1 - t0 + kSub - 1) / kSub;
  for (int64_t it = ntile - 1; it >= 0; --it) {
    const int64_t ts = t0 + it * kSub;
    const int nt = static_cast<int>(min<int64_t>(kSub, t1 - ts));
    __syncthreads();  // previous tile's LDS readers are done
    for (int i = tid; i < 2 * kSub * kStatePad; i += kThreads) {
      const int which = i / (kSub * kStatePad);
      const int tt = (i / kStatePad) % kSub;
      const int n = i % kStatePad;
      float v = 0.f;
      if (tt < nt && n < gm.N) {
        const int64_t row = token_row(tok, ts + tt, gm.L);
        v = ld(which ? Cm : Bm, bcbase + row * gm.bst + n);
      }
      sBC[which][tt][n] = v;
    }
    __syncthreads();

    float uu[kSub], dl[kSub], gg[kSub];
#pragma unroll
    for (int tt = 0; tt < kSub; ++tt) {
      uu[tt] = 0.f;
      dl[tt] = 0.f;
      gg[tt] = 0.f;
      if (tt < nt && dvalid) {
        const int64_t row = token_row(tok, ts + tt, gm.L);
        const int64_t off = xbase + row * gm.xst;
        uu[tt] = ld(u, off);
        dl[tt] = bf.delta[off];
        gg[tt] = ld(dy, off);
      }
    }

    // states entering the tile: the checkpoint after position ts-1
    float hs[kSub + 1][4];
    if (ts > 0 && dvalid) {
      const float4 h4 = *reinterpret_cast<const float4*>(
          bf.ckpt + ((bk * gm.nsub + ts / kSub - 1) * gm.D + d) * kStatePad + 4 * grp);
      hs[0][0] = h4.x; hs[0][1] = h4.y; hs[0][2] = h4.z; hs[0][3] = h4.w;
    } else {
      hs[0][0] = hs[0][1] = hs[0][2] = hs[0][3] = 0.f;
    }
    float ea[kSub][4];
    // per-tile partial sums of dA / dD, added to the running totals once per
    // tile (keeps fp32 rounding growth ~ tile + tiles, not chunk length)
    float tacc[4] = {0.f, 0.f, 0.f, 0.f};
    float tD = 0.f;
#pragma unroll
    for (int tt = 0; tt < kSub; ++tt) {
      const float4 b4 = *reinterpret_cast<const float4*>(&sBC[0][tt][4 * grp]);
      const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
      const float dxu = dl[tt] * uu[tt];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ea[tt][j] = fast_exp2(dl[tt] * a2[j]);
        hs[tt + 1][j] = fmaf(ea[tt][j], hs[tt][j], dxu * bv[j]);
      }
    }

#pragma unroll
    for (int tt = kSub - 1; tt >= 0; --tt) {
      if (tt < nt) {
        const float4 b4 = *reinterpret_cast<const float4*>(&sBC[0][tt][4 * grp]);
        const float4 c4 = *reinterpret_cast<const float4*>(&sBC[1][tt][4 * grp]);
        const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
        const float dxu = dl[tt] * uu[tt];
        float sa = 0.f, sb = 0.f;
        float xb[4], xc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lam = fmaf(cv[j], gg[tt], mu[j]);
          const float q = lam * ea[tt][j];
          const float w = q * hs[tt][j];
          sa = fmaf(w, an[j], sa);
          tacc[j] = fmaf(w, dl[tt], tacc[j]);
          sb = fmaf(lam, bv[j], sb);
          xb[j] = lam * dxu;
          xc[j] = gg[tt] * hs[tt + 1][j];
          mu[j] = q;
        }
        sa = sum_groups(sa);
        sb = sum_groups(sb);
        tD = fmaf(gg[tt], uu[tt], tD);
        if (grp == 0 && dvalid) {
          const int64_t row = token_row(tok, ts + tt, gm.L);
          const int64_t off = xbase + row * gm.xst;
          st(du_out, off, fmaf(dl[tt], sb, dskip * gg[tt]));
          bf.ddelta[off] = fmaf(uu[tt], sb, sa);
        }
        const float rb = channel_reduce4(xb[0], xb[1], xb[2], xb[3]);
        const float rc = channel_reduce4(xc[0], xc[1], xc[2], xc[3]);
        if (red_writer) {
          sRed[wave][tt][0][4 * grp + red_j] = rb;
          sRed[wave][tt][1][4 * grp + red_j] = rc;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) dacc[j] += static_cast<double>(tacc[j]);
    dDacc += static_cast<double>(tD);
    __syncthreads();
    // sum the 4 waves and publish this channel block's dB | dC partials
    for (int i = tid; i < nt * 2 * kStatePad; i += kThreads) {
      const int tt = i / (2 * kStatePad);
      const int w2 = (i / kStatePad) & 1;
      const int n = i % kStatePad;
      const float s = (sRed[0][tt][w2][n] + sRed[1][tt][w2][n]) + (sRed[2][tt][w2][n] + sRed[3][tt][w2][n]);
      bf.part_bc[((bk * gm.ncblk + blockIdx.x) * gm.L + ts + tt) * (2 * kStatePad) + w2 * kStatePad + n] = s;
    }
  }

  if (dvalid) {
    double* pa = bf.part_dA + slot * kStatePad + 4 * grp;
#pragma unroll
    for (int j = 0; j < 4; ++j) pa[j] = dacc[j];
    if (grp == 0) bf.part_dD[slot] = dDacc;
  }
}

// dB / dC: sum the channel-block partials in a fixed order and store at the
// token row each scan position read (mamba_metal_fused.py:221,224).
template <typename OT>
__global__ void __launch_bounds__(kThreads)
reduce_bc_kernel(Geom gm, BwdBufs bf) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t total = gm.B * gm.K * gm.L * 2 * kStatePad;
  if (idx >= total) return;
  const int n = static_cast<int>(idx % kStatePad);
  const int w2 = static_cast<int>((idx / kStatePad) & 1);
  const int64_t t = (idx / (2 * kStatePad)) % gm.L;
  const int64_t bk = idx / (2 * kStatePad * gm.L);
  if (n >= gm.N) return;
  float s = 0.f;
  for (int64_t cb = 0; cb < gm.ncblk; ++cb)
    s += bf.part_bc[((bk * gm.ncblk + cb) * gm.L + t) * (2 * kStatePad) + w2 * kStatePad + n];
  const int64_t b = bk / gm.K, k = bk % gm.K;
  const int64_t row = token_row(gm.tok ? gm.tok + k * gm.L : nullptr, t, gm.L);
  OT* out = static_cast<OT*>(w2 ? bf.dC : bf.dB);
  st(out, b * gm.bsb + k * gm.bsk + row * gm.bst + n, s);
}

// dA (K, D, N) and dD (K, D): sum per-(b, chunk) partials in a fixed order
// (mamba_metal_fused.py:214,218).
__global__ void __launch_bounds__(kThreads)
reduce_ad_kernel(Geom gm, BwdBufs bf) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t nA = gm.K * gm.D * kStatePad;
  if (idx < nA) {
    const int n = static_cast<int>(idx % kStatePad);
    const int64_t d = (idx / kStatePad) % gm.D;
    const int64_t k = idx / (kStatePad * gm.D);
    if (n >= gm.N) return;
    double s = 0.0;
    for (int64_t b = 0; b < gm.B; ++b)
      for (int64_t c = 0; c < gm.nchunk; ++c)
        s += bf.part_dA[(((b * gm.K + k) * gm.nchunk + c) * gm.D + d) * kStatePad + n];
    bf.dA[(k * gm.D + d) * gm.N + n] = static_cast<float>(s);
  } else if (idx < nA + gm.K * gm.D) {
    const int64_t i = idx - nA;
    const int64_t d = i % gm.D;
    const int64_t k = i / gm.D;
    double s = 0.0;
    for (int64_t b = 0; b < gm.B; ++b)
      for (int64_t c = 0; c < gm.nchunk; ++c)
        s += bf.part_dD[((b * gm.K + k) * gm.nchunk + c) * gm.D + d];
    bf.dD[k * gm.D + d] = static_cast<float>(s);
  }
}

template <typename XT, typename OT>
static hipError_t launch_bwd_t(const Geom& g, const BwdBufs& b, hipStream_t s) {
  const dim3 block(kThreads);
  const int64_t tot_state = g.B * g.K * g.D * kStatePad;
  if (g.nchunk > 1) {
    const dim3 grid_agg(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                        static_cast<unsigned>(g.nchunk - 1));
    hipLaunchKernelGGL((scan_bwd_agg_kernel<XT>), grid_agg, block, 0, s, g, b);
    hipLaunchKernelGGL(scan_bwd_carry_kernel, dim3(static_cast<unsigned>((tot_state + kThreads - 1) / kThreads)),
                       block, 0, s, g, b);
  }
  const dim3 grid(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                  static_cast<unsigned>(g.nchunk));
  hipLaunchKernelGGL((scan_bwd_kernel<XT, OT>), grid, block, 0, s, g, b);
  const int64_t nbc = g.B * g.K * g.L * 2 * kStatePad;
  hipLaunchKernelGGL((reduce_bc_kernel<OT>), dim3(static_cast<unsigned>((nbc + kThreads - 1) / kThreads)),
                     block, 0, s, g, b);
  const int64_t nad = g.K * g.D * (kStatePad + 1);
  hipLaunchKernelGGL(reduce_ad_kernel, dim3(static_cast<unsigned>((nad + kThreads - 1) / kThreads)),
                     block, 0, s, g, b);
  return hipGetLastError();
}

hipError_t launch_bwd(const Geom& g, const BwdBufs& b, int in_dtype, int out_dtype, hipStream_t s) {
  if (in_dtype == 0 && out_dtype == 0) return launch_bwd_t<float, float>(g, b, s);
  if (in_dtype == 1 && out_dtype == 1) return launch_bwd_t<bf16_t, bf16_t>(g, b, s);
  if (in_dtype == 1 && out_dtype == 0) return launch_bwd_t<bf16_t, float>(g, b, s);
  return launch_bwd_t<float, bf16_t>(g, b, s);
}

// --------------------------------------------------------------- utilities

__global__ void __launch_bounds__(kThreads) fill_kernel(float* p, int64_t n, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) p[i] = v;
}

hipError_t launch_fill(float* p, int64_t n, float v, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, s, p, n, v);
  return hipGetLastError();
}

// Lane-layout check of the cross-lane helpers: one wave, lane l holds
// x_j = 1000*j + l for j = 0..3.  out[0..63]: sum_groups(x_0);
// out[64..127]: channel_reduce4(x_0..x_3).
__global__ void __launch_bounds__(64) selftest_lanes_kernel(float* out) {
  const int l = threadIdx.x;
  const float x0 = static_cast<float>(l), x1 = 1000.f + l, x2 = 2000.f + l, x3 = 3000.f + l;
  out[l] = sum_groups(x0);
  out[64 + l] = channel_reduce4(x0, x1, x2, x3);
}

hipError_t launch_selftest_lanes(float* out, hipStream_t s) {
  hipLaunchKernelGGL(selftest_lanes_kernel, dim3(1), dim3(64), 0, s, out);
  return hipGetLastError();
}

}  // namespace mvm
