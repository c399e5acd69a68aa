// Forward selective scan for gfx950 (MI355X).
//
// Math (mamba_block.py:45-74; fused form mamba_metal_fused.py:21-63):
//   h_t = exp(delta_t * A) * h_{t-1} + delta_t * B_t * u_t,   h_{-1} = 0
//   y_t = sum_n C_t[n] * h_t[n] + D * u_t
//
// Work split.  Lane (c, g) of a wave owns states 4g..4g+3 of one channel
// (scan_common.h).  A 256-thread workgroup covers 64 channels of one
// (batch, direction) pair and one time chunk.  Per 16-step tile the
// workgroup stages B_t / C_t (shared by all its channels) in LDS, converted
// to fp32 once; u and delta are read straight from HBM, channel-contiguous.
//
// Long sequences are split into time chunks so that the grid fills the
// chip (the two-pass scheme whose carry step the reference left as TODO at
// mamba_metal_chunked.py:268-272):
//   pass 1 (kAgg)    each chunk scans from h = 0 and writes its end state
//                    and sum(delta) (the chunk's decay is exp(A*sum(delta)));
//   pass 2 (carry)   one thread per (b, k, d, n) folds the aggregates in
//                    order: H_c = exp(A*S_c) * H_{c-1} + e_c (mamba_fast.py:85-86);
//   pass 3 (kMain)   each chunk rescans from its carry-in, writes y and,
//                    when training, the state after every 16th position
//                    (the backward's checkpoints).
#include "scan_common.h"
#include "scan_kernels.h"

namespace mvm {

enum FwdMode { kAgg = 0, kMain = 1 };

template <typename XT, typename OT, int MODE>
__global__ void __launch_bounds__(kThreads)
scan_fwd_kernel(Geom gm, FwdBufs bf) {
  __shared__ float sBC[2][kSub][kStatePad];

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
  const float* __restrict__ delta = bf.delta;
  const XT* __restrict__ Bm = static_cast<const XT*>(bf.Bm);
  const XT* __restrict__ Cm = static_cast<const XT*>(bf.Cm);
  OT* __restrict__ y = static_cast<OT*>(bf.y);

  float a2[4], h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = 4 * grp + j;
    a2[j] = (dvalid && n < gm.N) ? bf.A[(k * gm.D + d) * gm.N + n] * kLog2e : 0.f;
    h[j] = 0.f;
  }
  const float dskip = (MODE == kMain && dvalid) ? bf.Dv[k * gm.D + d] : 0.f;
  const int64_t slot = (bk * gm.nchunk + chunk) * gm.D + dc;  // (bk, chunk, d)
  if (MODE == kMain && chunk > 0 && dvalid) {
    const float4 c4 = *reinterpret_cast<const float4*>(bf.agg_h + slot * kStatePad + 4 * grp);
    h[0] = c4.x; h[1] = c4.y; h[2] = c4.z; h[3] = c4.w;
  }
  float dsum = 0.f;

  for (int64_t ts = t0; ts < t1; ts += kSub) {
    const int nt = static_cast<int>(min<int64_t>(kSub, t1 - ts));
    __syncthreads();  // the previous tile's LDS readers are done
    constexpr int kStage = (MODE == kMain ? 2 : 1) * kSub * kStatePad;
    for (int i = tid; i < kStage; i += kThreads) {
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

    float uu[kSub], dl[kSub];
#pragma unroll
    for (int tt = 0; tt < kSub; ++tt) {
      uu[tt] = 0.f;
      dl[tt] = 0.f;
      if (tt < nt && dvalid) {
        const int64_t row = token_row(tok, ts + tt, gm.L);
        const int64_t off = xbase + row * gm.xst;
        uu[tt] = ld(u, off);
        dl[tt] = delta[off];
      }
    }

#pragma unroll
    for (int tt = 0; tt < kSub; ++tt) {
      if (tt < nt) {
        const float4 b4 = *reinterpret_cast<const float4*>(&sBC[0][tt][4 * grp]);
        const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
        const float du = dl[tt] * uu[tt];
        float yp = 0.f;
        float cv[4] = {0.f, 0.f, 0.f, 0.f};
        if (MODE == kMain) {
          const float4 c4 = *reinterpret_cast<const float4*>(&sBC[1][tt][4 * grp]);
          cv[0] = c4.x; cv[1] = c4.y; cv[2] = c4.z; cv[3] = c4.w;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = fast_exp2(dl[tt] * a2[j]);
          h[j] = fmaf(e, h[j], du * bv[j]);
          if (MODE == kMain) yp = fmaf(cv[j], h[j], yp);
        }
        if (MODE == kAgg) dsum += dl[tt];
        if (MODE == kMain) {
          yp = sum_groups(yp);
          if (y != nullptr && grp == 0 && dvalid) {
            const int64_t row = token_row(tok, ts + tt, gm.L);
            st(y, xbase + row * gm.xst, fmaf(dskip, uu[tt], yp));
          }
        }
      }
    }
    if (MODE == kMain && bf.ckpt != nullptr && dvalid) {
      float4 c4 = make_float4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<float4*>(bf.ckpt + ((bk * gm.nsub + ts / kSub) * gm.D + d) * kStatePad +
                                 4 * grp) = c4;
    }
  }

  if (MODE == kAgg && dvalid) {
    *reinterpret_cast<float4*>(bf.agg_h + slot * kStatePad + 4 * grp) =
        make_float4(h[0], h[1], h[2], h[3]);
    if (grp == 0) bf.agg_s[slot] = dsum;
  }
}

// Pass 2: fold chunk aggregates left to right; agg_h[c] becomes chunk c's
// carry-in (the state after the last position of chunk c-1).
__global__ void __launch_bounds__(kThreads)
scan_fwd_carry_kernel(Geom gm, FwdBufs bf) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t total = gm.B * gm.K * gm.D * kStatePad;
  if (idx >= total) return;
  const int n = static_cast<int>(idx % kStatePad);
  const int64_t d = (idx / kStatePad) % gm.D;
  const int64_t bk = idx / (kStatePad * gm.D);
  const int64_t k = bk % gm.K;
  const float a2 = n < gm.N ? bf.A[(k * gm.D + d) * gm.N + n] * kLog2e : 0.f;
  float carry = 0.f;
  for (int64_t c = 0; c < gm.nchunk; ++c) {
    const int64_t slot = (bk * gm.nchunk + c) * gm.D + d;
    float e = 0.f, s = 0.f;
    if (c + 1 < gm.nchunk) {
      e = bf.agg_h[slot * kStatePad + n];
      s = bf.agg_s[slot];
    }
    bf.agg_h[slot * kStatePad + n] = carry;
    carry = fmaf(fast_exp2(a2 * s), carry, e);
  }
}

template <typename XT, typename OT>
static hipError_t launch_fwd_t(const Geom& g, const FwdBufs& b, hipStream_t s) {
  const dim3 block(kThreads);
  if (g.nchunk > 1) {
    const dim3 grid_agg(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                        static_cast<unsigned>(g.nchunk - 1));
    hipLaunchKernelGGL((scan_fwd_kernel<XT, OT, kAgg>), grid_agg, block, 0, s, g, b);
    const int64_t total = g.B * g.K * g.D * kStatePad;
    hipLaunchKernelGGL(scan_fwd_carry_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                       block, 0, s, g, b);
  }
  const dim3 grid(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                  static_cast<unsigned>(g.nchunk));
  hipLaunchKernelGGL((scan_fwd_kernel<XT, OT, kMain>), grid, block, 0, s, g, b);
  return hipGetLastError();
}

hipError_t launch_fwd(const Geom& g, const FwdBufs& b, int in_dtype, int out_dtype, hipStream_t s) {
  if (in_dtype == 0 && out_dtype == 0) return launch_fwd_t<float, float>(g, b, s);
  if (in_dtype == 1 && out_dtype == 1) return launch_fwd_t<bf16_t, bf16_t>(g, b, s);
  if (in_dtype == 1 && out_dtype == 0) return launch_fwd_t<bf16_t, float>(g, b, s);
  return launch_fwd_t<float, bf16_t>(g, b, s);
}

}  // namespace mvm
