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
// sweep runs over the registers.  Inputs are staged tile by tile through
// double-buffered LDS with coalesced loads issued one tile ahead; du, ddelta
// and the dB | dC partials leave through LDS as coalesced rows.
//
// Reductions are atomic-free and in a fixed order (bitwise deterministic):
//   dB, dC   sum over 16 channels per wave with cross-lane ops, over the 4
//            waves in LDS, then over channel blocks in reduce_grads_kernel;
//   dA, dD   per-lane float32 sums over each 16-step tile, folded into
//            float64 running sums (a long chunk of unit-size terms can
//            cancel to ~1e-3, far below float32 running-sum error), float64
//            partials per (b, chunk), summed in float64 by reduce_grads_kernel.
// Long sequences: the adjoint carry between time chunks uses the same
// two-pass idea as the forward, run right to left: scan_bwd_agg_kernel
// writes each chunk's adjoint aggregate; they are folded by each chunk of
// the sweep itself (up to kFoldMax chunks) or by scan_bwd_carry_kernel.
//
// Fused form (FUSE, float32): delta = softplus(delta_raw + dt_bias) is
// applied as the delta tile is staged; the stored gradient is that of
// delta_raw, ddelta * sigmoid(delta_raw + dt_bias), the sigmoid formed from
// the softplus' own exponential when the tile is staged and kept in LDS
// until the tile is flushed; dt_bias's gradient is its sum
// over (b, t), reduced like dD.  The gate y = y_raw * silu(z) is undone as
// the upstream gradient is staged: the scan consumes g = dy * silu(z), and
// dz = dy * y_raw * silu'(z) is written from the same registers, so the
// gate's backward makes no pass of its own.
#include <type_traits>

#include "scan_common.h"
#include "scan_kernels.h"

namespace mvm {

// Pass 1: adjoint aggregate of chunks 1..nchunk-1: the mu that leaves the
// chunk's first position when mu = 0 enters its last, and sum(delta).
template <typename XT, bool FUSE, bool TOK, typename IdxT>
__global__ void __launch_bounds__(kThreads)
scan_bwd_agg_kernel(Geom gm, BwdBufs bf) {
  __shared__ float sX[2][2][kSub][kChPerBlock];  // delta, dy: one array (shared addresses)
  __shared__ float sC[2][kSub][kStatePad];
  float (*const sD)[kSub][kChPerBlock] = sX[0];
  float (*const sG)[kSub][kChPerBlock] = sX[1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = lane & 3;
  const int cl = wave * kChPerWave + (lane >> 2);
  const int64_t ch0 = static_cast<int64_t>(blockIdx.x) * kChPerBlock;
  const int64_t d = ch0 + cl;
  const int64_t dld = ch0 + lane;
  const bool dvalid = d < gm.D;
  const bool cok = dld < gm.D;
  const bool all_in = ch0 + kChPerBlock <= gm.D;  // block-uniform: no channel masked
  const int lc = cok ? lane : 0;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / gm.K;
  const int64_t k = bk - b * gm.K;
  const int64_t chunk = blockIdx.z + 1;
  const int32_t L = static_cast<int32_t>(gm.L);
  const int N = static_cast<int>(gm.N);
  const int32_t t0 = static_cast<int32_t>(chunk * gm.chunk_len);
  // the chunk's end in 64 bits: t0 + chunk_len may pass 2^31 - 1 in the last chunk
  const int32_t t1 = static_cast<int32_t>(min<int64_t>(gm.L, (chunk + 1) * gm.chunk_len));
  const int32_t* tok = TOK ? gm.tok + k * gm.L : nullptr;
  const float* __restrict__ delta = bf.delta + (b * gm.dsb + k * gm.dsk + ch0);
  const XT* __restrict__ dy = static_cast<const XT*>(bf.dy) + (b * gm.ysb + k * gm.ysk + ch0);
  const XT* __restrict__ Cm = static_cast<const XT*>(bf.Cm) + (b * gm.bsb + k * gm.bsk);
  const IdxT sd = static_cast<IdxT>(gm.dst), sy = static_cast<IdxT>(gm.yst);
  const IdxT sz = static_cast<IdxT>(gm.zst), sbc = static_cast<IdxT>(gm.bst);
  const float dbias_l = (FUSE && bf.dbias != nullptr && cok) ? bf.dbias[k * gm.D + dld] : 0.f;
  auto stage_delta = [&](float (&v)[4]) {
    if (FUSE) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = softplus_f(v[r] + dbias_l);
    }
  };
  // fused gate: the scan's upstream gradient is dy * silu(z)
  const bool gate = FUSE && bf.z != nullptr;
  const float* __restrict__ zin = gate ? bf.z + (b * gm.zsb + k * gm.zsk + ch0) : nullptr;
  float pz[4] = {0.f, 0.f, 0.f, 0.f};
  auto stage_g = [&](float (&gv)[4]) {
    if (gate) {
#pragma unroll
      for (int r = 0; r < 4; ++r) gv[r] *= pz[r] * sigmoid_f(pz[r]);
    }
  };

  float a2[4], mu[4];
  load_ax4(a2, bf.A, (k * gm.D + (dvalid ? d : 0)) * gm.N, grp, N, dvalid, gm.a_log);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a2[j] *= kLog2e;
    mu[j] = 0.f;
  }
  float dsum = 0.f;
  const int32_t ntile = (t1 - t0 + kSub - 1) / kSub;
  float pd[4], pg[4], pc;
  auto load_tile = [&](int32_t ts) {
    const TileRows rows = tile_rows<TOK>(tok, ts, L, tid);
    load_rows(pd, delta, rows, sd, lc);
    load_rows(pg, dy, rows, sy, lc);
    if (gate) load_rows(pz, zin, rows, sz, lc);
    pc = load_state(Cm, rows, sbc, N, tid);
  };
  auto store_tile = [&](int buf) {
    mask_xtile(pd, cok, all_in);
    mask_xtile(pg, cok, all_in);
    if (gate) mask_xtile(pz, cok, all_in);
    pc = mask_stile(pc, N, tid);
    stage_delta(pd);
    stage_g(pg);
    store_xtile(sD[buf], pd, tid);
    store_xtile(sG[buf], pg, tid);
    sC[buf][stile_row(tid)][tid & 15] = pc;
  };
  load_tile(t0 + (ntile - 1) * kSub);
  store_tile(0);
  for (int32_t j = 0; j < ntile; ++j) {
    const int buf = j & 1;
    const int32_t ts = t0 + (ntile - 1 - j) * kSub;
    const int nt = min(kSub, t1 - ts);
    __syncthreads();
    const bool more = j + 1 < ntile;
    if (more) load_tile(ts - kSub);
#pragma unroll
    for (int tt = kSub - 1; tt >= 0; --tt) {
      if (tt < nt) {
        const float dl = sD[buf][tt][cl];
        const float gy = sG[buf][tt][cl];
        const float4 c4 = *reinterpret_cast<const float4*>(&sC[buf][tt][4 * grp]);
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float lam = fmaf(cv[jj], gy, mu[jj]);
          mu[jj] = fast_exp2(dl * a2[jj]) * lam;
        }
        dsum += dl;
      }
    }
    if (more) store_tile(buf ^ 1);
  }
  if (dvalid) {
    const int64_t slot = (bk * gm.nchunk + chunk) * gm.D + d;
    *reinterpret_cast<float4*>(bf.agg_mu + slot * kStatePad + 4 * grp) =
        make_float4(mu[0], mu[1], mu[2], mu[3]);
    if (grp == 0) bf.agg_s[slot] = dsum;
  }
}

// Carry pass for many chunks: agg_mu[c] becomes the adjoint entering chunk
// c's last position, folded right to left, one thread per (b, k, d, n).
__global__ void __launch_bounds__(kThreads)
scan_bwd_carry_kernel(Geom gm, BwdBufs bf) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t total = gm.B * gm.K * gm.D * kStatePad;
  if (idx >= total) return;
  const int n = static_cast<int>(idx % kStatePad);
  const int64_t d = (idx / kStatePad) % gm.D;
  const int64_t bk = idx / (kStatePad * gm.D);
  const int64_t k = bk % gm.K;
  const float a2 = n < gm.N ? load_A(bf.A, (k * gm.D + d) * gm.N + n, gm.a_log) * kLog2e : 0.f;
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

// Pass 2: the reverse sweep.  Each 16-step tile is processed as two 8-step
// halves (later half first), each restarted from its checkpoint, so the
// register tile is 9 x 4 states + 8 x 4 decays.  IdxT is the row-offset
// type (see scan_common.h).
//
// Two resident-wave budgets.  The plain 32-bit-offset sweep (the long
// sequences) is built lean for 3 waves per SIMD (<= 168 VGPRs): its float64
// dA / dD sums live in LDS, its per-wave dB | dC channel sums are single-
// buffered (summed right after the tile's second barrier), delta * u and A
// are re-formed where they are used, and the next tile's two checkpoints are
// loaded one half-sweep apart.  The fused sweep (the block's scan, with the
// softplus / gate gradients) and the 64-bit-offset sweep hold more state and
// run at 2 waves per SIMD, where those trades cost more than they return.
template <bool FUSE, typename IdxT>
constexpr bool bwd_lean() {
  return !FUSE && std::is_same<IdxT, int32_t>::value;
}
template <typename XT, typename OT, bool FUSE, bool TOK, bool FOLD, typename IdxT>
__global__ void __launch_bounds__(kThreads, (bwd_lean<FUSE, IdxT>() ? 3 : 2))
scan_bwd_kernel(Geom gm, BwdBufs bf) {
  constexpr bool kLean = bwd_lean<FUSE, IdxT>();
  // double-buffered tile staging (u, delta, dy, B, C); du / ddelta are
  // written in place over u / dy of the same step once it is consumed (delta
  // stays for the fused softplus gradient); per-wave channel sums of dB | dC
  // (one buffer when lean); lean: each thread's float64 dA (4 states) and dD
  // running sums
  // one array, so that the three tiles sit at fixed distances: a thread's
  // accesses to its slot in all three share one address (immediate offsets)
  __shared__ float sX[3][2][kSub][kChPerBlock];
  __shared__ float sBC[2][2][kSub][kStatePad];
  float (*const sU)[kSub][kChPerBlock] = sX[0];
  float (*const sD)[kSub][kChPerBlock] = sX[1];
  float (*const sG)[kSub][kChPerBlock] = sX[2];
  float (*const sB)[kSub][kStatePad] = sBC[0];
  float (*const sC)[kSub][kStatePad] = sBC[1];
  __shared__ float sRed[kLean ? 1 : 2][4][kSub][2][kStatePad];
  __shared__ double sAcc[5][kLean ? kThreads : 1];
  __shared__ double sDb[4][kChPerBlock];  // fused: per-wave dt_bias gradient sums
  // fused: sigmoid(delta_raw + dt_bias) of the staged tile, the softplus
  // derivative applied to ddelta when the tile is flushed
  __shared__ float sSg[FUSE ? 2 : 1][FUSE ? kSub : 1][kChPerBlock];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = lane & 3;
  const int cl = wave * kChPerWave + (lane >> 2);
  const int64_t ch0 = static_cast<int64_t>(blockIdx.x) * kChPerBlock;
  const int64_t d = ch0 + cl;
  const int64_t dld = ch0 + lane;
  const bool dvalid = d < gm.D;
  const bool cok = dld < gm.D;
  const bool all_in = ch0 + kChPerBlock <= gm.D;  // block-uniform: no channel masked
  const int64_t dc = dvalid ? d : 0;
  const int lc = cok ? lane : 0;  // channel this thread stages / flushes (0 when out of range)
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / gm.K;
  const int64_t k = bk - b * gm.K;
  const int64_t chunk = blockIdx.z;
  const int32_t L = own_sc(static_cast<int32_t>(gm.L));
  const int N = own_sc(static_cast<int>(gm.N));
  const int32_t t0 = own_sc(static_cast<int32_t>(chunk * gm.chunk_len));
  // the chunk's end in 64 bits: t0 + chunk_len may pass 2^31 - 1 in the last chunk
  const int32_t t1 = own_sc(static_cast<int32_t>(min<int64_t>(gm.L, (chunk + 1) * gm.chunk_len)));
  const int32_t* tok = TOK ? own_ptr(gm.tok + k * gm.L) : nullptr;
  // the block's first channel of its (b, k) slab in every tensor, and the
  // row strides in IdxT
  const XT* __restrict__ u = own_ptr(static_cast<const XT*>(bf.u) + (b * gm.xsb + k * gm.xsk + ch0));
  const float* __restrict__ delta = own_ptr(bf.delta + (b * gm.dsb + k * gm.dsk + ch0));
  const XT* __restrict__ dy = own_ptr(static_cast<const XT*>(bf.dy) + (b * gm.ysb + k * gm.ysk + ch0));
  OT* __restrict__ du_out = own_ptr(static_cast<OT*>(bf.du) + (b * gm.xsb + k * gm.xsk + ch0));
  float* __restrict__ dd_out = own_ptr(bf.ddelta + (b * gm.dsb + k * gm.dsk + ch0));
  const XT* __restrict__ Bm = own_ptr(static_cast<const XT*>(bf.Bm) + (b * gm.bsb + k * gm.bsk));
  const XT* __restrict__ Cm = own_ptr(static_cast<const XT*>(bf.Cm) + (b * gm.bsb + k * gm.bsk));
  const IdxT sx = own_sc(static_cast<IdxT>(gm.xst)), sd = own_sc(static_cast<IdxT>(gm.dst));
  const IdxT sy = own_sc(static_cast<IdxT>(gm.yst)), sz = own_sc(static_cast<IdxT>(gm.zst));
  const IdxT sbc = own_sc(static_cast<IdxT>(gm.bst));

  // an = A (unused when lean: the sweep sums w * A * log2(e) and scales the
  // sum by ln 2 instead), a2 = A * log2(e)
  float a2[4], an[4], mu[4];
  double dacc[4], dDacc = 0.0;  // not lean: float64 dA / dD running sums
  const int64_t slot = (bk * gm.nchunk + chunk) * gm.D + dc;
  // the lean sweep issues the 4 A loads together; the 2-wave forms keep the
  // per-state loads, with which their scalar registers fit without spills
  if constexpr (kLean) {
    load_ax4(an, bf.A, (k * gm.D + dc) * gm.N, grp, N, dvalid, gm.a_log);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 4 * grp + j;
      an[j] = (dvalid && n < N) ? load_A(bf.A, (k * gm.D + d) * gm.N + n, gm.a_log) : 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a2[j] = an[j] * kLog2e;
    mu[j] = 0.f;
    dacc[j] = 0.0;
  }
  if constexpr (kLean) {
#pragma unroll
    for (int j = 0; j < 5; ++j) sAcc[j][tid] = 0.0;
  }
  if (chunk + 1 < gm.nchunk && dvalid) {
    if constexpr (FOLD) {
      // adjoint carry-in: fold the aggregates of chunks nchunk-1 .. chunk+1
      // right to left, mu = exp(A * S_c) * mu + M_c.  In the 32-bit form
      // all of them (at most kFoldMax) are loaded first, from in-bounds
      // chunk indices, so that their latencies overlap; the 64-bit form,
      // short of scalar registers, loads them one at a time.
      const int64_t s0 = bk * gm.nchunk * gm.D + dc;
      if constexpr (std::is_same<IdxT, int32_t>::value) {
        float4 m4[kFoldMax];
        float sdl[kFoldMax];
#pragma unroll
        for (int i = 0; i < kFoldMax; ++i) {
          const int64_t c = gm.nchunk - 1 - i;
          const int64_t sc = s0 + (c >= 0 ? c : 0) * gm.D;
          m4[i] = *reinterpret_cast<const float4*>(bf.agg_mu + sc * kStatePad + 4 * grp);
          sdl[i] = bf.agg_s[sc];
        }
#pragma unroll
        for (int i = 0; i < kFoldMax; ++i) {
          if (gm.nchunk - 1 - i > chunk) {
            const float m[4] = {m4[i].x, m4[i].y, m4[i].z, m4[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) mu[j] = fmaf(fast_exp2(a2[j] * sdl[i]), mu[j], m[j]);
          }
        }
      } else {
        for (int64_t c = gm.nchunk - 1; c > chunk; --c) {
          const int64_t sc = s0 + c * gm.D;
          const float4 m4 = *reinterpret_cast<const float4*>(bf.agg_mu + sc * kStatePad + 4 * grp);
          const float sdl = bf.agg_s[sc];
          const float m[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) mu[j] = fmaf(fast_exp2(a2[j] * sdl), mu[j], m[j]);
        }
      }
    } else {  // folded by scan_bwd_carry_kernel
      const float4 m4 = *reinterpret_cast<const float4*>(bf.agg_mu + slot * kStatePad + 4 * grp);
      mu[0] = m4.x; mu[1] = m4.y; mu[2] = m4.z; mu[3] = m4.w;
    }
  }
  const float dskip = dvalid ? bf.Dv[k * gm.D + d] : 0.f;
  // state j = (lane >> 4) & 3 of the lane's group holds its channel sum
  const int red_j = (lane >> 4) & 3;
  // checkpoint slot s of this lane's channel: float4 (cl * 4 + grp) of row s
  // (stride D * 16 floats) from the block's first channel
  const float4* ckb = own_ptr(reinterpret_cast<const float4*>(bf.ckpt + (bk * gm.nck * gm.D + ch0) * kStatePad));
  const IdxT ck_stride = own_sc(static_cast<IdxT>(gm.D * (kStatePad / 4)));
  // (a lane of a channel past D reads the block's first channel instead:
  // its u and dy are staged as 0, so its state enters no sum and no store)
  const int ck_lane = dvalid ? cl * 4 + grp : grp;
  const uint32_t ck_lane_b = static_cast<uint32_t>(ck_lane) * 16u;

  // state after position p - 1 (checkpoint slot p / 8 - 1), p a multiple of
  // 8; p is block-uniform, so the test is a scalar branch and the load needs
  // no per-lane default
  auto load_ckpt = [&](int32_t p) {
    float4 h4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p > 0) h4 = row_elem(ckb, p / kCk - 1, ck_stride, ck_lane, ck_lane_b);
    return h4;
  };
  // fused: the dt bias of the channel this thread stages / flushes, and its
  // gradient summed over the rows this thread flushes
  const float dbias_l = (FUSE && bf.dbias != nullptr && cok) ? bf.dbias[k * gm.D + dld] : 0.f;
  double dbacc = 0.0;
  // softplus of the staged delta_raw + dt bias, with its sigmoid (the
  // softplus derivative) from the same exponential
  float psg[4];
  auto stage_delta = [&](float (&v)[4]) {
    if (FUSE) {
#pragma unroll
      for (int r = 0; r < 4; ++r) softplus_sigmoid(v[r] + dbias_l, v[r], psg[r]);
    }
  };
  // fused gate: the upstream dy is the gradient of y_raw * silu(z); the scan
  // consumes g = dy * silu(z) and dz = dy * y_raw * silu'(z) leaves from the
  // staging registers of the tile (rows ts + tt, tt = wave + 4r)
  const bool gate = FUSE && bf.z != nullptr;
  const uint32_t lb4 = static_cast<uint32_t>(lc) * 4u;  // byte offset of the lane's channel (fp32)
  const int64_t zoff = b * gm.zsb + k * gm.zsk + ch0;
  const float* __restrict__ zin = gate ? own_ptr(bf.z + zoff) : nullptr;
  float* __restrict__ dz_out = gate ? own_ptr(bf.dz + zoff) : nullptr;
  // (an SGPR base whether or not there is a gate: only read when there is one)
  const float* __restrict__ yraw = own_ptr(bf.y_raw + (gate ? b * gm.ysb + k * gm.ysk + ch0 : 0));
  float pz[4] = {0.f, 0.f, 0.f, 0.f}, pyr[4] = {0.f, 0.f, 0.f, 0.f};
  auto stage_gate = [&](float (&gv)[4], const TileRows& rows, int nt) {
    if (gate) {
      const int wrow = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sg = sigmoid_f(pz[r]);
        const float dzv = gv[r] * pyr[r] * (sg * fmaf(pz[r], 1.f - sg, 1.f));
        gv[r] *= pz[r] * sg;
        const int tt = wrow + 4 * r;
        if (tt < nt && cok) row_elem(dz_out, rows.r[r], sz, lc, lb4) = dzv;
      }
    }
  };
  // this block's dB | dC partial rows: (position, dB|dC, state)
  float* __restrict__ pbc_blk = own_ptr(bf.part_bc + (bk * gm.ncblk + blockIdx.x) * gm.L * (2 * kStatePad));
  // write back the du / ddelta rows of a tile (token rows `rows`)
  auto flush = [&](int buf, const TileRows& rows, int nt) {
    const int wrow = __builtin_amdgcn_readfirstlane(wave);
    float dbt = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tt = wrow + 4 * r;
      if (tt < nt) {
        // values first (no divergent branch); only the stores are masked
        const int32_t row = rows.r[r];
        const float duv = sU[buf][tt][lane];
        float dd = sG[buf][tt][lane];
        if (FUSE) {
          dd *= sSg[buf][tt][lane];
          dbt += cok ? dd : 0.f;
        }
        if (cok) {
          row_elem(du_out, row, sx, lc, static_cast<uint32_t>(lc * sizeof(OT))) = from_f32<OT>(duv);
          row_elem(dd_out, row, sd, lc, lb4) = dd;
        }
      }
    }
    if (FUSE) dbacc += static_cast<double>(dbt);
  };
  // this block's dB | dC partials of a tile: the 4 waves' channel sums in
  // sRed[rb], added in a fixed order
  auto flush_red = [&](int rb, int32_t ts, int nt) {
    for (int i = tid; i < nt * 2 * kStatePad; i += kThreads) {
      const int tt = i / (2 * kStatePad);
      const int w2 = (i / kStatePad) & 1;
      const int n = i % kStatePad;
      const float v = (sRed[rb][0][tt][w2][n] + sRed[rb][1][tt][w2][n]) +
                      (sRed[rb][2][tt][w2][n] + sRed[rb][3][tt][w2][n]);
      if constexpr (std::is_same<IdxT, int32_t>::value)  // the block base plus a 32-bit offset
        *at_bytes(pbc_blk, static_cast<uint32_t>(ts * (2 * kStatePad) + i) * 4u) = v;
      else
        pbc_blk[static_cast<IdxT>(ts) * (2 * kStatePad) + i] = v;
    }
  };

  float tacc[4], tD;
  // reverse sweep over scan positions [h0, h0 + n) of tile buffer `buf`,
  // entering with the state after position h0 - 1.  The step body has no
  // divergent branches: lanes that share a result all store it.
  auto half = [&](auto full, int buf, int h0, int n, float4 hin) {
    constexpr bool kFull = decltype(full)::value;
    float hs[kCk + 1][4];
    float ea[kCk][4];
    float dxs[kCk];  // delta * u of each step, reused by the reverse loop (not lean)
    hs[0][0] = hin.x; hs[0][1] = hin.y; hs[0][2] = hin.z; hs[0][3] = hin.w;
#pragma unroll
    for (int i = 0; i < kCk; ++i) {
      const int tt = h0 + i;
      const float dl = sD[buf][tt][cl];
      const float dxu = dl * sU[buf][tt][cl];
      if constexpr (!kLean) dxs[i] = dxu;
      const float4 b4 = *reinterpret_cast<const float4*>(&sB[buf][tt][4 * grp]);
      const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        ea[i][jj] = fast_exp2(dl * a2[jj]);
        hs[i + 1][jj] = fmaf(ea[i][jj], hs[i][jj], dxu * bv[jj]);
      }
    }
    // the reverse loop reads its operands from LDS again rather than keeping
    // the forward loop's copies live (fewer VGPRs, earlier LDS issue); only
    // the product delta * u (dxs, one VALU per step) is kept
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = kCk - 1; i >= 0; --i) {
      if (kFull || i < n) {
        const int tt = h0 + i;
        const float uu = sU[buf][tt][cl];
        const float dl = sD[buf][tt][cl];
        const float gy = sG[buf][tt][cl];
        const float4 b4 = *reinterpret_cast<const float4*>(&sB[buf][tt][4 * grp]);
        const float4 c4 = *reinterpret_cast<const float4*>(&sC[buf][tt][4 * grp]);
        const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
        const float dxu = kLean ? dl * uu : dxs[i];
        float sa = 0.f, sb = 0.f;
        float xb[4], xc[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float lam = fmaf(cv[jj], gy, mu[jj]);
          const float q = lam * ea[i][jj];
          const float w = q * hs[i][jj];
          sa = fmaf(w, kLean ? a2[jj] : an[jj], sa);
          tacc[jj] = fmaf(w, dl, tacc[jj]);
          sb = fmaf(lam, bv[jj], sb);
          xb[jj] = lam * dxu;
          xc[jj] = gy * hs[i + 1][jj];
          mu[jj] = q;
        }
        sa = kLean ? sum_groups(sa) * kLn2 : sum_groups(sa);
        sb = sum_groups(sb);
        tD = fmaf(gy, uu, tD);
        // in place: this step's u / dy are consumed (the 4 lanes of the
        // channel store the same values)
        sU[buf][tt][cl] = fmaf(dl, sb, dskip * gy);
        sG[buf][tt][cl] = fmaf(uu, sb, sa);
        const float rb = channel_reduce4(xb[0], xb[1], xb[2], xb[3]);
        const float rc = channel_reduce4(xc[0], xc[1], xc[2], xc[3]);
        // lanes with equal (g, j) hold equal sums and store them together
        sRed[kLean ? 0 : buf][wave][tt][0][4 * grp + red_j] = rb;
        sRed[kLean ? 0 : buf][wave][tt][1][4 * grp + red_j] = rc;
      }
    }
  };

  const int32_t ntile = (t1 - t0 + kSub - 1) / kSub;
  float pu[4], pd[4], pg[4], pb, pc;
  // checkpoints entering the two halves of the staged tile (lean: the next
  // tile's pck0 is loaded after the first half-sweep, not with the prefetch)
  float4 pck0, pck1;
  auto load_tile = [&](const TileRows& rows, int32_t ts) {
    load_rows(pu, u, rows, sx, lc);
    load_rows(pd, delta, rows, sd, lc);
    load_rows(pg, dy, rows, sy, lc);
    if (gate) {
      load_rows(pz, zin, rows, sz, lc);
      load_rows(pyr, yraw, rows, sy, lc);
    }
    pb = load_state(Bm, rows, sbc, N, tid);
    pc = load_state(Cm, rows, sbc, N, tid);
    if constexpr (!kLean) pck0 = load_ckpt(ts);
    pck1 = load_ckpt(ts + kCk);
  };
  auto store_tile = [&](int buf, const TileRows& rows, int nt) {
    // the prefetched values are first consumed here, after the tile's math
    mask_xtile(pu, cok, all_in);
    mask_xtile(pd, cok, all_in);
    mask_xtile(pg, cok, all_in);
    if (gate) {
      mask_xtile(pz, cok, all_in);
      mask_xtile(pyr, cok, all_in);
    }
    pb = mask_stile(pb, N, tid);
    pc = mask_stile(pc, N, tid);
    stage_delta(pd);
    stage_gate(pg, rows, nt);
    store_xtile(sU[buf], pu, tid);
    store_xtile(sD[buf], pd, tid);
    store_xtile(sG[buf], pg, tid);
    if (FUSE) store_xtile(sSg[buf], psg, tid);
    sB[buf][stile_row(tid)][tid & 15] = pb;
    sC[buf][stile_row(tid)][tid & 15] = pc;
  };
  TileRows rc, rp;  // rows of the tile being computed, of the one before it
  {
    const int32_t ts = t0 + (ntile - 1) * kSub;
    rc = tile_rows<TOK>(tok, ts, L, tid);
    rp = rc;
    load_tile(rc, ts);
    if constexpr (kLean) pck0 = load_ckpt(ts);
    store_tile(0, rc, t1 - ts);
  }

  for (int32_t j = 0; j < ntile; ++j) {
    const int buf = j & 1;
    const int32_t ts = t0 + (ntile - 1 - j) * kSub;
    const int nt = min(kSub, t1 - ts);
    __syncthreads();  // tile j staged; the previous tile's outputs are complete
    if (j > 0) {
      flush(buf ^ 1, rp, min(kSub, t1 - ts - kSub));
      if constexpr (!kLean) flush_red(buf ^ 1, ts + kSub, min(kSub, t1 - ts - kSub));
    }
    const float4 hin0 = pck0, hin1 = pck1;
    const bool more = j + 1 < ntile;
    TileRows rn = rc;
    if (more) {  // prefetch the previous tile (next in processing order)
      rn = tile_rows<TOK>(tok, ts - kSub, L, tid);
      load_tile(rn, ts - kSub);
    }
    // per-tile partial sums of dA / dD, folded into float64 once per tile
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) tacc[jj] = 0.f;
    tD = 0.f;
    if (nt == kSub) {
      // raised wave priority over the tile's math: at 2 waves per SIMD, the
      // other wave's staging and flushes fill the gaps instead of taking
      // issue slots from it (measured 295 -> 282 us per call at the
      // VisionMamba step shape)
      __builtin_amdgcn_s_setprio(1);
      half(std::true_type{}, buf, kCk, kCk, hin1);
      if (kLean && more) pck0 = load_ckpt(ts - kSub);
      half(std::true_type{}, buf, 0, kCk, hin0);
      __builtin_amdgcn_s_setprio(0);
    } else {
      if (nt > kCk) half(std::false_type{}, buf, kCk, nt - kCk, hin1);
      if (kLean && more) pck0 = load_ckpt(ts - kSub);
      half(std::false_type{}, buf, 0, nt < kCk ? nt : kCk, hin0);
    }
    if constexpr (kLean) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) sAcc[jj][tid] += static_cast<double>(tacc[jj]);
      sAcc[4][tid] += static_cast<double>(tD);
      // the tile's dB | dC channel sums are complete and every flush of the
      // other buffer is done before it is refilled; the staging goes first
      // (its wait for the prefetched loads would otherwise also wait for
      // the partials' stores: one in-order counter covers both)
      __syncthreads();
      if (more) store_tile(buf ^ 1, rn, kSub);
      flush_red(0, ts, nt);
    } else {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dacc[jj] += static_cast<double>(tacc[jj]);
      dDacc += static_cast<double>(tD);
      // no barrier: each thread refills exactly the LDS slots of the other
      // buffer that it flushed at this tile's start (its dB | dC sums, read
      // by every thread, are not refilled), and this tile's math reads only
      // this buffer; the next tile's first barrier orders the refill before
      // that buffer's math
      if (more) store_tile(buf ^ 1, rn, kSub);
    }
    rp = rc;
    rc = rn;
  }
  if constexpr (!kLean) __syncthreads();  // lean: the last tile's second barrier
  flush((ntile - 1) & 1, rp, min(kSub, t1 - t0));
  if constexpr (!kLean) flush_red((ntile - 1) & 1, t0, min(kSub, t1 - t0));

  if (dvalid) {
    double* pa = bf.part_dA + slot * kStatePad + 4 * grp;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) pa[jj] = kLean ? sAcc[jj][tid] : dacc[jj];
    if (grp == 0) bf.part_dD[slot] = kLean ? sAcc[4][tid] : dDacc;
  }
  if (FUSE && bf.ddbias != nullptr) {  // dt_bias gradient: the 4 waves' rows, fixed order
    sDb[wave][lane] = dbacc;
    __syncthreads();
    if (wave == 0 && dld < gm.D)
      bf.part_db[(bk * gm.nchunk + chunk) * gm.D + dld] = (sDb[0][lane] + sDb[1][lane]) +
                                                          (sDb[2][lane] + sDb[3][lane]);
  }
}

// The two fixed-order reductions after the sweep, in one launch: blocks
// [0, nad_blocks) reduce dA, dD and the dt bias, the rest dB / dC.  The dA
// blocks go first: each waits on a chain of float64 partial loads, and
// dispatched last they formed the kernel's tail (16.0 -> 13.0 us at the
// VisionMamba step shape).
//
// dB / dC: sum the channel-block partials in a fixed order and store at the
// token row each scan position read (mamba_metal_fused.py:221,224).
template <typename OT>
__device__ __forceinline__ void reduce_bc_part(const Geom& gm, const BwdBufs& bf, int64_t blk) {
  static_assert(kStatePad == 16, "the (t, dB|dC, n) index below is a bit split");
  // blocks of one (batch, direction) row cover its L x 32 outputs; the
  // division is block-uniform (scalar), the split of j is shifts and masks
  const int64_t row_elems = gm.L * 2 * kStatePad;
  const int64_t bpr = (row_elems + kThreads - 1) / kThreads;
  const int64_t bk = blk / bpr;
  const int64_t j = (blk - bk * bpr) * kThreads + threadIdx.x;
  if (j >= row_elems) return;
  const int n = static_cast<int>(j & 15);
  const int w2 = static_cast<int>((j >> 4) & 1);
  const int64_t t = j >> 5;
  if (n >= gm.N) return;
  // the channel-block partials are summed left to right; each batch's
  // loads are in flight together (the bounds are block-uniform)
  const float* pp = bf.part_bc + (bk * gm.ncblk * gm.L + t) * (2 * kStatePad) + w2 * kStatePad + n;
  const int64_t cstride = gm.L * 2 * kStatePad;
  constexpr int kBatch = 16;
  float s = 0.f;
  for (int64_t cb0 = 0; cb0 < gm.ncblk; cb0 += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) v[u] = cb0 + u < gm.ncblk ? pp[(cb0 + u) * cstride] : 0.f;
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (cb0 + u < gm.ncblk) s += v[u];
  }
  const int64_t b = bk / gm.K, k = bk - b * gm.K;
  const int64_t row = token_row(gm.tok ? gm.tok + k * gm.L : nullptr, t, gm.L);
  OT* out = static_cast<OT*>(w2 ? bf.dC : bf.dB);
  st(out, b * gm.bsb + k * gm.bsk + row * gm.bst + n, s);
}

// dA (K, D, N), dD (K, D) and (fused, when requested) the dt_bias gradient
// (K, D): sum the per-(b, chunk) float64 partials in a fixed order
// (mamba_metal_fused.py:214,218).  A block covers 64 consecutive output
// columns; its 4 waves each sum a quarter of the B * nchunk partials and
// the quarters are added in wave order.
__device__ __forceinline__ void reduce_ad_part(const Geom& gm, const BwdBufs& bf, int64_t blk,
                                               double (*sq)[64]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t nA = gm.K * gm.D * kStatePad;
  const int64_t nKD = gm.K * gm.D;
  const int64_t col = blk * 64 + lane;
  int kind = 0;  // 0: dA, 1: dD, 2: dt_bias
  int64_t k = 0, d = 0;
  int n = 0;
  if (col < nA) {
    n = static_cast<int>(col % kStatePad);
    d = (col / kStatePad) % gm.D;
    k = col / (kStatePad * gm.D);
  } else {
    kind = col < nA + nKD ? 1 : 2;
    const int64_t i = col - nA - (kind == 2 ? nKD : 0);
    d = i % gm.D;
    k = i / gm.D;
  }
  const bool valid = col < nA + 2 * nKD && (kind != 0 || n < gm.N) &&
                     (kind != 2 || bf.ddbias != nullptr);
  const int64_t nparts = gm.B * gm.nchunk;
  const int64_t per = (nparts + 3) / 4;
  const int64_t q0 = wave * per, q1 = min(nparts, q0 + per);
  double s = 0.0;
  if (valid && q0 < q1) {
    // the lane's partial array: element (slot) at src[slot * smul + n]
    const double* src = kind == 0 ? bf.part_dA : (kind == 1 ? bf.part_dD : bf.part_db);
    const int64_t smul = kind == 0 ? kStatePad : 1;
    const int64_t sadd = kind == 0 ? n : 0;
    // q = b * nchunk + c, stepped without a division per partial; each
    // batch's loads are in flight together, then added in partial order
    constexpr int kBatch = 8;
    int64_t b = q0 / gm.nchunk, c = q0 - b * gm.nchunk;
    for (int64_t q = q0; q < q1; q += kBatch) {
      double v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        v[u] = 0.0;
        if (q + u < q1) {
          const int64_t slot = ((b * gm.K + k) * gm.nchunk + c) * gm.D + d;
          v[u] = src[slot * smul + sadd];
          if (++c == gm.nchunk) {
            c = 0;
            ++b;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (q + u < q1) s += v[u];
    }
  }
  sq[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && valid) {
    const double sum = (sq[0][lane] + sq[1][lane]) + (sq[2][lane] + sq[3][lane]);
    const float t = static_cast<float>(sum);
    if (kind == 0) {
      // with the A_log parametrisation, dA_log = dA * A (A = -exp(A_log))
      const int64_t ia = (k * gm.D + d) * gm.N + n;
      bf.dA[ia] = gm.a_log ? static_cast<float>(sum * static_cast<double>(load_A(bf.A, ia, 1)))
                           : t;
    }
    else
      (kind == 1 ? bf.dD : bf.ddbias)[k * gm.D + d] = t;
  }
}

template <typename OT>
__global__ void __launch_bounds__(kThreads)
reduce_grads_kernel(Geom gm, BwdBufs bf, int64_t nad_blocks) {
  __shared__ double sq[4][64];
  const int64_t blk = blockIdx.x;
  if (blk < nad_blocks)
    reduce_ad_part(gm, bf, blk, sq);  // block-uniform branch: its barrier is safe
  else
    reduce_bc_part<OT>(gm, bf, blk - nad_blocks);
}

template <typename XT, typename OT, bool FUSE, bool TOK, typename IdxT>
static hipError_t launch_bwd_tti(const Geom& g, const BwdBufs& b, hipStream_t s) {
  const dim3 block(kThreads);
  if (g.nchunk > 1) {
    const dim3 grid_agg(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                        static_cast<unsigned>(g.nchunk - 1));
    hipLaunchKernelGGL((scan_bwd_agg_kernel<XT, FUSE, TOK, IdxT>), grid_agg, block, 0, s, g, b);
    if (g.nchunk > kFoldMax) {
      const int64_t total = g.B * g.K * g.D * kStatePad;
      hipLaunchKernelGGL(scan_bwd_carry_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                         block, 0, s, g, b);
    }
  }
  const dim3 grid(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                  static_cast<unsigned>(g.nchunk));
  // the in-sweep fold is a separate instantiation: the one-chunk and
  // carry-pass kernels carry no code for it
  if (g.nchunk > 1 && g.nchunk <= kFoldMax)
    hipLaunchKernelGGL((scan_bwd_kernel<XT, OT, FUSE, TOK, true, IdxT>), grid, block, 0, s, g, b);
  else
    hipLaunchKernelGGL((scan_bwd_kernel<XT, OT, FUSE, TOK, false, IdxT>), grid, block, 0, s, g, b);
  const int64_t nbc_blocks = g.B * g.K * ((g.L * 2 * kStatePad + kThreads - 1) / kThreads);
  const int64_t nad_blocks = (g.K * g.D * (kStatePad + 2) + 63) / 64;
  hipLaunchKernelGGL((reduce_grads_kernel<OT>), dim3(static_cast<unsigned>(nbc_blocks + nad_blocks)),
                     block, 0, s, g, b, nad_blocks);
  return hipGetLastError();
}

template <typename XT, typename OT, bool FUSE, bool TOK>
static hipError_t launch_bwd_tt(const Geom& g, const BwdBufs& b, hipStream_t s) {
  return offsets_fit_i32(g) ? launch_bwd_tti<XT, OT, FUSE, TOK, int32_t>(g, b, s)
                            : launch_bwd_tti<XT, OT, FUSE, TOK, int64_t>(g, b, s);
}

// remapped (seq_to_tok given) and identity-order instantiations
template <typename XT, typename OT, bool FUSE = false>
static hipError_t launch_bwd_t(const Geom& g, const BwdBufs& b, hipStream_t s) {
  return g.tok ? launch_bwd_tt<XT, OT, FUSE, true>(g, b, s) : launch_bwd_tt<XT, OT, FUSE, false>(g, b, s);
}

hipError_t launch_bwd(const Geom& g, const BwdBufs& b, int in_dtype, int out_dtype, hipStream_t s) {
  if (in_dtype == 0 && out_dtype == 0) return launch_bwd_t<float, float>(g, b, s);
  if (in_dtype == 1 && out_dtype == 1) return launch_bwd_t<bf16_t, bf16_t>(g, b, s);
  if (in_dtype == 1 && out_dtype == 0) return launch_bwd_t<bf16_t, float>(g, b, s);
  return launch_bwd_t<float, bf16_t>(g, b, s);
}

hipError_t launch_fused_bwd(const Geom& g, const BwdBufs& b, hipStream_t s) {
  return launch_bwd_t<float, float, true>(g, b, s);
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
