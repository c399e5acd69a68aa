// Forward selective scan for gfx950 (MI355X).
//
// Math (mamba_block.py:45-74; fused form mamba_metal_fused.py:21-63):
//   h_t = exp(delta_t * A) * h_{t-1} + delta_t * B_t * u_t,   h_{-1} = 0
//   y_t = sum_n C_t[n] * h_t[n] + D * u_t
//
// Work split.  Lane (c, g) of a wave owns states 4g..4g+3 of one channel
// (scan_common.h).  A 256-thread workgroup covers 64 channels of one
// (batch, direction) pair and one time chunk, walking it in 16-step tiles.
// Each tile of u, delta (64 channels) and B, C (16 states, shared by all
// channels) is loaded with fully coalesced reads into a double-buffered LDS
// stage, converted to fp32 once; the next tile's loads are issued before the
// current tile's math so their latency is hidden.  y replaces u in the LDS
// stage and is written back one tile later as coalesced rows.  20 KiB of
// LDS and <= 80 VGPRs per block let six 4-wave blocks share a CU, so a
// VisionMamba-sized grid (B*K*D/64 = 1536 blocks) runs in one wave of
// blocks on 256 CUs.
//
// Long sequences are split into time chunks so that the grid fills the
// chip (the two-pass scheme whose carry step the reference left as TODO at
// mamba_metal_chunked.py:268-272):
//   pass 1 (kAgg)    each chunk but the last scans from h = 0 and writes its
//                    end state and sum(delta) (its decay is exp(A*sum(delta)));
//   carry            H_c = exp(A*S_c) * H_{c-1} + e_c (mamba_fast.py:85-86):
//                    folded by each chunk of the main pass itself for up to
//                    kFoldMax chunks, by scan_fwd_carry_kernel beyond;
//   pass 2 (kMain)   each chunk rescans from its carry-in, writes y and,
//                    when training, the state after every 8th position
//                    (the backward's checkpoints).
//
// Fused form (FUSE, float32): the block's prologue and epilogue around the
// scan (mamba_block.py:180-181, :190) run inside the staging and write-back
// of the same kernel: delta = softplus(delta_raw + dt_bias) as the delta tile
// is staged, and y = y_raw * silu(z) as y is written back (y_raw kept for
// the backward when requested), so neither delta nor the gate makes an
// extra pass over HBM.
#include "scan_common.h"
#include "scan_kernels.h"

namespace mvm {

enum FwdMode { kAgg = 0, kMain = 1 };

template <typename XT, typename OT, int MODE, bool FUSE, bool TOK, typename IdxT>
__global__ void __launch_bounds__(kThreads, 6)
scan_fwd_kernel(Geom gm, FwdBufs bf) {
  // double-buffered tile staging: u, delta (64 channels), B, C (16 states);
  // y replaces u in place and is written back coalesced one tile later (each
  // thread flushes exactly the LDS slots it refills with the next prefetch)
  // (one array per kind, so that a thread's slots in both tiles share one
  // address and immediate offsets)
  __shared__ float sX[2][2][kSub][kChPerBlock];
  __shared__ float sBC[2][2][kSub][kStatePad];
  float (*const sU)[kSub][kChPerBlock] = sX[0];
  float (*const sD)[kSub][kChPerBlock] = sX[1];
  float (*const sB)[kSub][kStatePad] = sBC[0];
  float (*const sC)[kSub][kStatePad] = sBC[1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = lane & 3;
  const int cl = wave * kChPerWave + (lane >> 2);          // compute channel within the block
  const int64_t ch0 = static_cast<int64_t>(blockIdx.x) * kChPerBlock;
  const int64_t d = ch0 + cl;
  const int64_t dld = ch0 + lane;                          // channel this thread loads / stores
  const bool dvalid = d < gm.D;
  const bool cok = dld < gm.D;
  const bool all_in = ch0 + kChPerBlock <= gm.D;  // block-uniform: no channel masked
  const int64_t dc = dvalid ? d : 0;
  const int lc = cok ? lane : 0;
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / gm.K;
  const int64_t k = bk - b * gm.K;
  const int64_t chunk = blockIdx.z;
  const int32_t L = static_cast<int32_t>(gm.L);
  const int N = static_cast<int>(gm.N);
  const int32_t t0 = static_cast<int32_t>(chunk * gm.chunk_len);
  // the chunk's end in 64 bits: t0 + chunk_len may pass 2^31 - 1 in the last chunk
  const int32_t t1 = static_cast<int32_t>(min<int64_t>(gm.L, (chunk + 1) * gm.chunk_len));
  const int32_t* tok = TOK ? gm.tok + k * gm.L : nullptr;
  // the block's first channel of its (b, k) slab in every tensor
  const XT* __restrict__ u = static_cast<const XT*>(bf.u) + (b * gm.xsb + k * gm.xsk + ch0);
  const float* __restrict__ delta = bf.delta + (b * gm.dsb + k * gm.dsk + ch0);
  const XT* __restrict__ Bm = static_cast<const XT*>(bf.Bm) + (b * gm.bsb + k * gm.bsk);
  const XT* __restrict__ Cm = static_cast<const XT*>(bf.Cm) + (b * gm.bsb + k * gm.bsk);
  const int64_t yoff = b * gm.ysb + k * gm.ysk + ch0;
  OT* __restrict__ y = bf.y != nullptr ? static_cast<OT*>(bf.y) + yoff : nullptr;
  const IdxT sx = static_cast<IdxT>(gm.xst), sd = static_cast<IdxT>(gm.dst);
  const IdxT sy = static_cast<IdxT>(gm.yst), sz = static_cast<IdxT>(gm.zst);
  const IdxT sbc = static_cast<IdxT>(gm.bst);
  // fused prologue: the dt bias of the channel this thread stages
  const float dbias_l = (FUSE && bf.dbias != nullptr && cok) ? bf.dbias[k * gm.D + dld] : 0.f;
  const bool gate = FUSE && MODE == kMain && bf.z != nullptr;
  const float* __restrict__ zin = gate ? bf.z + (b * gm.zsb + k * gm.zsk + ch0) : nullptr;
  float* __restrict__ y_raw = (FUSE && bf.y_raw != nullptr) ? bf.y_raw + yoff : nullptr;

  float a2[4], h[4];
  load_ax4(a2, bf.A, (k * gm.D + dc) * gm.N, grp, N, dvalid, gm.a_log);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a2[j] *= kLog2e;
    h[j] = 0.f;
  }
  const float dskip_v = bf.Dv[k * gm.D + dc];
  const float dskip = (MODE == kMain && dvalid) ? dskip_v : 0.f;
  const int64_t slot = (bk * gm.nchunk + chunk) * gm.D + dc;  // (bk, chunk, d)
  if (MODE == kMain && chunk > 0 && dvalid) {
    if (gm.nchunk <= kFoldMax) {
      // carry-in: fold the aggregates of chunks 0..chunk-1 left to right,
      // H = exp(A * S_c) * H + E_c (mamba_fast.py:85-86).  All (at most
      // kFoldMax) aggregates are loaded first, from in-bounds chunk indices,
      // so their latencies overlap; the fold then runs on registers.
      const int64_t s0 = bk * gm.nchunk * gm.D + dc;
      float4 e4[kFoldMax];
      float sdl[kFoldMax];
#pragma unroll
      for (int c = 0; c < kFoldMax; ++c) {
        const int64_t sc = s0 + (c < gm.nchunk ? c : 0) * gm.D;
        e4[c] = *reinterpret_cast<const float4*>(bf.agg_h + sc * kStatePad + 4 * grp);
        sdl[c] = bf.agg_s[sc];
      }
#pragma unroll
      for (int c = 0; c < kFoldMax; ++c) {
        if (c < chunk) {
          const float e[4] = {e4[c].x, e4[c].y, e4[c].z, e4[c].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) h[j] = fmaf(fast_exp2(a2[j] * sdl[c]), h[j], e[j]);
        }
      }
    } else {  // folded by scan_fwd_carry_kernel
      const float4 c4 = *reinterpret_cast<const float4*>(bf.agg_h + slot * kStatePad + 4 * grp);
      h[0] = c4.x; h[1] = c4.y; h[2] = c4.z; h[3] = c4.w;
    }
  }
  float dsum = 0.f;
  const bool write_y = MODE == kMain && y != nullptr;
  const bool write_ck = MODE == kMain && bf.ckpt != nullptr && dvalid;
  // checkpoint slot s holds the state after position 8s + 7
  float* ckp = write_ck ? bf.ckpt + (bk * gm.nck * gm.D + d) * kStatePad + 4 * grp : nullptr;
  const IdxT ck_stride = static_cast<IdxT>(gm.D * kStatePad);
  // y of a staged tile (held in sU, token rows `rows`) back to HBM; zv = the
  // gate values of the same rows and channel when fused
  auto flush_y = [&](int buf, const TileRows& rows, int nt, const float (&zv)[4]) {
    const int wrow = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tt = wrow + 4 * r;
      if (tt < nt && cok) {
        const IdxT roff = static_cast<IdxT>(rows.r[r]) * sy;
        float v = sU[buf][tt][lane];
        if (FUSE && y_raw != nullptr) (y_raw + roff)[lc] = v;
        if (gate) v *= zv[r] * sigmoid_f(zv[r]);
        st(y + roff, lc, v);
      }
    }
  };
  // fused prologue on the staged delta values
  auto stage_delta = [&](float (&v)[4]) {
    if (FUSE) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = softplus_f(v[r] + dbias_l);
    }
  };
  // one scan step at tile position tt of buffer buf
  auto step = [&](int buf, int tt) {
    const float uu = sU[buf][tt][cl];
    const float dl = sD[buf][tt][cl];
    const float4 b4 = *reinterpret_cast<const float4*>(&sB[buf][tt][4 * grp]);
    const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
    const float du = dl * uu;
    float yp = 0.f;
    float cv[4] = {0.f, 0.f, 0.f, 0.f};
    if (MODE == kMain) {
      const float4 c4 = *reinterpret_cast<const float4*>(&sC[buf][tt][4 * grp]);
      cv[0] = c4.x; cv[1] = c4.y; cv[2] = c4.z; cv[3] = c4.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e = fast_exp2(dl * a2[j]);
      h[j] = fmaf(e, h[j], du * bv[j]);
      if (MODE == kMain) yp = fmaf(cv[j], h[j], yp);
    }
    if (MODE == kAgg) dsum += dl;
    if (MODE == kMain) {  // the channel's 4 lanes store the same y (no branch)
      yp = sum_groups(yp);
      sU[buf][tt][cl] = fmaf(dskip, uu, yp);  // in place: u_t is consumed
    }
  };
  auto store_ck = [&](int32_t pos_end) {  // state after position pos_end (== 8s + 7)
    *reinterpret_cast<float4*>(ckp + static_cast<IdxT>(pos_end / kCk) * ck_stride) =
        make_float4(h[0], h[1], h[2], h[3]);
  };
  auto load_tile = [&](const TileRows& rows, float (&pu)[4], float (&pd)[4], float& pb, float& pc) {
    load_rows(pu, u, rows, sx, lc);
    load_rows(pd, delta, rows, sd, lc);
    pb = load_state(Bm, rows, sbc, N, tid);
    if (MODE == kMain) pc = load_state(Cm, rows, sbc, N, tid);
  };
  // zero the out-of-range channels / states of a prefetched tile: the first
  // use of its values, after the current tile's math
  auto mask_tile = [&](float (&pu)[4], float (&pd)[4], float& pb, float& pc) {
    mask_xtile(pu, cok, all_in);
    mask_xtile(pd, cok, all_in);
    pb = mask_stile(pb, N, tid);
    pc = mask_stile(pc, N, tid);
  };
  auto store_tile = [&](int buf, const float (&pu)[4], const float (&pd)[4], float pb, float pc) {
    store_xtile(sU[buf], pu, tid);
    store_xtile(sD[buf], pd, tid);
    sB[buf][stile_row(tid)][tid & 15] = pb;
    sC[buf][stile_row(tid)][tid & 15] = pc;
  };

  const int32_t ntile = (t1 - t0 + kSub - 1) / kSub;
  float pu[4], pd[4], pz[4] = {0.f, 0.f, 0.f, 0.f}, pb = 0.f, pc = 0.f;
  TileRows rc = tile_rows<TOK>(tok, t0, L, tid);  // rows of the tile being computed
  TileRows rp = rc;                                // rows of the previous tile
  load_tile(rc, pu, pd, pb, pc);
  mask_tile(pu, pd, pb, pc);
  stage_delta(pd);
  store_tile(0, pu, pd, pb, pc);

  for (int32_t it = 0; it < ntile; ++it) {
    const int buf = it & 1;
    const int32_t ts = t0 + it * kSub;
    const int nt = min(kSub, t1 - ts);
    __syncthreads();  // tile `it` staged; readers of the other buffer are done
    if (write_y && it > 0) flush_y(buf ^ 1, rp, kSub, pz);
    // gate values of this tile, used when it is flushed one tile later
    if (gate) load_rows(pz, zin, rc, sz, lc);
    const bool more = it + 1 < ntile;
    TileRows rn = rc;
    if (more) {  // prefetch the next tile; its latency overlaps this tile's math
      rn = tile_rows<TOK>(tok, ts + kSub, L, tid);
      load_tile(rn, pu, pd, pb, pc);
    }
    if (nt == kSub) {  // full tile: no per-step bounds checks
#pragma unroll
      for (int tt = 0; tt < kSub; ++tt) {
        step(buf, tt);
        if (write_ck && (tt == kCk - 1 || tt == kSub - 1)) store_ck(ts + tt);
      }
    } else {
      for (int tt = 0; tt < nt; ++tt) {
        step(buf, tt);
        if (write_ck && tt == kCk - 1) store_ck(ts + tt);
      }
    }
    if (more) {
      mask_tile(pu, pd, pb, pc);
      stage_delta(pd);
      store_tile(buf ^ 1, pu, pd, pb, pc);
    }
    rp = rc;
    rc = rn;
  }
  if (write_y) {
    __syncthreads();
    const int32_t ts = t0 + (ntile - 1) * kSub;
    flush_y((ntile - 1) & 1, rp, t1 - ts, pz);
  }

  if (MODE == kAgg && dvalid) {
    *reinterpret_cast<float4*>(bf.agg_h + slot * kStatePad + 4 * grp) =
        make_float4(h[0], h[1], h[2], h[3]);
    if (grp == 0) bf.agg_s[slot] = dsum;
  }
}

// Carry pass for many chunks: agg_h[c] becomes chunk c's carry-in (the state
// after the last position of chunk c-1), one thread per (b, k, d, n).
__global__ void __launch_bounds__(kThreads)
scan_fwd_carry_kernel(Geom gm, FwdBufs bf) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t total = gm.B * gm.K * gm.D * kStatePad;
  if (idx >= total) return;
  const int n = static_cast<int>(idx % kStatePad);
  const int64_t d = (idx / kStatePad) % gm.D;
  const int64_t bk = idx / (kStatePad * gm.D);
  const int64_t k = bk % gm.K;
  const float a2 = n < gm.N ? load_A(bf.A, (k * gm.D + d) * gm.N + n, gm.a_log) * kLog2e : 0.f;
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

template <typename XT, typename OT, bool FUSE, bool TOK, typename IdxT>
static hipError_t launch_fwd_tti(const Geom& g, const FwdBufs& b, hipStream_t s) {
  const dim3 block(kThreads);
  if (g.nchunk > 1) {
    const dim3 grid_agg(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                        static_cast<unsigned>(g.nchunk - 1));
    hipLaunchKernelGGL((scan_fwd_kernel<XT, OT, kAgg, FUSE, TOK, IdxT>), grid_agg, block, 0, s, g, b);
    if (g.nchunk > kFoldMax) {
      const int64_t total = g.B * g.K * g.D * kStatePad;
      hipLaunchKernelGGL(scan_fwd_carry_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                         block, 0, s, g, b);
    }
  }
  const dim3 grid(static_cast<unsigned>(g.ncblk), static_cast<unsigned>(g.B * g.K),
                  static_cast<unsigned>(g.nchunk));
  hipLaunchKernelGGL((scan_fwd_kernel<XT, OT, kMain, FUSE, TOK, IdxT>), grid, block, 0, s, g, b);
  return hipGetLastError();
}

template <typename XT, typename OT, bool FUSE, bool TOK>
static hipError_t launch_fwd_tt(const Geom& g, const FwdBufs& b, hipStream_t s) {
  return offsets_fit_i32(g) ? launch_fwd_tti<XT, OT, FUSE, TOK, int32_t>(g, b, s)
                            : launch_fwd_tti<XT, OT, FUSE, TOK, int64_t>(g, b, s);
}

// remapped (seq_to_tok given) and identity-order instantiations
template <typename XT, typename OT, bool FUSE = false>
static hipError_t launch_fwd_t(const Geom& g, const FwdBufs& b, hipStream_t s) {
  return g.tok ? launch_fwd_tt<XT, OT, FUSE, true>(g, b, s) : launch_fwd_tt<XT, OT, FUSE, false>(g, b, s);
}

hipError_t launch_fwd(const Geom& g, const FwdBufs& b, int in_dtype, int out_dtype, hipStream_t s) {
  if (in_dtype == 0 && out_dtype == 0) return launch_fwd_t<float, float>(g, b, s);
  if (in_dtype == 1 && out_dtype == 1) return launch_fwd_t<bf16_t, bf16_t>(g, b, s);
  if (in_dtype == 1 && out_dtype == 0) return launch_fwd_t<bf16_t, float>(g, b, s);
  return launch_fwd_t<float, bf16_t>(g, b, s);
}

hipError_t launch_fused_fwd(const Geom& g, const FwdBufs& b, hipStream_t s) {
  return launch_fwd_t<float, float, true>(g, b, s);
}

}  // namespace mvm
