// Kernel parameter blocks and launch entry points shared by the scan
// kernels (scan_fwd.hip, scan_bwd.hip) and the C ABI (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvm {

// Geometry of one scan call (all directions of one launch).
struct Geom {
  int64_t B, L, D, N, K;
  int64_t xsb, xsk, xst;   // u, du strides
  int64_t dsb, dsk, dst;   // delta, ddelta strides
  int64_t ysb, ysk, yst;   // y, dy (and the fused y_raw) strides
  int64_t zsb, zsk, zst;   // gate z, dz strides (fused form only)
  int64_t bsb, bsk, bst;   // B-like strides
  const int32_t* tok;      // (K, L) scan position -> token row, or nullptr
  int64_t chunk_len;       // multiple of kSub
  int64_t nchunk;          // ceil(L / chunk_len)
  int64_t nck;             // ceil(L / kCk), checkpoint slots per (b, k, d)
  int64_t ncblk;           // ceil(D / 64), channel blocks
  int32_t a_log;           // 1: the A array holds A_log, A = -exp(A_log)
};

// True when every element offset the kernels form within one (batch,
// direction) slab is below 2^30 (row strides, the checkpoint and partial
// rows included), so that they use the 32-bit row and byte-offset
// arithmetic; else the int64 instantiations run.
inline bool offsets_fit_i32(const Geom& g) {
  // element offsets below 2^30, so that byte offsets (elements of <= 4 bytes,
  // 16-byte checkpoint groups addressed as floats) fit in 32 bits; head-room
  // for the lane's channel
  constexpr int64_t lim = (int64_t{1} << 30) - 64;
  const int64_t lm = g.L > 0 ? g.L - 1 : 0;
  auto ok = [&](int64_t st) { return st >= 0 && st <= lim && lm * st <= lim; };
  return ok(g.xst) && ok(g.dst) && ok(g.yst) && ok(g.zst) && ok(g.bst) &&
         g.nck * g.D * 16 <= lim && g.L * 2 * 16 <= lim;  // 16 states per channel
}

struct FwdBufs {
  const void* u;
  const float* delta;
  const float* A;
  const void* Bm;
  const void* Cm;
  const float* Dv;
  void* y;         // may be null
  float* ckpt;     // may be null
  float* agg_h;    // (B*K, nchunk, D, 16): chunk end states, then carry-ins
  float* agg_s;    // (B*K, nchunk, D): sum of delta over each chunk
  // fused form: delta = softplus(delta_raw + dbias), y = y_raw * silu(z)
  const float* dbias;  // (K, D) or null (zero bias)
  const float* z;      // gate or null (no gate)
  float* y_raw;        // ungated output or null
};

struct BwdBufs {
  const void* u;
  const float* delta;
  const float* A;
  const void* Bm;
  const void* Cm;
  const float* Dv;
  const float* ckpt;
  const void* dy;
  void* du;
  float* ddelta;
  float* dA;
  void* dB;
  void* dC;
  float* dD;
  float* agg_mu;   // (B*K, nchunk, D, 16): adjoint aggregates, then carries
  float* agg_s;    // (B*K, nchunk, D)
  double* part_dA;  // (B*K, nchunk, D, 16) float64 partial sums
  double* part_dD;  // (B*K, nchunk, D)
  float* part_bc;  // (B*K, ncblk, L, 32): per channel-block dB | dC sums
  // fused form: delta_raw / ddelta_raw in place of delta / ddelta
  const float* dbias;  // (K, D) or null
  float* ddbias;       // (K, D) gradient of dbias (when dbias is given)
  double* part_db;     // (B*K, nchunk, D) float64 partials of ddbias
  // fused gate y = y_raw * silu(z): dy is the gradient of the gated y
  const float* z;      // z strides, or null (no gate)
  const float* y_raw;  // y strides
  float* dz;           // z strides
};

// in_dtype / out_dtype follow MVM_F32 / MVM_BF16.
hipError_t launch_fwd(const Geom& g, const FwdBufs& b, int in_dtype, int out_dtype,
                      hipStream_t s);
hipError_t launch_bwd(const Geom& g, const BwdBufs& b, int in_dtype, int out_dtype,
                      hipStream_t s);
// fused form (float32 only): softplus(delta_raw + dbias) on load, gate on store
hipError_t launch_fused_fwd(const Geom& g, const FwdBufs& b, hipStream_t s);
hipError_t launch_fused_bwd(const Geom& g, const BwdBufs& b, hipStream_t s);
hipError_t launch_fill(float* p, int64_t n, float v, hipStream_t s);
hipError_t launch_selftest_lanes(float* out, hipStream_t s);

}  // namespace mvm
