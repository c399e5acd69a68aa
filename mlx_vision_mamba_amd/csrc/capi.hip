// C ABI of libmvm_scan.so (declared in include/mvm_scan.h, mvm_conv.h,
// mvm_norm.h and mvm_optim.h).
//
// Host-side responsibilities: validate every argument before anything is
// enqueued, pick the time-chunk length, carve the caller's workspace into
// the kernels' scratch buffers, and map HIP failures to MVM_ERR_HIP with a
// thread-local message.  No device memory is allocated here.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <utility>

#include "conv_kernels.h"
#include "mvm_conv.h"
#include "mvm_norm.h"
#include "mvm_optim.h"
#include "norm_kernels.h"
#include "optim_kernels.h"
#include "mvm_scan.h"
#include "mvm_testing.h"
#include "scan_common.h"
#include "scan_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MVM_OK;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr int64_t kMaxSeqlen = INT32_MAX - 64;

// Time-chunk length.  One chunk (no carry passes) when the (batch x
// direction x channel-block) grid alone gives >= 4096 waves (four per SIMD
// on the 256-CU MI355X); otherwise the sequence is cut until the main passes
// launch ~16k waves, into at most ceil(tiles / 2) chunks (2 tiles = 32
// positions each; the last may hold one).  Measured on MI355X: B=32 L=196
// D=3072 is fastest unchunked; B=8 L=16384 D=1536 at 512-768 positions per
// chunk; B=2 L=196 D=1536 at 32 (fwd + VJP graph replay 50.3 us, against
// 54.8 at 48 and 60.7 at 16).
int64_t pick_chunk_len(const mvm_scan_desc* d) {
  if (d->chunk_len > 0) return d->chunk_len;
  const int64_t tiles = ceil_div(d->seqlen, mvm::kSub);
  const int64_t waves = d->batch * d->ndir * ceil_div(d->dim, mvm::kChPerBlock) * 4;
  int64_t nchunk = 1;
  if (waves < 4096) nchunk = ceil_div(16384, std::max<int64_t>(waves, 1));
  nchunk = std::min(nchunk, std::max<int64_t>(1, (tiles + 1) / 2));
  const int64_t tiles_per_chunk = ceil_div(tiles, nchunk);
  return std::max<int64_t>(1, tiles_per_chunk) * mvm::kSub;
}

// True when a strided layout maps no two index tuples to one element:
// ordered by stride, every dimension's stride clears the span of the
// smaller ones (dimensions of size <= 1 are skipped).  Outputs are written
// through the same strides as their inputs, so an overlapping layout would
// make writes race.  A layout with no elements cannot overlap.
bool no_overlap(std::initializer_list<std::pair<int64_t, int64_t>> dims) {  // (size, stride)
  std::pair<int64_t, int64_t> v[8];
  int n = 0;
  for (const auto& d : dims) {
    if (d.first == 0) return true;
    if (d.first > 1 && n < 8) v[n++] = {d.second, d.first};  // (stride, size)
  }
  std::sort(v, v + n);
  int64_t span = 1;
  for (int i = 0; i < n; ++i) {
    if (v[i].first < span) return false;
    span = v[i].first * v[i].second;
  }
  return true;
}

int check_desc(const mvm_scan_desc* d) {
  if (d == nullptr) return fail(MVM_ERR_INVALID_ARG, "desc is NULL");
  if (d->batch < 0 || d->seqlen < 0 || d->dim < 0)
    return fail(MVM_ERR_INVALID_ARG, "negative size (batch=%lld seqlen=%lld dim=%lld)",
                (long long)d->batch, (long long)d->seqlen, (long long)d->dim);
  if (d->dstate < 1 || d->dstate > MVM_MAX_DSTATE)
    return fail(MVM_ERR_UNSUPPORTED, "dstate=%lld unsupported (1..%d)", (long long)d->dstate,
                MVM_MAX_DSTATE);
  if (d->ndir < 1) return fail(MVM_ERR_INVALID_ARG, "ndir=%lld must be >= 1", (long long)d->ndir);
  if (d->in_dtype != MVM_F32 && d->in_dtype != MVM_BF16)
    return fail(MVM_ERR_UNSUPPORTED, "in_dtype=%d unsupported", d->in_dtype);
  if (d->out_dtype != MVM_F32 && d->out_dtype != MVM_BF16)
    return fail(MVM_ERR_UNSUPPORTED, "out_dtype=%d unsupported", d->out_dtype);
  if (d->chunk_len < 0 || d->chunk_len % mvm::kSub != 0)
    return fail(MVM_ERR_INVALID_ARG, "chunk_len=%d must be 0 or a positive multiple of %d",
                d->chunk_len, mvm::kSub);
  const int64_t strides[6] = {d->x_stride_b, d->x_stride_k, d->x_stride_t,
                              d->bc_stride_b, d->bc_stride_k, d->bc_stride_t};
  for (int64_t s : strides)
    if (s < 0) return fail(MVM_ERR_INVALID_ARG, "negative stride");
  if (!no_overlap({{d->batch, d->x_stride_b}, {d->ndir, d->x_stride_k}, {d->seqlen, d->x_stride_t},
                   {d->dim, 1}}))
    return fail(MVM_ERR_INVALID_ARG,
                "x strides (b=%lld k=%lld t=%lld) overlap for batch=%lld ndir=%lld seqlen=%lld dim=%lld",
                (long long)d->x_stride_b, (long long)d->x_stride_k, (long long)d->x_stride_t,
                (long long)d->batch, (long long)d->ndir, (long long)d->seqlen, (long long)d->dim);
  if (!no_overlap({{d->batch, d->bc_stride_b}, {d->ndir, d->bc_stride_k}, {d->seqlen, d->bc_stride_t},
                   {d->dstate, 1}}))
    return fail(MVM_ERR_INVALID_ARG,
                "bc strides (b=%lld k=%lld t=%lld) overlap for batch=%lld ndir=%lld seqlen=%lld dstate=%lld",
                (long long)d->bc_stride_b, (long long)d->bc_stride_k, (long long)d->bc_stride_t,
                (long long)d->batch, (long long)d->ndir, (long long)d->seqlen, (long long)d->dstate);
  if (d->batch * d->ndir > 65535)
    return fail(MVM_ERR_UNSUPPORTED, "batch*ndir=%lld exceeds 65535",
                (long long)(d->batch * d->ndir));
  if (d->seqlen > 0 && ceil_div(d->seqlen, pick_chunk_len(d)) > 65535)
    return fail(MVM_ERR_UNSUPPORTED, "too many time chunks; raise chunk_len");
  // positions are int32 in the kernels, and a tile's rows are formed as
  // position + up to 63 before they are clamped to seqlen - 1
  if (d->seqlen > kMaxSeqlen)
    return fail(MVM_ERR_UNSUPPORTED, "seqlen=%lld exceeds %lld", (long long)d->seqlen,
                (long long)kMaxSeqlen);
  return MVM_OK;
}

mvm::Geom make_geom(const mvm_scan_desc* d) {
  mvm::Geom g;
  g.B = d->batch;
  g.L = d->seqlen;
  g.D = d->dim;
  g.N = d->dstate;
  g.K = d->ndir;
  g.xsb = d->x_stride_b;
  g.xsk = d->x_stride_k;
  g.xst = d->x_stride_t;
  // the plain scan's delta / ddelta and y / dy share u's layout
  g.dsb = g.ysb = d->x_stride_b;
  g.dsk = g.ysk = d->x_stride_k;
  g.dst = g.yst = d->x_stride_t;
  g.zsb = g.zsk = g.zst = 0;
  g.bsb = d->bc_stride_b;
  g.bsk = d->bc_stride_k;
  g.bst = d->bc_stride_t;
  g.tok = d->seq_to_tok;
  g.chunk_len = pick_chunk_len(d);
  g.nchunk = d->seqlen > 0 ? ceil_div(d->seqlen, g.chunk_len) : 0;
  g.nck = ceil_div(d->seqlen, mvm::kCk);
  g.ncblk = ceil_div(d->dim, mvm::kChPerBlock);
  g.a_log = 0;
  return g;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Workspace layouts (byte sizes; every piece 256-byte aligned).
struct FwdWs {
  size_t agg_h = 0, agg_s = 0, total = 0;
};
FwdWs fwd_ws(const mvm::Geom& g) {
  FwdWs w;
  if (g.nchunk > 1) {
    const size_t slots = static_cast<size_t>(g.B * g.K * g.nchunk * g.D);
    w.agg_h = align_up(slots * mvm::kStatePad * sizeof(float));
    w.agg_s = align_up(slots * sizeof(float));
  }
  w.total = w.agg_h + w.agg_s;
  return w;
}

struct BwdWs {
  size_t agg_mu = 0, agg_s = 0, part_dA = 0, part_dD = 0, part_bc = 0, ckpt = 0, fwd = 0, total = 0;
};
BwdWs bwd_ws(const mvm::Geom& g, bool recompute_ckpt) {
  BwdWs w;
  const size_t slots = static_cast<size_t>(g.B * g.K * g.nchunk * g.D);
  if (g.nchunk > 1) {
    w.agg_mu = align_up(slots * mvm::kStatePad * sizeof(float));
    w.agg_s = align_up(slots * sizeof(float));
  }
  w.part_dA = align_up(slots * mvm::kStatePad * sizeof(double));
  w.part_dD = align_up(slots * sizeof(double));
  w.part_bc = align_up(static_cast<size_t>(g.B * g.K * g.ncblk * g.L) * 2 * mvm::kStatePad * sizeof(float));
  if (recompute_ckpt) {
    w.ckpt = align_up(static_cast<size_t>(g.B * g.K * g.nck * g.D) * mvm::kStatePad * sizeof(float));
    w.fwd = fwd_ws(g).total;
  }
  w.total = w.agg_mu + w.agg_s + w.part_dA + w.part_dD + w.part_bc + w.ckpt + w.fwd;
  return w;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(MVM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

int mvm_abi_version(void) { return MVM_ABI_VERSION; }

const char* mvm_last_error(void) { return g_err; }

int mvm_scan_validate(const mvm_scan_desc* desc) {
  const int rc = check_desc(desc);
  return rc == MVM_OK ? ok() : rc;
}

int64_t mvm_scan_ckpt_elems(const mvm_scan_desc* desc) {
  const int rc = check_desc(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = make_geom(desc);
  return g.B * g.K * g.nck * g.D * mvm::kStatePad;
}

int64_t mvm_scan_workspace_bytes(const mvm_scan_desc* desc, int which) {
  const int rc = check_desc(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = make_geom(desc);
  if (which == 0) return static_cast<int64_t>(fwd_ws(g).total);
  if (which == 1) return static_cast<int64_t>(bwd_ws(g, false).total);
  if (which == 2) return static_cast<int64_t>(bwd_ws(g, true).total);
  return fail(MVM_ERR_INVALID_ARG, "which=%d must be 0, 1 or 2", which);
}

int64_t mvm_scan_chunk_len(const mvm_scan_desc* desc) {
  const int rc = check_desc(desc);
  if (rc != MVM_OK) return rc;
  return make_geom(desc).chunk_len;
}

int mvm_scan_fwd(const mvm_scan_desc* desc, const void* u, const float* delta, const float* A,
                 const void* Bm, const void* Cm, const float* Dv, void* y, float* ckpt,
                 void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_desc(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = make_geom(desc);
  const bool empty = g.B == 0 || g.L == 0 || g.D == 0;
  if (!empty) {
    if (!u || !delta || !A || !Bm || !Cm || !Dv)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fwd: NULL input pointer");
    if (!y && !ckpt) return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fwd: y and ckpt are both NULL");
    if ((reinterpret_cast<uintptr_t>(ckpt) & 15u) != 0)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fwd: ckpt must be 16-byte aligned");
  }
  const FwdWs w = fwd_ws(g);
  if (workspace_bytes < w.total)
    return fail(MVM_ERR_WORKSPACE, "mvm_scan_fwd: workspace %zu bytes < %zu needed", workspace_bytes,
                w.total);
  if (w.total > 0 && workspace == nullptr)
    return fail(MVM_ERR_WORKSPACE, "mvm_scan_fwd: workspace is NULL");
  if ((reinterpret_cast<uintptr_t>(workspace) & (kAlign - 1)) != 0)
    return fail(MVM_ERR_WORKSPACE, "mvm_scan_fwd: workspace must be %zu-byte aligned", kAlign);
  if (empty) return ok();
  char* ws = static_cast<char*>(workspace);
  mvm::FwdBufs b{u, delta, A, Bm, Cm, Dv, y, ckpt,
                 reinterpret_cast<float*>(ws), reinterpret_cast<float*>(ws + w.agg_h)};
  return hip_status(mvm::launch_fwd(g, b, desc->in_dtype, desc->out_dtype,
                                    static_cast<hipStream_t>(stream)),
                    "mvm_scan_fwd launch");
}

int mvm_scan_bwd(const mvm_scan_desc* desc, const void* u, const float* delta, const float* A,
                 const void* Bm, const void* Cm, const float* Dv, const float* ckpt,
                 const void* dy, void* du, float* ddelta, float* dA, void* dB, void* dC,
                 float* dD, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_desc(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = make_geom(desc);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool empty = g.B == 0 || g.L == 0 || g.D == 0;
  if (g.D > 0 && (!dA || !dD)) return fail(MVM_ERR_INVALID_ARG, "mvm_scan_bwd: NULL dA or dD");
  if (!empty) {
    if (!u || !delta || !A || !Bm || !Cm || !Dv || !dy)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_bwd: NULL input pointer");
    if (!du || !ddelta || !dB || !dC)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_bwd: NULL output pointer");
    if ((reinterpret_cast<uintptr_t>(ckpt) & 15u) != 0)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_bwd: ckpt must be 16-byte aligned");
  }
  const bool recompute = ckpt == nullptr;
  const BwdWs w = bwd_ws(g, recompute);
  if (!empty) {
    if (workspace_bytes < w.total)
      return fail(MVM_ERR_WORKSPACE, "mvm_scan_bwd: workspace %zu bytes < %zu needed", workspace_bytes,
                  w.total);
    if (workspace == nullptr) return fail(MVM_ERR_WORKSPACE, "mvm_scan_bwd: workspace is NULL");
    if ((reinterpret_cast<uintptr_t>(workspace) & (kAlign - 1)) != 0)
      return fail(MVM_ERR_WORKSPACE, "mvm_scan_bwd: workspace must be %zu-byte aligned", kAlign);
  }
  if (empty) {
    // sums over an empty (b, t) range are zero
    hipError_t e = mvm::launch_fill(dA, g.K * g.D * g.N, 0.f, s);
    if (e == hipSuccess) e = mvm::launch_fill(dD, g.K * g.D, 0.f, s);
    return hip_status(e, "mvm_scan_bwd fill");
  }
  char* ws = static_cast<char*>(workspace);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    float* p = reinterpret_cast<float*>(ws + off);
    off += bytes;
    return bytes ? p : nullptr;
  };
  float* agg_mu = take(w.agg_mu);
  float* agg_s = take(w.agg_s);
  double* part_dA = reinterpret_cast<double*>(take(w.part_dA));
  double* part_dD = reinterpret_cast<double*>(take(w.part_dD));
  float* part_bc = take(w.part_bc);
  float* ck = take(w.ckpt);
  float* fws = take(w.fwd);
  if (recompute) {
    // the reference's VJP also recomputes the forward states
    // (mamba_metal_fused.py:241-244); here only the 16-step checkpoints
    const FwdWs fw = fwd_ws(g);
    float* fagg_s = fws ? reinterpret_cast<float*>(reinterpret_cast<char*>(fws) + fw.agg_h) : nullptr;
    mvm::FwdBufs fb{u, delta, A, Bm, Cm, Dv, nullptr, ck, fws, fagg_s};
    hipError_t e = mvm::launch_fwd(g, fb, desc->in_dtype, desc->out_dtype, s);
    if (e != hipSuccess) return hip_status(e, "mvm_scan_bwd checkpoint recompute");
    ckpt = ck;
  }
  mvm::BwdBufs b{u, delta, A, Bm, Cm, Dv, ckpt, dy, du, ddelta, dA, dB, dC, dD,
                 agg_mu, agg_s, part_dA, part_dD, part_bc};
  return hip_status(mvm::launch_bwd(g, b, desc->in_dtype, desc->out_dtype, s), "mvm_scan_bwd launch");
}

}  // extern "C"

// ------------------------------------------- backward without a workspace

namespace {

// Scratch of mvm_scan_bwd_noalloc: one array per GPU (each device that loads
// the library holds its own copy until the process ends).  Host code never
// uses the name `scratch` as an address: it is a host-side stand-in for the
// symbol, and the device address comes from hipGetSymbolAddress, once per
// device with that device current.
constexpr size_t kNoallocBytes = MVM_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kNoallocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the scratch array of the GPU `stream` runs on (the
// current device for the null stream).
int scratch_for_stream(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "mvm_scan_bwd_noalloc: device of the stream");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MVM_ERR_UNSUPPORTED, "mvm_scan_bwd_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return hip_status(e, "mvm_scan_bwd_noalloc: hipGetSymbolAddress(scratch)");
    if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & (kAlign - 1)) != 0)
      return fail(MVM_ERR_HIP, "mvm_scan_bwd_noalloc: scratch address %p is not %zu-byte aligned", p,
                  kAlign);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MVM_OK;
}

}  // namespace

extern "C" {

int64_t mvm_scan_noalloc_scratch_bytes(void) { return static_cast<int64_t>(kNoallocBytes); }

int mvm_scan_bwd_noalloc(const mvm_scan_desc* desc, const void* u, const float* delta,
                         const float* A, const void* Bm, const void* Cm, const float* Dv,
                         const float* ckpt, const void* dy, void* du, float* ddelta, float* dA,
                         void* dB, void* dC, float* dD, void* stream) {
  int rc = check_desc(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = make_geom(desc);
  const bool empty = g.B == 0 || g.L == 0 || g.D == 0;
  if (empty)  // only dA / dD are owed (zero fills): no scratch
    return mvm_scan_bwd(desc, u, delta, A, Bm, Cm, Dv, ckpt, dy, du, ddelta, dA, dB, dC, dD, nullptr,
                        0, stream);
  if (ckpt == nullptr)
    return fail(MVM_ERR_INVALID_ARG,
                "mvm_scan_bwd_noalloc: ckpt is required (recomputing it needs checkpoint-sized scratch)");
  const size_t need = bwd_ws(g, false).total;
  if (need > kNoallocBytes)
    return fail(MVM_ERR_WORKSPACE,
                "mvm_scan_bwd_noalloc: this shape needs %zu bytes of scratch, more than the %zu-byte "
                "static array; call mvm_scan_bwd with a workspace",
                need, kNoallocBytes);
  void* ws = nullptr;
  rc = scratch_for_stream(static_cast<hipStream_t>(stream), &ws);
  if (rc != MVM_OK) return rc;
  return mvm_scan_bwd(desc, u, delta, A, Bm, Cm, Dv, ckpt, dy, du, ddelta, dA, dB, dC, dD, ws,
                      kNoallocBytes, stream);
}

}  // extern "C"

// ----------------------------------------------------------- fused form

namespace {

int check_fused(const mvm_scan_fused_desc* fd) {
  if (fd == nullptr) return fail(MVM_ERR_INVALID_ARG, "fused desc is NULL");
  const int rc = check_desc(&fd->scan);
  if (rc != MVM_OK) return rc;
  if (fd->scan.in_dtype != MVM_F32 || fd->scan.out_dtype != MVM_F32)
    return fail(MVM_ERR_UNSUPPORTED, "the fused scan is float32 only");
  const int64_t st[9] = {fd->dt_stride_b, fd->dt_stride_k, fd->dt_stride_t,
                         fd->y_stride_b, fd->y_stride_k, fd->y_stride_t,
                         fd->z_stride_b, fd->z_stride_k, fd->z_stride_t};
  for (int64_t v : st)
    if (v < 0) return fail(MVM_ERR_INVALID_ARG, "negative stride in fused desc");
  const mvm_scan_desc& sd = fd->scan;
  if (!no_overlap({{sd.batch, fd->dt_stride_b}, {sd.ndir, fd->dt_stride_k}, {sd.seqlen, fd->dt_stride_t},
                   {sd.dim, 1}}) ||
      !no_overlap({{sd.batch, fd->y_stride_b}, {sd.ndir, fd->y_stride_k}, {sd.seqlen, fd->y_stride_t},
                   {sd.dim, 1}}))
    return fail(MVM_ERR_INVALID_ARG, "fused desc: delta_raw or y strides overlap (dim=%lld)",
                (long long)sd.dim);
  if (fd->scan.batch * fd->scan.ndir * fd->scan.seqlen > INT32_MAX)
    return fail(MVM_ERR_UNSUPPORTED, "batch*ndir*seqlen exceeds 2^31-1");
  if (fd->reserved != 0) return fail(MVM_ERR_INVALID_ARG, "fused desc: reserved must be 0");
  return MVM_OK;
}

// z / dz strides (checked only when a gate is given: without one they are 0)
bool z_ok(const mvm_scan_fused_desc* fd) {
  const mvm_scan_desc& sd = fd->scan;
  return no_overlap({{sd.batch, fd->z_stride_b}, {sd.ndir, fd->z_stride_k}, {sd.seqlen, fd->z_stride_t},
                     {sd.dim, 1}});
}

mvm::Geom fused_geom(const mvm_scan_fused_desc* fd) {
  mvm::Geom g = make_geom(&fd->scan);
  g.dsb = fd->dt_stride_b; g.dsk = fd->dt_stride_k; g.dst = fd->dt_stride_t;
  g.ysb = fd->y_stride_b;  g.ysk = fd->y_stride_k;  g.yst = fd->y_stride_t;
  g.zsb = fd->z_stride_b;  g.zsk = fd->z_stride_k;  g.zst = fd->z_stride_t;
  g.a_log = fd->a_is_log != 0 ? 1 : 0;
  return g;
}

// fused backward workspace: the plain backward's pieces and the dt_bias
// partials (the gate needs none: it is undone in the scan's staging)
struct FusedBwdWs {
  BwdWs base;
  size_t part_db = 0, total = 0;
};
FusedBwdWs fused_bwd_ws(const mvm::Geom& g) {
  FusedBwdWs w;
  w.base = bwd_ws(g, false);
  w.part_db = align_up(static_cast<size_t>(g.B * g.K * g.nchunk * g.D) * sizeof(double));
  w.total = w.base.total + w.part_db;
  return w;
}

int check_ws(const char* who, void* ws, size_t have, size_t need) {
  if (have < need) return fail(MVM_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu needed", who, have, need);
  if (need > 0 && ws == nullptr) return fail(MVM_ERR_WORKSPACE, "%s: workspace is NULL", who);
  if ((reinterpret_cast<uintptr_t>(ws) & (kAlign - 1)) != 0)
    return fail(MVM_ERR_WORKSPACE, "%s: workspace must be %zu-byte aligned", who, kAlign);
  return MVM_OK;
}

}  // namespace

extern "C" {

int mvm_scan_fused_validate(const mvm_scan_fused_desc* desc) {
  const int rc = check_fused(desc);
  return rc == MVM_OK ? ok() : rc;
}

int64_t mvm_scan_fused_workspace_bytes(const mvm_scan_fused_desc* desc, int which, int gate) {
  const int rc = check_fused(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = fused_geom(desc);
  if (which == 0) return static_cast<int64_t>(fwd_ws(g).total);
  (void)gate;  // the gate adds no workspace
  if (which == 1) return static_cast<int64_t>(fused_bwd_ws(g).total);
  return fail(MVM_ERR_INVALID_ARG, "which=%d must be 0 or 1", which);
}

int mvm_scan_fused_fwd(const mvm_scan_fused_desc* desc, const float* u, const float* delta_raw,
                       const float* delta_bias, const float* A, const float* Bm, const float* Cm,
                       const float* Dv, const float* z, float* y, float* y_raw, float* ckpt,
                       void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_fused(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = fused_geom(desc);
  const bool empty = g.B == 0 || g.L == 0 || g.D == 0;
  if (!empty) {
    if (!u || !delta_raw || !A || !Bm || !Cm || !Dv || !y)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_fwd: NULL input or y pointer");
    if (z && !z_ok(desc)) return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_fwd: z strides overlap");
    if ((reinterpret_cast<uintptr_t>(ckpt) & 15u) != 0)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_fwd: ckpt must be 16-byte aligned");
  }
  const FwdWs w = fwd_ws(g);
  rc = check_ws("mvm_scan_fused_fwd", workspace, workspace_bytes, w.total);
  if (rc != MVM_OK) return rc;
  if (empty) return ok();
  char* ws = static_cast<char*>(workspace);
  mvm::FwdBufs b{u, delta_raw, A, Bm, Cm, Dv, y, ckpt,
                 reinterpret_cast<float*>(ws), reinterpret_cast<float*>(ws + w.agg_h),
                 delta_bias, z, y_raw};
  return hip_status(mvm::launch_fused_fwd(g, b, static_cast<hipStream_t>(stream)),
                    "mvm_scan_fused_fwd launch");
}

int mvm_scan_fused_bwd(const mvm_scan_fused_desc* desc, const float* u, const float* delta_raw,
                       const float* delta_bias, const float* A, const float* Bm, const float* Cm,
                       const float* Dv, const float* z, const float* y_raw, const float* ckpt,
                       const float* dy, float* du, float* ddelta_raw, float* ddelta_bias,
                       float* dA, float* dB, float* dC, float* dD, float* dz, void* workspace,
                       size_t workspace_bytes, void* stream) {
  int rc = check_fused(desc);
  if (rc != MVM_OK) return rc;
  const mvm::Geom g = fused_geom(desc);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool empty = g.B == 0 || g.L == 0 || g.D == 0;
  const bool gate = z != nullptr;
  if (g.D > 0 && (!dA || !dD)) return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_bwd: NULL dA or dD");
  if (g.D > 0 && delta_bias && !ddelta_bias)
    return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_bwd: delta_bias given but ddelta_bias is NULL");
  if (!empty) {
    if (!u || !delta_raw || !A || !Bm || !Cm || !Dv || !dy || !ckpt)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_bwd: NULL input pointer (ckpt is required)");
    if (!du || !ddelta_raw || !dB || !dC)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_bwd: NULL output pointer");
    if (gate && (!y_raw || !dz))
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_bwd: a gate needs y_raw and dz");
    if (gate && !z_ok(desc)) return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_bwd: z strides overlap");
    if ((reinterpret_cast<uintptr_t>(ckpt) & 15u) != 0)
      return fail(MVM_ERR_INVALID_ARG, "mvm_scan_fused_bwd: ckpt must be 16-byte aligned");
  }
  const FusedBwdWs w = fused_bwd_ws(g);
  if (!empty) {
    rc = check_ws("mvm_scan_fused_bwd", workspace, workspace_bytes, w.total);
    if (rc != MVM_OK) return rc;
  }
  if (empty) {
    hipError_t e = mvm::launch_fill(dA, g.K * g.D * g.N, 0.f, s);
    if (e == hipSuccess) e = mvm::launch_fill(dD, g.K * g.D, 0.f, s);
    if (e == hipSuccess && ddelta_bias) e = mvm::launch_fill(ddelta_bias, g.K * g.D, 0.f, s);
    return hip_status(e, "mvm_scan_fused_bwd fill");
  }
  char* ws = static_cast<char*>(workspace);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = ws + off;
    off += bytes;
    return bytes ? p : nullptr;
  };
  float* agg_mu = reinterpret_cast<float*>(take(w.base.agg_mu));
  float* agg_s = reinterpret_cast<float*>(take(w.base.agg_s));
  double* part_dA = reinterpret_cast<double*>(take(w.base.part_dA));
  double* part_dD = reinterpret_cast<double*>(take(w.base.part_dD));
  float* part_bc = reinterpret_cast<float*>(take(w.base.part_bc));
  double* part_db = reinterpret_cast<double*>(take(w.part_db));
  mvm::BwdBufs b{u, delta_raw, A, Bm, Cm, Dv, ckpt, dy, du, ddelta_raw, dA, dB, dC, dD,
                 agg_mu, agg_s, part_dA, part_dD, part_bc, delta_bias,
                 delta_bias ? ddelta_bias : nullptr, part_db,
                 gate ? z : nullptr, gate ? y_raw : nullptr, gate ? dz : nullptr};
  return hip_status(mvm::launch_fused_bwd(g, b, s), "mvm_scan_fused_bwd launch");
}

}  // extern "C"

namespace {

int check_conv(const mvm_conv_desc* d) {
  if (d == nullptr) return fail(MVM_ERR_INVALID_ARG, "conv desc is NULL");
  if (d->batch < 0 || d->seqlen < 0 || d->dim < 0)
    return fail(MVM_ERR_INVALID_ARG, "negative size in conv desc");
  if (d->ndir < 1) return fail(MVM_ERR_INVALID_ARG, "conv ndir=%lld must be >= 1", (long long)d->ndir);
  if (d->kwidth < 1 || d->kwidth > MVM_CONV_MAX_KWIDTH)
    return fail(MVM_ERR_UNSUPPORTED, "kwidth=%lld unsupported (1..%d)", (long long)d->kwidth,
                MVM_CONV_MAX_KWIDTH);
  const int64_t st[9] = {d->x_stride_b, d->x_stride_k, d->x_stride_t,
                         d->y_stride_b, d->y_stride_k, d->y_stride_t,
                         d->dx_stride_b, d->dx_stride_k, d->dx_stride_t};
  for (int64_t v : st)
    if (v < 0) return fail(MVM_ERR_INVALID_ARG, "negative stride in conv desc");
  if (d->seqlen > 1 && (d->x_stride_t < d->dim || d->y_stride_t < d->dim || d->dx_stride_t < d->dim))
    return fail(MVM_ERR_INVALID_ARG, "conv row stride overlaps channels");
  if (d->batch * d->ndir > 65535) return fail(MVM_ERR_UNSUPPORTED, "batch*ndir exceeds 65535");
  return MVM_OK;
}

mvm::ConvGeom conv_geom(const mvm_conv_desc* d) {
  mvm::ConvGeom g;
  g.B = d->batch; g.L = d->seqlen; g.D = d->dim; g.K = d->ndir;
  g.xsb = d->x_stride_b; g.xsk = d->x_stride_k; g.xst = d->x_stride_t;
  g.ysb = d->y_stride_b; g.ysk = d->y_stride_k; g.yst = d->y_stride_t;
  g.dxsb = d->dx_stride_b; g.dxsk = d->dx_stride_k; g.dxst = d->dx_stride_t;
  g.tok = d->seq_to_tok;
  return g;
}

}  // namespace

extern "C" {

int mvm_conv_validate(const mvm_conv_desc* desc) {
  const int rc = check_conv(desc);
  return rc == MVM_OK ? ok() : rc;
}

int64_t mvm_conv_workspace_bytes(const mvm_conv_desc* desc) {
  const int rc = check_conv(desc);
  if (rc != MVM_OK) return rc;
  return static_cast<int64_t>(
      align_up(sizeof(float) * mvm::conv_partial_floats(conv_geom(desc), static_cast<int>(desc->kwidth))));
}

int mvm_conv_silu_fwd(const mvm_conv_desc* desc, const float* x, const float* w,
                      const float* bias, float* y, void* stream) {
  const int rc = check_conv(desc);
  if (rc != MVM_OK) return rc;
  const mvm::ConvGeom g = conv_geom(desc);
  if (g.B == 0 || g.L == 0 || g.D == 0) return ok();
  if (!x || !w || !bias || !y) return fail(MVM_ERR_INVALID_ARG, "mvm_conv_silu_fwd: NULL pointer");
  return hip_status(mvm::launch_conv_fwd(g, static_cast<int>(desc->kwidth), x, w, bias, y,
                                         static_cast<hipStream_t>(stream)),
                    "mvm_conv_silu_fwd launch");
}

int mvm_conv_silu_bwd(const mvm_conv_desc* desc, const float* x, const float* w,
                      const float* bias, const float* dy, float* dx, float* dw, float* dbias,
                      void* workspace, size_t workspace_bytes, void* stream) {
  const int rc = check_conv(desc);
  if (rc != MVM_OK) return rc;
  const mvm::ConvGeom g = conv_geom(desc);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int kc = static_cast<int>(desc->kwidth);
  if (g.D > 0 && (!dw || !dbias)) return fail(MVM_ERR_INVALID_ARG, "mvm_conv_silu_bwd: NULL dw/dbias");
  if (g.B == 0 || g.L == 0 || g.D == 0) {
    hipError_t e = mvm::launch_fill(dw, g.K * g.D * kc, 0.f, s);
    if (e == hipSuccess) e = mvm::launch_fill(dbias, g.K * g.D, 0.f, s);
    return hip_status(e, "mvm_conv_silu_bwd fill");
  }
  if (!x || !w || !bias || !dy || !dx) return fail(MVM_ERR_INVALID_ARG, "mvm_conv_silu_bwd: NULL pointer");
  const size_t need = align_up(sizeof(float) * mvm::conv_partial_floats(g, kc));
  if (workspace_bytes < need || workspace == nullptr)
    return fail(MVM_ERR_WORKSPACE, "mvm_conv_silu_bwd: workspace %zu bytes < %zu needed", workspace_bytes, need);
  return hip_status(mvm::launch_conv_bwd(g, kc, x, w, bias, dy, dx, dw, dbias,
                                         static_cast<float*>(workspace), s),
                    "mvm_conv_silu_bwd launch");
}

int mvm_selftest_lanes(float* out, void* stream) {
  if (out == nullptr) return fail(MVM_ERR_INVALID_ARG, "out is NULL");
  return hip_status(mvm::launch_selftest_lanes(out, static_cast<hipStream_t>(stream)), "selftest");
}

}  // extern "C"

namespace {

// MVM_NORM_MAX_ROWS: the forward's grid (4 rows per 256-thread workgroup)
// stays below 2^31 threads
constexpr int64_t kNormMaxRows = MVM_NORM_MAX_ROWS;

int check_norm(const mvm_norm_desc* d) {
  if (d == nullptr) return fail(MVM_ERR_INVALID_ARG, "norm desc is NULL");
  if (d->rows < 0) return fail(MVM_ERR_INVALID_ARG, "norm rows=%lld < 0", (long long)d->rows);
  if (d->rows > kNormMaxRows)
    return fail(MVM_ERR_UNSUPPORTED, "norm rows=%lld exceeds %lld", (long long)d->rows,
                (long long)kNormMaxRows);
  if (d->cols < 1 || d->cols > MVM_NORM_MAX_COLS)
    return fail(MVM_ERR_UNSUPPORTED, "norm cols=%lld unsupported (1..%d)", (long long)d->cols,
                MVM_NORM_MAX_COLS);
  if (d->x_stride < d->cols || d->y_stride < d->cols)
    return fail(MVM_ERR_INVALID_ARG, "norm row strides must be >= cols");
  if (!(d->eps >= 0.f) || d->eps > 1e30f)
    return fail(MVM_ERR_INVALID_ARG, "norm eps must be finite and >= 0");
  if (d->reserved != 0) return fail(MVM_ERR_INVALID_ARG, "norm desc reserved field must be 0");
  return MVM_OK;
}

mvm::NormGeom norm_geom(const mvm_norm_desc* d) {
  mvm::NormGeom g;
  g.rows = d->rows; g.cols = d->cols; g.xs = d->x_stride; g.ys = d->y_stride; g.eps = d->eps;
  return g;
}

}  // namespace

extern "C" {

int mvm_norm_validate(const mvm_norm_desc* desc) {
  const int rc = check_norm(desc);
  return rc == MVM_OK ? ok() : rc;
}

int64_t mvm_norm_workspace_bytes(const mvm_norm_desc* desc) {
  const int rc = check_norm(desc);
  if (rc != MVM_OK) return rc;
  return static_cast<int64_t>(align_up(sizeof(float) * mvm::norm_partial_floats(norm_geom(desc))));
}

int mvm_layernorm_fwd(const mvm_norm_desc* desc, const float* x, const float* gamma,
                      const float* beta, float* y, float* mean, float* rstd, void* stream) {
  const int rc = check_norm(desc);
  if (rc != MVM_OK) return rc;
  if (desc->rows == 0) return ok();
  if (!x || !gamma || !beta || !y || !mean || !rstd)
    return fail(MVM_ERR_INVALID_ARG, "mvm_layernorm_fwd: NULL pointer");
  return hip_status(mvm::launch_norm_fwd(norm_geom(desc), x, gamma, beta, y, mean, rstd,
                                         static_cast<hipStream_t>(stream)),
                    "mvm_layernorm_fwd launch");
}

int mvm_layernorm_bwd(const mvm_norm_desc* desc, const float* x, const float* gamma,
                      const float* mean, const float* rstd, const float* dy, const float* dres,
                      float* dx, float* dgamma, float* dbeta, void* workspace,
                      size_t workspace_bytes, void* stream) {
  int rc = check_norm(desc);
  if (rc != MVM_OK) return rc;
  if (!gamma || !dgamma || !dbeta)
    return fail(MVM_ERR_INVALID_ARG, "mvm_layernorm_bwd: NULL gamma, dgamma or dbeta");
  if (desc->rows > 0 && (!x || !mean || !rstd || !dy || !dx))
    return fail(MVM_ERR_INVALID_ARG, "mvm_layernorm_bwd: NULL pointer");
  const mvm::NormGeom g = norm_geom(desc);
  rc = check_ws("mvm_layernorm_bwd", workspace, workspace_bytes,
                align_up(sizeof(float) * mvm::norm_partial_floats(g)));
  if (rc != MVM_OK) return rc;
  return hip_status(mvm::launch_norm_bwd(g, x, gamma, mean, rstd, dy, dres, dx, dgamma, dbeta,
                                         static_cast<float*>(workspace),
                                         static_cast<hipStream_t>(stream)),
                    "mvm_layernorm_bwd launch");
}

}  // extern "C"

// ------------------------------------------------------------------ AdamW

static_assert(MVM_ADAMW_TENSORS_PER_LAUNCH == mvm::kAdamPerLaunch,
              "header and kernel agree on the tensors per launch");

extern "C" {

int mvm_adamw_step(const mvm_adamw_tensor* tensors, int32_t ntensors,
                   const mvm_adamw_hparams* hp, const float* step, float* exp_avg,
                   float* exp_avg_sq, void* stream) {
  if (hp == nullptr) return fail(MVM_ERR_INVALID_ARG, "mvm_adamw_step: hparams is NULL");
  if (hp->reserved != 0) return fail(MVM_ERR_INVALID_ARG, "mvm_adamw_step: reserved must be 0");
  if (!(hp->lr >= 0.f) || !(hp->beta1 >= 0.f && hp->beta1 < 1.f) ||
      !(hp->beta2 >= 0.f && hp->beta2 < 1.f) || !(hp->eps > 0.f) || !(hp->weight_decay >= 0.f))
    return fail(MVM_ERR_INVALID_ARG,
                "mvm_adamw_step: bad hyperparameters (lr=%g beta1=%g beta2=%g eps=%g wd=%g)",
                hp->lr, hp->beta1, hp->beta2, hp->eps, hp->weight_decay);
  if (ntensors < 0) return fail(MVM_ERR_INVALID_ARG, "mvm_adamw_step: ntensors=%d < 0", ntensors);
  if (ntensors == 0) return ok();
  if (tensors == nullptr) return fail(MVM_ERR_INVALID_ARG, "mvm_adamw_step: tensors is NULL");
  if (!step || !exp_avg || !exp_avg_sq)
    return fail(MVM_ERR_INVALID_ARG, "mvm_adamw_step: NULL step or state buffer");
  for (int32_t i = 0; i < ntensors; ++i) {
    const mvm_adamw_tensor& t = tensors[i];
    if (t.numel < 0 || t.state_offset < 0)
      return fail(MVM_ERR_INVALID_ARG, "mvm_adamw_step: tensor %d: numel=%lld state_offset=%lld",
                  i, (long long)t.numel, (long long)t.state_offset);
    if (t.numel > 0 && (!t.param || !t.grad))
      return fail(MVM_ERR_INVALID_ARG, "mvm_adamw_step: tensor %d: NULL param or grad", i);
    if (t.numel > (int64_t{1} << 40))
      return fail(MVM_ERR_UNSUPPORTED, "mvm_adamw_step: tensor %d: numel=%lld too large", i,
                  (long long)t.numel);
  }
  mvm::AdamLaunch a{};
  a.lr = hp->lr; a.beta1 = hp->beta1; a.beta2 = hp->beta2; a.eps = hp->eps;
  a.wd = hp->weight_decay;
  a.step = step; a.m = exp_avg; a.v = exp_avg_sq;
  auto flush = [&]() -> int {
    const int rc = hip_status(mvm::launch_adamw(a, static_cast<hipStream_t>(stream)),
                              "mvm_adamw_step launch");
    a.nt = 0;
    a.nblk = 0;
    return rc;
  };
  for (int32_t i = 0; i < ntensors; ++i) {
    const mvm_adamw_tensor& t = tensors[i];
    if (t.numel == 0) continue;
    const int64_t nb = ceil_div(t.numel, mvm::kAdamElems);
    if (a.nt == mvm::kAdamPerLaunch || a.nblk + nb > INT32_MAX) {
      const int rc = flush();
      if (rc != MVM_OK) return rc;
    }
    mvm::AdamSlice& sl = a.t[a.nt++];
    sl.p = t.param;
    sl.g = t.grad;
    sl.n = t.numel;
    sl.soff = t.state_offset;
    sl.blk0 = a.nblk;
    a.nblk += static_cast<int32_t>(nb);
  }
  return a.nt > 0 ? flush() : ok();
}

}  // extern "C"
