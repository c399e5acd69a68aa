// Shared device-side helpers for the gfx950 selective-scan kernels.
//
// Lane layout used by every scan kernel (wave64):
//   lane = 4 * c + g,  c = channel within the wave (0..15), g = state group
//   (0..3).  Lane (c, g) holds states n = 4g .. 4g+3 of channel c in VGPRs,
//   so a wave covers 16 channels x 16 states and a 256-thread workgroup
//   covers 64 channels.  Sums over the 16 states of one channel are two DPP
//   quad-permute adds; sums over the 16 channels of a wave use
//   v_permlane32_swap / v_permlane16_swap (gfx950) and two DPP row rotates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace mvm {

constexpr int kSub = 16;          // scan positions per staged tile
constexpr int kCk = 8;            // checkpoint interval (half a tile)
constexpr int kThreads = 256;     // threads per workgroup (4 waves)
constexpr int kChPerWave = 16;
constexpr int kChPerBlock = 64;
constexpr int kStatePad = 16;     // states per channel in every internal buffer
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Up to this many time chunks, each chunk of the main scan folds the chunk
// aggregates it needs itself (one launch fewer); beyond it a separate carry
// pass folds them once, so no block waits on a long chain of loads.
constexpr int64_t kFoldMax = 8;

struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
  // round to nearest even, NaN stays NaN: one v_cvt_pk_bf16_f32 on gfx950
  bf16_t r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  return r;
}

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }
template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = from_f32<T>(v); }

// Token row read / written at scan position t.  The table is read through
// the constant address space, so a wave-uniform lookup is a scalar load
// (K$, lgkmcnt) and never waits behind the vector loads in flight.  Table
// entries are clamped to [0, L) so that a malformed remap table cannot
// address outside the tensors (scalar work on a wave-uniform value).
typedef __attribute__((address_space(4))) const int32_t const_i32;
__device__ __forceinline__ int64_t token_row(const int32_t* tok, int64_t t, int64_t L) {
  if (tok == nullptr) return t;
  const int64_t r = ((const const_i32*)tok)[t];  // generic -> constant addrspacecast
  return r < 0 ? 0 : (r >= L ? L - 1 : r);
}

// Pointwise pieces of the fused block prologue / epilogue
// (mamba_block.py:180-181, :190), on the transcendental unit (v_exp_f32,
// v_log_f32, v_rcp_f32: a few ulp) rather than the libm routines, which
// cost ~10x the instructions in VALU-bound kernels.
//
// softplus: max(x, 0) + log(1 + y), y = e^-|x| in (0, 1].
// log(1 + y) = ln2 * log2(u) + (y - (u - 1)) with u = fl(1 + y): the second
// term is the rounding error of u (exact), so the sum keeps y's relative
// precision for small y (to first order in that rounding), and v_log_f32 is
// within 2 ulp of log2 near 1 (measured on MI355X); softplus within 30 ulp
// over x in [-30, 20], the error of e^-|x| from the rounded product
// |x| log2(e) included.  torch's threshold (x > 20 -> x) needs no branch of
// its own: there log(1 + y) < 2.1e-9 is below half an ulp of x, so the sum
// rounds to x (and +inf stays +inf, NaN stays NaN).
// The sigmoid of the same x comes from the same exponential:
// sigmoid(x) = (x >= 0 ? 1 : y) / (1 + y).
__device__ __forceinline__ float softplus_f(float x) {
  const float y = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e);
  const float u = 1.f + y;
  return fmaxf(x, 0.f) + fmaf(kLn2, __builtin_amdgcn_logf(u), y - (u - 1.f));
}
__device__ __forceinline__ void softplus_sigmoid(float x, float& sp, float& sg) {
  const float y = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e);
  const float u = 1.f + y;
  sp = fmaxf(x, 0.f) + fmaf(kLn2, __builtin_amdgcn_logf(u), y - (u - 1.f));
  sg = (x >= 0.f ? 1.f : y) * __builtin_amdgcn_rcpf(u);
}
// 1 / (1 + e^-x); saturates to 0 / 1 without NaN for large |x|
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
// A of one (direction, channel, state): the array holds A itself, or A_log
// with A = -exp(A_log) (mamba_block.py:184) when a_log is set.  Read once
// per (d, n) by each block, so the accurate expf costs nothing measurable.
__device__ __forceinline__ float load_A(const float* A, int64_t i, int a_log) {
  const float v = A[i];
  return a_log ? -expf(v) : v;
}

// a[j] = A[d, 4g + j] for the 4 states of a lane's group, 0 for states
// >= N or an invalid channel (A = -exp(A_log) when a_log is set).  The 4
// loads go to clamped, in-bounds indices and are issued together before
// any is used (a load under the validity branch would be waited for one at
// a time: 4 memory latencies in every block's prologue).
__device__ __forceinline__ void load_ax4(float (&a)[4], const float* A, int64_t row, int grp, int N,
                                         bool valid, int a_log) {
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = 4 * grp + j;
    v[j] = A[row + (n < N ? n : 0)];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) a[j] = (valid && 4 * grp + j < N) ? (a_log ? -expf(v[j]) : v[j]) : 0.f;
}

// 2^x on the transcendental unit (v_exp_f32); callers pre-scale by log2(e).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- DPP ops
// dpp_ctrl encodings (GCN/CDNA): quad_perm = sel0 | sel1<<2 | sel2<<4 | sel3<<6,
// row_ror:r = 0x120 + r.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kRowRor8 = 0x128;
constexpr int kRowRor4 = 0x124;

// Sum over the 4 lanes of a channel (lane bits 0-1); every lane gets the sum.
__device__ __forceinline__ float sum_groups(float x) {
  x += dpp<kQuadXor1>(x);
  x += dpp<kQuadXor2>(x);
  return x;
}

// v_permlane{32,16}_swap return both swapped registers.  The builtin's two
// results are read through a 64-bit bit_cast: in this toolchain, indexing
// the returned vector (r[1]) re-reads element 0, so the second half would be
// lost.
__device__ __forceinline__ float swap_sum32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a),
                                                 __builtin_bit_cast(unsigned, b), false, false);
  const unsigned long long w = __builtin_bit_cast(unsigned long long, r);
  return __builtin_bit_cast(float, static_cast<unsigned>(w)) +
         __builtin_bit_cast(float, static_cast<unsigned>(w >> 32));
}
__device__ __forceinline__ float swap_sum16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a),
                                                 __builtin_bit_cast(unsigned, b), false, false);
  const unsigned long long w = __builtin_bit_cast(unsigned long long, r);
  return __builtin_bit_cast(float, static_cast<unsigned>(w)) +
         __builtin_bit_cast(float, static_cast<unsigned>(w >> 32));
}

// v_permlane32_swap: lanes 32..63 of `a` trade places with lanes 0..31 of
// `b`.  Afterwards a + b holds, in lanes 0..31, a summed over lanes (l, l+32)
// and, in lanes 32..63, b summed over (l-32, l).
__device__ __forceinline__ float pair_reduce32(float a, float b) { return swap_sum32(a, b); }

// v_permlane16_swap: odd 16-lane rows of `a` trade places with even rows of
// `b`.  Afterwards a + b holds, in rows 0 and 2, a summed over row pairs
// (0,1) / (2,3) and, in rows 1 and 3, b summed over the same pairs.
__device__ __forceinline__ float pair_reduce16(float a, float b) { return swap_sum16(a, b); }

// Sum over the 16 channels of a wave of four per-lane values v[0..3] (the
// lane's states 4g+j).  Returns, in lane (c, g) with j = (lane >> 4) & 3, the
// channel sum of state 4g + j; lanes with equal (g, j) hold equal results.
__device__ __forceinline__ float channel_reduce4(float v0, float v1, float v2, float v3) {
  const float s02 = pair_reduce32(v0, v2);  // bit5=0 -> state j=0, bit5=1 -> j=2
  const float s13 = pair_reduce32(v1, v3);  // bit5=0 -> j=1,        bit5=1 -> j=3
  float s = pair_reduce16(s02, s13);        // row r=(bit5,bit4) -> j = r
  s += dpp<kRowRor8>(s);                    // lane bit 3
  s += dpp<kRowRor4>(s);                    // lane bit 2
  return s;
}

// ------------------------------------------------------ tile staging
// A tile is kSub consecutive scan positions of one workgroup's 64 channels.
// Wave w stages and writes back positions w + 4r (r = 0..3) of each tile:
// for channel-indexed tensors lane l holds channel l of those rows (one load
// instruction reads 64 consecutive channels of one token row); for
// state-indexed tensors (B, C) lane l holds state l & 15 of row
// w + 4 (l >> 4).  The 4 token rows of a wave are looked up once per tile
// (wave-uniform, in SGPRs) and shared by every tensor staged or written
// back for that tile.

// Token row of scan position p in [0, L): the remap table entry clamped to
// [0, L) (TOK), or p itself (identity order).  The table is read through the
// constant address space: a wave-uniform lookup is a scalar load.
template <bool TOK>
__device__ __forceinline__ int32_t row_of(const int32_t* tok, int64_t p, int64_t L) {
  if constexpr (TOK) {
    const int32_t r = ((const const_i32*)tok)[p];
    return r < 0 ? 0 : (r >= L ? static_cast<int32_t>(L - 1) : r);
  } else {
    return static_cast<int32_t>(p);
  }
}

struct TileRows {
  int32_t r[4];  // token rows of positions ts + wave + 4r
};

// Rows of a wave's 4 positions of the tile starting at ts.  Positions past
// L are clamped to L - 1: their values are staged but never used.  All in
// 32 bits (L < 2^31): wave-uniform values stay in SGPRs, with no 64-bit
// compares (which the scalar unit lacks) moved onto the VALU.
template <bool TOK>
__device__ __forceinline__ TileRows tile_rows(const int32_t* tok, int32_t ts, int32_t L, int tid) {
  const int32_t wrow = __builtin_amdgcn_readfirstlane(tid >> 6);
  TileRows t;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int32_t p = ts + wrow + 4 * r;
    const int32_t pc = p < L ? p : L - 1;
    if constexpr (TOK) {
      const int32_t v = ((const const_i32*)tok)[pc];
      t.r[r] = v < 0 ? 0 : (v >= L ? L - 1 : v);
    } else {
      t.r[r] = pc;
    }
  }
  return t;
}

// Row offsets are computed in IdxT: int32_t when every element offset of
// the call within one (batch, direction) slab is below 2^30 (checked on the
// host), so that its byte offset fits in 32 bits; else int64_t.  `p` points
// at the block's first channel of its (b, k) slab.
//
// In the int32_t instantiations an access is that block-uniform base plus a
// 32-bit byte offset: the row's part is wave-uniform (a scalar multiply),
// the lane's part a VGPR, so it compiles to one global access with the base
// in SGPRs and the offset in a VGPR (saddr form), with no 64-bit per-lane
// pointer held in VGPRs and no 64-bit address arithmetic on the VALU.
template <typename T>
__device__ __forceinline__ T* at_bytes(T* base, uint32_t off) {
  using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return reinterpret_cast<T*>(reinterpret_cast<C*>(base) + off);
}
// Element (row, lane) of a slab: p[row * st + lc], with lane_off = lc *
// sizeof(T) precomputed by the caller for the 32-bit form.
template <typename T, typename IdxT>
__device__ __forceinline__ T& row_elem(T* p, int32_t row, IdxT st, int lc, uint32_t lane_off) {
  if constexpr (std::is_same<IdxT, int32_t>::value) {
    return *at_bytes(p, static_cast<uint32_t>(row * st) * static_cast<uint32_t>(sizeof(T)) + lane_off);
  } else {
    return (p + static_cast<IdxT>(row) * st)[lc];
  }
}

// Channel-indexed tile rows: v[r] = p[rows.r[r] * st + lc], lc = the
// lane's channel, or channel 0 for out-of-range channels (always in bounds,
// so no load waits behind a divergent branch; mask_xtile zeroes them when
// the tile is staged).  Nothing here consumes the loaded values, so a
// prefetch issued before a tile's math is not waited for until the next
// tile is staged.
template <typename T, typename IdxT>
__device__ __forceinline__ void load_rows(float (&v)[4], const T* __restrict__ p, const TileRows& rows,
                                          IdxT st, int lc) {
  const uint32_t lb = static_cast<uint32_t>(lc) * static_cast<uint32_t>(sizeof(T));
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = to_f32(row_elem(p, rows.r[r], st, lc, lb));
}
// all_in: every channel of the block is < D (block-uniform), so nothing is
// masked and the selects are skipped by a scalar branch
__device__ __forceinline__ void mask_xtile(float (&v)[4], bool cok, bool all_in) {
  if (!all_in) {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = cok ? v[r] : 0.f;
  }
}

// LDS row of the state-indexed value a thread stages (row w + 4 (l >> 4)).
__device__ __forceinline__ int stile_row(int tid) { return (tid >> 6) + 4 * ((tid >> 4) & 3); }

// State-indexed tile value of this thread: state tid & 15 of row
// stile_row(tid), from p at the (b, k) slab's start; states >= N read
// state 0 and are zeroed by mask_stile when the tile is staged.
// In the 32-bit form the lane's row is chosen among the wave's four
// (scalar) rows with two bit-selects and its byte offset formed in a VGPR,
// so the address is the SGPR base plus one VGPR offset, with no per-lane
// pointer or branch.
template <typename T, typename IdxT>
__device__ __forceinline__ float load_state(const T* __restrict__ p, const TileRows& rows, IdxT st,
                                            int N, int tid) {
  const int q = (tid >> 4) & 3, n = tid & 15;
  const int nc = n < N ? n : 0;
  if constexpr (std::is_same<IdxT, int32_t>::value) {
    constexpr uint32_t kSz = static_cast<uint32_t>(sizeof(T));
    const int32_t lo = (q & 1) ? rows.r[1] : rows.r[0];
    const int32_t hi = (q & 1) ? rows.r[3] : rows.r[2];
    const int32_t row = (q & 2) ? hi : lo;
    return to_f32(*at_bytes(p, static_cast<uint32_t>(row * st + nc) * kSz));
  } else {
    const int32_t row = q == 0 ? rows.r[0] : (q == 1 ? rows.r[1] : (q == 2 ? rows.r[2] : rows.r[3]));
    return to_f32((p + static_cast<IdxT>(row) * st)[nc]);
  }
}
__device__ __forceinline__ float mask_stile(float x, int64_t N, int tid) {
  return (N >= kStatePad || (tid & 15) < N) ? x : 0.f;  // uniform test first
}

__device__ __forceinline__ void store_xtile(float (*s)[kChPerBlock], const float (&v)[4], int tid) {
#pragma unroll
  for (int r = 0; r < 4; ++r) s[(tid >> 6) + 4 * r][tid & 63] = v[r];
}

// Block-uniform kernel-argument values copied into SGPRs of their own, so
// that the registers of the 64-byte argument loads they came from do not
// stay live (and are not spilled whole) across the sweep.  A pointer keeps
// the global address space.
template <typename T>
__device__ __forceinline__ T own_sc(T v) {
  asm volatile("" : "+s"(v));
  return v;
}
template <typename T>
__device__ __forceinline__ T* own_ptr(T* p) {
  uint64_t v = reinterpret_cast<uint64_t>(p);
  asm volatile("" : "+s"(v));
  return (T*)(__attribute__((address_space(1))) T*)v;
}

}  // namespace mvm
