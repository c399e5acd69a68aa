/*
 * mvm_scan.h -- C ABI of the MI355X selective-scan library (libmvm_scan.so).
 *
 * This is the drop-in boundary for the reference's scan entry points.  The
 * reference binds its fused Metal kernels through mx.fast.metal_kernel; each
 * function below replaces one of those bindings (citations are relative to
 * the reference repository root):
 *
 *   mvm_scan_fwd   replaces _launch_fused_fwd + FUSED_FWD_SOURCE
 *                  (mlx_vision_mamba/mamba_metal_fused.py:148-179, :21-63),
 *                  which serves scan_fn(x, delta, A, B, C, D) -> y
 *                  (mamba_block.py:20-27, called at :187).  With ckpt == NULL
 *                  it is also the forward-only "metal" mode
 *                  (mamba_metal.py:230-242).
 *   mvm_scan_bwd   replaces _fused_scan_core_vjp + _launch_fused_bwd +
 *                  FUSED_BWD_SOURCE and its MLX reductions
 *                  (mamba_metal_fused.py:236-250, :182-226, :66-145); it
 *                  returns the six fully reduced gradients
 *                  (du, ddelta, dA, dB, dC, dD).
 *   direction descriptor (ndir, seq_to_tok)
 *                  replaces the materialised permute / reverse copies of
 *                  MultiDirectionalMambaBlock._apply_direction
 *                  (mamba_block.py:407-533) and the helpers at :254-338.
 *
 * Conventions
 *   - C linkage, no exceptions cross the boundary.  Every entry point returns
 *     MVM_OK (0) or a negative MVM_ERR_* code; mvm_last_error() gives a
 *     thread-local message for the last failure on the calling thread.
 *   - Arguments are validated on the host before anything is launched.
 *   - All device buffers are owned by the caller.  The library never
 *     allocates device memory: scratch space comes in through `workspace`,
 *     sized by mvm_scan_workspace_bytes().
 *   - Work is enqueued on `stream` (a hipStream_t) and is asynchronous.
 *   - Results are deterministic: no atomics, fixed reduction order.
 *   - Offsets are 64-bit everywhere (B*L*D*N may exceed 2^31).
 *
 * Layout
 *   Channel-indexed tensors u, delta, y, dy, du, ddelta hold element
 *   (b, k, t, d) at  b*x_stride_b + k*x_stride_k + t*x_stride_t + d.
 *   State-indexed tensors Bm, Cm, dB, dC hold (b, k, t, n) at
 *   b*bc_stride_b + k*bc_stride_k + t*bc_stride_t + n.
 *   A, dA: (ndir, dim, dstate) contiguous.  Dv, dD: (ndir, dim) contiguous.
 *   With ndir == 1 and contiguous (batch, seqlen, dim) tensors this is the
 *   reference's (B, L, D_inner) / (B, L, N) / (D_inner, N) / (D_inner,).
 *   t is a token row; when seq_to_tok != NULL, scan position s of
 *   direction k reads and writes token row seq_to_tok[k*seqlen + s].
 *   Outputs are written through the strides of their inputs, so every
 *   strided layout must be non-overlapping (ordered by stride, each stride
 *   at least the span of the smaller dimensions; a stride-0 broadcast over
 *   a dimension of size > 1 is rejected with MVM_ERR_INVALID_ARG).
 *   Each row of seq_to_tok must be a permutation of 0..seqlen-1: the kernels
 *   only clamp entries into [0, seqlen), so a row that misses a token leaves
 *   that token's outputs unwritten and a repeated token is written twice
 *   (the table lives in device memory and is not inspected on the host).
 */
#ifndef MVM_SCAN_H
#define MVM_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVM_ABI_VERSION 4

/* status codes */
#define MVM_OK 0
#define MVM_ERR_INVALID_ARG (-1)
#define MVM_ERR_UNSUPPORTED (-2)
#define MVM_ERR_WORKSPACE (-3)
#define MVM_ERR_HIP (-4)

/* dtype codes */
#define MVM_F32 0
#define MVM_BF16 1

/* largest d_state the kernels hold in registers (the reference's kernels
 * hard-code float h[16], mamba_metal_fused.py:28,76) */
#define MVM_MAX_DSTATE 16

typedef struct mvm_scan_desc {
  int64_t batch;    /* B */
  int64_t seqlen;   /* L (scan positions per direction), <= 2^31 - 65 */
  int64_t dim;      /* D = d_inner, channels */
  int64_t dstate;   /* N, 1..MVM_MAX_DSTATE */
  int64_t ndir;     /* K directions scanned in one call, >= 1 */
  int64_t x_stride_b, x_stride_k, x_stride_t;    /* element strides, u-like */
  int64_t bc_stride_b, bc_stride_k, bc_stride_t; /* element strides, B-like */
  const int32_t* seq_to_tok; /* device (ndir, seqlen) table or NULL */
  int32_t in_dtype;   /* u, Bm, Cm, dy: MVM_F32 or MVM_BF16 */
  int32_t out_dtype;  /* y, du, dB, dC: MVM_F32 or MVM_BF16 */
  int32_t chunk_len;  /* time-chunk length (multiple of 16) or 0 = auto */
  int32_t reserved;
} mvm_scan_desc;

/* ABI version of the loaded library (MVM_ABI_VERSION). */
int mvm_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* mvm_last_error(void);

/* Validates a descriptor without touching the GPU. */
int mvm_scan_validate(const mvm_scan_desc* desc);

/* Number of float32 elements of the state checkpoint buffer the forward
 * writes for the backward: states after every 8th scan position,
 * (batch*ndir, ceil(seqlen/8), dim, 16).  Returns < 0 on a bad desc. */
int64_t mvm_scan_ckpt_elems(const mvm_scan_desc* desc);

/* Workspace bytes needed by mvm_scan_fwd (which = 0) or mvm_scan_bwd
 * (which = 1, with a caller-provided checkpoint) or mvm_scan_bwd with
 * ckpt == NULL (which = 2, the checkpoints are then recomputed into the
 * workspace).  Returns < 0 on a bad desc. */
int64_t mvm_scan_workspace_bytes(const mvm_scan_desc* desc, int which);

/* Time-chunk length the library will use for this descriptor. */
int64_t mvm_scan_chunk_len(const mvm_scan_desc* desc);

/* Forward scan.  y may be NULL (checkpoints only); ckpt may be NULL
 * (inference).  delta is float32.  See the header comment for layouts. */
int mvm_scan_fwd(const mvm_scan_desc* desc, const void* u, const float* delta,
                 const float* A, const void* Bm, const void* Cm,
                 const float* Dv, void* y, float* ckpt, void* workspace,
                 size_t workspace_bytes, void* stream);

/* Backward (VJP).  dy is the upstream gradient of y.  ckpt is the buffer
 * the forward filled, or NULL to recompute it.  Every output is fully
 * written (no accumulation into existing contents). */
int mvm_scan_bwd(const mvm_scan_desc* desc, const void* u, const float* delta,
                 const float* A, const void* Bm, const void* Cm,
                 const float* Dv, const float* ckpt, const void* dy, void* du,
                 float* ddelta, float* dA, void* dB, void* dC, float* dD,
                 void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Backward without a workspace.  No counterpart in the reference: this is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Same as mvm_scan_bwd with a caller checkpoint, but the scratch space
 * (chunk aggregates, dA / dD and dB / dC partial sums) comes from a fixed
 * device array of MVM_NOALLOC_SCRATCH_BYTES that the library holds on each
 * GPU it runs on until the process ends; it calls no hipMalloc / hipFree.
 *   - ckpt is required (NULL fails with MVM_ERR_INVALID_ARG).
 *   - A shape whose scratch need, mvm_scan_workspace_bytes(desc, 1),
 *     exceeds MVM_NOALLOC_SCRATCH_BYTES fails with MVM_ERR_WORKSPACE before
 *     anything is launched (B=2 L=196 D=1536 needs ~5.6 MB; B*K=128 L=196
 *     D=768 needs ~52 MB).
 *   - All calls on one GPU share its array: calls that overlap in time on
 *     one GPU (other streams, other threads) race.  Calls in order on one
 *     stream are safe.  Nothing in the array needs clearing: every element
 *     the kernels read is written earlier in the same call.
 * ---------------------------------------------------------------------- */
#define MVM_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024)

/* MVM_NOALLOC_SCRATCH_BYTES, as compiled into the loaded library. */
int64_t mvm_scan_noalloc_scratch_bytes(void);

int mvm_scan_bwd_noalloc(const mvm_scan_desc* desc, const void* u, const float* delta,
                         const float* A, const void* Bm, const void* Cm,
                         const float* Dv, const float* ckpt, const void* dy, void* du,
                         float* ddelta, float* dA, void* dB, void* dC, float* dD,
                         void* stream);

/* ------------------------------------------------------------------------
 * Fused form: the Mamba block's prologue and epilogue around the scan.
 *
 * Replaces, for one block call, the ops around scan_fn in MambaBlock
 * (mlx_vision_mamba/mamba_block.py:180-190):
 *     delta = softplus(dt_proj(dt))          (:180-181; dt_proj's bias is
 *                                             delta_bias, its matmul output
 *                                             is delta_raw)
 *     y     = scan_fn(x, delta, A, B, C, D)  (:187)
 *     y     = y * silu(z)                    (:190)
 * plus their VJP, and optionally A = -exp(A_log) (:184).  softplus is
 * applied inside the scan kernels as delta is staged (forward and
 * backward), the gate as y is written back and its gradient as dy is
 * staged, so none of them makes its own pass over HBM.  float32 only
 * (in_dtype = out_dtype = MVM_F32).
 *
 * Layouts: `scan` gives the sizes, u / du strides (x_stride_*), the B-like
 * strides and the direction table.  delta_raw / ddelta_raw use dt_stride_*,
 * y / y_raw / dy use y_stride_*, z / dz use z_stride_* (all with channel
 * stride 1).  softplus(x) = x for x > 20, else log(1 + e^x) (torch's
 * threshold); silu(z) = z / (1 + e^-z).
 * ---------------------------------------------------------------------- */
typedef struct mvm_scan_fused_desc {
  mvm_scan_desc scan;
  int64_t dt_stride_b, dt_stride_k, dt_stride_t;  /* delta_raw, ddelta_raw */
  int64_t y_stride_b, y_stride_k, y_stride_t;     /* y, y_raw, dy */
  int64_t z_stride_b, z_stride_k, z_stride_t;     /* z, dz */
  /* Nonzero: the A argument holds A_log and the scan uses A = -exp(A_log)
   * (mamba_block.py:184), formed in the kernels; the backward's dA output
   * is then the gradient with respect to A_log (dA * A). */
  int32_t a_is_log;
  int32_t reserved; /* must be 0 */
} mvm_scan_fused_desc;

int mvm_scan_fused_validate(const mvm_scan_fused_desc* desc);

/* Workspace bytes of mvm_scan_fused_fwd (which = 0) or mvm_scan_fused_bwd
 * (which = 1); gate != 0 when z is given.  Checkpoints are sized by
 * mvm_scan_ckpt_elems(&desc->scan). */
int64_t mvm_scan_fused_workspace_bytes(const mvm_scan_fused_desc* desc, int which, int gate);

/* y = scan(u, softplus(delta_raw + delta_bias), A, Bm, Cm, Dv) * silu(z).
 * delta_bias (ndir, dim) may be NULL (zero bias); z may be NULL (no gate,
 * y is the scan output).  y_raw (the ungated scan output, needed by the
 * backward when z is given) and ckpt (training) may be NULL. */
int mvm_scan_fused_fwd(const mvm_scan_fused_desc* desc, const float* u, const float* delta_raw,
                       const float* delta_bias, const float* A, const float* Bm,
                       const float* Cm, const float* Dv, const float* z, float* y,
                       float* y_raw, float* ckpt, void* workspace, size_t workspace_bytes,
                       void* stream);

/* VJP of mvm_scan_fused_fwd for upstream dy (gradient of the gated y).
 * ckpt is required; y_raw and dz are required when z is given; ddelta_bias
 * (ndir, dim) is required when delta_bias is given.  ddelta_raw is the
 * gradient of delta_raw; every output is fully written. */
int mvm_scan_fused_bwd(const mvm_scan_fused_desc* desc, const float* u, const float* delta_raw,
                       const float* delta_bias, const float* A, const float* Bm,
                       const float* Cm, const float* Dv, const float* z, const float* y_raw,
                       const float* ckpt, const float* dy, float* du, float* ddelta_raw,
                       float* ddelta_bias, float* dA, float* dB, float* dC, float* dD,
                       float* dz, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MVM_SCAN_H */
