/*
 * mvm_conv.h -- C ABI of the causal depthwise conv1d + SiLU of the Mamba
 * block, run along each direction's scan order (libmvm_scan.so).
 *
 * Replaces, for the multi-directional blocks, the reference's
 * nn.Conv1d(d_inner, d_inner, kernel_size=d_conv, padding=d_conv-1,
 * groups=d_inner) + [:, :L] + nn.silu
 * (mlx_vision_mamba/mamba_block.py:129-132, :170-171) applied to the
 * permuted copies built by _permute_* / [:, ::-1]
 * (mamba_block.py:254-338, :443-533): here scan position s of direction k
 * reads and writes token row seq_to_tok[k*seqlen + s] directly.
 *
 *   pre[s] = bias + sum_{j<kwidth} w[j] * x[s - kwidth + 1 + j]   (x[<0] = 0)
 *   y[s]   = pre[s] * sigmoid(pre[s])
 *
 * Conventions are those of mvm_scan.h (status codes, mvm_last_error,
 * caller-owned buffers, host-side validation, deterministic results).
 * float32 only.  Layout: x holds (b, k, t, d) at
 * b*x_stride_b + k*x_stride_k + t*x_stride_t + d; y and dy use the
 * y_stride_* strides, dx the dx_stride_* strides (so dx can be written
 * straight into a slice of a larger gradient buffer); w is
 * (ndir, dim, kwidth) and bias (ndir, dim).
 */
#ifndef MVM_CONV_H
#define MVM_CONV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVM_CONV_MAX_KWIDTH 8

typedef struct mvm_conv_desc {
  int64_t batch;   /* B */
  int64_t seqlen;  /* L = tokens = scan positions */
  int64_t dim;     /* channels (d_inner) */
  int64_t ndir;    /* K */
  int64_t kwidth;  /* d_conv, 1..MVM_CONV_MAX_KWIDTH */
  int64_t x_stride_b, x_stride_k, x_stride_t;
  int64_t y_stride_b, y_stride_k, y_stride_t;
  const int32_t* seq_to_tok; /* device (ndir, seqlen) table or NULL */
  int64_t dx_stride_b, dx_stride_k, dx_stride_t;
} mvm_conv_desc;

/* Validates a descriptor without touching the GPU. */
int mvm_conv_validate(const mvm_conv_desc* desc);

/* Workspace bytes mvm_conv_silu_bwd needs (dw / dbias partial sums). */
int64_t mvm_conv_workspace_bytes(const mvm_conv_desc* desc);

/* y = silu(causal depthwise conv(x) + bias) along each direction. */
int mvm_conv_silu_fwd(const mvm_conv_desc* desc, const float* x, const float* w,
                      const float* bias, float* y, void* stream);

/* Gradients of mvm_conv_silu_fwd for upstream dy: dx (dx_stride_*), dw
 * (ndir, dim, kwidth), dbias (ndir, dim); all fully written. */
int mvm_conv_silu_bwd(const mvm_conv_desc* desc, const float* x, const float* w,
                      const float* bias, const float* dy, float* dx, float* dw,
                      float* dbias, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MVM_CONV_H */
