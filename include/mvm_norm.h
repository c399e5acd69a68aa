/*
 * mvm_norm.h -- C ABI of the LayerNorm that precedes every VisionMamba block
 * and follows the last one (libmvm_scan.so).
 *
 * Replaces the reference's nn.LayerNorm(d_model) (MLX: eps 1e-5, affine) at
 * mlx_vision_mamba/mamba_block.py:201,205 (ResidualMambaBlock),
 * :222,227 (BidirectionalMambaBlock), :401,548 (MultiDirectionalMambaBlock)
 * and vision_mamba.py:192,223 (the encoder's final norm).  Over each row r
 * of E = cols values:
 *
 *   mean_r = (1/E) sum_c x[r,c]
 *   rstd_r = 1 / sqrt((1/E) sum_c (x[r,c] - mean_r)^2 + eps)
 *   y[r,c] = (x[r,c] - mean_r) * rstd_r * gamma[c] + beta[c]
 *
 * Backward for an upstream dy, with xh = (x - mean) * rstd, g = dy * gamma:
 *
 *   dx[r,c]   = rstd_r * (g - (1/E) sum_c g - xh * (1/E) sum_c g * xh) + dres[r,c]
 *   dgamma[c] = sum_r dy * xh          dbeta[c] = sum_r dy
 *
 * dres (optional) is the gradient that reaches x through the block's
 * residual branch, x + f(norm(x)): adding it here replaces a separate
 * accumulation pass.
 *
 * Conventions are those of mvm_scan.h (status codes, mvm_last_error,
 * caller-owned buffers, host-side validation before any launch, no device
 * allocation).  float32 only.  Rows are x_stride (x) and y_stride (y, dy,
 * dres, dx) elements apart; columns are contiguous.  mean and rstd hold one
 * value per row.  dgamma and dbeta are summed over rows in a fixed order
 * (bitwise deterministic).  dx may be the dres buffer itself (in place);
 * no other output may alias an input.
 */
#ifndef MVM_NORM_H
#define MVM_NORM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVM_NORM_MAX_COLS 1024
#define MVM_NORM_MAX_ROWS (INT64_C(1) << 25)

typedef struct mvm_norm_desc {
  int64_t rows;      /* R, 0..MVM_NORM_MAX_ROWS */
  int64_t cols;      /* E, 1..MVM_NORM_MAX_COLS */
  int64_t x_stride;  /* >= cols */
  int64_t y_stride;  /* >= cols */
  float eps;         /* >= 0 */
  int32_t reserved;  /* must be 0 */
} mvm_norm_desc;

/* Validates a descriptor without touching the GPU. */
int mvm_norm_validate(const mvm_norm_desc* desc);

/* Workspace bytes mvm_layernorm_bwd needs (per-workgroup dgamma | dbeta
 * partial sums). */
int64_t mvm_norm_workspace_bytes(const mvm_norm_desc* desc);

/* y = LayerNorm(x) * gamma + beta; also writes mean and rstd (rows floats
 * each) for the backward. */
int mvm_layernorm_fwd(const mvm_norm_desc* desc, const float* x, const float* gamma,
                      const float* beta, float* y, float* mean, float* rstd, void* stream);

/* Gradients of mvm_layernorm_fwd for upstream dy: dx (+ dres when dres is
 * not NULL), dgamma and dbeta (cols floats each); all fully written. */
int mvm_layernorm_bwd(const mvm_norm_desc* desc, const float* x, const float* gamma,
                      const float* mean, const float* rstd, const float* dy, const float* dres,
                      float* dx, float* dgamma, float* dbeta, void* workspace,
                      size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MVM_NORM_H */
