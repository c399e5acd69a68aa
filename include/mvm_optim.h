/*
 * mvm_optim.h -- C ABI of the AdamW update of the VisionMamba training step
 * (libmvm_scan.so).
 *
 * No counterpart in the reference's scan path: the reference leaves the
 * optimiser to its training loop.  This entry point updates every float32
 * parameter tensor of a model in one kernel launch (a few launches for more
 * than MVM_ADAMW_TENSORS_PER_LAUNCH tensors), with all of the GPU's
 * workgroups busy, where a per-tensor-list optimiser runs many small
 * launches.
 *
 * AdamW with decoupled weight decay (the update of torch.optim.AdamW), for
 * every element of every tensor, with t = *step (the caller increments it
 * before the call, on the device, so a captured graph replays correctly):
 *
 *   p = p * (1 - lr * weight_decay)
 *   m = m + (1 - beta1) * (g - m)
 *   v = beta2 * v + (1 - beta2) * g * g
 *   p = p - lr / (1 - beta1^t) * m / (sqrt(v) / sqrt(1 - beta2^t) + eps)
 *
 * m and v of tensor i live at exp_avg + state_offset and exp_avg_sq +
 * state_offset (numel floats each, caller-owned, zero before the first
 * step).  Parameters and gradients are contiguous float32; no two tensors'
 * parameter or state ranges may overlap.  Conventions are those of
 * mvm_scan.h (status codes, mvm_last_error, host-side validation before any
 * launch, no device allocation).
 */
#ifndef MVM_OPTIM_H
#define MVM_OPTIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVM_ADAMW_TENSORS_PER_LAUNCH 64

typedef struct mvm_adamw_tensor {
  float* param;         /* numel floats, updated in place */
  const float* grad;    /* numel floats */
  int64_t numel;        /* >= 0 (0: skipped) */
  int64_t state_offset; /* element offset of this tensor's m and v */
} mvm_adamw_tensor;

typedef struct mvm_adamw_hparams {
  float lr;           /* >= 0 */
  float beta1;        /* [0, 1) */
  float beta2;        /* [0, 1) */
  float eps;          /* > 0 */
  float weight_decay; /* >= 0 */
  int32_t reserved;   /* must be 0 */
} mvm_adamw_hparams;

/* One AdamW step over ntensors tensors (host array `tensors`); step points
 * to one device float holding the step count t >= 1. */
int mvm_adamw_step(const mvm_adamw_tensor* tensors, int32_t ntensors,
                   const mvm_adamw_hparams* hp, const float* step, float* exp_avg,
                   float* exp_avg_sq, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MVM_OPTIM_H */
