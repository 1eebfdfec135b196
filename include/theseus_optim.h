/*
 * theseus_optim.h -- C ABI of the fused optimizer step in libtheseus_wkv7.so
 * (gfx950): the work the reference does between a layer's backward and its
 * next forward (train.py:198-209 with the optimizer built at theseus/stage.py:39-42):
 *
 *   for p in params: p.grad.mul_(world / count)                    (train.py:202-204)
 *   norm = clip_grad_norm_(params, clip_norm, error_if_nonfinite)   (train.py:205-206)
 *   AdamW step, two parameter groups (decay / no decay), fused      (train.py:208)
 *
 * as three launches on one stream with no host synchronisation in between:
 * per-chunk sums of squared gradients (float64, fixed chunks), one workgroup
 * that sums them in a fixed order and forms the norm, the clip factor and a
 * non-finite flag in device memory, and the AdamW update, which reads the
 * factor from device memory.  Results are deterministic (no atomics).  The
 * gradients are read, never written (the reference scales and clips them in
 * place and then drops them with zero_grad(set_to_none=True)).
 *
 * All tensors are float32 on the current device.  The tensor list is passed
 * by value from host memory (the library packs it into kernel arguments, 32
 * tensors per launch); nothing is copied to or allocated on the device.
 * Status codes are those of theseus_wkv7.h.
 */
#ifndef THESEUS_OPTIM_H
#define THESEUS_OPTIM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/* One parameter tensor of the step (host memory). */
typedef struct theseus_adamw_tensor {
    float* param;           /* updated in place                                   */
    const float* grad;      /* read only                                          */
    float* exp_avg;         /* AdamW first moment, updated in place               */
    float* exp_avg_sq;      /* AdamW second moment, updated in place              */
    long long numel;        /* elements (0: skipped)                              */
    float lr;               /* the group's learning rate for this step            */
    float weight_decay;     /* decoupled: param *= 1 - lr * weight_decay          */
    float step_size;        /* lr / (1 - beta1^step)                              */
    float bias_correction2_sqrt; /* sqrt(1 - beta2^step)                          */
} theseus_adamw_tensor;

/* Elements per workgroup chunk; the workspace holds one double per chunk. */
#define THESEUS_ADAMW_CHUNK 16384

/* Bytes of workspace theseus_adamw_step needs for these tensors (with a norm). */
size_t theseus_adamw_workspace_size(const theseus_adamw_tensor* tensors, int ntensors);

/* g = grad * grad_scale * clip, with clip = min(1, max_norm / (norm + 1e-6)) where
 * norm is the L2 norm of grad * grad_scale over all tensors (max_norm = +inf:
 * the norm without clipping; max_norm < 0: neither norm nor clipping, clip = 1,
 * result[0] = NaN, and no workspace is needed); then per element
 *   param *= 1 - lr * weight_decay
 *   exp_avg += (1 - beta1) * (g - exp_avg)
 *   exp_avg_sq = beta2 * exp_avg_sq + (1 - beta2) * g * g
 *   param -= step_size * exp_avg / (sqrt(exp_avg_sq) / bias_correction2_sqrt + eps)
 * (torch.optim.AdamW's update).  result: 3 floats of device memory, written
 * before the update runs: [0] the norm, [1] grad_scale * clip, [2] 1 when the
 * norm is not finite, else 0.  With skip_nonfinite != 0 a non-finite norm
 * leaves every param and moment unchanged (clip_grad_norm_'s
 * error_if_nonfinite=True raises before the update; the caller reads result[2]
 * to raise); with 0 the update runs with the non-finite factor, as torch does
 * with error_if_nonfinite=False.
 * Replaces the gradient loop, clip_grad_norm_ and optimizer.step() of
 * train.py:202-208 (the AdamW of theseus/stage.py:39-42). */
int theseus_adamw_step(const theseus_adamw_tensor* tensors, int ntensors, float grad_scale,
                       float max_norm, float beta1, float beta2, float eps, int skip_nonfinite,
                       float* result, void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* THESEUS_OPTIM_H */
