/*
 * theseus_gdn.h -- C ABI of the chunked gated-delta-rule forward in
 * libtheseus_wkv7.so (gfx950): the recurrence of the GDN layers of the
 * reference's teacher model, which the reference runs through transformers'
 * torch_chunk_gated_delta_rule / torch_recurrent_gated_delta_rule
 * (dispatched at theseus/hf_model.py:28-52), in the operand mapping its
 * converter states (convert_qwen2rwkv_lightning.py:381-385):
 *
 *   S_t = e^{g_t} S_{t-1} + beta_t k_t (v_t - e^{g_t} S_{t-1}^T k_t)^T,
 *   o_t = S_t^T q_t / sqrt(N)                  (S: [key][value], N = K = V)
 *
 * q is scaled by 1/sqrt(N) inside.  theseus_gdn_forward is the forward without
 * gradients (how the reference's teacher runs these layers); theseus_gdn_forward_train
 * and theseus_gdn_backward are the pair for calls that need them.
 * Status codes are those of theseus_wkv7.h.
 */
#ifndef THESEUS_GDN_H
#define THESEUS_GDN_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/* Chunked gated delta rule forward on the caller's stream.
 *   q, k, v, o  [B,T,H,N] contiguous, all of dtype (theseus_wkv7_dtype: BF16 or FP32;
 *               arithmetic is float32 either way, as in transformers' functions)
 *   g, beta     [B,T,H] float32          s0, sT  [B,H,N(key),N(value)] float32
 *   qk_l2norm   nonzero: q and k are L2-normalised first, x / sqrt(sum x^2 + 1e-6)
 *               (use_qk_l2norm_in_kernel); zero: used as given
 *   N = 64 or 128 (else THESEUS_WKV7_ERR_SHAPE); workspace of
 *   theseus_gdn_forward_workspace_size bytes (every 16-step chunk's operands,
 *   42 KB per chunk at N = 128, and, with few heads -- B*H*N/64 workgroups at
 *   most half the CUs, T > 112 -- the buffers of the time-split scan, which
 *   cuts each head's chunks into k = min(4, CUs / (B*H*N/64)) segments run at
 *   once; a workspace of just the operand records runs the one-pass scan, to
 *   float32 rounding the same), not shared with a call that can run at the
 *   same time.  Replaces the forward of transformers' torch_chunk_gated_delta_rule
 *   (chunk_size is not used) and torch_recurrent_gated_delta_rule. */
int theseus_gdn_forward(int B, int T, int H, int N, int dtype, int qk_l2norm, const void* q,
                        const void* k, const void* v, const float* g, const float* beta,
                        const float* s0, void* o, float* sT, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);
/* Workspace bytes of theseus_gdn_forward (0 for invalid sizes). */
size_t theseus_gdn_forward_workspace_size(int B, int T, int H, int N);

/* The forward of a call that needs gradients: as theseus_gdn_forward with q and k used as
 * given (a layer that normalises them does so before, differentiably), and also the saved
 * states ckpt [B,H,ceil(T/16)+1,N,N] float32 (the state after steps 0, 16, 32, ... and the
 * final one, in the library's own [value][key] order) for theseus_gdn_backward; the scan
 * runs in one pass (no time split).  Replaces the forward of transformers'
 * torch_chunk_gated_delta_rule under autograd (theseus/hf_model.py:37-48 keeps it for
 * such calls). */
int theseus_gdn_forward_train(int B, int T, int H, int N, int dtype, const void* q, const void* k,
                              const void* v, const float* g, const float* beta, const float* s0,
                              void* o, float* sT, float* ckpt, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* Backward of theseus_gdn_forward_train, N = 128 (else THESEUS_WKV7_ERR_SHAPE), on the
 * caller's stream: q, k, v, g, beta and ckpt as that forward had them, dout [B,T,H,N] in
 * dtype, dsT [B,H,key,value] float32 (may be NULL: zero); writes dq, dk, dv [B,T,H,N] in
 * dtype, dg, dbeta [B,T,H] float32 and ds0 [B,H,key,value] float32.  Workspace of
 * theseus_gdn_backward_workspace_size bytes (24.5 KB of scan records and a 64 KB float32
 * dL/dS per 16-step chunk and head), not shared with a call that can run at the same
 * time.  Replaces the backward of transformers' torch_chunk_gated_delta_rule. */
int theseus_gdn_backward(int B, int T, int H, int N, int dtype, const void* q, const void* k,
                         const void* v, const float* g, const float* beta, const float* ckpt,
                         const void* dout, const float* dsT, void* dq, void* dk, void* dv,
                         float* dg, float* dbeta, float* ds0, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);
/* Workspace bytes of theseus_gdn_backward (0 for invalid sizes or N != 128). */
size_t theseus_gdn_backward_workspace_size(int B, int T, int H, int N);

#ifdef __cplusplus
}
#endif

#endif /* THESEUS_GDN_H */
