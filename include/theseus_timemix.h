/*
 * theseus_timemix.h -- C ABI of the fused TimeMix elementwise kernels in
 * libtheseus_wkv7.so (gfx950).  They replace the torch op sequences around the
 * recurrence in TimeMix.forward (theseus/timemix.py:66-89); the reference has no
 * native counterpart (it runs ~20 separate torch kernels there).
 *
 * Activations are [B,T,C] contiguous bf16; the gate a = sigmoid(a0 + za) of
 * theseus/timemix.py:75 is formed inside the kernels from za (the bf16 LoRA output
 * (x_a @ a1) @ a2) and the parameter a0, in float32 as bf16 autocast over float32
 * parameters computes it; per-channel parameters are float32 [C] (r_k is [H,N] = [C]).  Parameter gradients are
 * reduced over B*T in a fixed order through a caller-provided float32 workspace
 * (theseus_tm_*_workspace gives its size), then written to [C] outputs.
 * Head size N must be 64 (8 lanes x 8 channels per head row), and B*T at most
 * 65535 * 64 tokens (status 1, THESEUS_WKV7_ERR_SHAPE, otherwise).  All calls are
 * asynchronous on `stream`; status codes are those of theseus_wkv7.h.
 */
#ifndef THESEUS_TIMEMIX_H
#define THESEUS_TIMEMIX_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/* mixed_n = x + (shift(x) - x) * coef_n for n in r,w,k,v,a,g
 * (theseus/timemix.py:70-71); shift(x)[t] = x[t-1], shift(x)[0] = shift_state.
 * coef: [6][C] float32 in the order r,w,k,v,a,g; out: 6 pointers, same order. */
int theseus_tm_shift_lerp_fwd(int B, int T, int C, const void* x, const void* shift_state,
                              const float* coef, void* const* out, hipStream_t stream);
size_t theseus_tm_shift_lerp_workspace(int B, int T, int C);
/* dmixed: 6 pointers (bf16); writes dx [B,T,C] bf16, dshift [B,C] bf16, dcoef [6][C] f32 */
int theseus_tm_shift_lerp_bwd(int B, int T, int C, const void* const* dmixed, const void* x,
                              const void* shift_state, const float* coef, void* dx, void* dshift,
                              float* dcoef, float* workspace, size_t workspace_bytes,
                              hipStream_t stream);

/* The decay input w = (w0 + zw).to(bf16) (theseus/timemix.py:73, 80): float32 parameter w0
 * [C] plus the bf16 LoRA output zw [B,T,C], rounded once to bf16.  Its backward needs no
 * kernel: dL/dzw is dL/dw itself and dL/dw0 its sum over B*T. */
int theseus_tm_add_param_fwd(int B, int T, int C, const void* zw, const float* w0, void* w,
                             hipStream_t stream);

/* WKV operands (theseus/timemix.py:75, 78-80): a = sigmoid(a0 + za), kk = normalize(k * k_k)
 * per head (eps 1e-12), kw = k * (1 + (a - 1) * k_a), aw = -kk, bw = kk * a, all written as
 * bf16. */
int theseus_tm_kk_fwd(int B, int T, int C, const void* k, const void* za, const float* a0, const float* k_k,
                      const float* k_a, void* kw, void* aw, void* bw, hipStream_t stream);
size_t theseus_tm_kk_workspace(int B, int T, int C);
/* writes dk (bf16), dza (bf16) = dL/d(a0 + za) and [C] f32 da0, dk_k, dk_a.  dzg
 * (float32 [B,T,C], or NULL for zero) is the rest of dL/da times a (1 - a), as
 * theseus_tm_gn_bwd writes it: the two parts are added in float32 before dza is rounded. */
int theseus_tm_kk_bwd(int B, int T, int C, const void* dkw, const void* daw, const void* dbw,
                      const void* k, const void* za, const float* a0, const float* dzg,
                      const float* k_k, const float* k_a, void* dk, void* dza, float* da0,
                      float* dk_k, float* dk_a, float* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* out = (GroupNorm_H(y; ln_w, ln_b, eps) + (sum_n r*kmod*r_k) v) * g, all float32
 * arithmetic, written as bf16 (theseus/timemix.py:83-88); kmod = k * (1 + (a - 1) * k_a),
 * a = sigmoid(a0 + za). */
int theseus_tm_gn_fwd(int B, int T, int C, const void* y, const void* r, const void* k,
                      const void* za, const float* a0, const float* k_a, const void* v,
                      const void* g, const float* r_k, const float* ln_w, const float* ln_b,
                      float eps, void* out, hipStream_t stream);
size_t theseus_tm_gn_workspace(int B, int T, int C);
/* writes dy, dr, dk, dv, dg (bf16), dzg (f32: this term's dL/da times a (1 - a), for
 * theseus_tm_kk_bwd), and [C] f32 dr_k, dln_w, dln_b, dk_a */
int theseus_tm_gn_bwd(int B, int T, int C, const void* dout, const void* y, const void* r,
                      const void* k, const void* za, const float* a0, const float* k_a,
                      const void* v, const void* g, const float* r_k, const float* ln_w,
                      const float* ln_b, float eps, void* dy, void* dr, void* dk, void* dv,
                      void* dg, float* dzg, float* dr_k, float* dln_w, float* dln_b,
                      float* dk_a, float* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* A TimeMix layer's parameters as a serving step reads them (theseus/timemix.py:18-59):
 * the stacked shift-lerp coefficients coef [6][C] float32 (x_r, x_w, x_k, x_v, x_a, x_g);
 * the projections w_r, w_k, w_v, w_o [C][C] bf16 in nn.Linear's [out][in] layout; the
 * LoRA matrices transposed to [out][in] bf16: w1t, a1t, g1t [rank][C] and w2t, a2t, g2t
 * [C][rank]; w0, a0, k_k, k_a, r_k, ln_w, ln_b [C] float32; ln_eps the GroupNorm eps. */
typedef struct theseus_tm_layer {
    int C, H, N, rank_w, rank_a, rank_g;
    const float* coef;
    const void *w_r, *w_k, *w_v, *w_o;
    const void *w1t, *a1t, *g1t, *w2t, *a2t, *g2t;
    const float *w0, *a0, *k_k, *k_a, *r_k, *ln_w, *ln_b;
    float ln_eps;
} theseus_tm_layer;

/* Workspace bytes of theseus_tm_serving_step for B lanes (0: sizes it refuses). */
size_t theseus_tm_serving_step_workspace(const theseus_tm_layer* layer, int B);

/* One serving step of TimeMix.forward (theseus/timemix.py:62-89) for x [B,1,C] bf16, no
 * autograd, N = 64, B <= THESEUS_GEMM_MAX_ROWS: the launches of the fused layer's
 * few-row path in one call (the same kernels, order and arguments, so the same bits),
 * every intermediate in the workspace.  shift_in [B,C] bf16 is the previous token; when
 * shift_out is not NULL, x is copied there at the end (the in-place step).  The WKV state
 * [B,H,N,N] float32 goes from wkv_in to wkv_out (the same pointer: in place); out [B,1,C]
 * bf16.  The step the reference's serving loop makes per token through AttentionAdapter
 * (theseus/hf_model.py:96-108) has no native counterpart there (~20 torch launches).
 * Asynchronous on `stream`; status codes of theseus_wkv7.h. */
int theseus_tm_serving_step(const theseus_tm_layer* layer, int B, const void* x, const void* shift_in,
                            void* shift_out, const float* wkv_in, float* wkv_out, void* out,
                            void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* THESEUS_TIMEMIX_H */
