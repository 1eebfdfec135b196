/*
 * theseus_wkv7.h -- C ABI of the MI355X (gfx950) WKV7 state-recurrence library
 * (libtheseus_wkv7.so).
 *
 * This ABI is the drop-in boundary for the reference's pybind11 module
 * `theseus_wkv7_state_v1` (kernels/wkv7_state.cpp:38-41), which
 * theseus/wkv7.py:31-36 JIT-builds and calls.  Python binds it with ctypes
 * (rwkv-theseus_amd/theseus/wkv7.py); no torch or HIP C++ types appear here.
 *
 * Conventions (identical to the reference kernels):
 *   token tensors r,w,k,v,a,b,y,dy and their gradients: [B,T,H,N], contiguous,
 *     element (b,t,h,n) at ((b*T+t)*H+h)*N+n   (kernels/wkv7_state.cu:25);
 *   w is the pre-sigmoid logit: decay = exp(-e^{-1/2} * sigmoid(w))  (cu:27);
 *   states s0, sT, ds0, dsT: [B,H,N,N] float32, element (b,h,i,j) at
 *     ((b*H+h)*N+i)*N+j with i = value row, j = key column  (cu:21);
 *   dtype: THESEUS_WKV7_BF16 or THESEUS_WKV7_FP32 for all token tensors of a
 *     call; the state is always float32.
 *
 * Ownership and threading: the caller allocates every buffer (outputs and
 * workspace included) in device memory of the current HIP device; the library
 * never allocates, frees or synchronises.  Each call enqueues its kernels on
 * `stream` and returns; a return code other than THESEUS_WKV7_OK means that
 * nothing was enqueued (argument errors) or that the launch failed
 * (THESEUS_WKV7_ERR_LAUNCH, checked with hipGetLastError like
 * C10_CUDA_KERNEL_LAUNCH_CHECK at kernels/wkv7_state.cpp:24,36).  The library
 * keeps no mutable global state, so calls are reentrant -- except
 * theseus_wkv7_forward_noalloc, whose calls on one device share a static
 * device scratch array (see its declaration).
 */
#ifndef THESEUS_WKV7_H
#define THESEUS_WKV7_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

enum theseus_wkv7_dtype { THESEUS_WKV7_BF16 = 0, THESEUS_WKV7_FP32 = 1 };

enum theseus_wkv7_status {
    THESEUS_WKV7_OK = 0,
    THESEUS_WKV7_ERR_SHAPE = 1,      /* B,H < 1, T < 1 or N outside 2..128 (cpp:12) */
    THESEUS_WKV7_ERR_DTYPE = 2,      /* dtype is not BF16/FP32 (cpp:13)             */
    THESEUS_WKV7_ERR_NULL = 3,       /* a required pointer is NULL                  */
    THESEUS_WKV7_ERR_WORKSPACE = 4,  /* workspace smaller than required             */
    THESEUS_WKV7_ERR_LAUNCH = 5,     /* hipGetLastError reported a failure          */
    THESEUS_WKV7_ERR_SCRATCH = 6,    /* theseus_wkv7_forward_noalloc: these sizes need
                                        more than THESEUS_WKV7_NOALLOC_SCRATCH_BYTES    */
    THESEUS_WKV7_ERR_FLAGS = 7       /* flags other than theseus_wkv7_flags bits        */
};

/* Options of the *_ex entry points (0 = the reference's operator). */
enum theseus_wkv7_flags {
    /* d = exp(w) with no clamp or sigmoid instead of exp(-e^{-1/2} sigmoid(w)): the
     * decay of the GDN teacher layers, w = g ("wkv_decay_operation",
     * convert_qwen2rwkv_lightning.py:383-384); dw is then dL/d(log d). */
    THESEUS_WKV7_DECAY_EXP = 1,
    /* s0, sT, dsT and ds0 are [B,H,key,value] (GDN's "B,Hv,K,V", :382) instead of
     * [B,H,value,key]; saved states keep the library's own layout. */
    THESEUS_WKV7_STATE_KEY_VALUE = 2
};

/* Kernel family a call of these sizes runs on (theseus_wkv7_kernel_family). */
enum theseus_wkv7_family {
    THESEUS_WKV7_FAMILY_CHUNKED = 0,    /* chunked MFMA kernels (bf16, N = 64)              */
    THESEUS_WKV7_FAMILY_FORCED = 1,     /* step-serial: THESEUS_WKV7_FAMILY=seq is set       */
    THESEUS_WKV7_FAMILY_FP32 = 2,       /* step-serial: fp32 token tensors                   */
    THESEUS_WKV7_FAMILY_HEAD_SIZE = 3,  /* step-serial: N != 64                              */
    THESEUS_WKV7_FAMILY_SIZE = 4,       /* step-serial: a token tensor >= 2 GiB or one head's
                                           saved states >= 4 GiB (32-bit buffer offsets)     */
    THESEUS_WKV7_FAMILY_FLAGS = 5,      /* step-serial: a call of the *_ex entry points with
                                           flags (exp decay or key-value states)             */
    THESEUS_WKV7_FAMILY_RECORDS = 6     /* bf16, N = 128: chunk-record kernels -- the forward
                                           when the workspace holds the records
                                           (theseus_wkv7_forward_workspace_size counts
                                           them; else step-serial), the backward always.
                                           Saved states in [value][key] order, as the
                                           step-serial kernels keep them                     */
};

/* ABI version of this header; bumped on any incompatible change. */
int theseus_wkv7_abi_version(void);

/* Static message for a status code (never NULL). */
const char* theseus_wkv7_error_string(int status);

/* Which kernel family theseus_wkv7_forward / _backward use for these sizes
 * (a theseus_wkv7_family value), or minus a status code for invalid sizes.
 * The step-serial kernels are exact but run one step at a time (config 2:
 * ~0.12 M tokens/s against ~9 M on the chunked kernels); callers can warn or
 * refuse when a call would fall back to them.  No counterpart in the
 * reference (its kernel is step-serial for every call, kernels/wkv7_state.cu:81-92). */
int theseus_wkv7_kernel_family(int B, int T, int H, int N, int dtype);

/* Time-outs of the chunked kernels' bounded waits on the current device since the
 * last reset: the cross-workgroup handoffs (heads cut between workgroups) and the
 * backward's in-workgroup rendezvous.  A wait that times out (about a second) writes
 * NaN in place of what depends on it instead of hanging; this count tells such a
 * result from NaN inputs.  Synchronous (waits for the device); reset != 0 zeroes the
 * count.  Not safe to call while such kernels run.  No counterpart in the reference,
 * whose kernel has no cross-wave waits (kernels/wkv7_state.cu:12-79). */
int theseus_wkv7_wait_timeouts(unsigned int* count, int reset);
/* Test hook: on = 0 makes every bounded wait of the chunked kernels give up at once
 * (each such wait then counts a time-out and poisons its outputs with NaN), so the
 * failure path can be exercised without any wave waiting; on = 1 restores them.
 * Synchronous; affects the current device only.  No counterpart in the reference. */
int theseus_wkv7_set_waits(int on);

/* Steps between saved states (16); the saved-state tensor of a T-step
 * forward holds theseus_wkv7_checkpoint_count(T) states
 * [B,H,count,N,N] float32: state after steps 0,16,32,... and, last, the final
 * state after step T.  Replaces the full [B,H,T+1,N,N] history that
 * kernels/wkv7_state.cpp:21-22 allocates.  The states are for the backward
 * of the same kernel family (theseus_wkv7_kernel_family of the same sizes):
 * the step-serial kernels keep every state in [value][key] order; the
 * chunked kernels keep the last (the final state, equal to sT) in that
 * order and states 0 .. count-2 in their tiled order, S[i][j] (value i,
 * key j) at float ((i/16*4 + j/16)*64 + 16*(j%16/4) + i%16)*4 + j%4 of
 * the N x N block. */
int theseus_wkv7_checkpoint_interval(void);
long long theseus_wkv7_checkpoint_count(int T);

/* Bytes of device workspace theseus_wkv7_forward / theseus_wkv7_backward
 * need for these sizes and dtype on the current device (0 when none).  The
 * chunked kernels use it when B*H heads outnumber the device's CUs: heads are
 * then cut between workgroups, which hand the carried state over through it;
 * the step-serial backward replays each 16-step segment into it.  For few
 * heads (chunked kernels, 2*B*H <= CUs, T > 112) the forward size also covers
 * the time-split forward: a forward without saved states given that much cuts
 * every head's steps into k = min(4, CUs / (B*H)) segments that run at once,
 * one workgroup each, and chains them with a fix-up kernel; it agrees with
 * the one-pass kernels to float32 rounding.  Given less (none is needed at
 * such sizes) it runs the one-pass kernels.  The split's buffers are
 * 4 * B*H * ((2k-1)*N*N + 2(k-1)*m*16*N) bytes, m the chunk count of each
 * segment after the first (segment 0, which carries one state instead of
 * two, takes ceil(T/16) - (k-1)m, about 1.2 m).  Contents need not be initialised (each
 * call clears what it uses, on its stream), and a workspace must not be
 * shared by calls that may run at the same time. */
size_t theseus_wkv7_forward_workspace_size(int B, int T, int H, int N, int dtype);
size_t theseus_wkv7_backward_workspace_size(int B, int T, int H, int N, int dtype);

/* Forward recurrence.  Replaces wkv_forward (kernels/wkv7_state.cpp:16-25)
 * and launch_forward (kernels/wkv7_state.cu:81-86).
 * ckpt may be NULL (no-grad path, like save_history=false at cpp:22); else it
 * must hold theseus_wkv7_checkpoint_count(T) states per (b,h). */
int theseus_wkv7_forward(int B, int T, int H, int N, int dtype,
                         const void* r, const void* w, const void* k, const void* v,
                         const void* a, const void* b, const float* s0,
                         void* y, float* sT, float* ckpt, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/* Backward (adjoint) pass.  Replaces wkv_backward (kernels/wkv7_state.cpp:26-37)
 * and launch_backward (kernels/wkv7_state.cu:87-92).  ckpt is the buffer the
 * forward filled; dsT may be NULL (treated as zero, as _WKV.backward does at
 * theseus/wkv7.py:53-54).  dr..db are written in `dtype` (the reference
 * returns float32 and casts at theseus/wkv7.py:56); ds0 is float32. */
int theseus_wkv7_backward(int B, int T, int H, int N, int dtype,
                          const void* r, const void* w, const void* k, const void* v,
                          const void* a, const void* b, const float* ckpt,
                          const void* dy, const float* dsT,
                          void* dr, void* dw, void* dk, void* dv, void* da, void* db,
                          float* ds0, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);

/* theseus_wkv7_forward / _backward with options (theseus_wkv7_flags; 0 gives exactly
 * the functions above).  With THESEUS_WKV7_DECAY_EXP and the GDN operand mapping
 * r = q/sqrt(N), w = g, k = k, v = beta v, a = k, b = -exp(g) beta k
 * ("wkv_inputs", convert_qwen2rwkv_lightning.py:385) they run the gated delta rule of
 * the reference's teacher layers (theseus/hf_model.py:28-52 dispatches those to
 * transformers' torch_chunk/recurrent_gated_delta_rule).  Calls with flags run on the
 * step-serial kernels (any N 2..128, bf16 or fp32); a T=1 forward without saved states
 * and without THESEUS_WKV7_STATE_KEY_VALUE runs the single-step kernel.  Workspace
 * sizes: theseus_wkv7_workspace_size_ex.  Unknown flags: THESEUS_WKV7_ERR_FLAGS. */
int theseus_wkv7_forward_ex(int B, int T, int H, int N, int dtype, int flags,
                            const void* r, const void* w, const void* k, const void* v,
                            const void* a, const void* b, const float* s0,
                            void* y, float* sT, float* ckpt, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);
int theseus_wkv7_backward_ex(int B, int T, int H, int N, int dtype, int flags,
                             const void* r, const void* w, const void* k, const void* v,
                             const void* a, const void* b, const float* ckpt,
                             const void* dy, const float* dsT,
                             void* dr, void* dw, void* dk, void* dv, void* da, void* db,
                             float* ds0, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);
/* Workspace bytes of theseus_wkv7_forward_ex (backward = 0) or _backward_ex (1). */
size_t theseus_wkv7_workspace_size_ex(int B, int T, int H, int N, int dtype, int flags, int backward);

/* One recurrent step (T = 1) that updates `state` [B,H,N,N] float32 IN PLACE
 * and writes y [B,H,N].  r..b are [B,H,N] (a [B,1,H,N] tensor).  The
 * reference has no in-place step: its decode is wkv_forward with T=1, which
 * allocates a new end state per call (kernels/wkv7_state.cpp:21). */
int theseus_wkv7_decode_step(int B, int H, int N, int dtype,
                             const void* r, const void* w, const void* k, const void* v,
                             const void* a, const void* b, float* state, void* y,
                             hipStream_t stream);

/* Bytes of the library's static device scratch array, which
 * theseus_wkv7_forward_noalloc uses in place of a caller workspace.  8 MiB
 * holds the forward's handoffs for up to ~500 workgroups (4.2 MB at most on
 * 256 CUs; theseus_wkv7_forward_workspace_size, except at sizes where that
 * also covers the time-split forward, which the handoffs never need). */
#define THESEUS_WKV7_NOALLOC_SCRATCH_BYTES (8u << 20)

/* theseus_wkv7_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, whose
 * forward allocates its outputs and history itself (kernels/wkv7_state.cpp:16-25).
 * Same arguments, kernels and results as theseus_wkv7_forward (bitwise), minus
 * workspace/workspace_bytes, except that it never takes the time-split path
 * (it runs the one-pass kernels theseus_wkv7_forward runs when given less
 * workspace than the split needs): the chunked kernels' handoffs go through a static
 * device array of THESEUS_WKV7_NOALLOC_SCRATCH_BYTES that the library owns (one
 * per device, held until the process ends).  Calls whose sizes need more
 * return THESEUS_WKV7_ERR_SCRATCH without enqueuing anything.  The call
 * allocates nothing (no hipMalloc/hipFree).  All calls on one device share
 * that array: calls that may run at the same time on one device (different
 * streams, or graphs holding this call replayed concurrently) race on its
 * handoff counters and carried states and give silently wrong or NaN results,
 * not an error.  Call it from one stream per device, or order the streams
 * (an event or stream wait between two such calls). */
int theseus_wkv7_forward_noalloc(int B, int T, int H, int N, int dtype,
                                 const void* r, const void* w, const void* k, const void* v,
                                 const void* a, const void* b, const float* s0,
                                 void* y, float* sT, float* ckpt, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* THESEUS_WKV7_H */
