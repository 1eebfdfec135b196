// Host-side launch descriptors shared by the kernel translation units and the
// C-ABI front end.  dtype: 0 = bf16, 1 = fp32 (theseus_wkv7_dtype).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace wkv7 {

constexpr int kCkptInterval = 16;  // must equal CKPT in wkv7_common.h
// theseus_wkv7_flags (include/theseus_wkv7.h)
constexpr int FLAG_DECAY_EXP = 1;  // d = exp(w), unclamped
constexpr int FLAG_STATE_KV = 2;   // caller states stored [key][value]
constexpr int FLAGS_ALL = FLAG_DECAY_EXP | FLAG_STATE_KV;

struct Fwd {
    int B, T, H, N, dtype;
    const void *r, *w, *k, *v, *a, *b;
    const float* s0;
    void* y;
    float* sT;
    float* ckpt;  // may be null
    void* ws;     // workspace (the chunked kernels' handoffs; the time split's buffers)
    hipStream_t stream;
    int flags = 0;
    size_t ws_bytes = 0;  // bytes at ws (0: take no path that needs more than forward_workspace)
};

struct Bwd {
    int B, T, H, N, dtype;
    const void *r, *w, *k, *v, *a, *b;
    const float* ckpt;
    const void* dy;
    const float* dsT;  // may be null (zero)
    void *dr, *dw, *dk, *dv, *da, *db;
    float* ds0;
    void* ws;
    hipStream_t stream;
    int flags = 0;
};

struct Dec {
    int B, H, N, dtype;
    const void *r, *w, *k, *v, *a, *b;
    const float* state_in;  // read; may equal state
    float* state;           // written
    void* y;
    hipStream_t stream;
    int flags = 0;          // FLAG_DECAY_EXP only
};

void launch_seq_forward(const Fwd& p);
void launch_seq_backward(const Bwd& p);
size_t seq_backward_workspace(int B, int H, int N);
void launch_decode(const Dec& p);
// bf16, N == 64; `cus` = CUs the schedule spreads the heads over
void launch_chunk_forward(const Fwd& p, int cus);
void launch_chunk_backward(const Bwd& p, int cus);
// time-outs of the chunked kernels' bounded waits on the current device (read, optionally
// zeroed), and the host switch that makes those waits give up at once (tests); 0 on success
int chunk_forward_wait_timeouts(uint32_t* out, int reset);
int chunk_backward_wait_timeouts(uint32_t* out, int reset);
int chunk_forward_waits(int on);
int chunk_backward_waits(int on);
size_t chunk_forward_workspace(int B, int T, int H, int cus);
size_t chunk_backward_workspace(int B, int T, int H, int cus);
// The time-split forward (no saved states, few heads): each head's chunks cut into
// k = chunk_forward_split_segments(...) >= 2 segments that run at once, then a fix-up
// kernel; its workspace holds the segments' states, transitions and outputs.
int chunk_forward_split_segments(int BH, int T, int cus);
void launch_chunk_forward_split(const Fwd& p, int cus);
size_t chunk_forward_split_workspace(int B, int T, int H, int cus);

// Gated delta rule forward on the chunked MFMA kernels (gdn_chunk.hip): q, k, v and o
// [B,T,H,N] in dtype (0 = bf16, 1 = fp32), g, beta [B,T,H] fp32, states [B,H,key,value]
// when kv, else [value][key]; N = 64 or 128; qk_norm: L2-normalise q and k first.  The
// workspace holds every chunk's operands.
struct Gdn {
    int B, T, H, N, dtype, qk_norm;
    const void *q, *k, *v;
    const float *g, *beta;
    const float* s0;
    void* o;
    float* sT;
    void* ws;
    int kv;
    hipStream_t stream;
    size_t ws_bytes = 0;  // bytes at ws: the time-split scan runs when they cover its buffers
    int cus = 0;          // CUs the time split may spread the segments over (0: no split)
    float* ckpt = nullptr;  // saved states for gdn backward ([value][key], every 16 steps + final); no split
};
// Its backward for N = 128 (wkv7_rec_bwd.hip): q, k as the forward used them (normalised
// by the caller), dout [B,T,H,N] and the gradients of q, k, v in dtype; g, beta and their
// gradients [B,T,H] float32; dsT (may be null) and ds0 [B,H,key,value]; the forward's
// saved states; a workspace of gdn_backward_workspace bytes.
struct GdnBwd {
    int B, T, H, N, dtype;
    const void *q, *k, *v;
    const float *g, *beta;
    const float* ckpt;
    const void* dout;
    const float* dsT;
    void *dq, *dk, *dv;
    float *dg, *dbeta, *ds0;
    void* ws;
    hipStream_t stream;
};
size_t gdn_backward_workspace(int B, int T, int H);
void launch_gdn_backward(const GdnBwd& p);
// the operand records (the least a call needs); with the time split's buffers when it
// applies (gdn_split_segments >= 2)
size_t gdn_forward_workspace(int B, int T, int H, int N);
size_t gdn_forward_workspace_split(int B, int T, int H, int N, int cus);
int gdn_split_segments(int B, int T, int H, int N, int cus);
void launch_gdn_forward(const Gdn& p);
// The WKV7 forward for bf16, N = 128 and flags 0 on the same two kernels (per-key
// decays in the records): wkv7_rec_workspace bytes of records, or
// wkv7_rec_workspace_split with the time split's buffers (few heads, no saved states).
size_t wkv7_rec_workspace(int B, int T, int H, int N);
size_t wkv7_rec_workspace_split(int B, int T, int H, int N, int cus);
void launch_wkv7_rec_forward(const Fwd& p, int cus);
// Its backward (wkv7_rec_bwd.hip), every chunk at once from the [value][key] saved
// states: a workspace of wkv7_rec_bwd_workspace bytes (the scan's records and dL/dS at
// every chunk's end).
size_t wkv7_rec_bwd_workspace(int B, int T, int H);
void launch_wkv7_rec_backward(const Bwd& p);

// Family dispatch (wkv7_capi.cpp): the chunked MFMA kernels when they cover
// the call, else the step-serial ones.
void launch_forward(const Fwd& p);
void launch_backward(const Bwd& p);
size_t forward_workspace(int B, int T, int H, int N, int dtype, int flags = 0);
// forward_workspace, or more where the time-split forward could take the call
size_t forward_workspace_fast(int B, int T, int H, int N, int dtype, int flags = 0);
size_t backward_workspace(int B, int T, int H, int N, int dtype, int flags = 0);

}  // namespace wkv7
