// C-ABI front end of libtheseus_wkv7.so (declared in include/theseus_wkv7.h).
//
// Validates sizes and pointers (the shape/dtype half of the reference's
// check(), kernels/wkv7_state.cpp:10-15; the torch-side half -- device,
// contiguity, same shapes -- is done by the Python wrapper, which owns the
// tensors), picks the kernel family, launches on the caller's stream and
// reports launch failures like C10_CUDA_KERNEL_LAUNCH_CHECK (cpp:24,36).
#include "../../include/theseus_wkv7.h"
#include "../../include/theseus_gdn.h"

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>

#include "wkv7_launch.h"

namespace {

constexpr int kAbiVersion = 2;

int check_dims(int B, int T, int H, int N, int dtype) {
    if (B < 1 || H < 1 || T < 1 || N < 2 || N > 128) return THESEUS_WKV7_ERR_SHAPE;
    if (dtype != THESEUS_WKV7_BF16 && dtype != THESEUS_WKV7_FP32) return THESEUS_WKV7_ERR_DTYPE;
    return THESEUS_WKV7_OK;
}

int launch_status() {
    return hipGetLastError() == hipSuccess ? THESEUS_WKV7_OK : THESEUS_WKV7_ERR_LAUNCH;
}

}  // namespace

namespace wkv7 {

// THESEUS_WKV7_FAMILY=seq forces the step-serial kernels (used by the tests to
// cross-check the two kernel families); anything else means automatic.
static bool force_seq() {
    const char* e = getenv("THESEUS_WKV7_FAMILY");
    return e && strcmp(e, "seq") == 0;
}
// Why the chunked kernels do not cover a call (0: they do).  They need bf16,
// N = 64, token tensors under 2 GiB and one head's saved states under 4 GiB:
// both are addressed with 32-bit buffer offsets (the token tensors' range
// check also drops rows past a partial chunk, so the limit is 2^31).
int chunk_refusal(int B, int T, int H, int N, int dtype, int flags) {
    if (force_seq()) return THESEUS_WKV7_FAMILY_FORCED;
    if (flags) return THESEUS_WKV7_FAMILY_FLAGS;
    if (dtype != THESEUS_WKV7_BF16) return THESEUS_WKV7_FAMILY_FP32;
    if (N != 64) return THESEUS_WKV7_FAMILY_HEAD_SIZE;
    if ((long long)B * T * H * N * 2 >= (1ll << 31) ||
        ((long long)(T + kCkptInterval - 1) / kCkptInterval + 1) * N * N * 4 >= (1ll << 32))
        return THESEUS_WKV7_FAMILY_SIZE;
    return 0;
}
static bool chunk_ok(int B, int T, int H, int N, int dtype, int flags) {
    return chunk_refusal(B, T, H, N, dtype, flags) == 0;
}

// bf16, N = 128 and no flags: the forward on the chunk-record kernels (gdn_chunk.hip)
// when the caller's workspace holds the records -- theseus_wkv7_forward_workspace_size
// counts them, theseus_wkv7_forward_noalloc brings none and stays step-serial -- and the
// backward on wkv7_rec_bwd.hip's (its workspace is required).  One head's records stay
// under 4 GiB (32-bit DMA offsets), B*H within the preps' grid y.
static bool rec_shape(int B, int T, int H, int N, int dtype, int flags) {
    return chunk_refusal(B, T, H, N, dtype, flags) == THESEUS_WKV7_FAMILY_HEAD_SIZE && N == 128 &&
           (long long)B * H <= 65535 && wkv7_rec_workspace(1, T, 1, N) < (1ull << 32);
}
static bool rec_ok(const Fwd& p) {
    return rec_shape(p.B, p.T, p.H, p.N, p.dtype, p.flags) && p.ws &&
           p.ws_bytes >= wkv7_rec_workspace(p.B, p.T, p.H, p.N);
}

// CUs of the current device, which the chunked kernels' schedule spreads the
// heads over (one workgroup each).  THESEUS_WKV7_CUS=<n> plans for n instead
// (the tests use it to cut heads at small sizes).
static int cu_count() {
    if (const char* e = getenv("THESEUS_WKV7_CUS")) {
        const int n = atoi(e);
        if (n > 0) return n;
    }
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
        n = 1;  // (cutting no head is always correct)
    return n;
}

// The time-split forward: few heads (at least two jobs per head, one CU each) and at
// least 8 chunks; it needs no saved states and its own workspace (split_ok below).
static bool split_shape(int B, int T, int H, int N, int dtype, int flags) {
    return chunk_ok(B, T, H, N, dtype, flags) && (T + kCkptInterval - 1) / kCkptInterval >= 8 &&
           2ll * B * H <= cu_count() && chunk_forward_split_segments(B * H, T, cu_count()) >= 2;
}
static bool split_ok(const Fwd& p) {
    return !p.ckpt && split_shape(p.B, p.T, p.H, p.N, p.dtype, p.flags) && p.ws &&
           p.ws_bytes >= chunk_forward_split_workspace(p.B, p.T, p.H, cu_count());
}

void launch_forward(const Fwd& p) {
    if (p.T == 1 && !p.ckpt && !force_seq() && !(p.flags & FLAG_STATE_KV)) {
        // one step without saved states (the serving step through the operator):
        // the single-step kernel, s0 -> sT
        Dec d{p.B, p.H, p.N, p.dtype, p.r, p.w, p.k, p.v, p.a, p.b, p.s0, p.sT, p.y, p.stream};
        d.flags = p.flags;
        launch_decode(d);
    } else if (split_ok(p)) launch_chunk_forward_split(p, cu_count());
    else if (chunk_ok(p.B, p.T, p.H, p.N, p.dtype, p.flags)) launch_chunk_forward(p, cu_count());
    else if (rec_ok(p)) launch_wkv7_rec_forward(p, cu_count());
    else launch_seq_forward(p);
}
void launch_backward(const Bwd& p) {
    if (chunk_ok(p.B, p.T, p.H, p.N, p.dtype, p.flags)) launch_chunk_backward(p, cu_count());
    else if (rec_shape(p.B, p.T, p.H, p.N, p.dtype, p.flags)) launch_wkv7_rec_backward(p);
    else launch_seq_backward(p);
}
// The chunked kernels' handoffs; the step-serial backward replays each
// 16-step segment into its workspace (its forward needs none).
size_t forward_workspace(int B, int T, int H, int N, int dtype, int flags) {
    return chunk_ok(B, T, H, N, dtype, flags) ? chunk_forward_workspace(B, T, H, cu_count()) : 0;
}
size_t forward_workspace_fast(int B, int T, int H, int N, int dtype, int flags) {
    if (rec_shape(B, T, H, N, dtype, flags)) return wkv7_rec_workspace_split(B, T, H, N, cu_count());
    const size_t need = forward_workspace(B, T, H, N, dtype, flags);
    if (!split_shape(B, T, H, N, dtype, flags)) return need;
    const size_t split = chunk_forward_split_workspace(B, T, H, cu_count());
    return split > need ? split : need;
}
size_t backward_workspace(int B, int T, int H, int N, int dtype, int flags) {
    if (chunk_ok(B, T, H, N, dtype, flags)) return chunk_backward_workspace(B, T, H, cu_count());
    if (rec_shape(B, T, H, N, dtype, flags)) return wkv7_rec_bwd_workspace(B, T, H);
    return seq_backward_workspace(B, H, N);
}

}  // namespace wkv7

extern "C" {

int theseus_wkv7_abi_version(void) { return kAbiVersion; }

const char* theseus_wkv7_error_string(int status) {
    switch (status) {
        case THESEUS_WKV7_OK: return "ok";
        case THESEUS_WKV7_ERR_SHAPE: return "invalid T or head size (2..128)";
        case THESEUS_WKV7_ERR_DTYPE: return "expected BF16 or FP32";
        case THESEUS_WKV7_ERR_NULL: return "null pointer argument";
        case THESEUS_WKV7_ERR_WORKSPACE: return "workspace too small";
        case THESEUS_WKV7_ERR_LAUNCH: return "HIP kernel launch failed";
        case THESEUS_WKV7_ERR_FLAGS: return "unknown flags (THESEUS_WKV7_DECAY_EXP | THESEUS_WKV7_STATE_KEY_VALUE)";
        case THESEUS_WKV7_ERR_SCRATCH:
            return "sizes need more handoff scratch than the library's static array holds "
                   "(THESEUS_WKV7_NOALLOC_SCRATCH_BYTES); use theseus_wkv7_forward with a workspace";
        default: return "unknown status";
    }
}

int theseus_wkv7_kernel_family(int B, int T, int H, int N, int dtype) {
    if (int e = check_dims(B, T, H, N, dtype)) return -e;
    if (wkv7::rec_shape(B, T, H, N, dtype, 0)) return THESEUS_WKV7_FAMILY_RECORDS;
    return wkv7::chunk_refusal(B, T, H, N, dtype, 0);
}

int theseus_wkv7_wait_timeouts(unsigned int* count, int reset) {
    if (!count) return THESEUS_WKV7_ERR_NULL;
    uint32_t f = 0, b = 0;
    if (wkv7::chunk_forward_wait_timeouts(&f, reset) || wkv7::chunk_backward_wait_timeouts(&b, reset))
        return THESEUS_WKV7_ERR_LAUNCH;
    *count = f + b;
    return THESEUS_WKV7_OK;
}

int theseus_wkv7_set_waits(int on) {
    if (wkv7::chunk_forward_waits(on) || wkv7::chunk_backward_waits(on)) return THESEUS_WKV7_ERR_LAUNCH;
    return THESEUS_WKV7_OK;
}

int theseus_wkv7_checkpoint_interval(void) { return wkv7::kCkptInterval; }

long long theseus_wkv7_checkpoint_count(int T) {
    return T < 1 ? 0 : (long long)(T + wkv7::kCkptInterval - 1) / wkv7::kCkptInterval + 1;
}

size_t theseus_wkv7_forward_workspace_size(int B, int T, int H, int N, int dtype) {
    if (check_dims(B, T, H, N, dtype) != THESEUS_WKV7_OK) return 0;
    return wkv7::forward_workspace_fast(B, T, H, N, dtype);
}

size_t theseus_wkv7_backward_workspace_size(int B, int T, int H, int N, int dtype) {
    if (check_dims(B, T, H, N, dtype) != THESEUS_WKV7_OK) return 0;
    return wkv7::backward_workspace(B, T, H, N, dtype);
}

int theseus_wkv7_forward_ex(int B, int T, int H, int N, int dtype, int flags, const void* r,
                            const void* w, const void* k, const void* v, const void* a, const void* b,
                            const float* s0, void* y, float* sT, float* ckpt, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
    if (int e = check_dims(B, T, H, N, dtype)) return e;
    if (flags & ~wkv7::FLAGS_ALL) return THESEUS_WKV7_ERR_FLAGS;
    if (!r || !w || !k || !v || !a || !b || !s0 || !y || !sT) return THESEUS_WKV7_ERR_NULL;
    const size_t need = wkv7::forward_workspace(B, T, H, N, dtype, flags);
    if (workspace_bytes < need || (need && !workspace)) return THESEUS_WKV7_ERR_WORKSPACE;
    wkv7::Fwd p{B, T, H, N, dtype, r, w, k, v, a, b, s0, y, sT, ckpt, workspace, stream};
    p.flags = flags;
    p.ws_bytes = workspace_bytes;
    wkv7::launch_forward(p);
    return launch_status();
}

int theseus_wkv7_forward(int B, int T, int H, int N, int dtype, const void* r, const void* w,
                         const void* k, const void* v, const void* a, const void* b,
                         const float* s0, void* y, float* sT, float* ckpt, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
    return theseus_wkv7_forward_ex(B, T, H, N, dtype, 0, r, w, k, v, a, b, s0, y, sT, ckpt, workspace,
                                   workspace_bytes, stream);
}

int theseus_wkv7_backward_ex(int B, int T, int H, int N, int dtype, int flags, const void* r,
                             const void* w, const void* k, const void* v, const void* a, const void* b,
                             const float* ckpt, const void* dy, const float* dsT, void* dr, void* dw,
                             void* dk, void* dv, void* da, void* db, float* ds0, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
    if (int e = check_dims(B, T, H, N, dtype)) return e;
    if (flags & ~wkv7::FLAGS_ALL) return THESEUS_WKV7_ERR_FLAGS;
    if (!r || !w || !k || !v || !a || !b || !ckpt || !dy || !dr || !dw || !dk || !dv || !da ||
        !db || !ds0)
        return THESEUS_WKV7_ERR_NULL;
    const size_t need = wkv7::backward_workspace(B, T, H, N, dtype, flags);
    if (workspace_bytes < need || (need && !workspace)) return THESEUS_WKV7_ERR_WORKSPACE;
    wkv7::Bwd p{B, T, H, N, dtype, r, w, k, v, a, b, ckpt, dy, dsT,
                dr, dw, dk, dv, da, db, ds0, workspace, stream};
    p.flags = flags;
    wkv7::launch_backward(p);
    return launch_status();
}

int theseus_wkv7_backward(int B, int T, int H, int N, int dtype, const void* r, const void* w,
                          const void* k, const void* v, const void* a, const void* b,
                          const float* ckpt, const void* dy, const float* dsT, void* dr,
                          void* dw, void* dk, void* dv, void* da, void* db, float* ds0,
                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return theseus_wkv7_backward_ex(B, T, H, N, dtype, 0, r, w, k, v, a, b, ckpt, dy, dsT, dr, dw, dk, dv,
                                    da, db, ds0, workspace, workspace_bytes, stream);
}

size_t theseus_wkv7_workspace_size_ex(int B, int T, int H, int N, int dtype, int flags, int backward) {
    if (check_dims(B, T, H, N, dtype) != THESEUS_WKV7_OK || (flags & ~wkv7::FLAGS_ALL)) return 0;
    return backward ? wkv7::backward_workspace(B, T, H, N, dtype, flags)
                    : wkv7::forward_workspace_fast(B, T, H, N, dtype, flags);
}

int theseus_wkv7_decode_step(int B, int H, int N, int dtype, const void* r, const void* w,
                             const void* k, const void* v, const void* a, const void* b,
                             float* state, void* y, hipStream_t stream) {
    if (int e = check_dims(B, 1, H, N, dtype)) return e;
    if (!r || !w || !k || !v || !a || !b || !state || !y) return THESEUS_WKV7_ERR_NULL;
    wkv7::Dec p{B, H, N, dtype, r, w, k, v, a, b, state, state, y, stream};
    wkv7::launch_decode(p);
    return launch_status();
}

// The chunked GDN kernels: N = 64 or 128, B*H workgroups (at most 65535 along the
// operand kernel's grid y), and one head's chunk records under 4 GiB (32-bit DMA offsets).
static int gdn_dims(int B, int T, int H, int N) {
    if (B < 1 || H < 1 || T < 1 || (N != 64 && N != 128) || (long long)B * H > 65535) return THESEUS_WKV7_ERR_SHAPE;
    return wkv7::gdn_forward_workspace(1, T, 1, N) >= (1ull << 32) ? THESEUS_WKV7_ERR_SHAPE : THESEUS_WKV7_OK;
}

size_t theseus_gdn_forward_workspace_size(int B, int T, int H, int N) {
    return gdn_dims(B, T, H, N) ? 0 : wkv7::gdn_forward_workspace_split(B, T, H, N, wkv7::cu_count());
}

int theseus_gdn_forward(int B, int T, int H, int N, int dtype, int qk_l2norm, const void* q, const void* k,
                        const void* v, const float* g, const float* beta, const float* s0, void* o, float* sT,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (int e = gdn_dims(B, T, H, N)) return e;
    if (dtype != THESEUS_WKV7_BF16 && dtype != THESEUS_WKV7_FP32) return THESEUS_WKV7_ERR_DTYPE;
    if (!q || !k || !v || !g || !beta || !s0 || !o || !sT) return THESEUS_WKV7_ERR_NULL;
    if (!workspace || workspace_bytes < wkv7::gdn_forward_workspace(B, T, H, N)) return THESEUS_WKV7_ERR_WORKSPACE;
    wkv7::Gdn p{B, T, H, N, dtype, qk_l2norm ? 1 : 0, q, k, v, g, beta, s0, o, sT, workspace, 1, stream};
    p.ws_bytes = workspace_bytes;
    p.cus = wkv7::cu_count();
    wkv7::launch_gdn_forward(p);
    return launch_status();
}

int theseus_gdn_forward_train(int B, int T, int H, int N, int dtype, const void* q, const void* k, const void* v,
                              const float* g, const float* beta, const float* s0, void* o, float* sT, float* ckpt,
                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (int e = gdn_dims(B, T, H, N)) return e;
    if (dtype != THESEUS_WKV7_BF16 && dtype != THESEUS_WKV7_FP32) return THESEUS_WKV7_ERR_DTYPE;
    if (!q || !k || !v || !g || !beta || !s0 || !o || !sT || !ckpt) return THESEUS_WKV7_ERR_NULL;
    if (!workspace || workspace_bytes < wkv7::gdn_forward_workspace(B, T, H, N)) return THESEUS_WKV7_ERR_WORKSPACE;
    wkv7::Gdn p{B, T, H, N, dtype, 0, q, k, v, g, beta, s0, o, sT, workspace, 1, stream};
    p.ws_bytes = workspace_bytes;
    p.ckpt = ckpt;
    wkv7::launch_gdn_forward(p);
    return launch_status();
}

size_t theseus_gdn_backward_workspace_size(int B, int T, int H, int N) {
    return gdn_dims(B, T, H, N) || N != 128 ? 0 : wkv7::gdn_backward_workspace(B, T, H);
}

int theseus_gdn_backward(int B, int T, int H, int N, int dtype, const void* q, const void* k, const void* v,
                         const float* g, const float* beta, const float* ckpt, const void* dout, const float* dsT,
                         void* dq, void* dk, void* dv, float* dg, float* dbeta, float* ds0, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
    if (int e = gdn_dims(B, T, H, N)) return e;
    if (N != 128) return THESEUS_WKV7_ERR_SHAPE;
    if (dtype != THESEUS_WKV7_BF16 && dtype != THESEUS_WKV7_FP32) return THESEUS_WKV7_ERR_DTYPE;
    if (!q || !k || !v || !g || !beta || !ckpt || !dout || !dq || !dk || !dv || !dg || !dbeta || !ds0)
        return THESEUS_WKV7_ERR_NULL;
    if (!workspace || workspace_bytes < wkv7::gdn_backward_workspace(B, T, H)) return THESEUS_WKV7_ERR_WORKSPACE;
    wkv7::GdnBwd p{B, T, H, N, dtype, q, k, v, g, beta, ckpt, dout, dsT, dq, dk, dv, dg, dbeta, ds0, workspace, stream};
    wkv7::launch_gdn_backward(p);
    return launch_status();
}

}  // extern "C"
