// theseus_wkv7_forward_noalloc: the forward recurrence for callers that may not
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  It runs exactly the kernels of
// theseus_wkv7_forward; the only difference is where the chunked forward's
// handoff workspace (boundary counters + carried states of heads cut between
// workgroups) lives: in `scratch`, a file-scope device array of
// THESEUS_WKV7_NOALLOC_SCRATCH_BYTES that the library owns, instead of a
// caller buffer.
//
// `scratch` is a symbol, not a device address, in host code: host code never
// passes it to a kernel or a copy.  On the first call on each device (with that
// device current) its address there is looked up once with hipGetSymbolAddress
// and kept per device; every launch uses that address.  Each device holds its
// own copy of the array until the process ends.  Every call on a device shares
// it, so calls that may run at the same time on one device (two streams) race;
// each call first clears the counters it uses with a fill kernel on its stream.
// Nothing here calls hipMalloc, hipFree or any allocating routine.
#include "../../include/theseus_wkv7.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "wkv7_launch.h"

static __device__ __align__(256) unsigned char scratch[THESEUS_WKV7_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];  // device address of `scratch`, per device
std::mutex g_lookup;

// This device's address of `scratch` (looked up on its first use), or null.
void* scratch_on_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> hold(g_lookup);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
        void* q = nullptr;
        if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return nullptr;
        g_scratch[dev].store(q, std::memory_order_release);
        p = q;
    }
    return p;
}

}  // namespace

extern "C" int theseus_wkv7_forward_noalloc(int B, int T, int H, int N, int dtype, const void* r,
                                            const void* w, const void* k, const void* v,
                                            const void* a, const void* b, const float* s0, void* y,
                                            float* sT, float* ckpt, hipStream_t stream) {
    if (B < 1 || H < 1 || T < 1 || N < 2 || N > 128) return THESEUS_WKV7_ERR_SHAPE;
    if (dtype != THESEUS_WKV7_BF16 && dtype != THESEUS_WKV7_FP32) return THESEUS_WKV7_ERR_DTYPE;
    if (!r || !w || !k || !v || !a || !b || !s0 || !y || !sT) return THESEUS_WKV7_ERR_NULL;
    const size_t need = wkv7::forward_workspace(B, T, H, N, dtype);
    if (need > (size_t)THESEUS_WKV7_NOALLOC_SCRATCH_BYTES) return THESEUS_WKV7_ERR_SCRATCH;
    void* ws = nullptr;
    if (need) {
        ws = scratch_on_current_device();
        if (!ws) return THESEUS_WKV7_ERR_LAUNCH;
    }
    wkv7::Fwd p{B, T, H, N, dtype, r, w, k, v, a, b, s0, y, sT, ckpt, ws, stream};
    wkv7::launch_forward(p);
    return hipGetLastError() == hipSuccess ? THESEUS_WKV7_OK : THESEUS_WKV7_ERR_LAUNCH;
}
