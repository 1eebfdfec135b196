// Load-balanced schedule of the chunked WKV7 kernels over the CUs.
//
// A job is one (b, h) head: n chunks that must be processed in order (forward:
// chunk 0 first; backward: chunk n-1 first).  The kernels keep one workgroup
// per CU (their LDS use admits no second), so J > CUs jobs of one workgroup
// each would run in ceil(J / CUs) rounds, the last one mostly idle (320 heads on
// 256 CUs: two rounds for 1.25 rounds of work).
//
// Instead the J*n (job, chunk) units are laid end to end, job after job, and
// "machine" m owns the global positions [m L, (m+1) L) with
// L = max(n, ceil(J n / CUs)) (wrap-around, McNaughton's rule).  A job that
// crosses the boundary m L is cut in two and rotated: its FIRST steps are the
// positions at the start of machine m, its LAST steps the positions at the end
// of machine m-1.  Machine m runs its first piece at local times [0, e) and
// hands the job's carried state over at step e; machine m-1 reaches that job's
// last piece at local time L - (n - e) >= e, so with machines moving at equal
// speed the handoff is ready L - n ticks before it is needed.  Every machine
// holds at most two cut pieces (one at each end), whole jobs in between.
//
// Machine m runs as workgroup G-1-m, so a waiting piece's workgroup has a
// higher index than the one it waits on: workgroups are dispatched in index
// order, so the awaited workgroup is already running (or done) whenever a
// waiter spins, whatever the number of CUs free.  The wait is bounded all the
// same (a missing handoff poisons the state with NaN instead of hanging).
//
// Handoffs go through a caller workspace: one 32-bit counter per boundary
// (zeroed by clear_words on the same stream before the kernel) and the carried
// state.  Every consumer wave of the handing workgroup stores its part and
// counts itself in; the waiting waves read it once the count is complete.
//
// Visibility across the XCDs (each has its own L2): every handoff word and
// counter is accessed only through agent-scope atomics, which compile to
// sc1 loads and stores that the hardware keeps coherent per location at agent
// scope (stores write through, loads do not hit a stale line).  The writer's
// s_waitcnt vmcnt(0) completes its stores before its counter increment is
// issued; the reader issues its data loads only after a counter load has
// returned the full count.  An agent-scope release/acquire fence pair would
// instead write back and invalidate the whole L2 of both XCDs at every
// handoff (measured: 10-17 % of the kernels' time).
#pragma once

#include "wkv7_common.h"

namespace wkv7 {

struct Sched {
    int J;  // jobs (B*H)
    int n;  // chunks per job
    int L;  // positions per machine
    int G;  // machines = workgroups
};

__host__ __device__ inline Sched plan_schedule(int J, int n, int cus) {
    const long total = (long)J * n, per = (total + cus - 1) / cus;
    const int L = (int)(per > n ? per : n);
    return Sched{J, n, L, (int)((total + L - 1) / L)};
}
// some job is cut in two (L a multiple of n places whole jobs only)
__host__ __device__ inline bool sched_cuts(const Sched& s) { return s.L % s.n != 0; }
// workspace: the boundary counters (256-byte aligned), then `per` floats per boundary
__host__ __device__ inline size_t sched_flag_bytes(const Sched& s) { return ((size_t)s.G * 4 + 255) / 256 * 256; }
__host__ __device__ inline size_t sched_workspace(const Sched& s, size_t per) {
    return sched_cuts(s) ? sched_flag_bytes(s) + (size_t)s.G * per * 4 : 0;
}

// One job's piece on one machine: steps [step0, step0 + count) of job `job`.
struct Seg {
    int job, step0, count;
    bool fresh;    // starts the job (else it continues from the handoff at boundary m + 1)
    bool handoff;  // hands the job over at boundary m (else it ends the job)
};
__device__ __forceinline__ Seg seg_of(const Sched& s, int m, int j) {
    const int p0 = m * s.L, p1 = min(p0 + s.L, s.J * s.n), j0 = j * s.n;
    const int lo = max(j0, p0), hi = min(j0 + s.n, p1);
    Seg g;
    g.job = j;
    g.count = hi - lo;
    g.handoff = lo > j0;                 // the job began at the end of machine m - 1: first steps here
    g.fresh = g.handoff || hi == j0 + s.n;  // else: the job runs on into machine m + 1, last steps here
    g.step0 = g.fresh ? 0 : s.n - g.count;
    return g;
}
// stream index x of machine m -> (job, step)
__device__ __forceinline__ int2 stream_at(const Sched& s, int m, int x) {
    const int p = m * s.L + x, j = p / s.n;
    const Seg g = seg_of(s, m, j);
    return make_int2(j, g.step0 + p - max(j * s.n, m * s.L));
}
__device__ __forceinline__ int stream_len(const Sched& s, int m) { return min(s.L, s.J * s.n - m * s.L); }
__device__ __forceinline__ int machine_of_block(const Sched& s) { return s.G - 1 - (int)blockIdx.x; }

// A stream position as (job j = bb H + h, offset r = p - j n within the job's n
// positions, and the job's step there), advanced without division: a producer
// wave visits every NPROD-th position and keeps a cursor on its current chunk
// and one on its next.
struct Cursor {
    int j, r, bb, h, step;
};
// the step of job j at offset r within it on machine m (as stream_at)
__device__ __forceinline__ int step_of(const Sched& s, int m, int j, int r) {
    return seg_of(s, m, j).step0 + r - max(0, m * s.L - j * s.n);
}
__device__ __forceinline__ Cursor cursor_at(const Sched& s, int m, int x, int H) {
    const int p = m * s.L + x, j = p / s.n, r = p - j * s.n;
    return Cursor{j, r, j / H, j % H, step_of(s, m, j, r)};
}
__device__ __forceinline__ void cursor_advance(Cursor& c, const Sched& s, int m, int k, int H) {
    c.r += k;
    while (c.r >= s.n) {
        c.r -= s.n;
        c.j++;
        if (++c.h == H) c.h = 0, c.bb++;
    }
    c.step = step_of(s, m, c.j, c.r);
}

// handoff words: agent-scope atomic stores / loads only
__device__ __forceinline__ void handoff_put(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float handoff_get(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void handoff_put4(float* p, float a, float b, float c, float d) {
    handoff_put(p, a), handoff_put(p + 1, b), handoff_put(p + 2, c), handoff_put(p + 3, d);
}
__device__ __forceinline__ float4 handoff_get4(const float* p) {
    return make_float4(handoff_get(p), handoff_get(p + 1), handoff_get(p + 2), handoff_get(p + 3));
}
// This wave's handoff stores have completed: count it in.
__device__ __forceinline__ void handoff_signal(uint32_t* cnt) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Bounded waits that time out poison what depends on them with NaN, and count the
// time-out here (one word per file that includes this header, per device), so that the
// host can tell a time-out from a NaN input (wait_timeouts_read, theseus_wkv7_wait_timeouts).
// g_wait_on = 0 (set from the host for tests, theseus_wkv7_set_waits) makes every bounded
// wait give up at once, which forces the time-out path without any wave waiting forever.
static __device__ uint32_t g_wait_timeouts;
static __device__ int g_wait_on = 1;
__device__ __forceinline__ void note_timeout() {
    if ((threadIdx.x & 63) == 0)
        __hip_atomic_fetch_add(&g_wait_timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// the spin bound of a wait (n, or 0 while the host has switched waits off), read once
__device__ __forceinline__ int wait_bound(int n) {
    return __builtin_amdgcn_readfirstlane(*(volatile const int*)&g_wait_on) ? n : 0;
}
// host side: read this file's time-out count on the current device (and zero it), or
// switch its waits on / off; synchronous
static inline int wait_timeouts_read(uint32_t* out, bool reset) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(g_wait_timeouts), sizeof(uint32_t)) != hipSuccess) return -1;
    const uint32_t zero = 0;
    if (reset && hipMemcpyToSymbol(HIP_SYMBOL(g_wait_timeouts), &zero, sizeof(uint32_t)) != hipSuccess) return -1;
    return 0;
}
static inline int wait_switch(int on) {
    const int v = on ? 1 : 0;
    return hipMemcpyToSymbol(HIP_SYMBOL(g_wait_on), &v, sizeof(int)) == hipSuccess ? 0 : -1;
}

// Wait (bounded, about a second) until `target` waves have counted in; the
// handoff loads come after it in program order (and the compiler may not move
// them above it).  Returns false on time-out (counted).
__device__ __forceinline__ bool handoff_wait(const uint32_t* cnt, uint32_t target) {
    bool ok = false;
    const int lim = wait_bound(1 << 21);
    for (int i = 0; i < lim && !ok; i++) {
        ok = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target;
        if (!ok) __builtin_amdgcn_s_sleep(8);
    }
    asm volatile("" ::: "memory");
    if (!ok) note_timeout();
    return ok;
}

// zero `n` 32-bit words (the boundary counters; a kernel, not a memset, so the
// sequence may be captured into a graph)
__global__ static void clear_words(uint32_t* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

}  // namespace wkv7
