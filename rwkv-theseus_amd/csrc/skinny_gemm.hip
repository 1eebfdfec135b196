// Y = act(X W^T) for few rows: the projections and LoRAs of a TimeMix serving step
// (theseus/timemix.py:63-69 run on B tokens of one step; B <= 128 rows).
//
// X [M][K] and W [N][K] are bf16, row-major (W in nn.Linear's [out][in] layout; the LoRA
// matrices, stored [in][out], are handed over transposed), Y [M][N] bf16, float32
// accumulation on v_mfma_f32_16x16x32_bf16.  With M this small the product is a stream
// over W (C=5120: 52 MB per projection against 0.6 MB of X), so the kernel is built to
// keep many bytes of W in flight:
//  * a workgroup (4 waves) owns 64 columns and a slice of K; wave w owns columns
//    16w..16w+15 and all MT 16-row tiles of X;
//  * W and X reach LDS by LDS DMA (buffer_load ... lds, wkv7_io.h) through a ring of D
//    stages of 128 k each (256 contiguous bytes of every row), issued D-1 stages ahead:
//    nothing is held in registers between a load and its use, and each workgroup keeps
//    D-1 stages (32-64 KB of W) in flight; each wave moves its own 16 rows of W and a
//    quarter of X, so the waves meet at one barrier per stage; a row's sixteen 16-byte
//    chunks are XOR-swizzled by row, so a 16-lane fragment read hits 16 bank groups;
//  * with the K range split over KS workgroups (split-K) each stores its float32 tile, and
//    gemm_reduce, launched after it on the same stream, sums the KS tiles in K order
//    (deterministic), applies the activation and stores bf16.
#include "../../include/theseus_gemm.h"
#include "../../include/theseus_wkv7.h"
#include "wkv7_io.h"

#include <algorithm>

namespace sg {
using namespace wkv7;

constexpr int KSMAX = 8;      // K slices at most

// A workgroup of WV waves owns 16 WV columns; a stage holds KST k of every row (2 KST
// contiguous bytes: whole DRAM bursts per row).
template <int MT, int WV, int KST>
struct Ring {
    static constexpr int COLS = 16 * WV;
    static constexpr int ROWB = 2 * KST;
    static constexpr int XB = 16 * MT * ROWB;                                // X bytes per stage
    static constexpr int SB = COLS * ROWB + XB;                               // bytes per stage (W first)
    static constexpr int D = (152 * 1024) / SB < 8 ? (152 * 1024) / SB : 8;  // stages
    static constexpr int CPR = ROWB / 16;                                     // 16-byte chunks per row
    static constexpr int RPI = 64 / CPR;                                      // rows per DMA instruction
    static constexpr int WI = 16 / RPI;                                       // W DMAs per wave and stage
    static constexpr int XI = (16 * MT / RPI + WV - 1) / WV;                 // X DMAs per wave and stage
    static constexpr int ND = WI + XI;
    static_assert(D >= 2 && (D - 2) * ND < 64, "ring depth");
};
// 16-byte chunk c of LDS row r holds logical chunk c ^ (r % chunks per row): a 16-lane
// fragment read (16 rows, one logical chunk) touches distinct bank groups
template <int CPR>
__device__ __forceinline__ int sw(int row) { return row & (CPR - 1) & 15; }

// s_waitcnt with vmcnt = n (gfx9 encoding; expcnt and lgkmcnt left unwaited)
template <int n>
__device__ __forceinline__ void vm_wait() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0f70 | (n & 15) | ((n >> 4) << 14));
    asm volatile("" ::: "memory");
}
// The activation is applied to the product rounded to bf16, as torch's bf16 matmul
// followed by torch.tanh / torch.sigmoid computes it under autocast (timemix.py:64, 67).
__device__ __forceinline__ float act(float x, int a) {
    if (a == THESEUS_GEMM_NONE) return x;
    x = bf16_to_f32(f32_to_bf16(x));
    return a == THESEUS_GEMM_TANH ? tanhf(x) : 1.f / (1.f + __expf(-x));
}

// One workgroup's part of a product: column tile `tile`, K slice ks of KS.
template <int MT, int WV, int KST>
__device__ __forceinline__ void gemm_tile(int M, int N, int K, int kchunk, int actf, int tile, int ks, int KS,
                                          const uint16_t* __restrict__ X, const uint16_t* __restrict__ W,
                                          uint16_t* __restrict__ Y, float* part) {
    using R = Ring<MT, WV, KST>;
    constexpr int CPR = R::CPR, ROWB = R::ROWB, COLS = R::COLS;
    extern __shared__ __align__(16) uint8_t lds[];  // R::D stages of R::SB bytes
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63, q = lane >> 4, r16 = lane & 15;
    const int n0 = tile * COLS + 16 * wv;  // this wave's first column
    const int k0 = ks * kchunk, kend = min(K, k0 + kchunk), nsteps = (kend - k0 + KST - 1) / KST;

    // DMA: one instruction fills RPI LDS rows, lane l row l / CPR, physical chunk l % CPR
    // with logical chunk (l % CPR) ^ sw(row); rows past M or N repeat the last row (never
    // stored).  Wave w moves rows 16w .. 16w+15 of W and X DMAs w, w + WV, ... (X rows
    // RPI i .. RPI i + RPI-1 of instruction i; waves past the count repeat one, which
    // writes the same bytes again)
    const i32x4_t wrs = dma_rsrc(W, (uint32_t)((long)N * K * 2)), xrs = dma_rsrc(X, (uint32_t)((long)M * K * 2));
    const int rl = lane / CPR, cl = lane % CPR;
    uint32_t w_off[R::WI], x_off[R::XI];
    int x_row0[R::XI];
#pragma unroll
    for (int i = 0; i < R::WI; i++) {
        const int row = 16 * wv + R::RPI * i + rl;  // LDS row of the W block
        w_off[i] = (uint32_t)((long)min(tile * COLS + row, N - 1) * K * 2 + 16 * (cl ^ sw<CPR>(row)));
    }
#pragma unroll
    for (int i = 0; i < R::XI; i++) {
        const int ins = (wv + WV * i) % (16 * MT / R::RPI);
        x_row0[i] = R::RPI * ins;
        const int row = x_row0[i] + rl;
        x_off[i] = (uint32_t)((long)min(row, M - 1) * K * 2 + 16 * (cl ^ sw<CPR>(row)));
    }
    auto issue = [&](int s) {  // stage s (clamped to the last: the same count of DMAs every time)
        const uint32_t kb = (uint32_t)((k0 + KST * min(s, nsteps - 1)) * 2);
        uint8_t* st = lds + (s % R::D) * R::SB;
#pragma unroll
        for (int i = 0; i < R::WI; i++)
            dma16(reinterpret_cast<const uint16_t*>(st + (16 * wv + R::RPI * i) * ROWB), wrs, w_off[i], kb);
#pragma unroll
        for (int i = 0; i < R::XI; i++)
            dma16(reinterpret_cast<const uint16_t*>(st + COLS * ROWB + __builtin_amdgcn_readfirstlane(x_row0[i]) * ROWB),
                  xrs, x_off[i], kb);
    };

    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = zero4();
#pragma unroll
    for (int s = 0; s < R::D - 1; s++) issue(s);
    for (int s = 0; s < nsteps; s++) {
        vm_wait<(R::D - 2) * R::ND>();  // this wave's DMAs of stage s have landed
        lds_barrier();                  // everyone's have; everyone is done with stage s - 1
        issue(s + R::D - 1);            // into the slot of stage s - 1
        const uint8_t* st = lds + (s % R::D) * R::SB;
        const int kleft = kend - k0 - KST * s;  // (a K tail ends the last stage early)
#pragma unroll
        for (int j = 0; j < KST / 32; j++) {  // k 32j .. 32j+31 of the stage: chunks 4j + q
            if (32 * j >= kleft) break;
            const int c = (4 * j + q) ^ sw<CPR>(r16);  // (every row read here is r16 mod 16)
            const uint4 b = *reinterpret_cast<const uint4*>(st + (16 * wv + r16) * ROWB + 16 * c);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const uint4 a = *reinterpret_cast<const uint4*>(st + COLS * ROWB + (16 * mt + r16) * ROWB + 16 * c);
                acc[mt] = mma32(acc[mt], a, b);
            }
        }
    }
    vm_wait<0>();  // (the ring's trailing DMAs, before the workgroup may end)

    if (KS > 1) {
        // split-K: this slice's tile in the accumulator layout, part[tile][ks][wave][mt][lane][4];
        // gemm_reduce sums the slices after the kernel
        float* dst = part + ((((long)tile * KS + ks) * WV + wv) * MT * 64 + lane) * 4;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) *reinterpret_cast<f32x4_t*>(dst + mt * 256) = acc[mt];
        return;
    }
    const int n = n0 + r16;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = 16 * mt + 4 * q + e;
            if (m < M && n < N) Y[(long)m * N + n] = f32_to_bf16(act(acc[mt][e], actf));
        }
}

template <int MT, int WV, int KST>
__global__ __launch_bounds__(WV * 64, 1) void skinny_gemm(int M, int N, int K, int kchunk, int actf,
                                                           const uint16_t* __restrict__ X,
                                                           const uint16_t* __restrict__ W,
                                                           uint16_t* __restrict__ Y, float* part) {
    gemm_tile<MT, WV, KST>(M, N, K, kchunk, actf, blockIdx.x, blockIdx.y, gridDim.y, X, W, Y, part);
}

// Several products with the same rows in one launch (a serving step's independent
// projections): problem i owns workgroups blk0 .. blk0 + tiles * KS - 1, in the order given.
constexpr int GMAX = THESEUS_GEMM_MAX_GROUP;
struct GemmProb {
    const uint16_t* X;
    const uint16_t* W;
    uint16_t* Y;
    float* part;
    int N, K, kchunk, KS, tiles, act, blk0, thr0;  // thr0: first reduce thread (KS > 1)
};
struct GemmGroup {
    int count;
    GemmProb p[GMAX];
};
template <int MT, int WV, int KST>
__global__ __launch_bounds__(WV * 64, 1) void skinny_gemm_group(int M, GemmGroup g) {
    const int b = blockIdx.x;
    int i = 0;
#pragma unroll
    for (int j = 1; j < GMAX; j++)
        if (j < g.count && b >= g.p[j].blk0) i = j;
    const GemmProb& p = g.p[i];
    const int local = b - p.blk0;
    gemm_tile<MT, WV, KST>(M, p.N, p.K, p.kchunk, p.act, local % p.tiles, local / p.tiles, p.KS, p.X, p.W, p.Y, p.part);
}

// Y from the KS float32 slices of every tile, summed in K order (deterministic), with the
// activation; one thread per (tile, wave, row tile, lane), as the GEMM's accumulator layout.
__device__ __forceinline__ void reduce_one(long t, int M, int N, int KS, int WV, int MT, int actf,
                                           const float* __restrict__ part, uint16_t* __restrict__ Y) {
    const int lane = (int)(t % 64), mt = (int)(t / 64 % MT), wv = (int)(t / (64 * MT) % WV);
    const long tile = t / (64L * MT * WV);
    const int n = (int)tile * 16 * WV + 16 * wv + (lane & 15), q = lane >> 4;
    if (n >= N || 16 * mt + 4 * q >= M) return;
    const long stride = (long)WV * MT * 64 * 4;  // between slices
    const float* p = part + ((tile * KS * WV + wv) * MT * 64 + mt * 64 + lane) * 4;
    f32x4_t s = zero4();
    for (int j = 0; j < KS; j++) s = s + *reinterpret_cast<const f32x4_t*>(p + j * stride);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int m = 16 * mt + 4 * q + e;
        if (m < M) Y[(long)m * N + n] = f32_to_bf16(act(s[e], actf));
    }
}
__global__ __launch_bounds__(256) void gemm_reduce(int M, int N, int KS, int WV, int MT, int actf,
                                                   const float* __restrict__ part, uint16_t* __restrict__ Y) {
    reduce_one((long)blockIdx.x * 256 + threadIdx.x, M, N, KS, WV, MT, actf, part, Y);
}
// the slices of a group's split products (those with KS > 1; thr0 their first thread)
__global__ __launch_bounds__(256) void gemm_reduce_group(int M, int WV, int MT, GemmGroup g) {
    const long t = (long)blockIdx.x * 256 + threadIdx.x;
    int i = -1;
#pragma unroll
    for (int j = 0; j < GMAX; j++)
        if (j < g.count && g.p[j].KS > 1 && t >= g.p[j].thr0) i = j;
    if (i < 0) return;
    const GemmProb& p = g.p[i];
    const long u = t - p.thr0;
    if (u >= (long)p.tiles * WV * MT * 64) return;
    reduce_one(u, M, p.N, p.KS, WV, MT, p.act, p.part, p.Y);
}

struct Plan {
    int MT, WV, KST, tiles, KS, kchunk;
};
// The shape: WV waves per workgroup and KST k per stage; K slices: about one workgroup per
// CU in all (the ring fills most of a CU's LDS), at most KSMAX slices of at least 2 stages.
constexpr int DEF_WV = 4, DEF_KST = 128;
inline Plan plan(int M, int N, int K, int cus, int wv = DEF_WV, int kst = DEF_KST, int per_cu = 1) {
    Plan p;
    const int mt = (M + 15) / 16;
    p.MT = mt <= 1 ? 1 : mt <= 2 ? 2 : mt <= 4 ? 4 : 8;
    p.WV = wv, p.KST = kst;
    p.tiles = (N + 16 * wv - 1) / (16 * wv);
    const int steps = (K + kst - 1) / kst;
    int ks = per_cu * cus / p.tiles;
    ks = std::max(1, std::min({ks, KSMAX, steps / 2}));
    p.kchunk = (steps + ks - 1) / ks * kst;
    p.KS = (K + p.kchunk - 1) / p.kchunk;
    return p;
}
inline size_t workspace(const Plan& p) { return p.KS > 1 ? (size_t)p.tiles * p.KS * p.WV * p.MT * 64 * 16 : 0; }
template <int MT, int WV, int KST>
inline int launch(const Plan& p, int M, int N, int K, int act, const uint16_t* X, const uint16_t* W, uint16_t* Y,
                  float* part, hipStream_t stream) {
    const size_t lds = (size_t)Ring<MT, WV, KST>::D * Ring<MT, WV, KST>::SB;
    // (beyond the default 64 KB of dynamic LDS; per function, cheap, so set before each launch)
    if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(&skinny_gemm<MT, WV, KST>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return THESEUS_WKV7_ERR_LAUNCH;
    hipLaunchKernelGGL((skinny_gemm<MT, WV, KST>), dim3(p.tiles, p.KS), dim3(WV * 64), lds, stream, M, N, K,
                       p.kchunk, act, X, W, Y, part);
    if (p.KS > 1) {
        const long threads = (long)p.tiles * WV * MT * 64;
        hipLaunchKernelGGL(gemm_reduce, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, M, N, p.KS, WV,
                           MT, act, part, Y);
    }
    return hipGetLastError() == hipSuccess ? THESEUS_WKV7_OK : THESEUS_WKV7_ERR_LAUNCH;
}
template <int WV, int KST>
inline int launch_mt(const Plan& p, int M, int N, int K, int act, const uint16_t* X, const uint16_t* W, uint16_t* Y,
                     float* part, hipStream_t stream) {
    switch (p.MT) {
        case 1: return launch<1, WV, KST>(p, M, N, K, act, X, W, Y, part, stream);
        case 2: return launch<2, WV, KST>(p, M, N, K, act, X, W, Y, part, stream);
        case 4: return launch<4, WV, KST>(p, M, N, K, act, X, W, Y, part, stream);
        default: return launch<8, WV, KST>(p, M, N, K, act, X, W, Y, part, stream);
    }
}

// A group's plan: each product gets a share of the CUs in proportion to its weight bytes
// and plans its K slices within that share (products of many column tiles then take one
// slice each: no partial tiles, no reduce).  Workgroups and reduce threads are numbered in
// the order of the products, partial tiles packed after one another in the workspace.
inline size_t plan_group(int M, int count, const theseus_gemm_problem* pr, int cus, GemmGroup& g, int& blocks,
                         long& rthreads, int& MT) {
    double tot = 0;
    for (int i = 0; i < count; i++) tot += (double)pr[i].N * pr[i].K;
    size_t ws = 0;
    blocks = 0, rthreads = 0;
    g.count = count;
    for (int i = 0; i < count; i++) {
        const int share = std::max(1, (int)(cus * ((double)pr[i].N * pr[i].K / tot)));
        const Plan p = plan(M, pr[i].N, pr[i].K, share);
        MT = p.MT;
        GemmProb& q = g.p[i];
        q.X = static_cast<const uint16_t*>(pr[i].x), q.W = static_cast<const uint16_t*>(pr[i].w);
        q.Y = static_cast<uint16_t*>(pr[i].y), q.part = nullptr;
        q.N = pr[i].N, q.K = pr[i].K, q.kchunk = p.kchunk, q.KS = p.KS, q.tiles = p.tiles, q.act = pr[i].act;
        q.blk0 = blocks, q.thr0 = (int)rthreads;
        blocks += p.tiles * p.KS;
        if (p.KS > 1) {
            q.part = reinterpret_cast<float*>(ws);  // (an offset until the workspace is known)
            ws += workspace(p);
            rthreads += (long)p.tiles * p.WV * p.MT * 64;
        }
    }
    for (int i = count; i < GMAX; i++) g.p[i] = GemmProb{};
    return ws;
}
template <int MT, int WV, int KST>
inline int launch_group(const GemmGroup& g, int M, int blocks, long rthreads, hipStream_t stream) {
    const size_t lds = (size_t)Ring<MT, WV, KST>::D * Ring<MT, WV, KST>::SB;
    if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(&skinny_gemm_group<MT, WV, KST>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return THESEUS_WKV7_ERR_LAUNCH;
    hipLaunchKernelGGL((skinny_gemm_group<MT, WV, KST>), dim3(blocks), dim3(WV * 64), lds, stream, M, g);
    if (rthreads)
        hipLaunchKernelGGL(gemm_reduce_group, dim3((unsigned)((rthreads + 255) / 256)), dim3(256), 0, stream, M, WV, MT, g);
    return hipGetLastError() == hipSuccess ? THESEUS_WKV7_OK : THESEUS_WKV7_ERR_LAUNCH;
}

int device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1)
        n = 256;
    return n;
}

}  // namespace sg

extern "C" {

// sizes the kernel takes: the shape rules of the header, and W, X and the partial tiles
// addressable with 32-bit buffer offsets
static bool gemm_shape_ok(int M, int N, int K) {
    if (M < 1 || M > THESEUS_GEMM_MAX_ROWS || N < 16 || N % 16 || K < 32 || K % 32) return false;
    return (long long)N * K * 2 < (1ll << 31) && (long long)M * K * 2 < (1ll << 31) && (long long)N * 128 * 16 * 8 < (1ll << 31);
}

size_t theseus_gemm_rows_workspace_size(int M, int N, int K) {
    if (!gemm_shape_ok(M, N, K)) return 0;
    return sg::workspace(sg::plan(M, N, K, sg::device_cus()));
}

int theseus_gemm_rows(int M, int N, int K, int act, const void* x, const void* w, void* y, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
    if (!gemm_shape_ok(M, N, K)) return THESEUS_WKV7_ERR_SHAPE;
    if (act < THESEUS_GEMM_NONE || act > THESEUS_GEMM_SIGMOID) return THESEUS_WKV7_ERR_FLAGS;
    if (!x || !w || !y) return THESEUS_WKV7_ERR_NULL;
    const sg::Plan p = sg::plan(M, N, K, sg::device_cus());
    const size_t need = sg::workspace(p);
    if (need && (!workspace || workspace_bytes < need)) return THESEUS_WKV7_ERR_WORKSPACE;
    return sg::launch_mt<sg::DEF_WV, sg::DEF_KST>(p, M, N, K, act, static_cast<const uint16_t*>(x),
                                                  static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y),
                                                  static_cast<float*>(workspace), stream);
}

static int group_ok(int M, int count, const theseus_gemm_problem* probs) {
    if (count < 1 || count > THESEUS_GEMM_MAX_GROUP || !probs) return THESEUS_WKV7_ERR_SHAPE;
    for (int i = 0; i < count; i++) {
        if (!gemm_shape_ok(M, probs[i].N, probs[i].K)) return THESEUS_WKV7_ERR_SHAPE;
        if (probs[i].act < THESEUS_GEMM_NONE || probs[i].act > THESEUS_GEMM_SIGMOID) return THESEUS_WKV7_ERR_FLAGS;
    }
    return THESEUS_WKV7_OK;
}

size_t theseus_gemm_rows_group_workspace_size(int M, int count, const theseus_gemm_problem* probs) {
    if (group_ok(M, count, probs)) return 0;
    sg::GemmGroup g;
    int blocks, MT;
    long rthreads;
    return sg::plan_group(M, count, probs, sg::device_cus(), g, blocks, rthreads, MT);
}

int theseus_gemm_rows_group(int M, int count, const theseus_gemm_problem* probs, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
    if (int e = group_ok(M, count, probs)) return e;
    for (int i = 0; i < count; i++)
        if (!probs[i].x || !probs[i].w || !probs[i].y) return THESEUS_WKV7_ERR_NULL;
    sg::GemmGroup g;
    int blocks, MT;
    long rthreads;
    const size_t need = sg::plan_group(M, count, probs, sg::device_cus(), g, blocks, rthreads, MT);
    if (need && (!workspace || workspace_bytes < need)) return THESEUS_WKV7_ERR_WORKSPACE;
    for (int i = 0; i < count; i++)
        if (g.p[i].KS > 1) g.p[i].part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) +
                                                                  reinterpret_cast<size_t>(g.p[i].part));
    switch (MT) {
        case 1: return sg::launch_group<1, sg::DEF_WV, sg::DEF_KST>(g, M, blocks, rthreads, stream);
        case 2: return sg::launch_group<2, sg::DEF_WV, sg::DEF_KST>(g, M, blocks, rthreads, stream);
        case 4: return sg::launch_group<4, sg::DEF_WV, sg::DEF_KST>(g, M, blocks, rthreads, stream);
        default: return sg::launch_group<8, sg::DEF_WV, sg::DEF_KST>(g, M, blocks, rthreads, stream);
    }
}

}  // extern "C"
