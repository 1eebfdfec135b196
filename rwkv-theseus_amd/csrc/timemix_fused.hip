// Fused elementwise kernels around the WKV7 recurrence in TimeMix (gfx950).
//
// Each replaces a chain of torch ops of theseus/timemix.py:66-89 with one pass
// over HBM (forward) or one pass plus a small fixed-order reduction of the
// parameter gradients (backward):
//   shift-lerp     mixed_n = x + (x[t-1] - x) * coef_n, six outputs   (:70-71)
//   kk / k-mod     kk = normalize(k*k_k), kw = k*(1+(a-1)k_a), -kk, kk*a  (:78-80)
//   GN+bonus+gate  ((GroupNorm(y) + (sum r*kmod*r_k) v) * g)        (:83-88)
// with a = sigmoid(a0 + za) (:75) formed inside the kernels that read it, from the bf16
// LoRA output za and the parameter a0; its backward is folded into theirs.
// Head rows of 64 channels are handled by 8 lanes x 8 channels (16-byte bf16
// vectors); row sums are 8-lane butterflies.  Parameter gradients are
// accumulated per (head, token block) and reduced over token blocks by
// reduce_blocks in a fixed order, so results are deterministic.
#include "../../include/theseus_timemix.h"
#include "../../include/theseus_wkv7.h"
#include "wkv7_common.h"

#include <algorithm>

namespace tmix {
using namespace wkv7;

constexpr int HN = 64;   // head size handled here
constexpr int TB = 64;   // tokens per block for the parameter-gradient partials
constexpr int HG = 8;    // heads per block of the kk / GroupNorm backward kernels

struct V8 {
    float x[8];
};
// Inputs read exactly once are loaded non-temporally (ld_str8, ld_row, ld_f8s): measured at
// config 3, kk_bwd 156 -> 138 µs and kk_fwd 91 -> 82 µs with them; the shift-lerp forward,
// whose threads re-read the row before their first token, keeps ordinary loads (it ran 4 %
// slower with them).  Stores stay ordinary: their results are read by the next kernel.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4v_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_raw8(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint4 ld_str8(const uint16_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ V8 cvt_bf8(uint4 u) {
    V8 r;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.x[2 * i] = bf16_to_f32((uint16_t)(w[i] & 0xffffu));
        r.x[2 * i + 1] = bf16_to_f32((uint16_t)(w[i] >> 16));
    }
    return r;
}
__device__ __forceinline__ V8 ld_f8s(const float* p) {
    const f32x4v_t a = __builtin_nontemporal_load(reinterpret_cast<const f32x4v_t*>(p));
    const f32x4v_t b = __builtin_nontemporal_load(reinterpret_cast<const f32x4v_t*>(p + 4));
    return V8{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
}
__device__ __forceinline__ V8 ld_f8(const float* p) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    return V8{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
}
__device__ __forceinline__ void st_bf8(uint16_t* p, const V8& v) {
    uint4 u;
    u.x = f32x2_to_bf16x2(v.x[0], v.x[1]);
    u.y = f32x2_to_bf16x2(v.x[2], v.x[3]);
    u.z = f32x2_to_bf16x2(v.x[4], v.x[5]);
    u.w = f32x2_to_bf16x2(v.x[6], v.x[7]);
    *reinterpret_cast<uint4*>(p) = u;
}
__device__ __forceinline__ void st_f8(float* p, const V8& v) {
    *reinterpret_cast<float4*>(p) = make_float4(v.x[0], v.x[1], v.x[2], v.x[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v.x[4], v.x[5], v.x[6], v.x[7]);
}
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }
// a = sigmoid(a0 + za) of theseus/timemix.py:75 in float32 (za, the LoRA output, is bf16 and
// the parameter a0 float32 under bf16 autocast): formed in every kernel that reads `a`, so
// no [B,T,C] float32 `a` is written or read
__device__ __forceinline__ V8 gate_a(const V8& a0, uint4 za) {
    const V8 z = cvt_bf8(za);
    V8 r;
#pragma unroll
    for (int e = 0; e < 8; e++) r.x[e] = 1.f / (1.f + expf(-(a0.x[e] + z.x[e])));
    return r;
}
__device__ __forceinline__ float sum8(float x) {  // over the 8 lanes of a head row
    x += __shfl_xor(x, 1, 8);
    x += __shfl_xor(x, 2, 8);
    x += __shfl_xor(x, 4, 8);
    return x;
}

// ---------------------------------------------------------------- shift-lerp
// Thread: 8 channels of SLT consecutive tokens (the six coefficient vectors loaded once,
// all x rows issued before use, x[t-1] taken from the previous token's registers).
constexpr int SLT = 8;
__global__ __launch_bounds__(256) void shift_lerp_fwd(long M, int T, int C, const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ st,
                                                      const float* __restrict__ coef, uint16_t* o0,
                                                      uint16_t* o1, uint16_t* o2, uint16_t* o3,
                                                      uint16_t* o4, uint16_t* o5) {
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;
    const int cv = C / 8;
    const long ng = (M + SLT - 1) / SLT;
    if (gid >= ng * cv) return;
    const long m0 = gid / cv * SLT, m1 = min(M, m0 + SLT);
    const int c = (int)(gid % cv) * 8;
    uint4 xr[SLT];
#pragma unroll
    for (int u = 0; u < SLT; u++) xr[u] = m0 + u < m1 ? ld_raw8(x + (m0 + u) * C + c) : make_uint4(0, 0, 0, 0);
    const uint4 prev0 = (m0 % T) > 0 ? ld_raw8(x + (m0 - 1) * C + c) : ld_raw8(st + (m0 / T) * C + c);
    V8 cf[6];
#pragma unroll
    for (int n = 0; n < 6; n++) cf[n] = ld_f8(coef + n * C + c);
    uint16_t* outs[6] = {o0, o1, o2, o3, o4, o5};
#pragma unroll
    for (int u = 0; u < SLT; u++) {
        const long m = m0 + u;
        if (m < m1) {
            const int t = (int)(m % T), b = (int)(m / T);
            const V8 xv = cvt_bf8(xr[u]);
            const V8 pv = cvt_bf8(t > 0 ? (u == 0 ? prev0 : xr[u - 1]) : ld_raw8(st + (long)b * C + c));
            float d[8];
#pragma unroll
            for (int e = 0; e < 8; e++) d[e] = round_bf16(pv.x[e] - xv.x[e]);  // delta is a bf16 tensor
#pragma unroll
            for (int n = 0; n < 6; n++) {
                V8 o;
#pragma unroll
                for (int e = 0; e < 8; e++) o.x[e] = xv.x[e] + d[e] * cf[n].x[e];
                st_bf8(outs[n] + m * C + c, o);
            }
        }
    }
}

// 1-D grid of ceil(C/(64 SV)) x ceil(M/TBk) waves (channel blocks fastest), SV channels
// per lane.  A wave walks its TBk tokens in order (the parameter-gradient partials are sums
// over them), UG tokens at a time: all loads of a group -- the six gradient rows of tokens
// m+1 .. m+UG (token m's are carried over) and the x rows of m .. m+UG-1 (x[m-1] is
// carried) -- are issued before any is used, and with PF the next group's loads are issued
// before the current group is used, so the wave waits on memory about once per group pair.
// Loads past the end of the tensors re-read its last row (their values are not used), so
// every group issues the same sequence of loads.  Measured at config 3 (B=2, T=4096,
// C=5120) against other shapes of the same kernel: 16-byte rows, 2 tokens per group,
// prefetch and 48 tokens per wave 146 µs (with the partials' reduction), 4-byte rows 152-171,
// 8-byte rows 149-167, 16-byte rows without prefetch 166-180; forcing more waves per SIMD
// than the registers allow spills.
//
// The registers hold one wave per SIMD, and a wave's time grows with its tokens, so TBk is
// planned (sl_tokens below) to give each SIMD of the device one wave: config 3's 8192 tokens
// x 10 channel blocks as 100 blocks of 82 tokens (1000 waves, one round) ran in 134 µs where
// 171 blocks of 48 (1710 waves, two rounds, the second two thirds full) ran in 145 µs;
// 900 or 960 waves of 92 or 86 tokens, leaving SIMDs idle, 149 and 136 µs.  Shapes that
// fit two or three waves per SIMD, each planned the same way (8-byte rows; or one token per
// group, with or without the prefetch), were no faster: 138-159 µs.
constexpr int SV = 8, UG = 2;
constexpr bool SPF = true;
template <int V>
struct RowT;
template <>
struct RowT<4> {
    typedef u32x2_t type;
};
template <>
struct RowT<8> {
    typedef u32x4_t type;
};
template <int V>
__device__ __forceinline__ typename RowT<V>::type ld_row(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const typename RowT<V>::type*>(p));
}
template <int V>
__device__ __forceinline__ float el(const typename RowT<V>::type& u, int e) {  // channel e
    const uint32_t w = u[e >> 1];
    return (e & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
}
template <int V>
__device__ __forceinline__ void st_row(uint16_t* p, const float (&v)[V]) {
    typename RowT<V>::type u;
#pragma unroll
    for (int w = 0; w < V / 2; w++) u[w] = f32x2_to_bf16x2(v[2 * w], v[2 * w + 1]);
    *reinterpret_cast<typename RowT<V>::type*>(p) = u;
}
template <int V, int G, bool PF>
__global__ __launch_bounds__(64) void shift_lerp_bwd(long M, int T, int C, int TBk, const uint16_t* d0,
                                                     const uint16_t* d1, const uint16_t* d2,
                                                     const uint16_t* d3, const uint16_t* d4,
                                                     const uint16_t* d5, const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ st,
                                                     const float* __restrict__ coef, uint16_t* dx,
                                                     uint16_t* dshift, float* __restrict__ part) {
    static_assert(V % 4 == 0, "coefficients and partials move as float4");
    typedef typename RowT<V>::type row_t;
    const int nbx = (C + 64 * V - 1) / (64 * V), bx = blockIdx.x % nbx, by = blockIdx.x / nbx;
    const int c = (bx * 64 + threadIdx.x) * V;
    if (c >= C) return;
    const long m0 = (long)by * TBk, m1 = min(M, m0 + TBk);
    const uint16_t* dn[6] = {d0, d1, d2, d3, d4, d5};
    float cf[6][V], acc[6][V];
#pragma unroll
    for (int n = 0; n < 6; n++)
#pragma unroll
        for (int e = 0; e < V; e += 4) {
            const float4 f = *reinterpret_cast<const float4*>(coef + n * C + c + e);
            cf[n][e] = f.x, cf[n][e + 1] = f.y, cf[n][e + 2] = f.z, cf[n][e + 3] = f.w;
        }
#pragma unroll
    for (int n = 0; n < 6; n++)
#pragma unroll
        for (int e = 0; e < V; e++) acc[n][e] = 0.f;
    row_t dcur[6];  // gradient rows of the group's first token
#pragma unroll
    for (int n = 0; n < 6; n++) dcur[n] = ld_row<V>(dn[n] + m0 * C + c);
    row_t xprev = ld_row<V>((m0 % T) > 0 ? x + (m0 - 1) * C + c : st + (m0 / T) * C + c);
    auto load = [&](long m, row_t (&dr)[G][6], row_t (&xr)[G]) {
#pragma unroll
        for (int u = 0; u < G; u++) {
            const long row = min(m + 1 + u, M - 1);  // (the last token's successor may lie past m1)
#pragma unroll
            for (int n = 0; n < 6; n++) dr[u][n] = ld_row<V>(dn[n] + row * C + c);
            xr[u] = ld_row<V>(x + min(m + u, M - 1) * C + c);
        }
    };
    auto compute = [&](long m, const row_t (&dr)[G][6], const row_t (&xr)[G]) {
#pragma unroll
        for (int u = 0; u < G; u++) {
            const long mm = m + u;
            if (mm < m1) {
                const int t = (int)(mm % T), b = (int)(mm / T);
                const row_t pr = t > 0 ? (u == 0 ? xprev : xr[u - 1]) : ld_row<V>(st + (long)b * C + c);
                const bool nxt = t + 1 < T;
                float gx[V], gs[V];
#pragma unroll
                for (int e = 0; e < V; e++) {
                    const float delta = round_bf16(el<V>(pr, e) - el<V>(xr[u], e));
                    float dsum = 0.f, dc = 0.f, nx = 0.f;
#pragma unroll
                    for (int n = 0; n < 6; n++) {
                        const float cu = el<V>(u == 0 ? dcur[n] : dr[u - 1][n], e);
                        dsum += cu;
                        dc += cu * cf[n][e];
                        nx += el<V>(dr[u][n], e) * cf[n][e];
                        acc[n][e] += cu * delta;
                    }
                    gx[e] = dsum - dc + (nxt ? nx : 0.f);
                    gs[e] = dc;
                }
                st_row<V>(dx + mm * C + c, gx);
                if (t == 0) st_row<V>(dshift + (long)b * C + c, gs);
            }
        }
        xprev = xr[G - 1];
#pragma unroll
        for (int n = 0; n < 6; n++) dcur[n] = dr[G - 1][n];
    };
    if (!PF) {
        for (long m = m0; m < m1; m += G) {
            row_t dr[G][6], xr[G];
            load(m, dr, xr);
            compute(m, dr, xr);
        }
    } else {
        row_t da[G][6], xa[G], db[G][6], xb[G];
        load(m0, da, xa);
        for (long m = m0; m < m1; m += 2 * G) {
            load(m + G, db, xb);
            compute(m, da, xa);
            if (m + G >= m1) break;
            load(m + 2 * G, da, xa);
            compute(m + G, db, xb);
        }
    }
    float* pb = part + (long)by * 6 * C;
#pragma unroll
    for (int n = 0; n < 6; n++)
#pragma unroll
        for (int e = 0; e < V; e += 4)
            *reinterpret_cast<float4*>(pb + n * C + c + e) =
                make_float4(acc[n][e], acc[n][e + 1], acc[n][e + 2], acc[n][e + 3]);
}

// part is [nblk][P][C]; outs[p][c] = sum_b part[b][p][c], summed in block order
struct Outs {
    float* p[6];
};
__global__ __launch_bounds__(256) void reduce_blocks(const float* __restrict__ part, int nblk, int P, int C,
                                                     Outs outs) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= P * C) return;
    const long stride = (long)P * C;
    float s = 0.f;
    int b = 0;
    for (; b + 16 <= nblk; b += 16) {  // 16 loads in flight, summed in block order
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = part[(b + u) * stride + j];
#pragma unroll
        for (int u = 0; u < 16; u++) s += v[u];
    }
    for (; b < nblk; b++) s += part[b * stride + j];
    outs.p[j / C][j % C] = s;
}

// ---------------------------------------------------------------- decay input
// w = (w0 + zw).to(bf16) of theseus/timemix.py:73, 80: the float32 parameter w0 plus the bf16
// LoRA output zw, rounded to bf16 once (the reference adds in float32 and casts); 8 channels
// per thread, whole rows of threads over whole rows of w.
__global__ __launch_bounds__(256) void add_param_bf16(long n8, int C, const uint16_t* __restrict__ z,
                                                      const float* __restrict__ p, uint16_t* __restrict__ out) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const int c = (int)(i % (C / 8)) * 8;
    const V8 zv = cvt_bf8(ld_str8(z + 8 * i)), pv = ld_f8(p + c);
    V8 o;
#pragma unroll
    for (int e = 0; e < 8; e++) o.x[e] = pv.x[e] + zv.x[e];
    st_bf8(out + 8 * i, o);
}

// ---------------------------------------------------------------- kk / k-mod
// The forward kernels: ceil(H / 8) x ceil(M / (4 U)) workgroups of 256 lanes, head groups
// first (workgroups next in line read neighbouring 1 KB runs of the same tokens; token-first
// order made both kernels 8-10 % slower); wave w takes 8 consecutive heads (a whole 1 KB run
// of a token per load) of the tokens 4 U tb + U w + u, u < U, all U tokens' loads issued
// before any is used and the parameter vectors loaded once (gn_fwd: 127 -> 121 µs at
// config 3 against one (token, head) row per 8 lanes).
// KU / FU tokens per wave: 4 for long inputs, 1 for short ones (a serving step's 64 tokens
// would fill only 40 workgroups with 4: 7.3 against 4.5 µs per gn_fwd call)
constexpr int U_LONG = 4;
template <int KU>
__global__ __launch_bounds__(256) void kk_fwd(long M, int H, int C, const uint16_t* __restrict__ k,
                                              const uint16_t* __restrict__ za, const float* __restrict__ a0p,
                                              const float* __restrict__ kkp, const float* __restrict__ kap,
                                              uint16_t* kw, uint16_t* aw, uint16_t* bw) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, sub = l & 7;
    const int ng = (H + 7) / 8, h = (int)(blockIdx.x % ng) * 8 + (l >> 3);
    const bool hok = h < H;
    const int c = (hok ? h : 0) * HN + 8 * sub;
    const long mb = ((long)(blockIdx.x / ng) * 4 + w) * KU;
    uint4 kr[KU], zr[KU];
#pragma unroll
    for (int u = 0; u < KU; u++) {
        const bool ok = hok && mb + u < M;
        const long o = ok ? (mb + u) * C + c : c;
        kr[u] = ld_str8(k + o);
        zr[u] = ld_str8(za + o);
    }
    const V8 kk_ = ld_f8(kkp + c), ka = ld_f8(kap + c), a0 = ld_f8(a0p + c);
#pragma unroll
    for (int u = 0; u < KU; u++) {
        const V8 kv = cvt_bf8(kr[u]), av = gate_a(a0, zr[u]);
        float uu[8], ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            uu[e] = kv.x[e] * kk_.x[e];
            ss += uu[e] * uu[e];
        }
        ss = sum8(ss);
        const float inv = 1.f / fmaxf(sqrtf(ss), 1e-12f);
        V8 ow, oa, ob;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float kkv = uu[e] * inv;
            ow.x[e] = kv.x[e] * (1.f + (av.x[e] - 1.f) * ka.x[e]);
            oa.x[e] = -kkv;
            ob.x[e] = kkv * av.x[e];
        }
        if (hok && mb + u < M) {
            const long o = (mb + u) * C + c;
            st_bf8(kw + o, ow);
            st_bf8(aw + o, oa);
            st_bf8(bw + o, ob);
        }
    }
}

// grid (ceil(H/HG), ceil(M/TB)), 256 lanes = 32 rows x 8 lanes
// dza = (this kernel's part of dL/da) a (1 - a) + dzg, where dzg is gn_bwd's part, already
// times a (1 - a) (float32, or null): the two parts meet in float32 and dza (bf16) is
// rounded once; partials dk_k, dk_a and a0's gradient (the sum of dza over tokens)
__global__ __launch_bounds__(256) void kk_bwd(long M, int H, int C, const uint16_t* __restrict__ dkw,
                                              const uint16_t* __restrict__ daw,
                                              const uint16_t* __restrict__ dbw, const uint16_t* __restrict__ k,
                                              const uint16_t* __restrict__ za, const float* __restrict__ a0p,
                                              const float* __restrict__ dzg, const float* __restrict__ kkp,
                                              const float* __restrict__ kap, uint16_t* dk, uint16_t* dza,
                                              float* __restrict__ part) {
    __shared__ float red[3][32][HN + 1];
    // 32 rows = 4 tokens x HG consecutive heads, so a wave reads whole 1 KB runs of a token;
    // the next step's rows are loaded before this step's arithmetic
    const int rs = threadIdx.x >> 3, sub = threadIdx.x & 7, hh = rs % HG, tt = rs / HG;
    const int h = blockIdx.x * HG + hh;
    const bool hok = h < H;
    const int c = (hok ? h : 0) * HN + 8 * sub;
    const V8 kk_ = ld_f8(kkp + c), ka = ld_f8(kap + c), a0 = ld_f8(a0p + c);
    float acc_kk[8] = {}, acc_ka[8] = {}, acc_a0[8] = {};
    uint4 nk, nz, nw, na, nb;
    V8 ngz;
    auto fetch = [&](int it) {
        const long m = (long)blockIdx.y * TB + it * 4 + tt;
        const long o = hok && m < M ? m * C + c : c;
        nk = ld_str8(k + o);
        nz = ld_str8(za + o);
        nw = ld_str8(dkw + o);
        na = ld_str8(daw + o);
        nb = ld_str8(dbw + o);
        ngz = dzg ? ld_f8s(dzg + o) : V8{};
    };
    fetch(0);
    for (int it = 0; it < TB / 4; it++) {
        const long m = (long)blockIdx.y * TB + it * 4 + tt;
        const bool ok = hok && m < M;
        const long o = m * C + c;
        V8 kv = cvt_bf8(nk), av = gate_a(a0, nz), gw = cvt_bf8(nw), ga = cvt_bf8(na), gb = cvt_bf8(nb), gz = ngz;
        if (!ok) kv = gw = ga = gb = gz = V8{};
        if (it + 1 < TB / 4) fetch(it + 1);
        float u[8], ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            u[e] = kv.x[e] * kk_.x[e];
            ss += u[e] * u[e];
        }
        ss = sum8(ss);
        const float nrm = sqrtf(ss);
        const bool clamped = nrm <= 1e-12f;
        const float inv = 1.f / fmaxf(nrm, 1e-12f);
        float kkv[8], dkk[8], dot = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kkv[e] = u[e] * inv;
            dkk[e] = -ga.x[e] + gb.x[e] * av.x[e];
            dot += kkv[e] * dkk[e];
        }
        dot = sum8(dot);
        V8 gk, gz_out;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float du = clamped ? dkk[e] * inv : (dkk[e] - kkv[e] * dot) * inv;
            gk.x[e] = du * kk_.x[e] + gw.x[e] * (1.f + (av.x[e] - 1.f) * ka.x[e]);
            const float gav = gb.x[e] * kkv[e] + gw.x[e] * kv.x[e] * ka.x[e];  // dL/da, this part
            const float dz = gav * (av.x[e] * (1.f - av.x[e])) + gz.x[e];
            gz_out.x[e] = dz;
            acc_kk[e] += du * kv.x[e];
            acc_ka[e] += gw.x[e] * kv.x[e] * (av.x[e] - 1.f);
            acc_a0[e] += dz;
        }
        if (ok) {
            st_bf8(dk + o, gk);
            st_bf8(dza + o, gz_out);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
        red[0][rs][8 * sub + e] = acc_kk[e];
        red[1][rs][8 * sub + e] = acc_ka[e];
        red[2][rs][8 * sub + e] = acc_a0[e];
    }
    __syncthreads();
    for (int q = threadIdx.x; q < 3 * HG * HN; q += 256) {  // sum the 4 token rows of each head
        const int p = q / (HG * HN), hq = (q / HN) % HG, n = q % HN, hd = blockIdx.x * HG + hq;
        if (hd < H) {
            float s = 0.f;
            for (int i = 0; i < 32 / HG; i++) s += red[p][i * HG + hq][n];
            part[((long)blockIdx.y * 3 + p) * C + hd * HN + n] = s;
        }
    }
}

// ---------------------------------------------------------------- GroupNorm + bonus + gate
template <int FU>  // tokens per wave (mapped as kk_fwd)
__global__ __launch_bounds__(256) void gn_fwd(long M, int H, int C, const uint16_t* __restrict__ y,
                                              const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
                                              const uint16_t* __restrict__ za, const float* __restrict__ a0p,
                                              const float* __restrict__ kap,
                                              const uint16_t* __restrict__ v, const uint16_t* __restrict__ g,
                                              const float* __restrict__ rkp, const float* __restrict__ lwp,
                                              const float* __restrict__ lbp, float eps, uint16_t* out) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, sub = l & 7;
    const int ng = (H + 7) / 8, h = (int)(blockIdx.x % ng) * 8 + (l >> 3);
    const bool hok = h < H;
    const int c = (hok ? h : 0) * HN + 8 * sub;
    const long mb = ((long)(blockIdx.x / ng) * 4 + w) * FU;
    uint4 yr[FU], rr[FU], kr[FU], vr[FU], gr[FU], zr[FU];
#pragma unroll
    for (int u = 0; u < FU; u++) {
        const bool ok = hok && mb + u < M;
        const long o = ok ? (mb + u) * C + c : c;
        yr[u] = ld_str8(y + o);
        rr[u] = ld_str8(r + o);
        kr[u] = ld_str8(k + o);
        vr[u] = ld_str8(v + o);
        gr[u] = ld_str8(g + o);
        zr[u] = ld_str8(za + o);
    }
    const V8 ka = ld_f8(kap + c), rk = ld_f8(rkp + c), lw = ld_f8(lwp + c), lb = ld_f8(lbp + c);
    const V8 a0 = ld_f8(a0p + c);
#pragma unroll
    for (int u = 0; u < FU; u++) {
        const V8 yv = cvt_bf8(yr[u]), rv = cvt_bf8(rr[u]), kv = cvt_bf8(kr[u]), vv = cvt_bf8(vr[u]), gv = cvt_bf8(gr[u]);
        const V8 av = gate_a(a0, zr[u]);
        float s = 0.f, cd = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            s += yv.x[e];
            cd += rv.x[e] * (kv.x[e] * (1.f + (av.x[e] - 1.f) * ka.x[e])) * rk.x[e];
        }
        const float mean = sum8(s) * (1.f / HN);
        cd = sum8(cd);
        float var = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) var += (yv.x[e] - mean) * (yv.x[e] - mean);
        const float rstd = rsqrtf(sum8(var) * (1.f / HN) + eps);
        V8 ov;
#pragma unroll
        for (int e = 0; e < 8; e++)
            ov.x[e] = ((yv.x[e] - mean) * rstd * lw.x[e] + lb.x[e] + cd * vv.x[e]) * gv.x[e];
        if (hok && mb + u < M) st_bf8(out + (mb + u) * C + c, ov);
    }
}

// grid (ceil(H/HG), ceil(M/TB)), 256 lanes = 32 rows x 8 lanes
// dzg = this kernel's part of dL/da times a (1 - a), float32, for kk_bwd to finish dza
__global__ __launch_bounds__(256) void gn_bwd(long M, int H, int C, const uint16_t* __restrict__ dout,
                                              const uint16_t* __restrict__ y, const uint16_t* __restrict__ r,
                                              const uint16_t* __restrict__ k, const uint16_t* __restrict__ za,
                                              const float* __restrict__ a0p, const float* __restrict__ kap,
                                              const uint16_t* __restrict__ v, const uint16_t* __restrict__ g,
                                              const float* __restrict__ rkp, const float* __restrict__ lwp,
                                              const float* __restrict__ lbp, float eps, uint16_t* dy,
                                              uint16_t* dr, uint16_t* dk, uint16_t* dv, uint16_t* dg,
                                              float* dzg, float* __restrict__ part) {
    __shared__ float red[4][32][HN + 1];
    // 32 rows = 4 tokens x HG consecutive heads, as kk_bwd
    const int rs = threadIdx.x >> 3, sub = threadIdx.x & 7, hh = rs % HG, tt = rs / HG;
    const int h = blockIdx.x * HG + hh;
    const bool hok = h < H;
    const int c = (hok ? h : 0) * HN + 8 * sub;
    const V8 ka = ld_f8(kap + c), rk = ld_f8(rkp + c), lw = ld_f8(lwp + c), lb = ld_f8(lbp + c);
    const V8 a0 = ld_f8(a0p + c);
    float acc[4][8] = {};  // dr_k, dln_w, dln_b, dk_a
    uint4 ny, nr, nk, nz, nv, ng, no;
    auto fetch = [&](int it) {
        const long m = (long)blockIdx.y * TB + it * 4 + tt;
        const long o = hok && m < M ? m * C + c : c;
        ny = ld_str8(y + o);
        nr = ld_str8(r + o);
        nk = ld_str8(k + o);
        nz = ld_str8(za + o);
        nv = ld_str8(v + o);
        ng = ld_str8(g + o);
        no = ld_str8(dout + o);
    };
    fetch(0);
    for (int it = 0; it < TB / 4; it++) {
        const long m = (long)blockIdx.y * TB + it * 4 + tt;
        const bool ok = hok && m < M;
        const long o = m * C + c;
        V8 yv = cvt_bf8(ny), rv = cvt_bf8(nr), kv = cvt_bf8(nk), av = gate_a(a0, nz), vv = cvt_bf8(nv), gv = cvt_bf8(ng),
           go = cvt_bf8(no);
        if (!ok) yv = rv = kv = av = vv = gv = go = V8{};
        if (it + 1 < TB / 4) fetch(it + 1);
        float km[8], s = 0.f, cd = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            km[e] = kv.x[e] * (1.f + (av.x[e] - 1.f) * ka.x[e]);
            s += yv.x[e];
            cd += rv.x[e] * km[e] * rk.x[e];
        }
        const float mean = sum8(s) * (1.f / HN);
        cd = sum8(cd);
        float var = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) var += (yv.x[e] - mean) * (yv.x[e] - mean);
        const float rstd = rsqrtf(sum8(var) * (1.f / HN) + eps);
        float yh[8], ds[8], dyh[8], m1 = 0.f, m2 = 0.f, dc = 0.f;
        V8 ogg, ogv;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            yh[e] = (yv.x[e] - mean) * rstd;
            const float sv = yh[e] * lw.x[e] + lb.x[e] + cd * vv.x[e];
            ds[e] = go.x[e] * gv.x[e];
            ogg.x[e] = go.x[e] * sv;
            ogv.x[e] = ds[e] * cd;
            dyh[e] = ds[e] * lw.x[e];
            m1 += dyh[e];
            m2 += dyh[e] * yh[e];
            dc += ds[e] * vv.x[e];
            acc[1][e] += ds[e] * yh[e];
            acc[2][e] += ds[e];
        }
        m1 = sum8(m1) * (1.f / HN);
        m2 = sum8(m2) * (1.f / HN);
        dc = sum8(dc);
        V8 ogy, ogr, ogk, oga;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            ogy.x[e] = rstd * (dyh[e] - m1 - yh[e] * m2);
            ogr.x[e] = dc * km[e] * rk.x[e];
            const float dkm = dc * rv.x[e] * rk.x[e];
            ogk.x[e] = dkm * (1.f + (av.x[e] - 1.f) * ka.x[e]);
            oga.x[e] = dkm * kv.x[e] * ka.x[e] * (av.x[e] * (1.f - av.x[e]));  // dL/da a (1 - a)
            acc[0][e] += dc * rv.x[e] * km[e];
            acc[3][e] += dkm * kv.x[e] * (av.x[e] - 1.f);
        }
        if (ok) {
            st_bf8(dy + o, ogy);
            st_bf8(dr + o, ogr);
            st_bf8(dk + o, ogk);
            st_bf8(dv + o, ogv);
            st_bf8(dg + o, ogg);
            st_f8(dzg + o, oga);
        }
    }
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int e = 0; e < 8; e++) red[p][rs][8 * sub + e] = acc[p][e];
    __syncthreads();
    for (int q = threadIdx.x; q < 4 * HG * HN; q += 256) {  // sum the 4 token rows of each head
        const int p = q / (HG * HN), hq = (q / HN) % HG, n = q % HN, hd = blockIdx.x * HG + hq;
        if (hd < H) {
            float s = 0.f;
            for (int i = 0; i < 32 / HG; i++) s += red[p][i * HG + hq][n];
            part[((long)blockIdx.y * 4 + p) * C + hd * HN + n] = s;
        }
    }
}

}  // namespace tmix

// ------------------------------------------------------------------ C ABI
namespace {
int tm_check(int B, int T, int C) {
    if (B < 1 || T < 1 || C < tmix::HN || C % tmix::HN) return THESEUS_WKV7_ERR_SHAPE;
    // token blocks run along the grid's y dimension (at most 65535 blocks)
    if ((long)B * T > 65535L * tmix::TB) return THESEUS_WKV7_ERR_SHAPE;
    return THESEUS_WKV7_OK;
}
int tm_status() { return hipGetLastError() == hipSuccess ? THESEUS_WKV7_OK : THESEUS_WKV7_ERR_LAUNCH; }
long nblk_t(int B, int T) { return ((long)B * T + tmix::TB - 1) / tmix::TB; }
int device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1)
        n = 256;
    return n;
}
// tokens per wave of shift_lerp_bwd: as many token blocks as one round of one wave per SIMD
// (4 per CU) holds over the channel blocks, but at least 16 tokens per wave (a block's
// partials, 24 bytes per channel, then cost at most a tenth of its inputs, 14 bytes per
// channel and token)
long sl_tokens(int B, int T, int C) {
    const long M = (long)B * T, nbx = (C + 64 * tmix::SV - 1) / (64 * tmix::SV);
    const long per_round = std::max(1L, 4L * device_cus() / nbx);
    return std::max(std::min(16L, M), (M + per_round - 1) / per_round);
}
long nblk_sl(int B, int T, int C) {
    const long tb = sl_tokens(B, T, C);
    return ((long)B * T + tb - 1) / tb;
}
}  // namespace

extern "C" {

int theseus_tm_shift_lerp_fwd(int B, int T, int C, const void* x, const void* st, const float* coef,
                              void* const* out, hipStream_t stream) {
    if (int e = tm_check(B, T, C)) return e;
    if (!x || !st || !coef || !out) return THESEUS_WKV7_ERR_NULL;
    for (int n = 0; n < 6; n++)
        if (!out[n]) return THESEUS_WKV7_ERR_NULL;
    const long M = (long)B * T, total = (M + tmix::SLT - 1) / tmix::SLT * (C / 8);
    hipLaunchKernelGGL(tmix::shift_lerp_fwd, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, M, T, C,
                       (const uint16_t*)x, (const uint16_t*)st, coef, (uint16_t*)out[0], (uint16_t*)out[1],
                       (uint16_t*)out[2], (uint16_t*)out[3], (uint16_t*)out[4], (uint16_t*)out[5]);
    return tm_status();
}

size_t theseus_tm_shift_lerp_workspace(int B, int T, int C) {
    return tm_check(B, T, C) ? 0 : (size_t)nblk_sl(B, T, C) * 6 * C * sizeof(float);
}

int theseus_tm_shift_lerp_bwd(int B, int T, int C, const void* const* dm, const void* x, const void* st,
                              const float* coef, void* dx, void* dshift, float* dcoef, float* ws,
                              size_t ws_bytes, hipStream_t stream) {
    if (int e = tm_check(B, T, C)) return e;
    if (!dm || !x || !st || !coef || !dx || !dshift || !dcoef) return THESEUS_WKV7_ERR_NULL;
    for (int n = 0; n < 6; n++)
        if (!dm[n]) return THESEUS_WKV7_ERR_NULL;
    if (!ws || ws_bytes < theseus_tm_shift_lerp_workspace(B, T, C)) return THESEUS_WKV7_ERR_WORKSPACE;
    const long M = (long)B * T;
    const int nb = (int)nblk_sl(B, T, C), tb = (int)sl_tokens(B, T, C);
    hipLaunchKernelGGL((tmix::shift_lerp_bwd<tmix::SV, tmix::UG, tmix::SPF>),
                       dim3((unsigned)((C + 64 * tmix::SV - 1) / (64 * tmix::SV) * (long)nb)), dim3(64), 0, stream, M,
                       T, C, tb, (const uint16_t*)dm[0], (const uint16_t*)dm[1], (const uint16_t*)dm[2],
                       (const uint16_t*)dm[3], (const uint16_t*)dm[4], (const uint16_t*)dm[5],
                       (const uint16_t*)x, (const uint16_t*)st, coef, (uint16_t*)dx, (uint16_t*)dshift, ws);
    tmix::Outs o6{{dcoef, dcoef + C, dcoef + 2 * C, dcoef + 3 * C, dcoef + 4 * C, dcoef + 5 * C}};
    hipLaunchKernelGGL(tmix::reduce_blocks, dim3((6 * C + 255) / 256), dim3(256), 0, stream, ws, nb, 6, C, o6);
    return tm_status();
}

int theseus_tm_add_param_fwd(int B, int T, int C, const void* z, const float* p, void* out, hipStream_t stream) {
    if (int e = tm_check(B, T, C)) return e;
    if (!z || !p || !out) return THESEUS_WKV7_ERR_NULL;
    const long n8 = (long)B * T * C / 8;
    hipLaunchKernelGGL(tmix::add_param_bf16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream, n8, C,
                       (const uint16_t*)z, p, (uint16_t*)out);
    return tm_status();
}

int theseus_tm_kk_fwd(int B, int T, int C, const void* k, const void* za, const float* a0, const float* k_k,
                      const float* k_a, void* kw, void* aw, void* bw, hipStream_t stream) {
    if (int e = tm_check(B, T, C)) return e;
    if (!k || !za || !a0 || !k_k || !k_a || !kw || !aw || !bw) return THESEUS_WKV7_ERR_NULL;
    const int H = C / tmix::HN;
    const long M = (long)B * T;
    const int U = M >= 4096 ? tmix::U_LONG : 1;
    hipLaunchKernelGGL(U == 1 ? tmix::kk_fwd<1> : tmix::kk_fwd<tmix::U_LONG>,
                       dim3((unsigned)((M + 4 * U - 1) / (4 * U) * ((H + 7) / 8))), dim3(256), 0, stream, M, H, C,
                       (const uint16_t*)k, (const uint16_t*)za, a0, k_k, k_a, (uint16_t*)kw, (uint16_t*)aw, (uint16_t*)bw);
    return tm_status();
}

size_t theseus_tm_kk_workspace(int B, int T, int C) {
    return tm_check(B, T, C) ? 0 : (size_t)nblk_t(B, T) * 3 * C * sizeof(float);
}

int theseus_tm_kk_bwd(int B, int T, int C, const void* dkw, const void* daw, const void* dbw, const void* k,
                      const void* za, const float* a0, const float* dzg, const float* k_k, const float* k_a,
                      void* dk, void* dza, float* da0, float* dk_k, float* dk_a, float* ws, size_t ws_bytes,
                      hipStream_t stream) {
    if (int e = tm_check(B, T, C)) return e;
    if (!dkw || !daw || !dbw || !k || !za || !a0 || !k_k || !k_a || !dk || !dza || !da0 || !dk_k || !dk_a)
        return THESEUS_WKV7_ERR_NULL;
    if (!ws || ws_bytes < theseus_tm_kk_workspace(B, T, C)) return THESEUS_WKV7_ERR_WORKSPACE;
    const int H = C / tmix::HN, nb = (int)nblk_t(B, T);
    hipLaunchKernelGGL(tmix::kk_bwd, dim3((H + tmix::HG - 1) / tmix::HG, nb), dim3(256), 0, stream, (long)B * T, H, C, (const uint16_t*)dkw,
                       (const uint16_t*)daw, (const uint16_t*)dbw, (const uint16_t*)k, (const uint16_t*)za, a0, dzg,
                       k_k, k_a, (uint16_t*)dk, (uint16_t*)dza, ws);
    tmix::Outs o3{{dk_k, dk_a, da0, nullptr, nullptr, nullptr}};
    hipLaunchKernelGGL(tmix::reduce_blocks, dim3((3 * C + 255) / 256), dim3(256), 0, stream, ws, nb, 3, C, o3);
    return tm_status();
}

int theseus_tm_gn_fwd(int B, int T, int C, const void* y, const void* r, const void* k, const void* za,
                      const float* a0, const float* k_a, const void* v, const void* g, const float* r_k,
                      const float* ln_w, const float* ln_b, float eps, void* out, hipStream_t stream) {
    if (int e = tm_check(B, T, C)) return e;
    if (!y || !r || !k || !za || !a0 || !k_a || !v || !g || !r_k || !ln_w || !ln_b || !out)
        return THESEUS_WKV7_ERR_NULL;
    const int H = C / tmix::HN;
    const long M = (long)B * T;
    const int U = M >= 4096 ? tmix::U_LONG : 1;
    hipLaunchKernelGGL(U == 1 ? tmix::gn_fwd<1> : tmix::gn_fwd<tmix::U_LONG>,
                       dim3((unsigned)((M + 4 * U - 1) / (4 * U) * ((H + 7) / 8))), dim3(256), 0, stream, M, H, C,
                       (const uint16_t*)y, (const uint16_t*)r, (const uint16_t*)k, (const uint16_t*)za, a0, k_a,
                       (const uint16_t*)v, (const uint16_t*)g, r_k, ln_w, ln_b, eps, (uint16_t*)out);
    return tm_status();
}

size_t theseus_tm_gn_workspace(int B, int T, int C) {
    return tm_check(B, T, C) ? 0 : (size_t)nblk_t(B, T) * 4 * C * sizeof(float);
}

int theseus_tm_gn_bwd(int B, int T, int C, const void* dout, const void* y, const void* r, const void* k,
                      const void* za, const float* a0, const float* k_a, const void* v, const void* g,
                      const float* r_k, const float* ln_w, const float* ln_b, float eps, void* dy, void* dr,
                      void* dk, void* dv, void* dg, float* dzg, float* dr_k, float* dln_w, float* dln_b,
                      float* dk_a, float* ws, size_t ws_bytes, hipStream_t stream) {
    if (int e = tm_check(B, T, C)) return e;
    if (!dout || !y || !r || !k || !za || !a0 || !k_a || !v || !g || !r_k || !ln_w || !ln_b || !dy || !dr ||
        !dk || !dv || !dg || !dzg || !dr_k || !dln_w || !dln_b || !dk_a)
        return THESEUS_WKV7_ERR_NULL;
    if (!ws || ws_bytes < theseus_tm_gn_workspace(B, T, C)) return THESEUS_WKV7_ERR_WORKSPACE;
    const int H = C / tmix::HN, nb = (int)nblk_t(B, T);
    hipLaunchKernelGGL(tmix::gn_bwd, dim3((H + tmix::HG - 1) / tmix::HG, nb), dim3(256), 0, stream, (long)B * T, H, C, (const uint16_t*)dout,
                       (const uint16_t*)y, (const uint16_t*)r, (const uint16_t*)k, (const uint16_t*)za, a0, k_a,
                       (const uint16_t*)v, (const uint16_t*)g, r_k, ln_w, ln_b, eps, (uint16_t*)dy, (uint16_t*)dr,
                       (uint16_t*)dk, (uint16_t*)dv, (uint16_t*)dg, dzg, ws);
    tmix::Outs o4{{dr_k, dln_w, dln_b, dk_a, nullptr, nullptr}};
    hipLaunchKernelGGL(tmix::reduce_blocks, dim3((4 * C + 255) / 256), dim3(256), 0, stream, ws, nb, 4, C, o4);
    return tm_status();
}

}  // extern "C"
