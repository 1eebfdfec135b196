// Chunked WKV7 backward on the matrix cores (bf16 I/O, fp32 state, N = 64).
//
// The forward's chunk form (see wkv7_chunk_fwd.hip for A~, R~, B-, K-, B^,
// K^, Aab, Aak, Brb, Brk, Ti, P, Q', SA) is differentiated per chunk.  With
// H = dL/dS at the chunk end (H = dsT for the last chunk) and dY the chunk's
// output gradient:
//   Q   = Ti^T (B^ H^T + Brb^T dY)         (Q[t] = dL/d sa_t)
//   dV  = K^ H^T + Aak^T Q + Brk^T dY
//   dK  = e^{-g} o [ (V H) diag(e^{gL}) + triu_s(V Q^T) A~ + triu(V dY^T) R~ ]
//   dB  = e^{-g} o [ (SA H) diag(e^{gL}) + triu_s(SA Q^T) A~ + triu(SA dY^T) R~ ]
//   dR  = e^{g}  o [ dY S0 + tril(dY SA^T) B- + tril(dY V^T) K- ]
//   dA  = e^{gp} o [ Q S0 + tril_s(Q SA^T) B- + tril_s(Q V^T) K- ]
//   H_0 = H diag(e^{gL}) + Q^T A~ + dY^T R~      (dL/dS at the chunk start)
// and the decay gradient uses the identity (derived from S_t = S_{t-1} D_t +
// sa_t b_t^T + v_t k_t^T)
//   dlogd_t = sum_{s>=t} (r dR - b dB - k dK)_s + sum_{s>t} (a dA)_s
//             + colsum(dsT o S_T),      dw = dlogd * (-e^{-1/2}) sig(w)(1-sig(w)),
// a reverse cumulative sum carried across chunks.  Together these equal the
// step adjoint of kernels/wkv7_state.cu:52-78 (checked against it on the CPU
// oracle in float64).
//
// Mapping: one 256-lane workgroup per (b,h), chunks in reverse.  Each wave w
// owns value rows 16w..16w+15: it keeps H^T and the chunk's S0^T (from the
// saved states) for those rows in registers, and computes Q, SA and dV for
// them without any barrier.  The key-indexed gradients contract over all
// value rows, so Q, SA, H and S0 are then shared through LDS and each wave
// produces one 16-key strip of dK, dB, dR, dA, dw in a fixed summation order
// (deterministic; the reference accumulates with fp32 atomics, cu:68-72).
#include "wkv7_launch.h"
#include "wkv7_mfma.h"

namespace wkv7 {
namespace {

constexpr int CH = CKPT;
constexpr int NK = 64;
constexpr int LD64 = 72;
constexpr int LD16 = 24;
constexpr int LD32 = 40;

typedef uint16_t Plane16[2][CH * LD64];   // [16][64] hi/lo
typedef uint16_t Plane64[2][NK * LD16];   // [64][16] hi/lo
typedef uint16_t PlaneC[2][CH * LD16];    // [16][16] hi/lo
typedef uint16_t PlaneC2[2][CH * LD32];   // [16][32] hi/lo
typedef uint16_t PlaneS[2][NK * LD64];    // [64][64] hi/lo

struct BwdLds {
    uint16_t raw[7][CH * LD64];  // r,w,k,v,a,b,dy bf16 bits, [t][x]
    union {
        struct {                  // chunk-matrix stage only
            Plane16 At, Rt, Bb, Kb;
        } a;
        struct {                  // state / gradient stages
            Plane16 Qs, SAs;      // Q, SA [t][i]
            PlaneC2 KC, BC, RC, AC;  // masked combine matrices [t][s']
        } b;
    } u;
    Plane16 Kh, P, Pb;            // K^, P, Pb [t][j]
    Plane64 AtT, RtT, BbT, KbT, BhT;  // [j][t]
    uint16_t VT[NK * LD16], dYT[NK * LD16];  // [i][t], exact bf16
    PlaneS HT, S0T;               // H^T, S0^T as [j][i]
    PlaneC Ti, TiT, BrbT, AakT, BrkT, Q1;  // [t][s]
    float g[CH * NK];             // cumulative log-decay [t][j]
    float zs[CH * NK];            // dlogd terms, then dlogd [t][j]
    float t2s[CH * NK];           // (a dA) terms [t][j]
    float part[8][NK];
    float egL[NK];
};

__device__ __forceinline__ Op op(Plane16& a) { return Op{a[0], a[1], LD64}; }
__device__ __forceinline__ Op op(Plane64& a) { return Op{a[0], a[1], LD16}; }
__device__ __forceinline__ Op op(PlaneC& a) { return Op{a[0], a[1], LD16}; }
__device__ __forceinline__ Op op(PlaneC2& a) { return Op{a[0], a[1], LD32}; }
__device__ __forceinline__ Op op(PlaneS& a) { return Op{a[0], a[1], LD64}; }

// acc += A(16 x 64, [t][x] plane) * B^T where B is a [64-row][x] plane (outer =
// output column), K = 64 over x, split precision on both sides.
__device__ __forceinline__ f32x4_t mm64(const Op& A, const Op& B, int b_x0, int lane) {
    return mma_k32<2>(zero4(), A, 0, B, b_x0, 0, lane);
}
// Same with A exact in bf16 (one plane, e.g. raw V or dY).
__device__ __forceinline__ f32x4_t mm64x(const uint16_t* A, const Op& B, int b_x0, int lane) {
    f32x4_t acc = zero4(), c1 = zero4();
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint4 ah = frag32(A, LD64, 0, 32 * s, lane);
        acc = mma32(acc, ah, frag32(B.hi, B.ld, b_x0, 32 * s, lane));
        c1 = mma32(c1, ah, frag32(B.lo, B.ld, b_x0, 32 * s, lane));
    }
    return acc + c1;
}

}  // namespace

__global__ __launch_bounds__(256) void chunk_backward_bf16(
    int Tn, int H, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
    const bf16_t* __restrict__ b, const float* __restrict__ ckpt, const bf16_t* __restrict__ dy,
    const float* __restrict__ dsT, bf16_t* __restrict__ dr, bf16_t* __restrict__ dw,
    bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, bf16_t* __restrict__ da,
    bf16_t* __restrict__ db, float* __restrict__ ds0) {
    __shared__ BwdLds sm;
    const int bh = blockIdx.x, bb = bh / H, h = bh % H;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    const long ncp = ckpt_count(Tn);
    const int i_own = 16 * wv + r16;   // value row (state registers, stage B)
    const int j_own = 16 * wv + r16;   // key column (gradient strip, stage C)

    const Op At = op(sm.u.a.At), Rt = op(sm.u.a.Rt), Bb = op(sm.u.a.Bb), Kb = op(sm.u.a.Kb);
    const Op Qs = op(sm.u.b.Qs), SAs = op(sm.u.b.SAs);
    const Op KC = op(sm.u.b.KC), BC = op(sm.u.b.BC), RC = op(sm.u.b.RC), AC = op(sm.u.b.AC);
    const Op Kh = op(sm.Kh), P = op(sm.P), Pb = op(sm.Pb);
    const Op AtT = op(sm.AtT), RtT = op(sm.RtT), BbT = op(sm.BbT), KbT = op(sm.KbT), BhT = op(sm.BhT);
    const Op HT = op(sm.HT), S0T = op(sm.S0T);
    const Op Ti = op(sm.Ti), TiT = op(sm.TiT), BrbT = op(sm.BrbT), AakT = op(sm.AakT), BrkT = op(sm.BrkT),
             Q1 = op(sm.Q1);

    // H^T tiles: Ht[tj][e] = H[i_own][16*tj + 4q + e]
    f32x4_t Ht[4];
    float carry = 0.f;  // dlogd carry for key j_own (meaningful in lanes q == 0)
    {
        f32x4_t STt[4];
#pragma unroll
        for (int tj = 0; tj < 4; tj++) {
            const long off = (long)i_own * NK + 16 * tj + 4 * q;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (dsT) x = *reinterpret_cast<const float4*>(dsT + bh * NN + off);
            Ht[tj] = f32x4_t{x.x, x.y, x.z, x.w};
            const float4 s = *reinterpret_cast<const float4*>(ckpt + (bh * ncp + ncp - 1) * NN + off);
            STt[tj] = f32x4_t{s.x, s.y, s.z, s.w};
        }
        // carry_j = sum_i dsT[i][j] * S_T[i][j]: reduce over the 16 rows of the
        // lane group, then over the 4 waves in a fixed order
#pragma unroll
        for (int tj = 0; tj < 4; tj++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float p = Ht[tj][e] * STt[tj][e];
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) p += __shfl_xor(p, off, 16);
                if (r16 == 0) sm.part[wv][16 * tj + 4 * q + e] = p;
            }
        __syncthreads();
        carry = sm.part[0][j_own] + sm.part[1][j_own] + sm.part[2][j_own] + sm.part[3][j_own];
    }

    const int nchunk = (Tn + CH - 1) / CH;
    // Inputs of the next chunk to process (c-1) are prefetched into registers:
    // slot m of lane tid covers tensor id>>7, row (id>>3)&15, segment id&7.
    uint4 pre[4];
    float4 S0n[4];
    auto load_chunk = [&](int cc) {
        const int tb = cc * CH, Lc = min(CH, Tn - tb);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int id = tid + 256 * m, ts = id >> 7, row = (id >> 3) & 15, seg = id & 7;
            pre[m] = make_uint4(0, 0, 0, 0);
            if (id < 7 * 128 && row < Lc) {
                const bf16_t* src = ts == 0 ? r : ts == 1 ? w : ts == 2 ? k : ts == 3 ? v : ts == 4 ? a : ts == 5 ? b : dy;
                pre[m] = *reinterpret_cast<const uint4*>(src + ((long)(bb * Tn + tb + row) * H + h) * NK + 8 * seg);
            }
        }
#pragma unroll
        for (int tj = 0; tj < 4; tj++)
            S0n[tj] = *reinterpret_cast<const float4*>(ckpt + (bh * ncp + cc) * NN + (long)i_own * NK + 16 * tj + 4 * q);
    };
    auto store_raw = [&]() {
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int id = tid + 256 * m, ts = id >> 7, row = (id >> 3) & 15, seg = id & 7;
            if (id < 7 * 128) *reinterpret_cast<uint4*>(&sm.raw[ts][row * LD64 + 8 * seg]) = pre[m];
        }
    };
    f32x4_t S0t[4];
    load_chunk(nchunk - 1);
    store_raw();
#pragma unroll
    for (int tj = 0; tj < 4; tj++) S0t[tj] = f32x4_t{S0n[tj].x, S0n[tj].y, S0n[tj].z, S0n[tj].w};
    for (int c = nchunk - 1; c >= 0; c--) {
        const int t0 = c * CH, L = min(CH, Tn - t0);
        // ---- A1: start loading chunk c-1; raw of chunk c is already in LDS ----
        if (c > 0) load_chunk(c - 1);
        __syncthreads();  // raw ready; the later chunk's stage C is done with LDS
        // ---- A2: decay cumsum and scaled operands; lane = key pair jp, token pair tp ----
        {
            const int jp = tid & 31, tp = tid >> 5, j0 = 2 * jp, tb = 2 * tp;
            float lw[2][2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t wb = *reinterpret_cast<const uint32_t*>(&sm.raw[1][(tb + u) * LD64 + j0]);
#pragma unroll
                for (int x = 0; x < 2; x++)
                    lw[u][x] = tb + u < L ? log_decay(bf16_to_f32((uint16_t)(wb >> (16 * x)))) : 0.f;
            }
#pragma unroll
            for (int x = 0; x < 2; x++) sm.part[tp][j0 + x] = lw[0][x] + lw[1][x];
            __syncthreads();
            float pre_[2] = {0.f, 0.f}, tot[2] = {0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int x = 0; x < 2; x++) {
                    const float p = sm.part[u][j0 + x];
                    tot[x] += p;
                    if (u < tp) pre_[x] += p;
                }
            float vat[2][2], vrt[2][2], vbb[2][2], vkb[2][2], vbh[2][2], vkh[2][2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int t = tb + u;
                const uint32_t rb = *reinterpret_cast<const uint32_t*>(&sm.raw[0][t * LD64 + j0]);
                const uint32_t kb = *reinterpret_cast<const uint32_t*>(&sm.raw[2][t * LD64 + j0]);
                const uint32_t ab = *reinterpret_cast<const uint32_t*>(&sm.raw[4][t * LD64 + j0]);
                const uint32_t bb2 = *reinterpret_cast<const uint32_t*>(&sm.raw[5][t * LD64 + j0]);
                float gv[2];
#pragma unroll
                for (int x = 0; x < 2; x++) {
                    const float g = pre_[x] + lw[0][x] + (u ? lw[1][x] : 0.f), gp = g - lw[u][x];
                    gv[x] = g;
                    const float eg = __expf(g), eng = __expf(-g), egp = __expf(gp), eL = __expf(tot[x] - g);
                    const float rr = bf16_to_f32((uint16_t)(rb >> (16 * x)));
                    const float kk = bf16_to_f32((uint16_t)(kb >> (16 * x)));
                    const float aa = bf16_to_f32((uint16_t)(ab >> (16 * x)));
                    const float bv = bf16_to_f32((uint16_t)(bb2 >> (16 * x)));
                    vat[u][x] = aa * egp;
                    vrt[u][x] = rr * eg;
                    vbb[u][x] = bv * eng;
                    vkb[u][x] = kk * eng;
                    vbh[u][x] = bv * eL;
                    vkh[u][x] = kk * eL;
                }
                *reinterpret_cast<float2*>(&sm.g[t * NK + j0]) = make_float2(gv[0], gv[1]);
            }
            auto put_row = [&](const Op& o, const float (&vv)[2][2]) {  // [t][j] pairs along j
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    uint32_t hh, ll;
                    split2(vv[u][0], vv[u][1], hh, ll);
                    *reinterpret_cast<uint32_t*>(&o.hi[(tb + u) * o.ld + j0]) = hh;
                    *reinterpret_cast<uint32_t*>(&o.lo[(tb + u) * o.ld + j0]) = ll;
                }
            };
            auto put_col = [&](const Op& o, const float (&vv)[2][2]) {  // [j][t] pairs along t
#pragma unroll
                for (int x = 0; x < 2; x++) {
                    uint32_t hh, ll;
                    split2(vv[0][x], vv[1][x], hh, ll);
                    *reinterpret_cast<uint32_t*>(&o.hi[(j0 + x) * o.ld + tb]) = hh;
                    *reinterpret_cast<uint32_t*>(&o.lo[(j0 + x) * o.ld + tb]) = ll;
                }
            };
            put_row(At, vat);
            put_col(AtT, vat);
            put_row(Rt, vrt);
            put_col(RtT, vrt);
            put_row(Bb, vbb);
            put_col(BbT, vbb);
            put_row(Kb, vkb);
            put_col(KbT, vkb);
            put_col(BhT, vbh);
            put_row(Kh, vkh);
            auto put_raw_col = [&](int ts, uint16_t* dst) {  // exact bf16 plane, transposed
                const uint32_t v0 = *reinterpret_cast<const uint32_t*>(&sm.raw[ts][tb * LD64 + j0]);
                const uint32_t v1 = *reinterpret_cast<const uint32_t*>(&sm.raw[ts][(tb + 1) * LD64 + j0]);
                *reinterpret_cast<uint32_t*>(&dst[j0 * LD16 + tb]) = (v0 & 0xffffu) | (v1 << 16);
                *reinterpret_cast<uint32_t*>(&dst[(j0 + 1) * LD16 + tb]) = (v0 >> 16) | (v1 & 0xffff0000u);
            };
            put_raw_col(3, sm.VT);
            put_raw_col(6, sm.dYT);
            if (tp == 0) {
                sm.egL[j0] = __expf(tot[0]);
                sm.egL[j0 + 1] = __expf(tot[1]);
            }
        }
        __syncthreads();
        // ---- A3: chunk matrices; wave 0: Aab, Aab^T -> Ti, Ti^T; waves 1-3: Aak, Brb, Brk ----
        f32x4_t cm = zero4();
        if (wv == 0) {
            f32x4_t Lm = mm64(At, Bb, 0, lane);
            f32x4_t LT = mm64(Bb, At, 0, lane);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (r16 >= 4 * q + e) Lm[e] = 0.f;
                if (r16 <= 4 * q + e) LT[e] = 0.f;
            }
            f32x4_t ti, tiT;
            tri_inverse(Lm, LT, lane, ti, tiT);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                Ti.put(4 * q + e, r16, ti[e]);
                TiT.put(4 * q + e, r16, tiT[e]);
            }
        } else {
            if (wv == 1) cm = mm64(At, Kb, 0, lane);        // Aak
            else if (wv == 2) cm = mm64(Rt, Bb, 0, lane);   // Brb
            else cm = mm64(Rt, Kb, 0, lane);                // Brk
#pragma unroll
            for (int e = 0; e < 4; e++) {  // D layout: row t = 4q+e, column s = r16
                const int t = 4 * q + e, s = r16;
                if (wv == 1 ? s >= t : s > t) cm[e] = 0.f;
                if (wv == 1) AakT.put(s, t, cm[e]);
                if (wv == 2) BrbT.put(s, t, cm[e]);
                if (wv == 3) BrkT.put(s, t, cm[e]);
            }
        }
        __syncthreads();
        // ---- A5: P = Ti A~, Pb = Ti^T B^ on key strip 16wv..; wave 1: Q' = Ti Aak ----
        {
            const int j = 16 * wv + r16;
            const f32x4_t p = mma_k16(zero4(), Ti, 0, AtT, 16 * wv, 0, lane);
            const f32x4_t pb = mma_k16(zero4(), TiT, 0, BhT, 16 * wv, 0, lane);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                P.put(4 * q + e, j, p[e]);
                Pb.put(4 * q + e, j, pb[e]);
            }
            if (wv == 1) {  // cm = Aak in D layout: rows s = 4q+e (the K index), column s' = r16
                uint2 ah, al;
                pack4(cm, ah, al);
                const uint2 th = frag16(Ti.hi, LD16, 0, 0, lane), tl = frag16(Ti.lo, LD16, 0, 0, lane);
                f32x4_t q1 = mma16(zero4(), th, ah);
                f32x4_t c1 = mma16(zero4(), th, al);
                c1 = mma16(c1, tl, ah);
                q1 += c1;
#pragma unroll
                for (int e = 0; e < 4; e++) Q1.put(4 * q + e, r16, q1[e]);
            }
        }
        __syncthreads();
        // ---- B: wave-local rows i_own: SA, Q, dV, and H update ----
        f32x4_t Hn[4];
        f32x4_t dvk;              // dV[t = 4q+e][i_own], stored at the end of the chunk
        float gk_[4], gb_[4], gr_[4], ga_[4], gw_[4];  // key-strip gradients, stored at the end
        {
            const uint2 vfr = ld8B(&sm.VT[i_own * LD16 + 4 * q]);   // V[t=4q..][i_own]
            const uint2 dyf = ld8B(&sm.dYT[i_own * LD16 + 4 * q]);  // dY[t=4q..][i_own]
            // X = Brb^T dY ; Qc = Ti^T X
            f32x4_t X = mma16(zero4(), frag16(BrbT.hi, LD16, 0, 0, lane), dyf);
            X = mma16(X, frag16(BrbT.lo, LD16, 0, 0, lane), dyf);
            uint2 xh, xl;
            pack4(X, xh, xl);
            const uint2 tth = frag16(TiT.hi, LD16, 0, 0, lane), ttl = frag16(TiT.lo, LD16, 0, 0, lane);
            f32x4_t Qc = mma16(zero4(), tth, xh);
            f32x4_t c0 = mma16(zero4(), tth, xl);
            c0 = mma16(c0, ttl, xh);
            Qc += c0;
            // SA = P S0^T + Q' V ; Q = Pb H^T + Qc ; dV (K^ H^T part)
            f32x4_t sa = zero4(), qq = zero4(), dvv = zero4();
#pragma unroll
            for (int s = 0; s < 2; s++) {
                float sv[8], hv[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sv[e] = S0t[2 * s][e];
                    sv[4 + e] = S0t[2 * s + 1][e];
                    hv[e] = Ht[2 * s][e];
                    hv[4 + e] = Ht[2 * s + 1][e];
                }
                uint4 sh, sl, hh, hl;
                pack8(sv, sh, sl);
                pack8(hv, hh, hl);
                const int k0 = 32 * s;
                const uint4 pah = fragp(P.hi, LD64, r16, k0, lane), pal = fragp(P.lo, LD64, r16, k0, lane);
                const uint4 bah = fragp(Pb.hi, LD64, r16, k0, lane), bal = fragp(Pb.lo, LD64, r16, k0, lane);
                const uint4 kah = fragp(Kh.hi, LD64, r16, k0, lane), kal = fragp(Kh.lo, LD64, r16, k0, lane);
                sa = mma32(sa, pah, sh);
                sa = mma32(sa, pah, sl);
                sa = mma32(sa, pal, sh);
                qq = mma32(qq, bah, hh);
                qq = mma32(qq, bah, hl);
                qq = mma32(qq, bal, hh);
                dvv = mma32(dvv, kah, hh);
                dvv = mma32(dvv, kah, hl);
                dvv = mma32(dvv, kal, hh);
            }
            {
                f32x4_t sv2 = mma16(zero4(), frag16(Q1.hi, LD16, 0, 0, lane), vfr);
                sv2 = mma16(sv2, frag16(Q1.lo, LD16, 0, 0, lane), vfr);
                sa += sv2;
            }
            qq += Qc;
            // dV += Aak^T Q + Brk^T dY
            uint2 qh, ql;
            pack4(qq, qh, ql);
            {
                const uint2 aah = frag16(AakT.hi, LD16, 0, 0, lane), aal = frag16(AakT.lo, LD16, 0, 0, lane);
                f32x4_t d2 = mma16(zero4(), aah, qh);
                f32x4_t d3 = mma16(zero4(), aah, ql);
                d3 = mma16(d3, aal, qh);
                d2 = mma16(d2, frag16(BrkT.hi, LD16, 0, 0, lane), dyf);
                d2 = mma16(d2, frag16(BrkT.lo, LD16, 0, 0, lane), dyf);
                dvv += d2 + d3;
            }
            dvk = dvv;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 4 * q + e;
                Qs.put(t, i_own, qq[e]);
                SAs.put(t, i_own, sa[e]);
            }
#pragma unroll
            for (int tj = 0; tj < 4; tj++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    HT.put(16 * tj + 4 * q + e, i_own, Ht[tj][e]);
                    S0T.put(16 * tj + 4 * q + e, i_own, S0t[tj][e]);
                }
            // H_new^T = H^T diag(e^{gL}) + [A~^T R~^T] [Q; dY]
            const uint4 bhi = cat(qh, dyf), blo = cat(ql, make_uint2(0, 0));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const int jr = 16 * tj + r16;
                const uint4 ah = cat(ld8B(&AtT.hi[jr * LD16 + 4 * q]), ld8B(&RtT.hi[jr * LD16 + 4 * q]));
                const uint4 al = cat(ld8B(&AtT.lo[jr * LD16 + 4 * q]), ld8B(&RtT.lo[jr * LD16 + 4 * q]));
                f32x4_t acc;
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = Ht[tj][e] * sm.egL[16 * tj + 4 * q + e];
                acc = mma32(acc, ah, bhi);
                f32x4_t c1 = mma32(zero4(), ah, blo);
                c1 = mma32(c1, al, bhi);
                Hn[tj] = acc + c1;
            }
        }
        __syncthreads();
        // ---- C1: the 16x16 contractions over i (one per wave) and masked combine forms ----
        {
            const uint16_t* Vr = sm.raw[3];
            const uint16_t* dYr = sm.raw[6];
            f32x4_t m;
            if (wv == 0) m = mm64x(Vr, Qs, 0, lane);            // M1 = V Q^T
            else if (wv == 1) {                                 // M2 = V dY^T (exact x exact)
                m = zero4();
#pragma unroll
                for (int s = 0; s < 2; s++)
                    m = mma32(m, frag32(Vr, LD64, 0, 32 * s, lane), frag32(dYr, LD64, 0, 32 * s, lane));
            } else if (wv == 2) m = mm64(SAs, Qs, 0, lane);     // N1 = SA Q^T
            else m = mm64x(dYr, SAs, 0, lane);                  // N2^T = dY SA^T
            // element (t = 4q+e, s = r16)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 4 * q + e, s = r16;
                const float x = m[e];
                if (wv == 0) {  // M1: dK uses triu_s(M1); dA uses tril_s(M1^T)
                    KC.put(t, s, s > t ? x : 0.f);
                    AC.put(s, 16 + t, t < s ? x : 0.f);
                } else if (wv == 1) {  // M2: dK uses triu(M2); dR uses tril(M2^T)
                    KC.put(t, 16 + s, s >= t ? x : 0.f);
                    RC.put(s, 16 + t, t <= s ? x : 0.f);
                } else if (wv == 2) {  // N1: dB uses triu_s(N1); dA uses tril_s(N1^T)
                    BC.put(t, s, s > t ? x : 0.f);
                    AC.put(s, t, t < s ? x : 0.f);
                } else {  // x = (dY SA^T)[t][s] = N2[s][t]: dR uses tril(dY SA^T); dB uses triu(N2)
                    RC.put(t, s, s <= t ? x : 0.f);
                    BC.put(s, 16 + t, t >= s ? x : 0.f);
                }
            }
        }
        __syncthreads();
        // ---- C2: key strip j_own: dK, dB, dR, dA and the decay gradient ----
        {
            const uint16_t* Vr = sm.raw[3];
            const uint16_t* dYr = sm.raw[6];
            const int x0 = 16 * wv;
            // [A~; R~] and [B-; K-] as B operands with K = 32 (rows s' of the combine matrices)
            uint4 arh, arl, bkh, bkl;
            {
                const int jr = x0 + r16;
                const bool fst = q < 2;
                const int kk0 = 8 * (q & 1);
                arh = *reinterpret_cast<const uint4*>((fst ? AtT.hi : RtT.hi) + jr * LD16 + kk0);
                arl = *reinterpret_cast<const uint4*>((fst ? AtT.lo : RtT.lo) + jr * LD16 + kk0);
                bkh = *reinterpret_cast<const uint4*>((fst ? BbT.hi : KbT.hi) + jr * LD16 + kk0);
                bkl = *reinterpret_cast<const uint4*>((fst ? BbT.lo : KbT.lo) + jr * LD16 + kk0);
            }
            auto combine = [&](const Op& M, const uint4& bh_, const uint4& bl_) {
                const uint4 mh = frag32(M.hi, LD32, 0, 0, lane), ml = frag32(M.lo, LD32, 0, 0, lane);
                f32x4_t acc = mma32(zero4(), mh, bh_);
                f32x4_t c1 = mma32(zero4(), mh, bl_);
                c1 = mma32(c1, ml, bh_);
                return acc + c1;
            };
            f32x4_t gK = mm64x(Vr, HT, x0, lane);      // (V H)[t][j]
            f32x4_t gB = mm64(SAs, HT, x0, lane);      // (SA H)[t][j]
            f32x4_t gR = mm64x(dYr, S0T, x0, lane);    // (dY S0)[t][j]
            f32x4_t gA = mm64(Qs, S0T, x0, lane);      // (Q S0)[t][j]
            const f32x4_t cK = combine(KC, arh, arl);
            const f32x4_t cB = combine(BC, arh, arl);
            const f32x4_t cR = combine(RC, bkh, bkl);
            const f32x4_t cA = combine(AC, bkh, bkl);
            const float eL = sm.egL[j_own];
            float z[4], t2v[4], sg[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 4 * q + e;
                const float g = sm.g[t * NK + j_own];
                const float gp = t > 0 ? sm.g[(t - 1) * NK + j_own] : 0.f;
                const float vK = __expf(-g) * (gK[e] * eL + cK[e]);
                const float vB = __expf(-g) * (gB[e] * eL + cB[e]);
                const float vR = __expf(g) * (gR[e] + cR[e]);
                const float vA = __expf(gp) * (gA[e] + cA[e]);
                const float rr = bf16_to_f32(sm.raw[0][t * LD64 + j_own]);
                const float kk = bf16_to_f32(sm.raw[2][t * LD64 + j_own]);
                const float aa = bf16_to_f32(sm.raw[4][t * LD64 + j_own]);
                const float bv = bf16_to_f32(sm.raw[5][t * LD64 + j_own]);
                const float wv_ = bf16_to_f32(sm.raw[1][t * LD64 + j_own]);
                sg[e] = sigmoidf_(wv_);
                z[e] = rr * vR - bv * vB - kk * vK;
                t2v[e] = aa * vA;
                gk_[e] = vK;
                gb_[e] = vB;
                gr_[e] = vR;
                ga_[e] = vA;
                sm.zs[t * NK + j_own] = z[e];
                sm.t2s[t * NK + j_own] = t2v[e];
            }
            __syncthreads();
            // dlogd_t = carry + sum_{s>=t} z_s + sum_{s>t} (a dA)_s  (16 lanes, one key each)
            if (q == 0) {
                float run = carry;
#pragma unroll
                for (int t = CH - 1; t >= 0; t--) {
                    run += sm.zs[t * NK + j_own] + (t + 1 < CH ? sm.t2s[(t + 1) * NK + j_own] : 0.f);
                    sm.zs[t * NK + j_own] = run;
                }
                carry = run + sm.t2s[j_own];
            }
            __syncthreads();
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 4 * q + e;
                gw_[e] = sm.zs[t * NK + j_own] * (-DECAY_SCALE) * sg[e] * (1.f - sg[e]);
            }
        }
#pragma unroll
        for (int tj = 0; tj < 4; tj++) Ht[tj] = Hn[tj];
        // ---- D: next chunk's inputs into LDS, then this chunk's gradient stores ----
        // (the prefetch wait comes before the stores are issued, so it never waits on them)
        if (c > 0) {
            __syncthreads();  // every wave is done reading raw
            store_raw();
#pragma unroll
            for (int tj = 0; tj < 4; tj++) S0t[tj] = f32x4_t{S0n[tj].x, S0n[tj].y, S0n[tj].z, S0n[tj].w};
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 4 * q + e;
            if (t < L) {
                dv[((long)(bb * Tn + t0 + t) * H + h) * NK + i_own].bits = f32_to_bf16(dvk[e]);
                const long o = ((long)(bb * Tn + t0 + t) * H + h) * NK + j_own;
                dk[o].bits = f32_to_bf16(gk_[e]);
                db[o].bits = f32_to_bf16(gb_[e]);
                dr[o].bits = f32_to_bf16(gr_[e]);
                da[o].bits = f32_to_bf16(ga_[e]);
                dw[o].bits = f32_to_bf16(gw_[e]);
            }
        }
    }
#pragma unroll
    for (int tj = 0; tj < 4; tj++)
        *reinterpret_cast<float4*>(ds0 + bh * NN + (long)i_own * NK + 16 * tj + 4 * q) =
            make_float4(Ht[tj][0], Ht[tj][1], Ht[tj][2], Ht[tj][3]);
}

void launch_chunk_backward(const Bwd& p) {
    hipLaunchKernelGGL(chunk_backward_bf16, dim3(p.B * p.H), dim3(256), 0, p.stream, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.ckpt, (const bf16_t*)p.dy, p.dsT,
                       (bf16_t*)p.dr, (bf16_t*)p.dw, (bf16_t*)p.dk, (bf16_t*)p.dv, (bf16_t*)p.da,
                       (bf16_t*)p.db, p.ds0);
}

}  // namespace wkv7
