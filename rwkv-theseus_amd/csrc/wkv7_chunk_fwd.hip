// Chunked WKV7 forward on the matrix cores (bf16 I/O, fp32 state, N = 64).
//
// Algebra (per batch*head, chunk of C = 16 steps, local t = 0..C-1; i = value
// row, j = key column; g_t = cumulative log-decay inside the chunk, gp_t =
// g_{t-1}, gL = g_{C-1}):
//   A~ = a*e^{gp},  R~ = r*e^{g},  B- = b*e^{-g},  K- = k*e^{-g},
//   B^ = b*e^{gL-g} = e^{gL} B-,  K^ = e^{gL} K-
//   Aab = tril_strict(A~ B-^T)  Aak = tril_strict(A~ K-^T)
//   Brb = tril(R~ B-^T)          Brk = tril(R~ K-^T)
//   Ti  = (I - Aab)^{-1};  P = Ti A~;  Q' = Ti Aak;  P2 = R~ + Brb P;  Q2 = Brk + Brb Q'
//   SA  = P S0^T + Q' V          (SA[t] = S_{t-1} a_t, the "sa" of the recurrence)
//   Y   = P2 S0^T + Q2 V
//   S_C = S0 diag(e^{gL}) + SA^T B^ + V^T K^
// which is the step recurrence of theseus/wkv7.py:16-28 rewritten in the
// WY / diagonal-plus-low-rank chunk form (exact in exact arithmetic).
//
// Mapping: one 512-lane workgroup per (b,h), two roles, lock-step "ticks"
// that each end in one LDS barrier (no global-memory fence, so prefetches stay
// in flight across it).
//  * Producers (waves 0-3).  Everything above that does not involve the
//    state depends only on the chunk's inputs, so producer p builds the
//    operands of chunks p, p+4, p+8, ... alone -- no barrier inside -- in four
//    phases spread over the four ticks before the chunk is consumed; at any
//    tick the four producers are in four different phases.  A lane holds one
//    token and 16 keys (X[t = l%16][32 hf + 8q + e], the K=32 operand layout),
//    so the decay cumsum over tokens is a 16-lane DPP scan, the key
//    contractions (Aab, ...) take the operands straight from registers, and the products over tokens
//    read their transposed operand back with ds_read_b64_tr_b16.
//  * Consumers (waves 4-7).  Wave 4+c keeps value rows 16c..16c+15 of the
//    state in registers (value rows never interact) and advances them by one
//    chunk per tick from the operands the producers left in a 4-slot LDS ring.
#include "wkv7_launch.h"
#include "wkv7_mfma.h"

namespace wkv7 {
namespace {

constexpr int CH = CKPT;  // chunk length
constexpr int NK = 64;    // head size of this kernel
constexpr int LDA = 72;   // row stride of [16][64] planes (elements)
constexpr int LDC = 24;   // row stride of [16][16] planes

// One chunk's operands, as the consumers read them.
struct Slot {
    uint16_t P[2][CH * LDA];    // P [t][j] (hi, lo); A~ [t][j] until the producer replaces it
    uint16_t P2[2][CH * LDA];   // P2 [t][j]; R~ [t][j] until the producer replaces it
    uint16_t Bh[2][CH * LDA];   // B^ [t][j]
    uint16_t Kh[2][CH * LDA];   // K^ [t][j]
    uint16_t Q1T[2][CH * LDC];  // Q'^T [s][t]
    uint16_t Q2[2][CH * LDC];   // Q2 [t][s]
    uint16_t V[CH * LDA];       // V [t][i], exact bf16
    float egL[NK];              // e^{gL} per key
};
struct FwdLds {
    Slot slot[4];
};

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void st8(uint16_t* p, uint2 v) { *reinterpret_cast<uint2*>(p) = v; }
__device__ __forceinline__ float lo_bf(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_bf(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
// element e of 4 / 8 packed bf16
__device__ __forceinline__ float bf_el(uint2 u, int e) {
    const uint32_t w = e < 2 ? u.x : u.y;
    return (e & 1) ? hi_bf(w) : lo_bf(w);
}
__device__ __forceinline__ float bf_el8(uint4 u, int e) {
    const uint32_t w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
    return (e & 1) ? hi_bf(w) : lo_bf(w);
}
__device__ __forceinline__ void st16(uint16_t* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
// X Y^T over the 64 keys for operands in the standard K=32 layout
// (x[hf] = X[t = l%16][32 hf + 8q .. +7], split into hi / lo)
__device__ __forceinline__ f32x4_t mm_keys8(const uint4 (&xh)[2], const uint4 (&xl)[2], const uint4 (&yh)[2],
                                            const uint4 (&yl)[2]) {
    f32x4_t acc = zero4(), c1 = zero4(), c2 = zero4();
#pragma unroll
    for (int s = 0; s < 2; s++) {
        acc = mma32(acc, xh[s], yh[s]);
        c1 = mma32(c1, xh[s], yl[s]);
        c2 = mma32(c2, xl[s], yh[s]);
    }
    return acc + c1 + c2;
}

}  // namespace

__global__ __launch_bounds__(512) void chunk_forward_bf16(
    int Tn, int H, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
    const bf16_t* __restrict__ b, const float* __restrict__ s0, bf16_t* __restrict__ y,
    float* __restrict__ sT, float* __restrict__ ckpt) {
    __shared__ FwdLds sm;
    const int bh = blockIdx.x, bb = bh / H, h = bh % H;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    const long ncp = ckpt_count(Tn);
    const int nchunk = (Tn + CH - 1) / CH;
    const bool producer = wv < 4;

    // ---------------- producer state (lane: token r16, keys 32 hf + 8q + e) ----------------
    uint4 pre[6][2];             // prefetched inputs r, w, k, v, a, b
    float eg[2][8], eng[2][8];   // e^{g}, e^{-g} (phase 0 -> 1)
    f32x4_t Aab, AabT, Aak, BrbT, BrkT;  // phase 1 -> 2, 3
    f32x4_t Ti, TiT;             // phase 2 -> 3
    auto load_chunk = [&](int cc) {
        const int Lc = min(CH, Tn - cc * CH);
        const long row = ((long)(bb * Tn + cc * CH + r16) * H + h) * NK + 8 * q;
        const bf16_t* src[6] = {r, w, k, v, a, b};
        if (Lc == CH) {  // wave-uniform: full chunks load without predication
#pragma unroll
            for (int ts = 0; ts < 6; ts++)
#pragma unroll
                for (int hf = 0; hf < 2; hf++) pre[ts][hf] = *reinterpret_cast<const uint4*>(src[ts] + row + 32 * hf);
        } else {
#pragma unroll
            for (int ts = 0; ts < 6; ts++)
#pragma unroll
                for (int hf = 0; hf < 2; hf++)
                    pre[ts][hf] = r16 < Lc ? *reinterpret_cast<const uint4*>(src[ts] + row + 32 * hf) : make_uint4(0, 0, 0, 0);
        }
    };

    // ---------------- consumer state: S^T tiles St[tj][e] = S[i_own][16tj + 4q + e] ----------------
    const int cw = wv - 4, i_own = 16 * cw + r16;
    f32x4_t St[4];
    if (producer) {
        if (wv < nchunk) load_chunk(wv);
    } else {
#pragma unroll
        for (int tj = 0; tj < 4; tj++) {
            const long off = bh * NN + (long)i_own * NK + 16 * tj + 4 * q;
            const float4 x = *reinterpret_cast<const float4*>(s0 + off);
            St[tj] = f32x4_t{x.x, x.y, x.z, x.w};
            if (ckpt) *reinterpret_cast<float4*>(ckpt + bh * ncp * NN + (long)i_own * NK + 16 * tj + 4 * q) = x;
        }
        // nothing else is loaded by consumers: drain here so the tick loop never
        // waits on the (in-order) memory counter, which also counts its stores
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    }

    for (int n = -4; n < nchunk; n++) {
        if (producer) {
            // the chunk this producer works on at tick n, and its phase; chunk x
            // owns slot x & 3 from tick x-3 (its last reader was chunk x-4)
            const int x = n + 1 + ((wv - n - 1) & 3);
            const int ph = n + 4 - x;
            Slot& S = sm.slot[x & 3];
            const int o = r16 * LDA + 4 * q;  // [t][j] position of a 4-key D-layout piece (plus 16 tj)
            const int o8 = r16 * LDA + 8 * q; // [t][j] position of this lane's 8-key run (plus 32 hf)
            if (x >= 0 && x < nchunk) {  // (prologue ticks have no chunk for some producers)
                if (ph == 0) {
                    // ---- phase 0: log-decays, their cumulative sum, e^{+-g} ----
                    const int L = min(CH, Tn - x * CH);
#pragma unroll
                    for (int hf = 0; hf < 2; hf++)
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            float ld = log_decay(bf_el8(pre[1][hf], e));
                            if (L < CH) ld = r16 < L ? ld : 0.f;  // padded steps keep the state
                            const float gv = row_prefix_sum(ld);
                            eg[hf][e] = __expf(gv);
                            eng[hf][e] = __expf(-gv);
                        }
                } else if (ph == 1) {
                    // ---- phase 1: scaled operands, the chunk matrices over the keys (from
                    //      registers), and the slot planes P <- A~, P2 <- R~, Bh, Kh, V,
                    //      e^{gL}; then prefetch this producer's next chunk ----
                    uint4 ath[2], atl[2], rth[2], rtl[2], bbh[2], bbl[2], kbh[2], kbl[2];
#pragma unroll
                    for (int hf = 0; hf < 2; hf++) {
                        float el[8];
#pragma unroll
                        for (int e = 0; e < 8; e++) el[e] = row_last(eg[hf][e]);
                        float at[8], rt[8], bbv[8], kbv[8], bhv[8], khv[8];
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            at[e] = bf_el8(pre[4][hf], e) * row_prev(eg[hf][e], 1.f);
                            rt[e] = bf_el8(pre[0][hf], e) * eg[hf][e];
                            bbv[e] = bf_el8(pre[5][hf], e) * eng[hf][e];
                            kbv[e] = bf_el8(pre[2][hf], e) * eng[hf][e];
                            bhv[e] = bbv[e] * el[e];
                            khv[e] = kbv[e] * el[e];
                        }
                        pack8(at, ath[hf], atl[hf]);
                        pack8(rt, rth[hf], rtl[hf]);
                        pack8(bbv, bbh[hf], bbl[hf]);
                        pack8(kbv, kbh[hf], kbl[hf]);
                        uint4 hh, ll;
                        pack8(bhv, hh, ll);
                        st16(&S.Bh[0][o8 + 32 * hf], hh);
                        st16(&S.Bh[1][o8 + 32 * hf], ll);
                        pack8(khv, hh, ll);
                        st16(&S.Kh[0][o8 + 32 * hf], hh);
                        st16(&S.Kh[1][o8 + 32 * hf], ll);
                        st16(&S.P[0][o8 + 32 * hf], ath[hf]);
                        st16(&S.P[1][o8 + 32 * hf], atl[hf]);
                        st16(&S.P2[0][o8 + 32 * hf], rth[hf]);
                        st16(&S.P2[1][o8 + 32 * hf], rtl[hf]);
                        st16(&S.V[o8 + 32 * hf], pre[3][hf]);
                        if (r16 == 0) {
                            *reinterpret_cast<float4*>(&S.egL[32 * hf + 8 * q]) = make_float4(el[0], el[1], el[2], el[3]);
                            *reinterpret_cast<float4*>(&S.egL[32 * hf + 8 * q + 4]) = make_float4(el[4], el[5], el[6], el[7]);
                        }
                    }
                    if (x + 4 < nchunk) load_chunk(x + 4);
                    Aab = mm_keys8(ath, atl, bbh, bbl);
                    AabT = mm_keys8(bbh, bbl, ath, atl);
                    Aak = mm_keys8(ath, atl, kbh, kbl);
                    BrbT = mm_keys8(bbh, bbl, rth, rtl);
                    BrkT = mm_keys8(kbh, kbl, rth, rtl);
                } else if (ph == 2) {
                    // ---- phase 2: triangular inverse, Q' = Ti Aak, P^T = A~^T Ti^T ----
#pragma unroll
                    for (int e = 0; e < 4; e++) {  // D layout: row 4q+e, column r16
                        const int rw = 4 * q + e;
                        if (r16 >= rw) Aab[e] = 0.f, Aak[e] = 0.f;   // [t][s]: s < t
                        if (rw >= r16) AabT[e] = 0.f;                // [s][t]: s < t
                        if (rw > r16) BrbT[e] = 0.f, BrkT[e] = 0.f;  // [s][t]: s <= t
                    }
                    tri_inverse(Aab, AabT, lane, Ti, TiT);
                    const Pk pTiT = pk(TiT);
                    // Q' (D layout [t][s]) stored as Q'^T [s][t]
                    const Pk pq1 = pk(mm16s(pTiT, pk(Aak)));
                    st8(&S.Q1T[0][r16 * LDC + 4 * q], pq1.h);
                    st8(&S.Q1T[1][r16 * LDC + 4 * q], pq1.l);
                    // P^T per 16-key tile; tile tj of A~ (read transposed) is replaced by tile tj of P
#pragma unroll
                    for (int tj = 0; tj < 4; tj++) {
                        const Pk pa = {ldtr(&S.P[0][16 * tj], LDA, lane), ldtr(&S.P[1][16 * tj], LDA, lane)};
                        const Pk pp = pk(mm16s(pa, pTiT));  // lane: P[t = r16][16tj + 4q + e]
                        st8(&S.P[0][o + 16 * tj], pp.h);
                        st8(&S.P[1][o + 16 * tj], pp.l);
                    }
                    // Q2^T = Brk^T + Q'^T Brb^T  (lane: Q2[t = r16][s = 4q + e])
                    const Pk q2 = pk(BrkT + mm16s(pq1, pk(BrbT)));
                    st8(&S.Q2[0][r16 * LDC + 4 * q], q2.h);
                    st8(&S.Q2[1][r16 * LDC + 4 * q], q2.l);
                } else {
                    // ---- phase 3: P2^T = R~^T + P^T Brb^T (R~ read from the P2 plane first) ----
                    const Pk pB = pk(BrbT);
#pragma unroll
                    for (int tj = 0; tj < 4; tj++) {
                        const uint2 hh = ld8B(&S.P2[0][o + 16 * tj]), ll = ld8B(&S.P2[1][o + 16 * tj]);
                        f32x4_t rt;
#pragma unroll
                        for (int e = 0; e < 4; e++) rt[e] = bf_el(hh, e) + bf_el(ll, e);
                        const Pk pp = {ldtr(&S.P[0][16 * tj], LDA, lane), ldtr(&S.P[1][16 * tj], LDA, lane)};
                        const Pk p2 = pk(rt + mm16s(pp, pB));
                        st8(&S.P2[0][o + 16 * tj], p2.h);
                        st8(&S.P2[1][o + 16 * tj], p2.l);
                    }
                }
            }
        } else if (n >= 0) {
            // ---------------- consumer: rows i_own through chunk n ----------------
            const Slot& S = sm.slot[n & 3];
            const int t0 = n * CH, L = min(CH, Tn - t0);
            f32x4_t sa = zero4(), yy = zero4();
#pragma unroll
            for (int s = 0; s < 2; s++) {  // K = 64 over keys in two permuted K=32 steps
                float sv[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sv[e] = St[2 * s][e];
                    sv[4 + e] = St[2 * s + 1][e];
                }
                uint4 sh, sl;
                pack8(sv, sh, sl);
                const uint4 pah = fragp(S.P[0], LDA, r16, 32 * s, lane), pal = fragp(S.P[1], LDA, r16, 32 * s, lane);
                const uint4 p2h = fragp(S.P2[0], LDA, r16, 32 * s, lane), p2l = fragp(S.P2[1], LDA, r16, 32 * s, lane);
                sa = mma32(sa, pah, sh);
                sa = mma32(sa, pah, sl);
                sa = mma32(sa, pal, sh);
                yy = mma32(yy, p2h, sh);
                yy = mma32(yy, p2h, sl);
                yy = mma32(yy, p2l, sh);
            }
            // V parts on the K=16 instruction, in their own accumulators
            const uint2 vfr = ldtr(&S.V[16 * cw], LDA, lane);  // V[s = 4q+e][i_own]
            {
                f32x4_t sv = mma16(zero4(), ldtr(S.Q1T[0], LDC, lane), vfr);
                sv = mma16(sv, ldtr(S.Q1T[1], LDC, lane), vfr);
                f32x4_t yv = mma16(zero4(), frag16(S.Q2[0], LDC, 0, 0, lane), vfr);
                yv = mma16(yv, frag16(S.Q2[1], LDC, 0, 0, lane), vfr);
                sa += sv;
                yy += yv;
            }
            // S_new^T = S^T diag(e^{gL}) + [B^^T K^^T] [SA; V]   (K = 32: SA rows, then V rows)
            uint2 sah, sal;
            pack4(sa, sah, sal);
            const uint4 bhi = cat(sah, vfr), blo = cat(sal, make_uint2(0, 0));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const uint4 ah = cat(ldtr(&S.Bh[0][16 * tj], LDA, lane), ldtr(&S.Kh[0][16 * tj], LDA, lane));
                const uint4 al = cat(ldtr(&S.Bh[1][16 * tj], LDA, lane), ldtr(&S.Kh[1][16 * tj], LDA, lane));
                const float4 el = *reinterpret_cast<const float4*>(&S.egL[16 * tj + 4 * q]);
                f32x4_t acc = St[tj] * f32x4_t{el.x, el.y, el.z, el.w};
                acc = mma32(acc, ah, bhi);
                f32x4_t c1 = mma32(zero4(), ah, blo);
                c1 = mma32(c1, al, bhi);
                St[tj] = acc + c1;
            }
            bf16_t* yp = y + ((long)(bb * Tn + t0 + 4 * q) * H + h) * NK + i_own;
            if (L == CH) {
#pragma unroll
                for (int e = 0; e < 4; e++) yp[(long)e * H * NK].bits = f32_to_bf16(yy[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (4 * q + e < L) yp[(long)e * H * NK].bits = f32_to_bf16(yy[e]);
            }
            if (ckpt) {
#pragma unroll
                for (int tj = 0; tj < 4; tj++)
                    *reinterpret_cast<float4*>(ckpt + (bh * ncp + n + 1) * NN + (long)i_own * NK + 16 * tj + 4 * q) =
                        make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
            }
        }
        lds_barrier();
    }
    if (!producer) {
#pragma unroll
        for (int tj = 0; tj < 4; tj++)
            *reinterpret_cast<float4*>(sT + bh * NN + (long)i_own * NK + 16 * tj + 4 * q) =
                make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
    }
}

void launch_chunk_forward(const Fwd& p) {
    hipLaunchKernelGGL(chunk_forward_bf16, dim3(p.B * p.H), dim3(512), 0, p.stream, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.s0, (bf16_t*)p.y, p.sT, p.ckpt);
}

}  // namespace wkv7
