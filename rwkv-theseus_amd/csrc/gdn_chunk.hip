// Chunked forward of the gated delta rule (the GDN layers of the reference's
// teacher: one decay per head and step) on the matrix cores, head sizes 64 and 128.
//
// The recurrence is the WKV7 one with the converter's GDN operands
// (convert_qwen2rwkv_lightning.py:381-385): r = q/sqrt(N), a = k, b = -e^{g} beta k,
// v <- beta v, and a decay e^{g_t} shared by all keys.  In [value][key] form
// X_t = e^{g_t} X_{t-1} + beta_t (v_t - e^{g_t} X_{t-1} k_t) k_t^T, y_t = X_t r_t.
//
// Over a chunk of 16 steps with gamma_t = g_0 + ... + g_t (gamma_{-1} = 0, L = last
// step) the WY form of the WKV7 kernels becomes, because the decay is one scalar
// per step, a set of products of UNSCALED operands times a 16x16 matrix of decay
// ratios e^{gamma_t - gamma_s} (s <= t: never above 1, so no clamp is needed):
//   Aab[t][s] = -beta_s (k_t.k_s) e^{gamma_{t-1} - gamma_{s-1}}   (s < t)
//   Aak[t][s] =          (k_t.k_s) e^{gamma_{t-1} - gamma_s}       (s < t)
//   Brb[t][s] = -beta_s (r_t.k_s) e^{gamma_t - gamma_{s-1}}       (s <= t)
//   Brk[t][s] =          (r_t.k_s) e^{gamma_t - gamma_s}           (s <= t)
//   A~ = k e^{gamma_{t-1}},  R~ = r e^{gamma_t},
//   B^ = -beta k e^{gamma_L - gamma_{t-1}},  K^ = k e^{gamma_L - gamma_t},  V = beta v
//   Ti = (I - Aab)^{-1}; P = Ti A~; Q' = Ti Aak; P2 = R~ + Brb P; Q2 = Brk + Brb Q'
//   SA = P X0^T + Q' V;  Y = P2 X0^T + Q2 V;  X_L = e^{gamma_L} X0 + SA^T B^ + V^T K^
// (checked in float64 against the oracle's step recurrence before the kernels).
//
// Two kernels.  gdn_prep forms every chunk's operands at once (one wave per chunk,
// all chunks of all heads in parallel: nothing in them depends on the state) and
// writes them to the workspace already in the register layouts of the scan:
// P and P2 as split-bf16 A operands of the K=32 products over the keys, the
// update operand [B^^T | K^^T] per 16-key tile, Q'^T and Q2^T as K=16 A
// operands, beta v as the K=16 B operand of each 16-row block, and e^{gamma_L}.
// gdn_scan then walks each head's chunks in order, one workgroup per head and one
// wave per 16 value rows of the fp32 state, which stays in registers.  The next
// chunk's record comes into LDS by DMA while the current one is used (all waves
// read the same record), so the scan reads nothing else from memory.
// Products use split-bf16 operands (hi + lo, three MFMAs), as the WKV7 kernels.
//
// With few heads (the teacher's 32 heads of 128 keys fill 64 of 256 CUs) the scan is
// cut in time like the WKV7 forward's time split: X after a chunk is affine in X before
// it, X_{c+1} = X_c M_c + U_c, so each head's chunks form k segments scanned at once.
// Segment 0 starts from s0; segment s >= 1 carries two states in every wave, one from
// zero (its output y0 and final U_s) and one from the identity with v = 0 (its output
// z_t = Phi_t r_t and final Phi_s), both on the same record.  gdn_split_fixup then
// chains X_{s+1} = X_s Phi_s + U_s and forms y_t = y0_t + X_s z_t.
#include "wkv7_io.h"
#include "wkv7_launch.h"

namespace wkv7 {
namespace {

constexpr int GC = 16;  // chunk length

// One chunk's record in the workspace (byte offsets; 256-byte aligned records).  PK: the
// WKV7 operator's records (wkv7_rec_prep), whose decay is one per key, so EL holds
// e^{g_L} for every key instead of one e^{gamma_L}.
template <int NK, bool PK = false>
struct GdnRec {
    static constexpr int KS = NK / 32, TJ = NK / 16;
    static constexpr size_t PF = 0;                                // [KS][hi, lo][64 lanes] uint4
    static constexpr size_t P2F = PF + (size_t)KS * 2 * 64 * 16;   // same for P2
    static constexpr size_t UF = P2F + (size_t)KS * 2 * 64 * 16;   // [TJ][hi, lo][64] uint4
    static constexpr size_t QF = UF + (size_t)TJ * 2 * 64 * 16;    // [Q'^T hi, lo, Q2^T hi, lo][64] uint2
    static constexpr size_t VF = QF + 4 * 64 * 8;                  // [TJ row blocks][hi, lo][64] uint2
    static constexpr size_t EL = VF + (size_t)TJ * 2 * 64 * 8;     // e^{gamma_L} (PK: [NK] per key)
    static constexpr size_t BYTES = EL + (PK ? ((size_t)NK * 4 + 255) / 256 * 256 : 256);
    static constexpr int DMA_BLOCKS = (int)((BYTES + 1023) / 1024);  // 1 KB LDS DMA blocks
};
static_assert(GdnRec<128>::BYTES % 256 == 0 && GdnRec<64>::BYTES % 256 == 0 && GdnRec<128, true>::BYTES % 256 == 0,
              "record alignment");

// ---------------------------------------------------------------------------
// Operands of chunk blockIdx.x of head blockIdx.y (one wave).
// Lane (q4, r16) holds token t = r16's keys of K-step ks in the permuted K=32
// order (32ks + 4q4 + e, then 32ks + 16 + 4q4 + e), and D-layout tiles with
// rows 4q4 + e, column r16.  q, k, v are float32 or bfloat16 (TI); with qk_norm, q
// and k are L2-normalised here, x / sqrt(sum x^2 + 1e-6) as the layers do it
// (use_qk_l2norm_in_kernel).
// ---------------------------------------------------------------------------
template <int NK, typename TI>
__global__ __launch_bounds__(64) void gdn_prep(int Tn, int H, int qk_norm, const TI* __restrict__ q,
                                               const TI* __restrict__ k, const TI* __restrict__ v,
                                               const float* __restrict__ g, const float* __restrict__ beta,
                                               uint8_t* __restrict__ ws) {
    using R = GdnRec<NK>;
    constexpr int KS = R::KS;
    const int c = blockIdx.x, bh = blockIdx.y, nchunk = gridDim.x;
    const int bb = bh / H, h = bh - bb * H;
    const int lane = threadIdx.x, q4 = lane >> 4, r16 = lane & 15;
    const int t0 = c * GC, L = min(GC, Tn - t0);
    const long tok0 = (long)bb * Tn + t0;
    auto row = [&](int t) { return ((tok0 + t) * H + h) * (long)NK; };
    const float rs = 1.f / __builtin_sqrtf((float)NK);
    __shared__ float gsh[4][GC];  // gamma_t, gamma_{t-1}, beta_t, k_t's norm factor (past the end: 0)
    // v as rows [t][value] (past the end: 0), loaded with k and q and read back per block of
    // 16 values: the V operand's elementwise loads at the end of the kernel had cost 18 µs
    // of a 189 µs teacher-geometry call
    __shared__ float vsh[GC][NK + 4];

    const bool tv = r16 < L;
    const int tl = tv ? r16 : 0;  // (clamped: every lane loads, lane_mask in wkv7_io.h)
    const float g_ = g[(tok0 + tl) * H + h], b_ = beta[(tok0 + tl) * H + h];
    const uint32_t tm = lane_mask(tv);
    const float gt = keep(tm, g_), bt = keep(tm, b_);
    const float gam = row_prefix_sum(gt);
    const float gm1 = row_prev(gam, 0.f);
    const float gL = row_last(gam);
    // rows of k and q (zero past the end); q kept for R~
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int c0 = 32 * ks + 4 * q4;
        *reinterpret_cast<float4*>(&vsh[r16][c0]) = keep4(tm, ld4f(v + row(tl) + c0));
        *reinterpret_cast<float4*>(&vsh[r16][c0 + 16]) = keep4(tm, ld4f(v + row(tl) + c0 + 16));
    }
    float kr[KS][8], qr[KS][8];
    float ssk = 0.f, ssq = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int c0 = 32 * ks + 4 * q4;
        const float4 a = keep4(tm, ld4f(k + row(tl) + c0)), b = keep4(tm, ld4f(k + row(tl) + c0 + 16));
        const float4 x = keep4(tm, ld4f(q + row(tl) + c0)), y = keep4(tm, ld4f(q + row(tl) + c0 + 16));
        kr[ks][0] = a.x, kr[ks][1] = a.y, kr[ks][2] = a.z, kr[ks][3] = a.w;
        kr[ks][4] = b.x, kr[ks][5] = b.y, kr[ks][6] = b.z, kr[ks][7] = b.w;
        qr[ks][0] = x.x, qr[ks][1] = x.y, qr[ks][2] = x.z, qr[ks][3] = x.w;
        qr[ks][4] = y.x, qr[ks][5] = y.y, qr[ks][6] = y.z, qr[ks][7] = y.w;
#pragma unroll
        for (int e = 0; e < 8; e++) ssk += kr[ks][e] * kr[ks][e], ssq += qr[ks][e] * qr[ks][e];
    }
    float nk = 1.f, nq = 1.f;  // the rows' L2-norm factors (the four lane groups of a token hold its keys)
    if (qk_norm) {
        ssk += __shfl_xor(ssk, 16), ssq += __shfl_xor(ssq, 16);
        ssk += __shfl_xor(ssk, 32), ssq += __shfl_xor(ssq, 32);
        nk = __frsqrt_rn(ssk + 1e-6f), nq = __frsqrt_rn(ssq + 1e-6f);
    }
    if (q4 == 0) {
        gsh[0][r16] = gam;
        gsh[1][r16] = gm1;
        gsh[2][r16] = bt;
        gsh[3][r16] = nk;
    }
    uint4 kh[KS], kl[KS], qh[KS], ql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
#pragma unroll
        for (int e = 0; e < 8; e++) kr[ks][e] *= nk, qr[ks][e] *= nq;
        pack8(kr[ks], kh[ks], kl[ks]);
        pack8(qr[ks], qh[ks], ql[ks]);
    }
    // KK[t][s] = k_t.k_s, KR[t][s] = k_t.q_s (contractions over the keys)
    f32x4_t KK = zero4(), KR = zero4();
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        KK = mma32(mma32(mma32(KK, kh[ks], kh[ks]), kh[ks], kl[ks]), kl[ks], kh[ks]);
        KR = mma32(mma32(mma32(KR, kh[ks], qh[ks]), kh[ks], ql[ks]), kl[ks], qh[ks]);
    }
    __syncthreads();  // gsh, vsh
    // the chunk matrices in D layout (element [rr][cc], rr = 4q4 + e, cc = r16); the
    // decay ratios are exponentials of differences that are <= 0 where the mask keeps them
    const int cc = r16;
    f32x4_t Aab, AabT, Aak, BrbT, BrkT;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        const float gr = gsh[0][rr], gm1r = gsh[1][rr], br = gsh[2][rr];
        const float kk = KK[e], kq = KR[e] * rs;  // k_rr.k_cc, k_rr.r_cc
        Aab[e] = cc < rr ? -bt * kk * __expf(gm1r - gm1) : 0.f;   // Aab[rr][cc]
        AabT[e] = rr < cc ? -br * kk * __expf(gm1 - gm1r) : 0.f;  // Aab[cc][rr]
        Aak[e] = cc < rr ? kk * __expf(gm1r - gam) : 0.f;         // Aak[rr][cc]
        BrbT[e] = rr <= cc ? -br * kq * __expf(gam - gm1r) : 0.f; // Brb[cc][rr]
        BrkT[e] = rr <= cc ? kq * __expf(gam - gr) : 0.f;         // Brk[cc][rr]
    }
    f32x4_t Ti, TiT;
    tri_inverse(Aab, AabT, lane, Ti, TiT);
    const Pk pTiT = pk(TiT), pAak = pk(Aak), pBrbT = pk(BrbT);
    const f32x4_t Q1 = mm16s(pTiT, pAak);                      // Q' = Ti Aak        [t][s]
    const Pk pQ1T = pk(mm16s(pAak, pTiT));                      // Q'^T               [s][t]
    const Pk pQ2T = pk(BrkT + mm16s(pk(Q1), pBrbT));            // Q2^T = Brk^T + Q'^T Brb^T
    uint8_t* const rec = ws + ((size_t)bh * nchunk + c) * R::BYTES;
    {
        uint2* qf = reinterpret_cast<uint2*>(rec + R::QF) + lane;
        qf[0] = pQ1T.h, qf[64] = pQ1T.l, qf[128] = pQ2T.h, qf[192] = pQ2T.l;
        if (lane == 0) *reinterpret_cast<float*>(rec + R::EL) = __expf(gL);
    }
    // V = beta v as the K=16 B operand of each block of 16 value rows (lane: value
    // 16rb + r16, steps 4q4 + e), split
#pragma unroll
    for (int rb = 0; rb < R::TJ; rb++) {
        f32x4_t vv;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 4 * q4 + e;
            vv[e] = gsh[2][t] * vsh[t][16 * rb + r16];  // (zero past the end)
        }
        const Pk pv = pk(vv);
        uint2* vf = reinterpret_cast<uint2*>(rec + R::VF) + (size_t)(2 * rb) * 64 + lane;
        vf[0] = pv.h;
        vf[64] = pv.l;
    }
    // per pair of 16-key tiles (one K-step): P, P2 and the update operands
    const float egam = __expf(gam) * rs;  // R~ row scale of token r16
    float ea[4], eb[4], ek[4];  // the tiles' token scalings (t = 4q4 + e), formed once
    const TI* krow[4];          // and k's row of token t, key r16
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = 4 * q4 + e;
        krow[e] = k + row(t < L ? t : 0) + r16;
        ea[e] = __expf(gsh[1][t]);
        eb[e] = -gsh[2][t] * __expf(gL - gsh[1][t]);
        ek[e] = __expf(gL - gsh[0][t]);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        Pk pPT[2], pP2T[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int tj = 2 * ks + u;
            // A~, B^, K^ of tile tj in D layout [t][j] (t = 4q4 + e, j = 16tj + r16)
            f32x4_t at, bhat, khat;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 4 * q4 + e;
                const float kx = io<TI>::ld(krow[e], 16 * tj);  // (krow: clamped)
                const float kv = keep(lane_mask(t < L), kx) * gsh[3][t];  // (gsh[3]: 0 past the end)
                at[e] = kv * ea[e];
                bhat[e] = kv * eb[e];
                khat[e] = kv * ek[e];
            }
            const Pk pA = pk(at);
            const f32x4_t Pt = mm16s(pTiT, pA);   // P tile [t][j]
            pPT[u] = pk(mm16s(pA, pTiT));          // P^T tile [j][t]: lane (t = r16) holds P[t][16tj + 4q4 + e]
            f32x4_t rt;
#pragma unroll
            for (int e = 0; e < 4; e++) rt[e] = qr[ks][4 * u + e] * egam;  // R~[t][16tj + 4q4 + e]
            pP2T[u] = pk(rt + mm16s(pk(Pt), pBrbT));  // P2^T = R~^T + P^T Brb^T
            const Pk pb = pk(bhat), pkh = pk(khat);
            uint4* uf = reinterpret_cast<uint4*>(rec + R::UF) + (size_t)(2 * tj) * 64 + lane;
            uf[0] = cat(pb.h, pkh.h);
            uf[64] = cat(pb.l, pkh.l);
        }
        uint4* pf = reinterpret_cast<uint4*>(rec + R::PF) + (size_t)(2 * ks) * 64 + lane;
        pf[0] = cat(pPT[0].h, pPT[1].h);
        pf[64] = cat(pPT[0].l, pPT[1].l);
        uint4* p2 = reinterpret_cast<uint4*>(rec + R::P2F) + (size_t)(2 * ks) * 64 + lane;
        p2[0] = cat(pP2T[0].h, pP2T[1].h);
        p2[64] = cat(pP2T[0].l, pP2T[1].l);
    }
}

// ---------------------------------------------------------------------------
// The WKV7 operator's records (bf16 r, w, k, v, a, b; kernels/wkv7_state.cu:12-40's
// recurrence, chunk algebra of wkv7_chunk_fwd.hip).  The decay is one per key, so the
// decay ratios ride on the operands rather than on a 16x16 matrix: per key, with g the
// chunk's inclusive cumulative log-decay (|g| < 16 e^{-1/2}, so e^{-g} < 2e4 stays
// finite and every product below is of moderate size), gp = g_{t-1} and gL = g_{L-1},
//   A~ = a e^{gp}, R~ = r e^{g}, B- = b e^{-g}, K- = k e^{-g}, B^ = b e^{gL-g}, K^ = k e^{gL-g}
//   Aab = tril_s(A~ B-^T), Aak = tril_s(A~ K-^T), Brb = tril(R~ B-^T), Brk = tril(R~ K-^T)
// (contractions over the keys on the matrix cores), V = v, and e^{gL} per key.  One wave
// per chunk as gdn_prep, writing the same record layout (GdnRec<NK, true>).  Lane (q4,
// r16) holds token r16's keys 32ks + 4q4 + e and 32ks + 16 + 4q4 + e; the D-layout tiles
// of A~, B^ and K^ ([t][j], rows t = 4q4 + e) are read back from LDS planes.
// ---------------------------------------------------------------------------
template <int NK>
__global__ __launch_bounds__(64) void wkv7_rec_prep(int Tn, int H, const bf16_t* __restrict__ r,
                                                    const bf16_t* __restrict__ w, const bf16_t* __restrict__ k,
                                                    const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
                                                    const bf16_t* __restrict__ b, uint8_t* __restrict__ ws) {
    using R = GdnRec<NK, true>;
    constexpr int KS = R::KS, LP = NK + 4;
    const int c = blockIdx.x, bh = blockIdx.y, nchunk = gridDim.x;
    const int bb = bh / H, h = bh - bb * H;
    const int lane = threadIdx.x, q4 = lane >> 4, r16 = lane & 15;
    const int t0 = c * GC, L = min(GC, Tn - t0);
    const long tok0 = (long)bb * Tn + t0;
    const bool tv = r16 < L;
    const long row = ((tok0 + (tv ? r16 : 0)) * H + h) * (long)NK;  // token r16's row (clamped: every lane loads)
    const uint32_t tm = lane_mask(tv);
    // A~, B^, K^ as rows [t][j] for the D-layout reads; v as rows [t][i]
    __shared__ __attribute__((aligned(16))) float pa[GC][LP], pb[GC][LP], pkh[GC][LP], vsh[GC][LP];
    uint8_t* const rec = ws + ((size_t)bh * nchunk + c) * R::BYTES;
    f32x4_t Aab = zero4(), AabT = zero4(), Aak = zero4(), BrbT = zero4(), BrkT = zero4();
    float rt[KS][8];  // R~ of the lane's keys, kept for P2
    auto ld8 = [&](const bf16_t* x, int c0, float (&o)[8]) {
        const float4 p = keep4(tm, ld4f(x + row + c0)), q = keep4(tm, ld4f(x + row + c0 + 16));
        o[0] = p.x, o[1] = p.y, o[2] = p.z, o[3] = p.w, o[4] = q.x, o[5] = q.y, o[6] = q.z, o[7] = q.w;
    };
    auto st8 = [&](float (*pl)[LP], int c0, const float (&x)[8]) {
        *reinterpret_cast<float4*>(&pl[r16][c0]) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(&pl[r16][c0 + 16]) = make_float4(x[4], x[5], x[6], x[7]);
    };
    // split products over one K=32 step: acc += X Y^T (X, Y: the lanes' token rows)
    auto mm3 = [](f32x4_t acc, uint4 xh, uint4 xl, uint4 yh, uint4 yl) {
        return mma32(mma32(mma32(acc, xh, yh), xh, yl), xl, yh);
    };
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int c0 = 32 * ks + 4 * q4;
        float wv[8], av[8], bv[8], kv[8], vv[8];
        ld8(w, c0, wv), ld8(a, c0, av), ld8(b, c0, bv), ld8(k, c0, kv), ld8(r, c0, rt[ks]), ld8(v, c0, vv);
        st8(vsh, c0, vv);
        float At[8], Bm[8], Km[8], Bh[8], Kh[8], eL[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float g = row_prefix_sum(tv ? log_decay(wv[e]) : 0.f);  // (0 past the end)
            const float gp = row_prev(g, 0.f), gL = row_last(g);
            const float em = __expf(-g), eh = __expf(gL - g);
            At[e] = av[e] * __expf(gp);
            rt[ks][e] *= __expf(g);
            Bm[e] = bv[e] * em, Km[e] = kv[e] * em;
            Bh[e] = bv[e] * eh, Kh[e] = kv[e] * eh;
            eL[e] = __expf(gL);
        }
        st8(pa, c0, At), st8(pb, c0, Bh), st8(pkh, c0, Kh);
        if (r16 == 0) {
            float* el = reinterpret_cast<float*>(rec + R::EL);
            *reinterpret_cast<float4*>(el + c0) = make_float4(eL[0], eL[1], eL[2], eL[3]);
            *reinterpret_cast<float4*>(el + c0 + 16) = make_float4(eL[4], eL[5], eL[6], eL[7]);
        }
        uint4 ah, al, bh_, bl, kh, kl, rh, rl;
        pack8(At, ah, al), pack8(Bm, bh_, bl), pack8(Km, kh, kl), pack8(rt[ks], rh, rl);
        Aab = mm3(Aab, ah, al, bh_, bl);     // [rr][cc] = A~_rr . B-_cc
        AabT = mm3(AabT, bh_, bl, ah, al);   // B-_rr . A~_cc
        Aak = mm3(Aak, ah, al, kh, kl);      // A~_rr . K-_cc
        BrbT = mm3(BrbT, bh_, bl, rh, rl);   // B-_rr . R~_cc
        BrkT = mm3(BrkT, kh, kl, rh, rl);    // K-_rr . R~_cc
    }
    // the chunk matrices in D layout (element [rr][cc], rr = 4q4 + e, cc = r16), masked
    const int cc = r16;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        Aab[e] = cc < rr ? Aab[e] : 0.f;     // Aab[rr][cc]
        AabT[e] = rr < cc ? AabT[e] : 0.f;   // Aab[cc][rr]
        Aak[e] = cc < rr ? Aak[e] : 0.f;     // Aak[rr][cc]
        BrbT[e] = rr <= cc ? BrbT[e] : 0.f;  // Brb[cc][rr]
        BrkT[e] = rr <= cc ? BrkT[e] : 0.f;  // Brk[cc][rr]
    }
    f32x4_t Ti, TiT;
    tri_inverse(Aab, AabT, lane, Ti, TiT);
    const Pk pTiT = pk(TiT), pAak = pk(Aak), pBrbT = pk(BrbT);
    const f32x4_t Q1 = mm16s(pTiT, pAak);                      // Q' = Ti Aak        [t][s]
    const Pk pQ1T = pk(mm16s(pAak, pTiT));                      // Q'^T               [s][t]
    const Pk pQ2T = pk(BrkT + mm16s(pk(Q1), pBrbT));            // Q2^T = Brk^T + Q'^T Brb^T
    {
        uint2* qf = reinterpret_cast<uint2*>(rec + R::QF) + lane;
        qf[0] = pQ1T.h, qf[64] = pQ1T.l, qf[128] = pQ2T.h, qf[192] = pQ2T.l;
    }
    __syncthreads();  // the planes
    // V as the K=16 B operand of each block of 16 value rows (lane: value 16rb + r16,
    // steps 4q4 + e; zero past the end), split
#pragma unroll
    for (int rb = 0; rb < R::TJ; rb++) {
        f32x4_t vq;
#pragma unroll
        for (int e = 0; e < 4; e++) vq[e] = vsh[4 * q4 + e][16 * rb + r16];
        const Pk pv = pk(vq);
        uint2* vf = reinterpret_cast<uint2*>(rec + R::VF) + (size_t)(2 * rb) * 64 + lane;
        vf[0] = pv.h;
        vf[64] = pv.l;
    }
    // per pair of 16-key tiles (one K-step): P, P2 and the update operands
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        Pk pPT[2], pP2T[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int tj = 2 * ks + u;
            f32x4_t at, bhat, khat;  // D layout [t][j], t = 4q4 + e, j = 16tj + r16
#pragma unroll
            for (int e = 0; e < 4; e++) {
                at[e] = pa[4 * q4 + e][16 * tj + r16];
                bhat[e] = pb[4 * q4 + e][16 * tj + r16];
                khat[e] = pkh[4 * q4 + e][16 * tj + r16];
            }
            const Pk pA = pk(at);
            const f32x4_t Pt = mm16s(pTiT, pA);   // P tile [t][j]
            pPT[u] = pk(mm16s(pA, pTiT));          // P^T tile [j][t]
            f32x4_t rr4;                            // R~[t = r16][16tj + 4q4 + e]
#pragma unroll
            for (int e = 0; e < 4; e++) rr4[e] = rt[ks][4 * u + e];
            pP2T[u] = pk(rr4 + mm16s(pk(Pt), pBrbT));  // P2^T = R~^T + P^T Brb^T
            const Pk pb4 = pk(bhat), pk4 = pk(khat);
            uint4* uf = reinterpret_cast<uint4*>(rec + R::UF) + (size_t)(2 * tj) * 64 + lane;
            uf[0] = cat(pb4.h, pk4.h);
            uf[64] = cat(pb4.l, pk4.l);
        }
        uint4* pf = reinterpret_cast<uint4*>(rec + R::PF) + (size_t)(2 * ks) * 64 + lane;
        pf[0] = cat(pPT[0].h, pPT[1].h);
        pf[64] = cat(pPT[0].l, pPT[1].l);
        uint4* p2 = reinterpret_cast<uint4*>(rec + R::P2F) + (size_t)(2 * ks) * 64 + lane;
        p2[0] = cat(pP2T[0].h, pP2T[1].h);
        p2[64] = cat(pP2T[0].l, pP2T[1].l);
    }
}

// ---------------------------------------------------------------------------
// Each head's chunks in order.  A head's value rows are split over `row groups`
// (workgroups rg * BH + bh, so that with BH a multiple of 8 a head's groups share an
// XCD and its L2); wave w of group rg keeps the 16 rows of block rb = rg * NW + w,
// St[tj][e] = X[i_own][16tj + 4q4 + e] (as the WKV7 forward's consumers).  States
// s0 / sT are [key][value] when kv (GDN's layout), else [value][key].  Records are
// double-buffered in LDS: chunk c + 1's comes in by DMA (each wave moves every NW-th
// kilobyte) while chunk c's is read; one barrier per chunk.
// ---------------------------------------------------------------------------
// The time split's buffers (float32): X_1 [BH][N][N] (internal [value][key] layout), U_s
// and Phi_s [k - 1][BH][N][N], and the y0 and z tiles [k - 1][BH][m][N/16 row blocks][64
// lanes][4] (lane (q4, r16) of row block rb: y[4q4 + e][16rb + r16]).
struct GdnSplit {
    int m = 0, k = 0;  // chunks of each segment after the first, segments
    int m0 = 0;        // chunks of segment 0
    float *send0 = nullptr, *uend = nullptr, *phi = nullptr, *y0 = nullptr, *z = nullptr;
};

// PK: WKV7 records (a decay per key: the state's key columns scale by e^{g_L} each);
// ckpt (not with SPLIT; may be null): the state at every chunk's start and the final one,
// [bh][count][value][key] as the step-serial kernels keep saved states.
template <int NK, typename TO, bool SPLIT, bool PK = false>
__global__ __launch_bounds__(256) void gdn_scan(int Tn, int H, int BH, int kv, const float* __restrict__ s0,
                                                   TO* __restrict__ o, float* __restrict__ sT,
                                                   const uint8_t* __restrict__ ws, GdnSplit sp,
                                                   float* __restrict__ ckpt) {
    using R = GdnRec<NK, PK>;
    constexpr int KS = R::KS, TJ = R::TJ;
    __shared__ __attribute__((aligned(1024))) uint8_t recs[2][R::DMA_BLOCKS * 1024];
    // workgroup (segment * row groups + rg) * BH + bh (SPLIT; else rg * BH + bh)
    constexpr int RGS = NK / 64;
    const int bh = blockIdx.x % BH, rest = blockIdx.x / BH, rg = SPLIT ? rest % RGS : rest;
    const int sgm = SPLIT ? rest / RGS : 0, bb = bh / H, h = bh - bb * H;
    const bool dual = SPLIT && sgm > 0;  // the zero and identity runs
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // waves per group (the host launches whole waves, at least one: the DMA loop steps by NW)
    const int NW = max(1, __builtin_amdgcn_readfirstlane((int)(blockDim.x >> 6)));
    const int lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
    const int rb = rg * NW + wv, i_own = 16 * rb + r16;
    const long NN = (long)NK * NK, ei = kv ? 1 : NK, ej = kv ? NK : 1;
    const int nchunk = (Tn + GC - 1) / GC;
    // this segment's chunks (segment 0: m0, the others m)
    const int c0 = SPLIT ? (sgm == 0 ? 0 : sp.m0 + (sgm - 1) * sp.m) : 0;
    const int c1 = SPLIT ? min(nchunk, c0 + (sgm == 0 ? sp.m0 : sp.m)) : nchunk;
    // this head's records (the host keeps them under 4 GB, so 32-bit offsets reach them)
    const i32x4_t rs = dma_rsrc(ws + (size_t)bh * nchunk * R::BYTES, (uint32_t)((size_t)nchunk * R::BYTES));
    auto fetch = [&](int c, int buf) {
        uint32_t so = (uint32_t)((size_t)c * R::BYTES);
        asm volatile("" : "+s"(so));  // (an SGPR even where it is a constant)
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)recs[buf];
        for (int j = wv; j < R::DMA_BLOCKS; j += NW) dma_kb(base + 1024 * j, rs, (uint32_t)(1024 * j + 16 * lane), so);
    };
    fetch(c0, 0);
    f32x4_t St[TJ], Sp[TJ];  // (Sp: the identity run)
#pragma unroll
    for (int tj = 0; tj < TJ; tj++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            St[tj][e] = dual ? 0.f : s0[bh * NN + i_own * ei + (16 * tj + 4 * q4 + e) * ej];
            Sp[tj][e] = i_own == 16 * tj + 4 * q4 + e ? 1.f : 0.f;
        }
    vm_wait0();
    __syncthreads();
    const long ncp = nchunk + 1;  // saved states per head
    // The wave's 16 rows of a saved state are 16 * NK contiguous floats; regrouped through
    // LDS, each of its TJ stores writes 1 KB of them (from the registers, each would write
    // 64-byte pieces of 16 rows)
    constexpr int SQ = NK + 4;  // padded row (floats)
    __shared__ __attribute__((aligned(16))) float sq[SPLIT ? 1 : 4][SPLIT ? 4 : 16 * SQ];
    auto save = [&](int slot) {
        if constexpr (!SPLIT) {
            float* const q = sq[wv];
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
                *reinterpret_cast<float4*>(q + r16 * SQ + 16 * tj + 4 * q4) =
                    make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
            float* const dst = ckpt + ((long)bh * ncp + slot) * NN + (long)(16 * rb) * NK;
#pragma unroll
            for (int u = 0; u < TJ; u++) {  // (16 NK floats = TJ runs of 256)
                const int f = 256 * u + 4 * lane, row = f / NK, col = f % NK;
                *reinterpret_cast<float4*>(dst + f) = *reinterpret_cast<const float4*>(q + row * SQ + col);
            }
        }
    };
    for (int c = c0; c < c1; c++) {
        if (c + 1 < c1) fetch(c + 1, (c - c0 + 1) & 1);
        const uint8_t* const rec = recs[(c - c0) & 1];
        const int t0 = c * GC, L = min(GC, Tn - t0);
        const long tok0 = (long)bb * Tn + t0;
        // SA = P X0^T and Y = P2 X0^T over the keys (permuted K=32 steps)
        f32x4_t sa = zero4(), yy = zero4(), sa2 = zero4(), yy2 = zero4();
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const float sv[8] = {St[2 * ks][0], St[2 * ks][1], St[2 * ks][2], St[2 * ks][3],
                                 St[2 * ks + 1][0], St[2 * ks + 1][1], St[2 * ks + 1][2], St[2 * ks + 1][3]};
            uint4 sh, sl;
            pack8(sv, sh, sl);
            const uint4* pf = reinterpret_cast<const uint4*>(rec + R::PF) + (2 * ks) * 64 + lane;
            const uint4* p2 = reinterpret_cast<const uint4*>(rec + R::P2F) + (2 * ks) * 64 + lane;
            const uint4 ph = pf[0], pl = pf[64], p2h = p2[0], p2l = p2[64];
            sa = mma32(mma32(mma32(sa, ph, sh), ph, sl), pl, sh);
            yy = mma32(mma32(mma32(yy, p2h, sh), p2h, sl), p2l, sh);
            if (dual) {  // the identity run on the same record
                const float sw[8] = {Sp[2 * ks][0], Sp[2 * ks][1], Sp[2 * ks][2], Sp[2 * ks][3],
                                     Sp[2 * ks + 1][0], Sp[2 * ks + 1][1], Sp[2 * ks + 1][2], Sp[2 * ks + 1][3]};
                pack8(sw, sh, sl);
                sa2 = mma32(mma32(mma32(sa2, ph, sh), ph, sl), pl, sh);
                yy2 = mma32(mma32(mma32(yy2, p2h, sh), p2h, sl), p2l, sh);
            }
        }
        // + Q' V and Q2 V on the K=16 instruction, in their own accumulators
        const uint2* vf = reinterpret_cast<const uint2*>(rec + R::VF) + (2 * rb) * 64 + lane;
        const uint2 vh = vf[0], vl = vf[64];
        {
            const uint2* qf = reinterpret_cast<const uint2*>(rec + R::QF) + lane;
            const uint2 q1h = qf[0], q1l = qf[64], q2h = qf[128], q2l = qf[192];
            sa += mma16(mma16(mma16(zero4(), q1h, vh), q1h, vl), q1l, vh);
            yy += mma16(mma16(mma16(zero4(), q2h, vh), q2h, vl), q2l, vh);
        }
        if (!dual) {
#pragma unroll
            for (int e = 0; e < 4; e++) {  // y[t][i_own], t = 4q4 + e
                const int t = 4 * q4 + e;
                if (t < L) io<TO>::st(o, ((tok0 + t) * H + h) * NK + i_own, yy[e]);
            }
        } else {  // the tiles for gdn_split_fixup
            const long f4 = ((((long)(sgm - 1) * BH + bh) * sp.m + (c - c0)) * TJ + rb) * 64 + lane;
            reinterpret_cast<float4*>(sp.y0)[f4] = make_float4(yy[0], yy[1], yy[2], yy[3]);
            reinterpret_cast<float4*>(sp.z)[f4] = make_float4(yy2[0], yy2[1], yy2[2], yy2[3]);
        }
        // the saved state of this chunk's start, issued after the next record's DMA: the wait
        // below lets these TJ stores stay in flight (a vmcnt(0) there had waited for every
        // store to complete each chunk: 0.49 -> 0.23 ms of scan at B=4, T=2048, H=32, N=128
        // without them)
        if (!SPLIT && ckpt) save(c);
        // X^T <- e^{gamma_L} X^T + [B^^T K^^T] [SA; V]   (K = 32: SA rows, then V rows;
        // the identity run has no V rows)
        uint2 sah, sal, sah2, sal2;
        pack4(sa, sah, sal);
        if (dual) pack4(sa2, sah2, sal2);
        const uint4 bhi = cat(sah, vh), blo = cat(sal, vl);
        const uint4 bhi2 = cat(sah2, make_uint2(0, 0)), blo2 = cat(sal2, make_uint2(0, 0));
        const float egL = *reinterpret_cast<const float*>(rec + R::EL);
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            const uint4* uf = reinterpret_cast<const uint4*>(rec + R::UF) + (2 * tj) * 64 + lane;
            const uint4 ah = uf[0], al = uf[64];
            // the decay of the lane's keys 16 tj + 4 q4 + e (one for all keys unless PK)
            const f32x4_t eg = PK ? *reinterpret_cast<const f32x4_t*>(rec + R::EL + 4 * (16 * tj + 4 * q4))
                                  : f32x4_t{egL, egL, egL, egL};
            St[tj] = mma32(mma32(mma32(St[tj] * eg, ah, bhi), ah, blo), al, bhi);
            if (dual) Sp[tj] = mma32(mma32(mma32(Sp[tj] * eg, ah, bhi2), ah, blo2), al, bhi2);
        }
        // this wave's part of the next record is in LDS (the DMA precedes the saved-state
        // stores, and the memory counter completes in order)
        if (!SPLIT && ckpt) vm_wait_n<TJ>();
        else vm_wait0();
        __syncthreads();  // every wave's part is, and nobody still reads this one
    }
    if (!SPLIT) {
        if (ckpt) save(nchunk);
#pragma unroll
        for (int tj = 0; tj < TJ; tj++)
#pragma unroll
            for (int e = 0; e < 4; e++) sT[bh * NN + i_own * ei + (16 * tj + 4 * q4 + e) * ej] = St[tj][e];
    } else {  // X_1, or U_s and Phi_s, in the internal layout (float4 per tile)
        const long o4 = ((dual ? (long)(sgm - 1) * BH : 0) + bh) * NN + (long)i_own * NK;
        float* const dst = dual ? sp.uend : sp.send0;
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            *reinterpret_cast<float4*>(dst + o4 + 16 * tj + 4 * q4) = make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
            if (dual)
                *reinterpret_cast<float4*>(sp.phi + o4 + 16 * tj + 4 * q4) =
                    make_float4(Sp[tj][0], Sp[tj][1], Sp[tj][2], Sp[tj][3]);
        }
    }
}

// ---------------------------------------------------------------------------
// The time split's fix-up, two kernels.  gdn_split_chain (one workgroup per head, N/16
// waves, wave w on rows 16w .. 16w+15) chains X_{s+1} = X_s Phi_s + U_s in LDS on the
// matrix cores (split-bf16 operands), storing X_{s+1} over U_s (which only it reads; the
// same lane reads each U element before writing it) and X_k as sT in the caller's
// layout.  Phi_s (as split B operands in LDS) and U_s (registers) come one step ahead.  gdn_split_y then forms y_t = y0_t + X_s z_t for every chunk of segments
// 1 .. k-1: workgroup (chunk group, head), wave w keeps output columns 16w .. 16w+15
// (rows of X_s as its B operand in registers); per chunk the z tile is turned into rows in
// LDS, y0 comes in the accumulator layout, o leaves in whole rows through LDS.
// ---------------------------------------------------------------------------
constexpr int GFY = 8;  // chunks per gdn_split_y workgroup (2 measured slower: 21.6 against 19.3 us)
__device__ __forceinline__ void op8f(const float* p, uint4& hi, uint4& lo) {  // 8 floats, split
    const float4 x0 = *reinterpret_cast<const float4*>(p), x1 = *reinterpret_cast<const float4*>(p + 4);
    const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    pack8(v, hi, lo);
}
// X_s of segment s >= 1: X_1 in send0, X_s (s >= 2) in the U_{s-1} slot
__device__ __forceinline__ const float* seg_state(const GdnSplit& sp, int BH, int bh, int s, long NN) {
    return s == 1 ? sp.send0 + bh * NN : sp.uend + ((long)(s - 2) * BH + bh) * NN;
}

template <int NK>
__global__ __launch_bounds__(64 * (NK / 16)) void gdn_split_chain(int BH, int kv, GdnSplit sp, float* __restrict__ sT) {
    constexpr int KS = NK / 32, TJ = NK / 16, XR = NK + 4, NT = 64 * TJ;
    __shared__ float st[NK * XR];              // X_s [i][j]
    __shared__ uint4 fr[TJ * KS * 2 * 64];     // Phi_s as split B operands [n][t][hi, lo][lane]
    const int bh = blockIdx.x, tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    // Fragment entries (n, t, lane') = KS per thread, number v*NT + tid: Phi[32t + 8q' + e][16n + r']
    // for e = 0..7, loaded a step ahead and split once here, not by every wave.  (Plain
    // float arrays in macros: arrays behind lambdas end up in scratch memory.)
    float pv[KS][8];
    float uf[TJ][4];  // U_u[16w + 4q + e][16n + r16]
#define GDN_CHAIN_LOAD(u_)                                                                                    \
    do {                                                                                                      \
        const long ol_ = ((long)((u_) - 1) * BH + bh) * NN;                                                   \
        _Pragma("unroll") for (int v = 0; v < KS; v++) {                                                      \
            const int x_ = v * NT + tid, l_ = x_ & 63, t_ = (x_ >> 6) % KS, n_ = (x_ >> 6) / KS;              \
            _Pragma("unroll") for (int e = 0; e < 8; e++)                                                     \
                pv[v][e] = sp.phi[ol_ + (32 * t_ + 8 * (l_ >> 4) + e) * NK + 16 * n_ + (l_ & 15)];            \
        }                                                                                                     \
        _Pragma("unroll") for (int n = 0; n < TJ; n++)                                                        \
            _Pragma("unroll") for (int e = 0; e < 4; e++) uf[n][e] = sp.uend[ol_ + (16 * w + 4 * q + e) * NK + 16 * n + r16]; \
    } while (0)
#define GDN_CHAIN_STAGE()                                                                                     \
    do {                                                                                                      \
        _Pragma("unroll") for (int v = 0; v < KS; v++) {                                                      \
            const int x_ = v * NT + tid, l_ = x_ & 63, f_ = x_ >> 6;                                          \
            uint4 h_, lo_;                                                                                    \
            pack8(pv[v], h_, lo_);                                                                            \
            fr[(2 * f_) * 64 + l_] = h_;                                                                      \
            fr[(2 * f_ + 1) * 64 + l_] = lo_;                                                                 \
        }                                                                                                     \
    } while (0)
#pragma unroll
    for (int u = 0; u < NK / 16; u++) {  // rows 16w .. 16w+15 of X_1 (float4 u*64 + lane of the strip)
        const int f = 4 * (u * 64 + lane), r = 16 * w + f / NK, c = f % NK;
        *reinterpret_cast<float4*>(&st[r * XR + c]) = *reinterpret_cast<const float4*>(sp.send0 + bh * NN + r * NK + c);
    }
    GDN_CHAIN_LOAD(1);
    GDN_CHAIN_STAGE();
    __syncthreads();
    for (int u = 1; u < sp.k; u++) {  // X_{u+1} = X_u Phi_u + U_u, this wave's rows
        const long ob = ((long)(u - 1) * BH + bh) * NN;
        float acc0[TJ][4];
#pragma unroll
        for (int n = 0; n < TJ; n++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc0[n][e] = uf[n][e];
        if (u + 1 < sp.k) GDN_CHAIN_LOAD(u + 1);  // the next step's operands, in flight during this one
        uint4 ah[KS], al[KS];  // A operand X_u: lane (q, r16) holds X_u[16w + r16][32t + 8q .. +7]
#pragma unroll
        for (int t = 0; t < KS; t++) op8f(&st[(16 * w + r16) * XR + 32 * t + 8 * q], ah[t], al[t]);
        wave_lds_fence();  // (the strip is overwritten below)
        // the TJ output tiles' products interleaved (independent accumulator chains)
        f32x4_t acc[TJ];
#pragma unroll
        for (int n = 0; n < TJ; n++) acc[n] = f32x4_t{acc0[n][0], acc0[n][1], acc0[n][2], acc0[n][3]};
#pragma unroll
        for (int t = 0; t < KS; t++)
#pragma unroll
            for (int n = 0; n < TJ; n++) {
                const uint4 bhv = fr[(2 * (n * KS + t)) * 64 + lane], blv = fr[(2 * (n * KS + t) + 1) * 64 + lane];
                acc[n] = mma32(acc[n], ah[t], bhv);
                acc[n] = mma32(acc[n], ah[t], blv);
                acc[n] = mma32(acc[n], al[t], bhv);
            }
#pragma unroll
        for (int n = 0; n < TJ; n++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                st[(16 * w + 4 * q + e) * XR + 16 * n + r16] = acc[n][e];
                if (u + 1 < sp.k) sp.uend[ob + (16 * w + 4 * q + e) * NK + 16 * n + r16] = acc[n][e];  // X_{u+1}
            }
        __syncthreads();  // everyone is done with Phi_u
        if (u + 1 < sp.k) GDN_CHAIN_STAGE();
        __syncthreads();  // (and, after the last step, every row of X_k is in st)
    }
#undef GDN_CHAIN_LOAD
#undef GDN_CHAIN_STAGE
    // sT = X_k in the caller's layout, whole rows: float4 number v*NT + tid of row a,
    // columns c .. c+3 (kv: sT[a = j][c = i] = X[i][j], read down a column of st)
#pragma unroll
    for (int v = 0; v < NK * NK / 4 / NT; v++) {
        const int f = 4 * (v * NT + tid), a = f / NK, c = f % NK;
        const float4 x = kv ? make_float4(st[c * XR + a], st[(c + 1) * XR + a], st[(c + 2) * XR + a], st[(c + 3) * XR + a])
                            : *reinterpret_cast<const float4*>(&st[a * XR + c]);
        *reinterpret_cast<float4*>(sT + bh * NN + f) = x;
    }
}

template <int NK, typename TO>
__global__ __launch_bounds__(64 * (NK / 16)) void gdn_split_y(int Tn, int H, int BH, GdnSplit sp, TO* __restrict__ o) {
    constexpr int KS = NK / 32, TJ = NK / 16, XR = NK + 4, NT = 64 * TJ;
    __shared__ float zt[GC * XR];    // the chunk's z tile as rows [t][j]
    __shared__ TO yt[GC * NK];       // its o tile [t][i]
    const int ngy = (sp.m + GFY - 1) / GFY;  // chunk groups per segment
    const int sgm = 1 + blockIdx.x / ngy, cg = blockIdx.x % ngy, bh = blockIdx.y, bb = bh / H, h = bh - bb * H;
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    // B operand X_s^T for output columns 16w .. 16w+15: lane (q, r16) holds X_s[16w + r16][32t + 8q .. +7]
    const float* const X = seg_state(sp, BH, bh, sgm, NN);
    uint4 bhv[KS], blv[KS];
#pragma unroll
    for (int t = 0; t < KS; t++) op8f(X + (16 * w + r16) * NK + 32 * t + 8 * q, bhv[t], blv[t]);
    // this group's chunks that hold steps; each chunk's tiles are loaded one chunk ahead
    const int cfirst = sp.m0 + (sgm - 1) * sp.m;  // the segment's first chunk
    const int cend = min(min(sp.m, (cg + 1) * GFY), (Tn + GC - 1) / GC - cfirst);
    const long tile0 = (((long)(sgm - 1) * BH + bh) * sp.m) * TJ * 64;  // float4 index of the segment's tiles
    float4 zn = {}, yn = {};  // float4 tid of the z tile; y0[4q + e][16w + r16]
    auto load = [&](int c) {
        zn = reinterpret_cast<const float4*>(sp.z)[tile0 + (long)c * TJ * 64 + tid];
        yn = reinterpret_cast<const float4*>(sp.y0)[tile0 + (long)c * TJ * 64 + w * 64 + lane];
    };
    if (cg * GFY < cend) load(cg * GFY);
    for (int c = cg * GFY; c < cend; c++) {  // (block-uniform)
        const float4 zc = zn, x = yn;
        if (c + 1 < cend) load(c + 1);
        {   // z tile: float4 tid (row block tid / 64, lane tid % 64) holds z[4q' + e][16 (tid / 64) + r']
            float* const d = zt + 4 * ((tid >> 4) & 3) * XR + 16 * (tid >> 6) + (tid & 15);
            d[0] = zc.x, d[XR] = zc.y, d[2 * XR] = zc.z, d[3 * XR] = zc.w;
        }
        __syncthreads();
        f32x4_t acc = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int t = 0; t < KS; t++) {
            uint4 ah, al;  // A operand Z: lane (q, r16) holds z[r16][32t + 8q .. +7]
            op8f(zt + r16 * XR + 32 * t + 8 * q, ah, al);
            acc = mma32(acc, ah, bhv[t]);
            acc = mma32(acc, ah, blv[t]);
            acc = mma32(acc, al, bhv[t]);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) io<TO>::st(yt, (4 * q + e) * NK + 16 * w + r16, acc[e]);
        __syncthreads();
        // 16 rows of NK outputs in 16-byte pieces
        constexpr int PR = NK * (int)sizeof(TO) / 16;
        for (int idx = tid; idx < GC * PR; idx += NT) {
            const int rr = idx / PR, pc = idx - rr * PR, tabs = GC * (cfirst + c) + rr;
            if (tabs < Tn)
                reinterpret_cast<uint4*>(o + ((long)(bb * Tn + tabs) * H + h) * NK)[pc] =
                    reinterpret_cast<const uint4*>(yt + rr * NK)[pc];
        }
        __syncthreads();  // (zt and yt are rewritten by the next chunk)
    }
}

// chunks per segment for k segments of n chunks
// Lengths of k segments over n chunks: m0 = n - (k-1) m chunks go to segment 0 with m
// minimising max(GDN_R0 m0, GDN_R1 m), every segment non-empty.  Unlike the WKV7 forward's,
// the scan's tick hardly grows with the second state: at the teacher's geometry (T=2048,
// 32 heads, K=V=128) equal lengths took 186.8 us per call against 202.8 / 210.0 / 220.9
// with segment 0 given 1.4 / 1.8 / 2.2 times the others' chunks.
constexpr int GDN_R0 = 1, GDN_R1 = 1;
void gdn_split_lengths(int n, int k, int& m0, int& m) {
    int best = 1 << 30;
    m0 = n, m = 0;
    for (int mm = 1; n - (k - 1) * mm >= 1; mm++) {
        const int r = n - (k - 1) * mm, cost = max(GDN_R0 * r, GDN_R1 * mm);
        if (cost < best) best = cost, m0 = r, m = mm;
    }
}
}  // namespace

template <bool PK>
static size_t records(int B, int T, int H, int N) {
    const size_t rec = N == 128 ? GdnRec<128, PK>::BYTES : GdnRec<64, PK>::BYTES;
    return (size_t)B * H * ((T + GC - 1) / GC) * rec;
}
size_t gdn_forward_workspace(int B, int T, int H, int N) { return records<false>(B, T, H, N); }
// Segments of the time-split scan: with at least 8 chunks, as many as fit one workgroup
// per CU (B*H*N/64 per segment), at most 4, each with at least one chunk; 1 = no split.
int gdn_split_segments(int B, int T, int H, int N, int cus) {
    const int n = (T + GC - 1) / GC, per = B * H * (N / 64);
    if (n < 8 || per < 1) return 1;
    return max(1, min(min(4, cus / per), n));
}
template <bool PK>
static size_t split_workspace(int B, int T, int H, int N, int cus) {
    const int k = gdn_split_segments(B, T, H, N, cus);
    if (k < 2) return records<PK>(B, T, H, N);
    int m0, mi;
    gdn_split_lengths((T + GC - 1) / GC, k, m0, mi);
    const size_t m = mi, BH = (size_t)B * H, NN = (size_t)N * N;
    const size_t recs = (records<PK>(B, T, H, N) + 255) / 256 * 256;
    return recs + BH * ((2 * k - 1) * NN + 2 * (k - 1) * m * GC * N) * sizeof(float);
}
size_t gdn_forward_workspace_split(int B, int T, int H, int N, int cus) {
    return split_workspace<false>(B, T, H, N, cus);
}
size_t wkv7_rec_workspace(int B, int T, int H, int N) { return records<true>(B, T, H, N); }
size_t wkv7_rec_workspace_split(int B, int T, int H, int N, int cus) { return split_workspace<true>(B, T, H, N, cus); }

// Row groups per head for the scan: groups of four waves (64 value rows).  Measured at
// B=1, T=2048 (MI355X): N=128 in 2 groups 0.248 ms against 0.279 (1), 0.292 (4) and
// 0.380 (8); N=64 in 1 group 0.168 ms against 0.192 (2) -- every group moves the whole
// record into its LDS, and groups of fewer waves wait on that more than they gain.
static int gdn_row_groups(int N) { return N / 64; }  // (256 lanes each: the kernel's bound)

// The scan over the records at ws: in one pass (with saved states when ckpt), or cut in
// time when cus allows at least two segments and ws_bytes covers the split's buffers.
template <int NK, typename TO, bool PK>
static void scan_records(int B, int T, int H, int kv, const float* s0, TO* o, float* sT, float* ckpt, void* ws,
                         size_t ws_bytes, int cus, hipStream_t stream) {
    const int nchunk = (T + GC - 1) / GC, BH = B * H;
    const int rgs = gdn_row_groups(NK), lanes = 64 * (NK / 16) / rgs;
    const uint8_t* const recs = static_cast<const uint8_t*>(ws);
    const int k = ckpt ? 1 : gdn_split_segments(B, T, H, NK, cus);
    if (k < 2 || ws_bytes < split_workspace<PK>(B, T, H, NK, cus)) {
        hipLaunchKernelGGL((gdn_scan<NK, TO, false, PK>), dim3(BH * rgs), dim3(lanes), 0, stream, T, H, BH, kv, s0, o,
                           sT, recs, GdnSplit{}, ckpt);
        return;
    }
    // the time split: buffers after the records
    GdnSplit sp;
    sp.k = k;
    gdn_split_lengths(nchunk, k, sp.m0, sp.m);
    const size_t NN = (size_t)NK * NK, per = (size_t)(k - 1) * BH;
    float* const base = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + (records<PK>(B, T, H, NK) + 255) / 256 * 256);
    sp.send0 = base, sp.uend = base + BH * NN, sp.phi = sp.uend + per * NN;
    sp.y0 = sp.phi + per * NN, sp.z = sp.y0 + per * sp.m * GC * NK;
    hipLaunchKernelGGL((gdn_scan<NK, TO, true, PK>), dim3(k * BH * rgs), dim3(lanes), 0, stream, T, H, BH, kv, s0, o,
                       sT, recs, sp, nullptr);
    hipLaunchKernelGGL((gdn_split_chain<NK>), dim3(BH), dim3(64 * (NK / 16)), 0, stream, BH, kv, sp, sT);
    // chunk groups of segments 1 .. k-1; heads along y
    hipLaunchKernelGGL((gdn_split_y<NK, TO>), dim3((k - 1) * ((sp.m + GFY - 1) / GFY), BH), dim3(64 * (NK / 16)), 0,
                       stream, T, H, BH, sp, o);
}
template <int NK, typename TI>
static void launch_gdn(const Gdn& p) {
    const int nchunk = (p.T + GC - 1) / GC, BH = p.B * p.H;
    hipLaunchKernelGGL((gdn_prep<NK, TI>), dim3(nchunk, BH), dim3(64), 0, p.stream, p.T, p.H, p.qk_norm,
                       static_cast<const TI*>(p.q), static_cast<const TI*>(p.k), static_cast<const TI*>(p.v), p.g,
                       p.beta, static_cast<uint8_t*>(p.ws));
    scan_records<NK, TI, false>(p.B, p.T, p.H, p.kv, p.s0, static_cast<TI*>(p.o), p.sT, p.ckpt, p.ws, p.ws_bytes,
                                p.cus, p.stream);
}
void launch_gdn_forward(const Gdn& p) {
    if (p.N == 128) {
        if (p.dtype == 0) launch_gdn<128, bf16_t>(p);
        else launch_gdn<128, float>(p);
    } else {
        if (p.dtype == 0) launch_gdn<64, bf16_t>(p);
        else launch_gdn<64, float>(p);
    }
}

// The WKV7 forward on records: bf16, N = 128, flags 0 ([value][key] states), a
// workspace of at least wkv7_rec_workspace bytes; saved states (ckpt) in the step-serial
// kernels' [value][key] order.
void launch_wkv7_rec_forward(const Fwd& p, int cus) {
    const int nchunk = (p.T + GC - 1) / GC, BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_rec_prep<128>), dim3(nchunk, BH), dim3(64), 0, p.stream, p.T, p.H,
                       static_cast<const bf16_t*>(p.r), static_cast<const bf16_t*>(p.w), static_cast<const bf16_t*>(p.k),
                       static_cast<const bf16_t*>(p.v), static_cast<const bf16_t*>(p.a), static_cast<const bf16_t*>(p.b),
                       static_cast<uint8_t*>(p.ws));
    scan_records<128, bf16_t, true>(p.B, p.T, p.H, 0, p.s0, static_cast<bf16_t*>(p.y), p.sT, p.ckpt, p.ws, p.ws_bytes,
                                    cus, p.stream);
}

}  // namespace wkv7
