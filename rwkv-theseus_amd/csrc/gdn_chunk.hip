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
#include "wkv7_io.h"
#include "wkv7_launch.h"

namespace wkv7 {
namespace {

constexpr int GC = 16;  // chunk length

// One chunk's record in the workspace (byte offsets; 256-byte aligned records).
template <int NK>
struct GdnRec {
    static constexpr int KS = NK / 32, TJ = NK / 16;
    static constexpr size_t PF = 0;                                // [KS][hi, lo][64 lanes] uint4
    static constexpr size_t P2F = PF + (size_t)KS * 2 * 64 * 16;   // same for P2
    static constexpr size_t UF = P2F + (size_t)KS * 2 * 64 * 16;   // [TJ][hi, lo][64] uint4
    static constexpr size_t QF = UF + (size_t)TJ * 2 * 64 * 16;    // [Q'^T hi, lo, Q2^T hi, lo][64] uint2
    static constexpr size_t VF = QF + 4 * 64 * 8;                  // [TJ row blocks][hi, lo][64] uint2
    static constexpr size_t EL = VF + (size_t)TJ * 2 * 64 * 8;     // e^{gamma_L}
    static constexpr size_t BYTES = EL + 256;
    static constexpr int DMA_BLOCKS = (int)((BYTES + 1023) / 1024);  // 1 KB LDS DMA blocks
};
static_assert(GdnRec<128>::BYTES % 256 == 0 && GdnRec<64>::BYTES % 256 == 0, "record alignment");

// four consecutive elements as float
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4(const bf16_t* p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
}

// LDS DMA of 1 KB: lane l moves 16 bytes from the buffer at soff + voff to lds_off + 16 l
// (lds_off: byte address in LDS, made scalar for M0).  Issued from inline asm like
// wkv7_io.h's dma16, so the compiler does not wait for it; vm_wait0 does.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_kb(uint32_t lds_off, i32x4_t rs, uint32_t voff, uint32_t soff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_off);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(m0), "v"(voff), "s"(rs), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop

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

    const bool tv = r16 < L;
    const float gt = tv ? g[(tok0 + r16) * H + h] : 0.f;
    const float bt = tv ? beta[(tok0 + r16) * H + h] : 0.f;
    const float gam = row_prefix_sum(gt);
    const float gm1 = row_prev(gam, 0.f);
    const float gL = row_last(gam);
    // rows of k and q (zero past the end); q kept for R~
    float kr[KS][8], qr[KS][8];
    float ssk = 0.f, ssq = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int c0 = 32 * ks + 4 * q4;
        if (tv) {
            const float4 a = ld4(k + row(r16) + c0), b = ld4(k + row(r16) + c0 + 16);
            const float4 x = ld4(q + row(r16) + c0), y = ld4(q + row(r16) + c0 + 16);
            kr[ks][0] = a.x, kr[ks][1] = a.y, kr[ks][2] = a.z, kr[ks][3] = a.w;
            kr[ks][4] = b.x, kr[ks][5] = b.y, kr[ks][6] = b.z, kr[ks][7] = b.w;
            qr[ks][0] = x.x, qr[ks][1] = x.y, qr[ks][2] = x.z, qr[ks][3] = x.w;
            qr[ks][4] = y.x, qr[ks][5] = y.y, qr[ks][6] = y.z, qr[ks][7] = y.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) kr[ks][e] = qr[ks][e] = 0.f;
        }
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
    __syncthreads();  // gsh
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
            vv[e] = t < L ? gsh[2][t] * io<TI>::ld(v, row(t) + 16 * rb + r16) : 0.f;
        }
        const Pk pv = pk(vv);
        uint2* vf = reinterpret_cast<uint2*>(rec + R::VF) + (size_t)(2 * rb) * 64 + lane;
        vf[0] = pv.h;
        vf[64] = pv.l;
    }
    // per pair of 16-key tiles (one K-step): P, P2 and the update operands
    const float egam = __expf(gam) * rs;  // R~ row scale of token r16
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
                const float kv = t < L ? io<TI>::ld(k, row(t) + 16 * tj + r16) * gsh[3][t] : 0.f;
                at[e] = kv * __expf(gsh[1][t]);
                bhat[e] = -gsh[2][t] * kv * __expf(gL - gsh[1][t]);
                khat[e] = kv * __expf(gL - gsh[0][t]);
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
// Each head's chunks in order.  A head's value rows are split over `row groups`
// (workgroups rg * BH + bh, so that with BH a multiple of 8 a head's groups share an
// XCD and its L2); wave w of group rg keeps the 16 rows of block rb = rg * NW + w,
// St[tj][e] = X[i_own][16tj + 4q4 + e] (as the WKV7 forward's consumers).  States
// s0 / sT are [key][value] when kv (GDN's layout), else [value][key].  Records are
// double-buffered in LDS: chunk c + 1's comes in by DMA (each wave moves every NW-th
// kilobyte) while chunk c's is read; one barrier per chunk.
// ---------------------------------------------------------------------------
template <int NK, typename TO>
__global__ __launch_bounds__(256) void gdn_scan(int Tn, int H, int BH, int kv, const float* __restrict__ s0,
                                                   TO* __restrict__ o, float* __restrict__ sT,
                                                   const uint8_t* __restrict__ ws) {
    using R = GdnRec<NK>;
    constexpr int KS = R::KS, TJ = R::TJ;
    __shared__ __attribute__((aligned(1024))) uint8_t recs[2][R::DMA_BLOCKS * 1024];
    const int bh = blockIdx.x % BH, rg = blockIdx.x / BH, bb = bh / H, h = bh - bb * H;
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // waves per group (the host launches whole waves, at least one: the DMA loop steps by NW)
    const int NW = max(1, __builtin_amdgcn_readfirstlane((int)(blockDim.x >> 6)));
    const int lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
    const int rb = rg * NW + wv, i_own = 16 * rb + r16;
    const long NN = (long)NK * NK, ei = kv ? 1 : NK, ej = kv ? NK : 1;
    const int nchunk = (Tn + GC - 1) / GC;
    // this head's records (the host keeps them under 4 GB, so 32-bit offsets reach them)
    const i32x4_t rs = dma_rsrc(ws + (size_t)bh * nchunk * R::BYTES, (uint32_t)((size_t)nchunk * R::BYTES));
    auto fetch = [&](int c, int buf) {
        uint32_t so = (uint32_t)((size_t)c * R::BYTES);
        asm volatile("" : "+s"(so));  // (an SGPR even where it is a constant)
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)recs[buf];
        for (int j = wv; j < R::DMA_BLOCKS; j += NW) dma_kb(base + 1024 * j, rs, (uint32_t)(1024 * j + 16 * lane), so);
    };
    fetch(0, 0);
    f32x4_t St[TJ];
#pragma unroll
    for (int tj = 0; tj < TJ; tj++)
#pragma unroll
        for (int e = 0; e < 4; e++) St[tj][e] = s0[bh * NN + i_own * ei + (16 * tj + 4 * q4 + e) * ej];
    vm_wait0();
    __syncthreads();
    for (int c = 0; c < nchunk; c++) {
        if (c + 1 < nchunk) fetch(c + 1, (c + 1) & 1);
        const uint8_t* const rec = recs[c & 1];
        const int t0 = c * GC, L = min(GC, Tn - t0);
        const long tok0 = (long)bb * Tn + t0;
        // SA = P X0^T and Y = P2 X0^T over the keys (permuted K=32 steps)
        f32x4_t sa = zero4(), yy = zero4();
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
#pragma unroll
        for (int e = 0; e < 4; e++) {  // y[t][i_own], t = 4q4 + e
            const int t = 4 * q4 + e;
            if (t < L) io<TO>::st(o, ((tok0 + t) * H + h) * NK + i_own, yy[e]);
        }
        // X^T <- e^{gamma_L} X^T + [B^^T K^^T] [SA; V]   (K = 32: SA rows, then V rows)
        uint2 sah, sal;
        pack4(sa, sah, sal);
        const uint4 bhi = cat(sah, vh), blo = cat(sal, vl);
        const float egL = *reinterpret_cast<const float*>(rec + R::EL);
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            const uint4* uf = reinterpret_cast<const uint4*>(rec + R::UF) + (2 * tj) * 64 + lane;
            const uint4 ah = uf[0], al = uf[64];
            St[tj] = mma32(mma32(mma32(St[tj] * egL, ah, bhi), ah, blo), al, bhi);
        }
        vm_wait0();      // this wave's part of the next record is in LDS
        __syncthreads();  // every wave's part is, and nobody still reads this one
    }
#pragma unroll
    for (int tj = 0; tj < TJ; tj++)
#pragma unroll
        for (int e = 0; e < 4; e++) sT[bh * NN + i_own * ei + (16 * tj + 4 * q4 + e) * ej] = St[tj][e];
}

}  // namespace

size_t gdn_forward_workspace(int B, int T, int H, int N) {
    const size_t rec = N == 128 ? GdnRec<128>::BYTES : GdnRec<64>::BYTES;
    return (size_t)B * H * ((T + GC - 1) / GC) * rec;
}
// Row groups per head for the scan: groups of four waves (64 value rows).  Measured at
// B=1, T=2048 (MI355X): N=128 in 2 groups 0.248 ms against 0.279 (1), 0.292 (4) and
// 0.380 (8); N=64 in 1 group 0.168 ms against 0.192 (2) -- every group moves the whole
// record into its LDS, and groups of fewer waves wait on that more than they gain.
static int gdn_row_groups(int N) { return N / 64; }  // (256 lanes each: the kernel's bound)
template <int NK, typename TI>
static void launch_gdn(const Gdn& p) {
    const int nchunk = (p.T + GC - 1) / GC, BH = p.B * p.H;
    const int rgs = gdn_row_groups(NK), lanes = 64 * (NK / 16) / rgs;
    hipLaunchKernelGGL((gdn_prep<NK, TI>), dim3(nchunk, BH), dim3(64), 0, p.stream, p.T, p.H, p.qk_norm,
                       static_cast<const TI*>(p.q), static_cast<const TI*>(p.k), static_cast<const TI*>(p.v), p.g,
                       p.beta, static_cast<uint8_t*>(p.ws));
    hipLaunchKernelGGL((gdn_scan<NK, TI>), dim3(BH * rgs), dim3(lanes), 0, p.stream, p.T, p.H, BH, p.kv, p.s0,
                       static_cast<TI*>(p.o), p.sT, static_cast<const uint8_t*>(p.ws));
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

}  // namespace wkv7
