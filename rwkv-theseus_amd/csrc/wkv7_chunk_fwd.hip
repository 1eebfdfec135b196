// Chunked WKV7 forward on the matrix cores (bf16 I/O, fp32 state, N = 64).
//
// Algebra (per batch*head, chunk of C = 16 steps, local t = 0..C-1; i = value
// row, j = key column; g_t = cumulative log-decay inside the chunk, gp_t =
// g_{t-1}, gL = g_{C-1}):
//   A~ = a*e^{gp},  R~ = r*e^{g},  B- = b*e^{-g},  K- = k*e^{-g},
//   B^ = b*e^{gL-g},  K^ = k*e^{gL-g}
//   Aab = tril_strict(A~ B-^T)  Aak = tril_strict(A~ K-^T)
//   Brb = tril(R~ B-^T)          Brk = tril(R~ K-^T)
//   Ti  = (I - Aab)^{-1};  P = Ti A~;  Q' = Ti Aak;  P2 = R~ + Brb P;  Q2 = Brk + Brb Q'
//   SA  = P S0^T + Q' V          (SA[t] = S_{t-1} a_t, the "sa" of the recurrence)
//   Y   = P2 S0^T + Q2 V
//   S_C = S0 diag(e^{gL}) + SA^T B^ + V^T K^
// which is the step recurrence of theseus/wkv7.py:16-28 rewritten in the
// WY / diagonal-plus-low-rank chunk form (exact in exact arithmetic).
//
// Mapping: one 256-lane workgroup per (b,h).  Everything that does not
// depend on the state (the chunk operands above) is built cooperatively in
// LDS; then each wave w owns value rows 16w..16w+15 and advances its slice of
// the state with no barrier: value rows never interact, so S^T (rows j,
// columns i) stays in that wave's accumulator registers for the whole
// sequence and feeds the next chunk's MFMAs directly as B operands.
#include "wkv7_launch.h"
#include "wkv7_mfma.h"

namespace wkv7 {
namespace {

constexpr int CH = CKPT;  // chunk length
constexpr int NK = 64;    // head size of this kernel
constexpr int LD64 = 72;  // row stride of [16][64] operand planes
constexpr int LD16 = 24;  // row stride of [64][16] and [16][16] operand planes

struct FwdLds {
    uint16_t raw[6][CH * LD64];                   // r,w,k,v,a,b bf16 bits, [t][j]
    uint16_t At[2][CH * LD64], Rt[2][CH * LD64];  // A~, R~ [t][j]
    uint16_t Bb[2][CH * LD64], Kb[2][CH * LD64];  // B-, K- [s][j]
    uint16_t P[2][CH * LD64], P2[2][CH * LD64];   // P, P2 [t][j]
    uint16_t AtT[2][NK * LD16];                   // A~^T [j][s]
    uint16_t BhT[2][NK * LD16], KhT[2][NK * LD16];  // B^^T, K^^T [j][t]
    uint16_t VT[NK * LD16];                       // V^T [i][t] (exact bf16)
    uint16_t Ti[2][CH * LD16], Brb[2][CH * LD16];  // [t][s]
    uint16_t Q1[2][CH * LD16], Q2[2][CH * LD16];   // Q', Q2 [t][s]
    float Brk[CH * CH];   // fp32 [t][s]
    float part[8][NK];
    float egL[NK];
};

__device__ __forceinline__ Op op(uint16_t (&a)[2][CH * LD64]) { return Op{a[0], a[1], LD64}; }
__device__ __forceinline__ Op op16(uint16_t (&a)[2][NK * LD16]) { return Op{a[0], a[1], LD16}; }
__device__ __forceinline__ Op opc(uint16_t (&a)[2][CH * LD16]) { return Op{a[0], a[1], LD16}; }

}  // namespace

__global__ __launch_bounds__(256) void chunk_forward_bf16(
    int Tn, int H, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
    const bf16_t* __restrict__ b, const float* __restrict__ s0, bf16_t* __restrict__ y,
    float* __restrict__ sT, float* __restrict__ ckpt) {
    __shared__ FwdLds sm;
    const int bh = blockIdx.x, bb = bh / H, h = bh % H;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    const long ncp = ckpt_count(Tn);
    const int i_own = 16 * wv + r16;  // value row this lane holds in the state registers

    const Op At = op(sm.At), Rt = op(sm.Rt), Bb = op(sm.Bb), Kb = op(sm.Kb), P = op(sm.P), P2 = op(sm.P2);
    const Op AtT = op16(sm.AtT), BhT = op16(sm.BhT), KhT = op16(sm.KhT);
    const Op Ti = opc(sm.Ti), Brb = opc(sm.Brb), Q1 = opc(sm.Q1), Q2 = opc(sm.Q2);

    // S^T tiles: St[tj][e] = S[i_own][16*tj + 4q + e]
    f32x4_t St[4];
#pragma unroll
    for (int tj = 0; tj < 4; tj++) {
        const long off = bh * NN + (long)i_own * NK + 16 * tj + 4 * q;
        const float4 x = *reinterpret_cast<const float4*>(s0 + off);
        St[tj] = f32x4_t{x.x, x.y, x.z, x.w};
        if (ckpt) *reinterpret_cast<float4*>(ckpt + bh * ncp * NN + (long)i_own * NK + 16 * tj + 4 * q) = x;
    }

    const int nchunk = (Tn + CH - 1) / CH;
    // raw chunk inputs are prefetched into registers one chunk ahead:
    // lane-slot m covers tensor id>>7, row (id>>3)&15, 8-element segment id&7
    uint4 pre[3];
    auto load_chunk = [&](int cc) {
        const int tb = cc * CH, Lc = min(CH, Tn - tb);
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const int id = tid + 256 * m, ts = id >> 7, row = (id >> 3) & 15, seg = id & 7;
            const bf16_t* src = ts == 0 ? r : ts == 1 ? w : ts == 2 ? k : ts == 3 ? v : ts == 4 ? a : b;
            pre[m] = make_uint4(0, 0, 0, 0);
            if (row < Lc) pre[m] = *reinterpret_cast<const uint4*>(src + ((long)(bb * Tn + tb + row) * H + h) * NK + 8 * seg);
        }
    };
    auto store_raw = [&]() {
#pragma unroll
        for (int m = 0; m < 3; m++) {
            const int id = tid + 256 * m, ts = id >> 7, row = (id >> 3) & 15, seg = id & 7;
            *reinterpret_cast<uint4*>(&sm.raw[ts][row * LD64 + 8 * seg]) = pre[m];
        }
    };
    load_chunk(0);
    store_raw();
    if (nchunk > 1) load_chunk(1);
    for (int c = 0; c < nchunk; c++) {
        const int t0 = c * CH, L = min(CH, Tn - t0);
        // ---- A1: inputs of chunk c were put in LDS during the previous chunk ----
        __syncthreads();  // raw ready; previous chunk's state phase done with all operands
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
#pragma unroll
                for (int x = 0; x < 2; x++) {
                    const float g = pre_[x] + lw[0][x] + (u ? lw[1][x] : 0.f), gp = g - lw[u][x];
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
            put_row(Rt, vrt);
            put_row(Bb, vbb);
            put_row(Kb, vkb);
            put_col(AtT, vat);
            put_col(BhT, vbh);
            put_col(KhT, vkh);
            {
                const uint32_t v0 = *reinterpret_cast<const uint32_t*>(&sm.raw[3][tb * LD64 + j0]);
                const uint32_t v1 = *reinterpret_cast<const uint32_t*>(&sm.raw[3][(tb + 1) * LD64 + j0]);
                *reinterpret_cast<uint32_t*>(&sm.VT[j0 * LD16 + tb]) = (v0 & 0xffffu) | (v1 << 16);
                *reinterpret_cast<uint32_t*>(&sm.VT[(j0 + 1) * LD16 + tb]) = (v0 >> 16) | (v1 & 0xffff0000u);
            }
            if (tp == 0) {
                sm.egL[j0] = __expf(tot[0]);
                sm.egL[j0 + 1] = __expf(tot[1]);
            }
        }
        __syncthreads();
        // ---- A3: chunk matrices; wave 0: Aab, Aab^T -> Ti; wave 1: Aak; wave 2: Brb; wave 3: Brk ----
        f32x4_t cm = zero4();
        if (wv == 0) {
            f32x4_t L = mma_k32<2>(zero4(), At, 0, Bb, 0, 0, lane);
            f32x4_t LT = mma_k32<2>(zero4(), Bb, 0, At, 0, 0, lane);
#pragma unroll
            for (int e = 0; e < 4; e++) {  // keep s < t (L), row < column (L^T)
                if (r16 >= 4 * q + e) L[e] = 0.f;
                if (r16 <= 4 * q + e) LT[e] = 0.f;
            }
            f32x4_t ti, tiT;
            tri_inverse(L, LT, lane, ti, tiT);
#pragma unroll
            for (int e = 0; e < 4; e++) Ti.put(4 * q + e, r16, ti[e]);
        } else {
            if (wv == 1) cm = mma_k32<2>(zero4(), At, 0, Kb, 0, 0, lane);
            else if (wv == 2) cm = mma_k32<2>(zero4(), Rt, 0, Bb, 0, 0, lane);
            else cm = mma_k32<2>(zero4(), Rt, 0, Kb, 0, 0, lane);
#pragma unroll
            for (int e = 0; e < 4; e++) {  // D layout: row t = 4q+e, column s = r16
                const int t = 4 * q + e, s = r16;
                if (wv == 1 ? s >= t : s > t) cm[e] = 0.f;
                if (wv == 2) Brb.put(t, s, cm[e]);
                if (wv == 3) sm.Brk[t * CH + s] = cm[e];
            }
        }
        __syncthreads();
        // ---- A5: P = Ti A~ and P2 = R~ + Brb P on key strip 16wv..; wave 1: Q' = Ti Aak, Q2 = Brk + Brb Q' ----
        {
            const int j = 16 * wv + r16;
            f32x4_t p = mma_k16(zero4(), Ti, 0, AtT, 16 * wv, 0, lane);
            f32x4_t p2;
#pragma unroll
            for (int e = 0; e < 4; e++) p2[e] = Rt.get(4 * q + e, j);
            uint2 ph, pl;
            pack4(p, ph, pl);
            {  // Brb (A, from LDS) x P (B, straight from the accumulator: rows = k)
                const uint2 ah = frag16(Brb.hi, LD16, 0, 0, lane), al = frag16(Brb.lo, LD16, 0, 0, lane);
                p2 = mma16(p2, ah, ph);
                f32x4_t c2 = mma16(zero4(), ah, pl);
                c2 = mma16(c2, al, ph);
                p2 += c2;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                P.put(4 * q + e, j, p[e]);
                P2.put(4 * q + e, j, p2[e]);
            }
            if (wv == 1) {  // cm holds Aak (rows s = 4q+e, column s' = r16): B operand as is
                uint2 ah_, al_;
                pack4(cm, ah_, al_);
                const uint2 th = frag16(Ti.hi, LD16, 0, 0, lane), tl = frag16(Ti.lo, LD16, 0, 0, lane);
                f32x4_t q1 = mma16(zero4(), th, ah_);
                f32x4_t c1 = mma16(zero4(), th, al_);
                c1 = mma16(c1, tl, ah_);
                q1 += c1;
                uint2 qh, ql;
                pack4(q1, qh, ql);
                const uint2 bh_ = frag16(Brb.hi, LD16, 0, 0, lane), bl_ = frag16(Brb.lo, LD16, 0, 0, lane);
                f32x4_t q2 = mma16(zero4(), bh_, qh);
                f32x4_t c3 = mma16(zero4(), bh_, ql);
                c3 = mma16(c3, bl_, qh);
#pragma unroll
                for (int e = 0; e < 4; e++) q2[e] += c3[e] + sm.Brk[(4 * q + e) * CH + r16];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    Q1.put(4 * q + e, r16, q1[e]);
                    Q2.put(4 * q + e, r16, q2[e]);
                }
            }
        }
        __syncthreads();
        // ---- B: state phase, wave-local (value rows i_own) ----
        // raw is dead after A2: park the prefetched chunk c+1 there and start
        // loading chunk c+2 before this phase issues its y / state stores, so
        // the next wait on the prefetch never waits on those stores
        if (c + 1 < nchunk) {
            store_raw();
            if (c + 2 < nchunk) load_chunk(c + 2);
        }
        {
            // V fragment, B operand for K=16 (rows t = 4q.., column i_own); exact in bf16
            const uint2 vfr = ld8B(&sm.VT[i_own * LD16 + 4 * q]);
            f32x4_t sa = zero4(), yy = zero4();
#pragma unroll
            for (int s = 0; s < 2; s++) {  // K = 64 over j, as 2 steps of 32 (k-slots permuted)
                float sv[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sv[e] = St[2 * s][e];
                    sv[4 + e] = St[2 * s + 1][e];
                }
                uint4 sh, sl;
                pack8(sv, sh, sl);
                const int k0 = 32 * s + 4 * q;
                const uint4 pah = cat(ld8B(&P.hi[r16 * LD64 + k0]), ld8B(&P.hi[r16 * LD64 + k0 + 16]));
                const uint4 pal = cat(ld8B(&P.lo[r16 * LD64 + k0]), ld8B(&P.lo[r16 * LD64 + k0 + 16]));
                const uint4 p2h = cat(ld8B(&P2.hi[r16 * LD64 + k0]), ld8B(&P2.hi[r16 * LD64 + k0 + 16]));
                const uint4 p2l = cat(ld8B(&P2.lo[r16 * LD64 + k0]), ld8B(&P2.lo[r16 * LD64 + k0 + 16]));
                sa = mma32(sa, pah, sh);
                sa = mma32(sa, pah, sl);
                sa = mma32(sa, pal, sh);
                yy = mma32(yy, p2h, sh);
                yy = mma32(yy, p2h, sl);
                yy = mma32(yy, p2l, sh);
            }
            {  // V part on the K=16 instruction, in its own accumulators
                const uint2 qh = frag16(Q1.hi, LD16, 0, 0, lane), ql = frag16(Q1.lo, LD16, 0, 0, lane);
                f32x4_t sv = mma16(zero4(), qh, vfr);
                sv = mma16(sv, ql, vfr);
                const uint2 q2h = frag16(Q2.hi, LD16, 0, 0, lane), q2l = frag16(Q2.lo, LD16, 0, 0, lane);
                f32x4_t yv = mma16(zero4(), q2h, vfr);
                yv = mma16(yv, q2l, vfr);
                sa += sv;
                yy += yv;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 4 * q + e;
                if (t < L) y[((long)(bb * Tn + t0 + t) * H + h) * NK + i_own].bits = f32_to_bf16(yy[e]);
            }
            // S_new^T = S^T diag(e^{gL}) + [B^^T K^^T] [SA; V]   (K = 32, slots: SA rows, V rows)
            uint2 sah, sal;
            pack4(sa, sah, sal);
            const uint4 bhi = cat(sah, vfr), blo = cat(sal, make_uint2(0, 0));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const int jr = 16 * tj + r16;  // A-fragment row (key j)
                const uint4 ah = cat(ld8B(&BhT.hi[jr * LD16 + 4 * q]), ld8B(&KhT.hi[jr * LD16 + 4 * q]));
                const uint4 al = cat(ld8B(&BhT.lo[jr * LD16 + 4 * q]), ld8B(&KhT.lo[jr * LD16 + 4 * q]));
                f32x4_t acc;
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = St[tj][e] * sm.egL[16 * tj + 4 * q + e];
                acc = mma32(acc, ah, bhi);
                f32x4_t c1 = mma32(zero4(), ah, blo);
                c1 = mma32(c1, al, bhi);
                St[tj] = acc + c1;
                if (ckpt)
                    *reinterpret_cast<float4*>(ckpt + (bh * ncp + c + 1) * NN + (long)i_own * NK + 16 * tj + 4 * q) =
                        make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
            }
        }
    }
#pragma unroll
    for (int tj = 0; tj < 4; tj++)
        *reinterpret_cast<float4*>(sT + bh * NN + (long)i_own * NK + 16 * tj + 4 * q) =
            make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
}

void launch_chunk_forward(const Fwd& p) {
    hipLaunchKernelGGL(chunk_forward_bf16, dim3(p.B * p.H), dim3(256), 0, p.stream, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.s0, (bf16_t*)p.y, p.sT, p.ckpt);
}

}  // namespace wkv7
