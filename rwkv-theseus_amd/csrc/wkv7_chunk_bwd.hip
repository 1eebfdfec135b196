// Chunked WKV7 backward on the matrix cores (bf16 I/O, fp32 state, N = 64).
//
// The forward's chunk form (see wkv7_chunk_fwd.hip for A~, R~, B-, K-, Aab,
// Aak, Brb, Brk, Ti) is differentiated per chunk.  With H = dL/dS at the chunk
// end (H = dsT for the last chunk), H' = H diag(e^{gL}), S0 the state at the
// chunk start (a saved state) and dY the chunk's output gradient:
//   SA  = Ti (A~ S0^T + Aak V)                 (SA[t] = S_{t-1} a_t)
//   Q   = Ti^T (B- H'^T + Brb^T dY)            (Q[t] = dL/d sa_t)
//   dV  = K- H'^T + Aak^T Q + Brk^T dY
//   dK  = e^{-g} o [ V H' + triu_s(V Q^T) A~ + triu(V dY^T) R~ ]
//   dB  = e^{-g} o [ SA H' + triu_s(SA Q^T) A~ + triu(SA dY^T) R~ ]
//   dR  = e^{g}  o [ dY S0 + tril(dY SA^T) B- + tril(dY V^T) K- ]
//   dA  = e^{gp} o [ Q S0 + tril_s(Q SA^T) B- + tril_s(Q V^T) K- ]
//   H_0 = H' + Q^T A~ + dY^T R~                (dL/dS at the chunk start)
// and the decay gradient uses the identity (derived from S_t = S_{t-1} D_t +
// sa_t b_t^T + v_t k_t^T)
//   dlogd_t = sum_{s>=t} (r dR - b dB - k dK)_s + sum_{s>t} (a dA)_s
//             + colsum(dsT o S_T),      dw = dlogd * (-e^{-1/2}) sig(w)(1-sig(w)),
// a reverse cumulative sum carried across chunks (r dR = R~ o [..], b dB =
// B- o [..], ...), with sig(w_t) = (g_{t-1} - g_t) / e^{-1/2}.  Together these
// equal the step adjoint of kernels/wkv7_state.cu:52-78 (checked against it on
// the CPU oracle in float64).
//
// Mapping: one 448-lane workgroup per (b,h), chunks in reverse, lock-step
// ticks of two LDS barriers (no global-memory fence).
//  * Producers (waves 4-6) build everything that depends only on a chunk's
//    inputs -- A~, R~, B-, K-, g, e^{gL}, Ti, Aak, Brb, Brk, V dY^T -- one
//    chunk each, in three phases over the three ticks before it is consumed,
//    into a 3-slot LDS ring (as the forward's producers do).  Their inputs
//    arrive by LDS DMA (global_load_lds_dwordx4) two ticks ahead, so no
//    prefetch registers are held across ticks.  Each phase is split in two
//    parts, one run beside each consumer stage, so the producers' work spans
//    the whole tick.
//  * Consumers (waves 0-3).  Stage B: wave c owns value rows 16c..16c+15 of H
//    in registers and computes SA, Q, dV and the new H for them; it publishes
//    H', S0, Q^T and SA^T rows.  Barrier.  Stage C: wave c produces the key
//    strip 16c..16c+15 of dK, dB, dR, dA and dw, contracting over all value
//    rows in a fixed order (deterministic; the reference accumulates with fp32
//    atomics, cu:68-72), reading the other orientation of every exchanged
//    matrix with ds_read_b64_tr_b16.
#include "wkv7_launch.h"
#include "wkv7_io.h"

namespace wkv7 {
namespace {

constexpr int CH = CKPT;
constexpr int NK = 64;
constexpr int NPROD = 3;  // producer waves = ring slots
constexpr int LDQ = 16;   // [64][16] exchange planes
constexpr int LDC = 16;   // [16][16] matrices
constexpr int LDG = 68;   // fp32 [16][64] plane

// [16][64] and [64][64] bf16 planes are unpadded and row-swizzled (pl<>):
// planes written by lanes use SwLane, planes filled by LDS DMA SwDma; the
// [*][16] planes (Q^T, SA^T, 16x16 matrices) use pl16.
typedef uint16_t Plane[CH * NK];
// A 16x16 matrix M from its D-layout tile is stored as M^T rows (lane (q, r16)
// writes M[4q..4q+3][r16] at row r16): a plain fragment read of it is the A
// operand of M^T, a transpose read the A operand of M.
typedef uint16_t Mat[2][CH * LDC];

struct Slot {
    Plane At[2], Rt[2], Bb[2], Kb[2];  // A~, R~, B-, K- [t][j] (hi, lo)
    Plane V, dY;                       // [t][i], exact bf16
    Mat Ti, Aak, Brb, Brk, M2;         // M2 = triu(V dY^T); Ti..Brk are dead after stage B
    float g[CH * LDG];                 // cumulative log-decay [t][j]
    float egL[NK];
};
struct BwdLds {
    Slot slot[NPROD];
    uint16_t Hx[2][NK * NK], S0x[2][NK * NK];    // H', S0 [i][j] (swizzled)
    uint16_t QT[2][NK * LDQ], SAT[2][NK * LDQ];  // Q^T, SA^T [i][t]
    Plane raw[NPROD][5];                         // producer input staging: r, w, k, a, b
};
static_assert(sizeof(BwdLds) <= 160 * 1024, "backward LDS budget");

__device__ __forceinline__ void st8(uint16_t* p, uint2 v) { *reinterpret_cast<uint2*>(p) = v; }
__device__ __forceinline__ float lo_bf(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_bf(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float bf_el8(uint4 u, int e) {
    const uint32_t w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
    return (e & 1) ? hi_bf(w) : lo_bf(w);
}
__device__ __forceinline__ void put_mat(Mat& m, const f32x4_t& d, int lane) {
    uint2 h, l;
    pack4(d, h, l);
    const int o = pl16(lane & 15, 4 * (lane >> 4));
    st8(&m[0][o], h);
    st8(&m[1][o], l);
}
__device__ __forceinline__ Pk mat_t(const Mat& m, int lane) {  // A operand of M^T
    const int o = pl16(lane & 15, 4 * (lane >> 4));
    return Pk{*reinterpret_cast<const uint2*>(&m[0][o]), *reinterpret_cast<const uint2*>(&m[1][o])};
}
__device__ __forceinline__ Pk mat_n(const Mat& m, int lane) {  // A operand of M
    return Pk{ldtr16(m[0], 0, lane), ldtr16(m[1], 0, lane)};
}
// split-precision K=32 product (both operands split)
__device__ __forceinline__ f32x4_t mm32s(uint4 ah, uint4 al, uint4 bh, uint4 bl) {
    const f32x4_t acc = mma32(zero4(), ah, bh);
    f32x4_t c = mma32(zero4(), ah, bl);
    c = mma32(c, al, bh);
    return acc + c;
}
// X Y^T over 64 keys, both in the K=32 operand layout (x[hf] = X[t][32hf + 8q ..])
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
// permuted K=32 fragments over the rows of a [64][*] plane (k = 32s + 4q + e, 32s + 16 + 4q + e)
__device__ __forceinline__ uint4 rows_tr(const uint16_t* x, int s, int lane) {  // [64][16] plane
    return cat(ldtr16(x, 32 * s, lane), ldtr16(x, 32 * s + 16, lane));
}
__device__ __forceinline__ uint4 rows_tr_sw(const uint16_t* x, int s, int col0, int lane) {  // [64][64] SwLane plane
    return cat(ldtr_sw<SwLane>(x, 32 * s, col0, lane), ldtr_sw<SwLane>(x, 32 * s + 16, col0, lane));
}

// the value of x, hidden from the optimiser: lane-derived addresses recomputed
// per tick instead of being hoisted out of the loop into spilled registers
__device__ __forceinline__ int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

}  // namespace

__global__ __launch_bounds__(448) void chunk_backward_bf16(
    int Tn, int H, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
    const bf16_t* __restrict__ b, const float* __restrict__ ckpt, const bf16_t* __restrict__ dy,
    const float* __restrict__ dsT, bf16_t* __restrict__ dr, bf16_t* __restrict__ dw,
    bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, bf16_t* __restrict__ da,
    bf16_t* __restrict__ db, float* __restrict__ ds0) {
    __shared__ BwdLds sm;
    const int bh = blockIdx.x, bb = bh / H, h = bh % H;
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    int lane = tid & 63, q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    const long ncp = ckpt_count(Tn);
    const int nchunk = (Tn + CH - 1) / CH;
    const bool consumer = wv < 4;
    const int cw = wv;      // consumer: value-row block / key strip
    const int pw = wv - 4;  // producer index
    int i_own = 16 * cw + r16;
    int j_own = 16 * cw + r16;
    const int lane0 = lane;
    const long rstride = (long)H * NK;  // between consecutive tokens of one head

    // ---------------- producer (lane: token r16, keys 32 hf + 8q + e) ----------------
    float gq[2][8];  // cumulative log-decay, phase 0 -> 1
    // processing index xx -> chunk nchunk-1-xx: byte offset of its first row, valid length
    auto chunk_off = [&](int xx) { return (uint32_t)(((long)(bb * Tn + (nchunk - 1 - xx) * CH) * H + h) * NK * 2); };
    auto chunk_len = [&](int xx) { return min(CH, Tn - (nchunk - 1 - xx) * CH); };
    const uint32_t tbytes = (uint32_t)((long)gridDim.x * Tn * NK * 2);  // bytes of one [B,T,H,64] tensor
    uint32_t voff[2];  // this lane's LDS DMA offsets
    dma_lane_offsets(voff, rstride, lane);
    const bf16_t* const rsrc_src[5] = {r, w, k, a, b};

    // ---------------- consumer ----------------
    // H^T tiles Ht[tj][e] = H[i_own][16tj + 4q + e]; the next chunk's saved state in the same layout
    f32x4_t Ht[4], S0n[4];
    float carry = 0.f;  // dlogd carry for key j_own
    auto load_state = [&](int cc) {
#pragma unroll
        for (int tj = 0; tj < 4; tj++) {
            const float4 s = *reinterpret_cast<const float4*>(ckpt + (bh * ncp + cc) * NN + (long)i_own * NK + 16 * tj + 4 * q);
            S0n[tj] = f32x4_t{s.x, s.y, s.z, s.w};
        }
    };
    if (consumer) {
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
        load_state(nchunk - 1);
        // carry_j = sum_i dsT[i][j] S_T[i][j]: 16 rows per lane group, then the 4 waves in order
        float* part = reinterpret_cast<float*>(&sm.Hx[0][0]);
#pragma unroll
        for (int tj = 0; tj < 4; tj++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float p = Ht[tj][e] * STt[tj][e];
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) p += __shfl_xor(p, off, 16);
                if (r16 == 0) part[cw * NK + 16 * tj + 4 * q + e] = p;
            }
        // consumers load nothing else before use: drain, so the tick loop never
        // waits on the (in-order) memory counter for earlier stores
        vm_wait0();
    } else if (pw < nchunk) {
        // the first chunk of each producer; only processing index 0 can be partial,
        // and its V, dY go into its slot here too so the loop only ever runs DMA
#pragma unroll
        for (int ts = 0; ts < 5; ts++)
            stage_plane(sm.raw[pw][ts], dma_rsrc(rsrc_src[ts], tbytes), rsrc_src[ts], chunk_off(pw), voff, rstride,
                        chunk_len(pw), lane);
        if (pw == 0) {
            stage_plane(sm.slot[0].V, dma_rsrc(v, tbytes), v, chunk_off(0), voff, rstride, chunk_len(0), lane);
            stage_plane(sm.slot[0].dY, dma_rsrc(dy, tbytes), dy, chunk_off(0), voff, rstride, chunk_len(0), lane);
        }
    }
    lds_barrier();
    if (consumer) {
        const float* part = reinterpret_cast<const float*>(&sm.Hx[0][0]);
        carry = part[j_own] + part[NK + j_own] + part[2 * NK + j_own] + part[3 * NK + j_own];
    }
    lds_barrier();

    // Producer work for chunk x (processing order) in phase ph, split into the part
    // done while consumers run stage B (part 0) and the part done during stage C.
    f32x4_t Aab, AabT, Aak, Brb, Brk, M2;  // phase 2, part 0 -> part 1
    auto produce = [&](int x, int ph, int part) {
        Slot& S = sm.slot[x % NPROD];
        const Plane* raw = sm.raw[pw];
        if (ph == 0) {
            if (part == 0) {
                // ---- phase 0: log-decays and their cumulative sum ----
                vm_wait0();  // this chunk's inputs (LDS DMA issued two ticks ago)
                const int L = chunk_len(x);
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const uint4 wr = ld16_sw<SwDma>(raw[1], r16, 32 * hf + 8 * q);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        float ld = log_decay(bf_el8(wr, e));
                        if (L < CH) ld = r16 < L ? ld : 0.f;
                        gq[hf][e] = row_prefix_sum(ld);
                    }
                }
            }
        } else if (ph == 1) {
            // ---- phase 1: scaled operands, g and e^{gL} into the slot (keys 0-31 in
            //      part 0, 32-63 in part 1); then V, dY of this chunk and the inputs of
            //      this producer's next chunk by LDS DMA ----
            auto half = [&](auto hfc) {
                constexpr int hf = decltype(hfc)::value;
                const int c8 = 32 * hf + 8 * q;
                const uint4 rr = ld16_sw<SwDma>(raw[0], r16, c8), kk = ld16_sw<SwDma>(raw[2], r16, c8);
                const uint4 aa = ld16_sw<SwDma>(raw[3], r16, c8), bv = ld16_sw<SwDma>(raw[4], r16, c8);
                float at[8], rt[8], bbv[8], kbv[8], el[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float eg = __expf(gq[hf][e]), eng = __expf(-gq[hf][e]);
                    at[e] = bf_el8(aa, e) * row_prev(eg, 1.f);
                    rt[e] = bf_el8(rr, e) * eg;
                    bbv[e] = bf_el8(bv, e) * eng;
                    kbv[e] = bf_el8(kk, e) * eng;
                    el[e] = row_last(eg);
                }
                uint4 hh, ll;
                pack8(at, hh, ll);
                st16_sw<SwLane>(S.At[0], r16, c8, hh);
                st16_sw<SwLane>(S.At[1], r16, c8, ll);
                pack8(rt, hh, ll);
                st16_sw<SwLane>(S.Rt[0], r16, c8, hh);
                st16_sw<SwLane>(S.Rt[1], r16, c8, ll);
                pack8(bbv, hh, ll);
                st16_sw<SwLane>(S.Bb[0], r16, c8, hh);
                st16_sw<SwLane>(S.Bb[1], r16, c8, ll);
                pack8(kbv, hh, ll);
                st16_sw<SwLane>(S.Kb[0], r16, c8, hh);
                st16_sw<SwLane>(S.Kb[1], r16, c8, ll);
                float* gp_ = &S.g[r16 * LDG + 32 * hf + 8 * q];
                *reinterpret_cast<float4*>(gp_) = make_float4(gq[hf][0], gq[hf][1], gq[hf][2], gq[hf][3]);
                *reinterpret_cast<float4*>(gp_ + 4) = make_float4(gq[hf][4], gq[hf][5], gq[hf][6], gq[hf][7]);
                if (r16 == 0) {
                    *reinterpret_cast<float4*>(&S.egL[32 * hf + 8 * q]) = make_float4(el[0], el[1], el[2], el[3]);
                    *reinterpret_cast<float4*>(&S.egL[32 * hf + 8 * q + 4]) = make_float4(el[4], el[5], el[6], el[7]);
                }
            };
            if (part == 0) {
                half(std::integral_constant<int, 0>{});
            } else {
                half(std::integral_constant<int, 1>{});
                if (x > 0) {  // (chunk 0's V, dY were staged before the loop)
                    dma_plane(S.V, dma_rsrc(v, tbytes), chunk_off(x), voff);
                    dma_plane(S.dY, dma_rsrc(dy, tbytes), chunk_off(x), voff);
                }
                wave_lds_fence();  // staging reads done before the DMA overwrites it
                if (x + NPROD < nchunk) {
#pragma unroll
                    for (int ts = 0; ts < 5; ts++)
                        dma_plane(sm.raw[pw][ts], dma_rsrc(rsrc_src[ts], tbytes), chunk_off(x + NPROD), voff);
                }
            }
        } else if (part == 0) {
            // ---- phase 2: chunk matrices over keys / value rows, triangular inverse ----
            // V, dY of this chunk: the 10 staging DMA ops issued after them may still run
            if (x + NPROD < nchunk) vm_wait10();
            else vm_wait0();
            auto rd = [&](const Plane (&pl2)[2], uint4 (&xh)[2], uint4 (&xl)[2]) {
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    xh[hf] = ld16_sw<SwLane>(pl2[0], r16, 32 * hf + 8 * q);
                    xl[hf] = ld16_sw<SwLane>(pl2[1], r16, 32 * hf + 8 * q);
                }
            };
            {
                uint4 ath[2], atl[2], xh[2], xl[2];
                rd(S.At, ath, atl);
                rd(S.Bb, xh, xl);
                Aab = mm_keys8(ath, atl, xh, xl);
                AabT = mm_keys8(xh, xl, ath, atl);
                rd(S.Kb, xh, xl);
                Aak = mm_keys8(ath, atl, xh, xl);
                __builtin_amdgcn_sched_barrier(0);
            }
            {
                uint4 rth[2], rtl[2], xh[2], xl[2];
                rd(S.Rt, rth, rtl);
                rd(S.Bb, xh, xl);
                Brb = mm_keys8(rth, rtl, xh, xl);
                rd(S.Kb, xh, xl);
                Brk = mm_keys8(rth, rtl, xh, xl);
                __builtin_amdgcn_sched_barrier(0);
            }
            {
                uint4 vv[2], yy[2];
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    vv[hf] = ld16_sw<SwDma>(S.V, r16, 32 * hf + 8 * q);
                    yy[hf] = ld16_sw<SwDma>(S.dY, r16, 32 * hf + 8 * q);
                }
                M2 = mma32(mma32(zero4(), vv[0], yy[0]), vv[1], yy[1]);  // V dY^T (exact operands)
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) {  // D layout: row 4q+e, column r16
                const int rw = 4 * q + e;
                if (r16 >= rw) Aab[e] = 0.f, Aak[e] = 0.f;  // [t][s]: s < t
                if (rw >= r16) AabT[e] = 0.f;               // [s][t]: s < t
                if (r16 > rw) Brb[e] = 0.f, Brk[e] = 0.f;   // [t][s]: s <= t
                if (r16 < rw) M2[e] = 0.f;                  // [t][s]: s >= t
            }
            f32x4_t Ti, TiT;
            tri_inverse(Aab, AabT, lane, Ti, TiT);
            put_mat(S.Ti, Ti, lane);
            put_mat(S.Aak, Aak, lane);
            put_mat(S.Brb, Brb, lane);
            put_mat(S.Brk, Brk, lane);
            put_mat(S.M2, M2, lane);
        }
    };

    for (int n = -NPROD; n < nchunk; n++) {
        lane = opaque(lane0);
        q = lane >> 4;
        r16 = lane & 15;
        i_own = 16 * cw + r16;
        j_own = i_own;
        // the chunk a producer works on at tick n (x = pw mod 3, so slot x % 3 is its
        // own) and its phase; prologue ticks have no chunk for some producers
        const int x = n + 1 + ((pw - n - 1) % NPROD + NPROD) % NPROD;
        const int ph = n + NPROD - x;
        const bool pact = !consumer && x >= 0 && x < nchunk;
        if (pact) produce(x, ph, 0);
        // ================= consumers, stage B (chunk n, rows i_own) =================
        if (consumer && n >= 0) {
            const Slot& S = sm.slot[n % NPROD];
            const int c = nchunk - 1 - n, t0 = c * CH, L = min(CH, Tn - t0);
            f32x4_t S0r[4], Hp[4];
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                S0r[tj] = S0n[tj];
                const float4 el = *reinterpret_cast<const float4*>(&S.egL[16 * tj + 4 * q]);
                Hp[tj] = Ht[tj] * f32x4_t{el.x, el.y, el.z, el.w};
            }
            const uint2 vfr = ldtr_sw<SwDma>(S.V, 0, 16 * cw, lane);   // V[s = 4q+e][i_own]
            const uint2 dyf = ldtr_sw<SwDma>(S.dY, 0, 16 * cw, lane);  // dY[s = 4q+e][i_own]
            // X1 = A~ S0^T + Aak V ; X2 = B- H'^T + Brb^T dY ; dV0 = K- H'^T + Brk^T dY
            f32x4_t x1 = zero4(), x2 = zero4(), dv0 = zero4();
#pragma unroll
            for (int s = 0; s < 2; s++) {
                float hv[8], sv[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    hv[e] = Hp[2 * s][e];
                    hv[4 + e] = Hp[2 * s + 1][e];
                    sv[e] = S0r[2 * s][e];
                    sv[4 + e] = S0r[2 * s + 1][e];
                }
                uint4 hbh, hbl, sbh, sbl;
                pack8(hv, hbh, hbl);
                pack8(sv, sbh, sbl);
                // the halves are this lane's 4-key pieces of H' and S0 (tiles 2s, 2s+1):
                // publish them for stage C now (no second split)
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int col = 16 * (2 * s + u) + 4 * q;
                    st8_sw<SwLane>(sm.Hx[0], i_own, col, u ? make_uint2(hbh.z, hbh.w) : make_uint2(hbh.x, hbh.y));
                    st8_sw<SwLane>(sm.Hx[1], i_own, col, u ? make_uint2(hbl.z, hbl.w) : make_uint2(hbl.x, hbl.y));
                    st8_sw<SwLane>(sm.S0x[0], i_own, col, u ? make_uint2(sbh.z, sbh.w) : make_uint2(sbh.x, sbh.y));
                    st8_sw<SwLane>(sm.S0x[1], i_own, col, u ? make_uint2(sbl.z, sbl.w) : make_uint2(sbl.x, sbl.y));
                }
                const uint4 ah = fragp_sw<SwLane>(S.At[0], r16, 32 * s, lane), al = fragp_sw<SwLane>(S.At[1], r16, 32 * s, lane);
                x1 = mma32(x1, ah, sbh);
                x1 = mma32(x1, ah, sbl);
                x1 = mma32(x1, al, sbh);
                const uint4 bh_ = fragp_sw<SwLane>(S.Bb[0], r16, 32 * s, lane), bl_ = fragp_sw<SwLane>(S.Bb[1], r16, 32 * s, lane);
                x2 = mma32(x2, bh_, hbh);
                x2 = mma32(x2, bh_, hbl);
                x2 = mma32(x2, bl_, hbh);
                const uint4 kh = fragp_sw<SwLane>(S.Kb[0], r16, 32 * s, lane), kl = fragp_sw<SwLane>(S.Kb[1], r16, 32 * s, lane);
                dv0 = mma32(dv0, kh, hbh);
                dv0 = mma32(dv0, kh, hbl);
                dv0 = mma32(dv0, kl, hbh);
            }
            {
                f32x4_t c1 = zero4(), c2 = zero4(), c3 = zero4();
                const Pk aak = mat_n(S.Aak, lane), brbT = mat_t(S.Brb, lane), brkT = mat_t(S.Brk, lane);
                c1 = mma16(c1, aak.h, vfr);
                c1 = mma16(c1, aak.l, vfr);
                c2 = mma16(c2, brbT.h, dyf);
                c2 = mma16(c2, brbT.l, dyf);
                c3 = mma16(c3, brkT.h, dyf);
                c3 = mma16(c3, brkT.l, dyf);
                x1 += c1;
                x2 += c2;
                dv0 += c3;
            }
            const f32x4_t sa = mm16s(mat_n(S.Ti, lane), pk(x1));   // SA = Ti X1
            const f32x4_t qq = mm16s(mat_t(S.Ti, lane), pk(x2));   // Q  = Ti^T X2
            const Pk pq = pk(qq), psa = pk(sa);
            const f32x4_t dvv = dv0 + mm16s(mat_t(S.Aak, lane), pq);
            // publish this block's rows for stage C
            st8(&sm.QT[0][pl16(i_own, 4 * q)], pq.h);
            st8(&sm.QT[1][pl16(i_own, 4 * q)], pq.l);
            st8(&sm.SAT[0][pl16(i_own, 4 * q)], psa.h);
            st8(&sm.SAT[1][pl16(i_own, 4 * q)], psa.l);
            // H_0^T = H'^T + [A~^T R~^T] [Q; dY]
            const uint4 bhi = cat(pq.h, dyf), blo = cat(pq.l, make_uint2(0, 0));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const uint4 ah = cat(ldtr_sw<SwLane>(S.At[0], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Rt[0], 0, 16 * tj, lane));
                const uint4 al = cat(ldtr_sw<SwLane>(S.At[1], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Rt[1], 0, 16 * tj, lane));
                f32x4_t acc = mma32(Hp[tj], ah, bhi);
                f32x4_t c1 = mma32(zero4(), ah, blo);
                c1 = mma32(c1, al, bhi);
                Ht[tj] = acc + c1;
            }
            {  // lane (q, 4m + jj) stores row 4q + jj, values 16c + 4m .. +3
                const int tr = 4 * q + (lane & 3);
                const uint32_t o = tr < L ? (uint32_t)((((long)(bb * Tn + t0 + tr) * H + h) * NK + 16 * cw + 4 * (r16 >> 2)) * 2)
                                          : OUT_OF_RANGE;
                store8(dv, tbytes, o, quad_rows_bf16(dvv, lane));
            }
        }
        lds_barrier();
        if (consumer) {
            // ================= consumers, stage C (chunk n, key strip j_own) =================
            if (n >= 0) {
                Slot& S = sm.slot[n % NPROD];
                const int c = nchunk - 1 - n, t0 = c * CH, L = min(CH, Tn - t0);
                if (c > 0) load_state(c - 1);  // saved state of the next chunk processed
                // contractions over all value rows i (each fragment read once)
                f32x4_t m1 = zero4(), n1 = zero4(), xm = zero4(), gK = zero4(), gB = zero4(), gR = zero4(), gA = zero4();
                {
                    f32x4_t c1 = zero4(), c2 = zero4(), c3 = zero4();
#pragma unroll
                    for (int s = 0; s < 2; s++) {
                        const uint4 va = fragp_sw<SwDma>(S.V, r16, 32 * s, lane);    // V[t][i], exact
                        const uint4 ya = fragp_sw<SwDma>(S.dY, r16, 32 * s, lane);   // dY[t][i], exact
                        const uint4 qh = rows_tr(sm.QT[0], s, lane), ql = rows_tr(sm.QT[1], s, lane);
                        const uint4 sh = rows_tr(sm.SAT[0], s, lane), sl = rows_tr(sm.SAT[1], s, lane);
                        const uint4 hh = rows_tr_sw(sm.Hx[0], s, 16 * cw, lane), hl = rows_tr_sw(sm.Hx[1], s, 16 * cw, lane);
                        const uint4 oh = rows_tr_sw(sm.S0x[0], s, 16 * cw, lane), ol = rows_tr_sw(sm.S0x[1], s, 16 * cw, lane);
                        m1 = mma32(m1, va, qh);   // V Q^T
                        m1 = mma32(m1, va, ql);
                        gK = mma32(gK, va, hh);   // V H'
                        gK = mma32(gK, va, hl);
                        xm = mma32(xm, ya, sh);   // dY SA^T
                        xm = mma32(xm, ya, sl);
                        gR = mma32(gR, ya, oh);   // dY S0
                        gR = mma32(gR, ya, ol);
                        n1 = mma32(n1, sh, qh);   // SA Q^T
                        n1 = mma32(n1, sh, ql);
                        c1 = mma32(c1, sl, qh);
                        gB = mma32(gB, sh, hh);   // SA H'
                        gB = mma32(gB, sh, hl);
                        c2 = mma32(c2, sl, hh);
                        gA = mma32(gA, qh, oh);   // Q S0
                        gA = mma32(gA, qh, ol);
                        c3 = mma32(c3, ql, oh);
                    }
                    n1 += c1;
                    gB += c2;
                    gA += c3;
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {  // D layout: row t = 4q+e, column s = r16
                    const int t = 4 * q + e;
                    if (r16 <= t) m1[e] = 0.f, n1[e] = 0.f;  // keep s > t
                    if (r16 > t) xm[e] = 0.f;                // keep s <= t
                }
                // [A~; R~] and [B-; K-] strips as K=32 B operands (also their values in D layout)
                const uint4 arh = cat(ldtr_sw<SwLane>(S.At[0], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Rt[0], 0, 16 * cw, lane));
                const uint4 arl = cat(ldtr_sw<SwLane>(S.At[1], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Rt[1], 0, 16 * cw, lane));
                const uint4 bkh = cat(ldtr_sw<SwLane>(S.Bb[0], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Kb[0], 0, 16 * cw, lane));
                const uint4 bkl = cat(ldtr_sw<SwLane>(S.Bb[1], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Kb[1], 0, 16 * cw, lane));
                // the 16x16 masked products go through this wave's scratch matrix (in the
                // slot's Ti/Aak/Brb/Brk area, dead after stage B) to get both orientations
                Mat& P = cw == 0 ? S.Ti : cw == 1 ? S.Aak : cw == 2 ? S.Brb : S.Brk;
                const Pk m2n = mat_n(S.M2, lane), m2t = mat_t(S.M2, lane);
                put_mat(P, m1, lane);
                wave_lds_fence();
                const Pk m1n = mat_n(P, lane), m1t = mat_t(P, lane);
                wave_lds_fence();
                const f32x4_t cK = mm32s(cat(m1n.h, m2n.h), cat(m1n.l, m2n.l), arh, arl);  // [triu_s(M1) | triu(M2)]
                put_mat(P, xm, lane);
                wave_lds_fence();
                const Pk xmn = mat_n(P, lane), xmt = mat_t(P, lane);
                wave_lds_fence();
                const f32x4_t cR = mm32s(cat(xmn.h, m2t.h), cat(xmn.l, m2t.l), bkh, bkl);  // [tril(dY SA^T) | tril(dY V^T)]
                put_mat(P, n1, lane);
                wave_lds_fence();
                const Pk n1n = mat_n(P, lane), n1t = mat_t(P, lane);
                const f32x4_t cB = mm32s(cat(n1n.h, xmt.h), cat(n1n.l, xmt.l), arh, arl);  // [triu_s(N1) | triu(SA dY^T)]
                const f32x4_t cA = mm32s(cat(n1t.h, m1t.h), cat(n1t.l, m1t.l), bkh, bkl);  // [tril_s(Q SA^T) | tril_s(Q V^T)]
                float gk_[4], gb_[4], gr_[4], ga_[4], gw_[4], z[4], t2[4], fw[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = 4 * q + e;
                    const float gv = S.g[t * LDG + j_own];
                    const float gp = t > 0 ? S.g[(t - 1) * LDG + j_own] : 0.f;
                    const float uK = gK[e] + cK[e], uB = gB[e] + cB[e], uR = gR[e] + cR[e], uA = gA[e] + cA[e];
                    const float eng = __expf(-gv);
                    gk_[e] = eng * uK;
                    gb_[e] = eng * uB;
                    gr_[e] = __expf(gv) * uR;
                    ga_[e] = __expf(gp) * uA;
                    const float At_ = bf_el8(arh, e) + bf_el8(arl, e);
                    const float Rt_ = bf_el8(arh, 4 + e) + bf_el8(arl, 4 + e);
                    const float Bb_ = bf_el8(bkh, e) + bf_el8(bkl, e);
                    const float Kb_ = bf_el8(bkh, 4 + e) + bf_el8(bkl, 4 + e);
                    z[e] = Rt_ * uR - Bb_ * uB - Kb_ * uK;
                    t2[e] = At_ * uA;
                    const float sg = (gp - gv) * (1.f / DECAY_SCALE);  // sigmoid(w_t)
                    fw[e] = -DECAY_SCALE * sg * (1.f - sg);
                }
                // dlogd_t = carry + sum_{s>=t} z_s + sum_{s>t} t2_s over the chunk (t = 4q + e)
                float tot = 0.f;
#pragma unroll
                for (int e = 0; e < 4; e++) tot += z[e] + t2[e];
                const float s1 = __shfl(tot, (lane & 15) + 16), s2 = __shfl(tot, (lane & 15) + 32),
                            s3 = __shfl(tot, (lane & 15) + 48), s0 = __shfl(tot, lane & 15);
                float run = carry + (q < 1 ? s1 : 0.f) + (q < 2 ? s2 : 0.f) + (q < 3 ? s3 : 0.f);
#pragma unroll
                for (int e = 3; e >= 0; e--) {
                    run += z[e];
                    gw_[e] = run * fw[e];
                    run += t2[e];
                }
                carry += ((s0 + s1) + s2) + s3;
                // lane (q, 4m + jj) stores row 4q + jj, keys 16c + 4m .. +3 of each gradient
                const int tr = 4 * q + (lane & 3);
                const uint32_t o = tr < L ? (uint32_t)((((long)(bb * Tn + t0 + tr) * H + h) * NK + 16 * cw + 4 * (r16 >> 2)) * 2)
                                          : OUT_OF_RANGE;
                store8(dk, tbytes, o, quad_rows_bf16(f32x4_t{gk_[0], gk_[1], gk_[2], gk_[3]}, lane));
                store8(db, tbytes, o, quad_rows_bf16(f32x4_t{gb_[0], gb_[1], gb_[2], gb_[3]}, lane));
                store8(dr, tbytes, o, quad_rows_bf16(f32x4_t{gr_[0], gr_[1], gr_[2], gr_[3]}, lane));
                store8(da, tbytes, o, quad_rows_bf16(f32x4_t{ga_[0], ga_[1], ga_[2], ga_[3]}, lane));
                store8(dw, tbytes, o, quad_rows_bf16(f32x4_t{gw_[0], gw_[1], gw_[2], gw_[3]}, lane));
            }
        } else {
            // ================= producers, second part of the tick's phase =================
            if (pact) produce(x, ph, 1);
        }
        lds_barrier();
    }
    if (consumer) {
#pragma unroll
        for (int tj = 0; tj < 4; tj++)
            *reinterpret_cast<float4*>(ds0 + bh * NN + (long)i_own * NK + 16 * tj + 4 * q) =
                make_float4(Ht[tj][0], Ht[tj][1], Ht[tj][2], Ht[tj][3]);
    }
}

void launch_chunk_backward(const Bwd& p) {
    hipLaunchKernelGGL(chunk_backward_bf16, dim3(p.B * p.H), dim3(448), 0, p.stream, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.ckpt, (const bf16_t*)p.dy, p.dsT,
                       (bf16_t*)p.dr, (bf16_t*)p.dw, (bf16_t*)p.dk, (bf16_t*)p.dv, (bf16_t*)p.da,
                       (bf16_t*)p.db, p.ds0);
}

}  // namespace wkv7
