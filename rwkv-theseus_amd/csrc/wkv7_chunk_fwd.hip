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
// Mapping: 512-lane workgroups, one per CU, each running a stream of chunks
// (b,h heads one after another, the first and last possibly cut pieces of a
// head shared with another workgroup: wkv7_sched.h), two roles, lock-step
// "ticks" that each end in one LDS barrier (no global-memory fence, so
// prefetches stay in flight across it).  The producers' pipeline runs on across
// head boundaries; only the consumers see them (initial and final state).
//  * Producers (waves 0-3).  Everything above that does not involve the
//    state depends only on the chunk's inputs, so producer p builds the
//    operands of chunks p, p+4, p+8, ... alone -- no barrier inside -- in four
//    phases over the four ticks before the chunk is consumed (one loop
//    iteration per chunk); at any tick the four producers are in four different
//    phases, each phase about a quarter of the work.  A chunk's inputs arrive
//    by LDS DMA two ticks ahead into the producer's staging planes (no
//    prefetch registers).  A lane
//    holds one token and 8 keys of a 32-key half (X[t = l%16][32 hf + 8q + e],
//    the K=32 operand layout), so the decay cumsum over tokens is a 16-lane
//    DPP scan, the key contractions (Aab, ...) take the operands straight from
//    registers, and the products over tokens read their transposed operand
//    back with ds_read_b64_tr_b16.
//  * Consumers (waves 4-7).  Wave 4+c keeps value rows 16c..16c+15 of the
//    state in registers (value rows never interact) and advances them by one
//    chunk per tick from the operands the producers left in a 5-slot LDS ring
//    (chunk x in slot x % 5, free from tick x-4 since its last reader was
//    chunk x-5).  Their outputs leave in whole lines: y through LDS in
//    128-byte rows, stored a tick late by all four waves; the saved states S_c
//    straight from the registers in a tiled order (whole KBs), in chunk c's tick
//    while its first products run; the final saved state in [value][key] rows
//    regrouped through LDS eight at a time.
#include "wkv7_launch.h"
#include "wkv7_io.h"
#include "wkv7_sched.h"

namespace wkv7 {
namespace {

constexpr int CH = CKPT;   // chunk length
constexpr int NK = 64;     // head size of this kernel
constexpr int NPROD = 4;   // producer waves (= phases per chunk)
constexpr int NSLOT = 5;   // operand ring

// [16][64] bf16 planes are unpadded and row-swizzled (pl<>): SwLane for planes
// the producers write from registers, SwDma for planes filled by LDS DMA;
// [16][16] matrices use pl16.
typedef uint16_t Plane[CH * NK];
typedef uint16_t Mat[2][CH * 16];

// One chunk's operands, as the consumers read them.
struct Slot {
    Plane P[2];    // P [t][j] (hi, lo); A~ until phases 2-3 replace it
    Plane P2[2];   // P2 [t][j]; R~ until phase 3 replaces it
    Plane Bh[2];   // B^ [t][j]
    Plane Kh[2];   // K^ [t][j]
    Mat Q1T;       // Q'^T [s][t]
    Mat Q2;        // Q2 [t][s]
    Plane V;       // V [t][i], exact bf16 (SwDma)
    float egL[NK]; // e^{gL} per key
};
// Outputs leave in whole lines: a wave's own pieces of y are 32-byte parts of 128-byte
// lines, and stores of such parts cost far more than their bytes (the forward ran 7 %
// faster with y regrouped, 6 % with the saved states regrouped, before those were stored
// in the tiled order instead).
constexpr int LDR = NK + 4;  // padded row (floats) of the final state's regrouping planes
struct FwdLds {
    Slot slot[NSLOT];
    Plane raw[NPROD][5];     // producer input staging: r, w, k, a, b (SwDma)
    uint16_t yq[2][CH * NK]; // y tiles of the last two ticks [t][i], stored a tick late
    float sq[4][8 * LDR];    // per consumer wave: 8 of its 16 final-state rows at a time
};
static_assert(sizeof(FwdLds) <= 160 * 1024, "forward LDS budget");

__device__ __forceinline__ void st8(uint16_t* p, uint2 v) { *reinterpret_cast<uint2*>(p) = v; }
__device__ __forceinline__ uint2 ld8(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }
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
// X Y^T over the 64 keys for operands in the standard K=32 layout
// (x[hf] = X[t = l%16][32 hf + 8q .. +7], split into hi / lo)
__device__ __forceinline__ f32x4_t mm_keys8(const uint4 (&xh)[2], const uint4 (&xl)[2], const uint4 (&yh)[2],
                                            const uint4 (&yl)[2]) {
    f32x4_t acc = zero4();  // one accumulator chain: no VALU adds
#pragma unroll
    for (int s = 0; s < 2; s++) {
        acc = mma32(acc, xh[s], yh[s]);
        acc = mma32(acc, xh[s], yl[s]);
        acc = mma32(acc, xl[s], yh[s]);
    }
    return acc;
}
}  // namespace

// The time-split forward (SPLIT): the state after a chunk is affine in the state before
// it, S_{c+1} = S_c M_c + U_c, so with few heads each head's chunks are cut into k
// segments that all run at once, one job (workgroup) per (segment, head), segment 0 of m0
// chunks and the others of m (segment 0 carries one state and ticks faster, so it takes
// more chunks):
//  * segment 0 runs from s0 and writes y as usual, its final state S_1 to the workspace;
//  * segment s >= 1 runs two states side by side on the same chunk operands, each
//    consumer wave holding its rows of both: one from zero (y0 and the final state U_s),
//    one from the identity with v = 0 ("y" z_t = Phi_t r_t and the final state, the
//    segment's transition Phi_s).
// split_fixup then chains S_{s+1} = S_s Phi_s + U_s, forms y_t = y0_t + S_s z_t over
// segment s and writes sT = S_k (wkv7_capi.cpp decides when).
struct SplitArgs {
    int BH = 0, m = 0, k = 0;  // heads, chunks of segments 1 .., segments
    int m0 = 0;                // chunks of segment 0
    float* send0 = nullptr;    // S_1 [BH][64][64]
    float* uend = nullptr;     // U_s [k - 1][BH][64][64]
    float* phi = nullptr;      // Phi_s, the same layout
    float* y0 = nullptr;       // segments 1.. from zero: y tiles [k - 1][BH][m][4 waves][64 lanes][4] float32
    float* z = nullptr;        // the identity runs' tiles, the same layout
};

// Saved states.  State c < ceil(T/16) (the state chunk c starts from) is stored in the
// tiled order: S[i][j] (value i, key j) at float
//   ((i/16 * 4 + j/16) * 64 + 16 * (j%16/4) + i%16) * 4 + j%4,
// which is each consumer wave's register layout (wave i/16, tile j/16, lane, element), so
// every store is a whole KB.  The last one, the final state, is stored in the plain
// [value][key] order (it equals sT) by FWD_SAVE_STATE: this wave's 16 rows of St, 8 at a
// time through its sq plane, four whole 256-byte rows per store.
#define FWD_SAVE_STATE(e)                                                                                     \
    do {                                                                                                      \
        float* const sq_ = sm.sq[cw];                                                                         \
        float* const dst_ = ckpt + (bh * ncp + (e)) * NN + (long)(16 * cw) * NK;                             \
        _Pragma("unroll") for (int p_ = 0; p_ < 2; p_++) {                                                    \
            if ((r16 >> 3) == p_) {                                                                           \
                _Pragma("unroll") for (int tj_ = 0; tj_ < 4; tj_++)                                           \
                    *reinterpret_cast<float4*>(sq_ + (r16 & 7) * LDR + 16 * tj_ + 4 * q) =                   \
                        make_float4(St[tj_][0], St[tj_][1], St[tj_][2], St[tj_][3]);                          \
            }                                                                                                 \
            _Pragma("unroll") for (int u_ = 0; u_ < 2; u_++) {                                                \
                const int rr_ = 4 * u_ + (lane >> 4), cc_ = 4 * (lane & 15);                                  \
                *reinterpret_cast<float4*>(dst_ + (8 * p_ + rr_) * NK + cc_) =                                \
                    *reinterpret_cast<const float4*>(sq_ + rr_ * LDR + cc_);                                  \
            }                                                                                                 \
        }                                                                                                     \
    } while (0)

// CKPT: saved states are written (ckpt is not null); a template argument so that the
// forward without them keeps its tick in one basic block.
template <bool SPLIT, bool CKPT>
__global__ __launch_bounds__(512) void chunk_forward_bf16(
    Sched sc, int Tn, int H, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
    const bf16_t* __restrict__ b, const float* __restrict__ s0, bf16_t* __restrict__ y,
    float* __restrict__ sT, float* __restrict__ ckpt, uint32_t* __restrict__ flags, float* __restrict__ hand,
    SplitArgs sp) {
    __shared__ FwdLds sm;
    const int m = machine_of_block(sc);
    // (SPLIT: one job per machine, job m; its segment's length)
    const int nstream = SPLIT ? (m < sp.BH ? sp.m0 : sp.m) : stream_len(sc, m);
    auto seg_first = [&](int sg) { return sg == 0 ? 0 : sp.m0 + (sg - 1) * sp.m; };  // (SPLIT) first chunk
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int lane = tid & 63, q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    const long ncp = ckpt_count(Tn);
    const bool producer = wv < NPROD;
    const int pw = wv, cw = wv - NPROD;
    const long rstride = (long)H * NK;                              // between consecutive tokens of one head
    // bytes of one [B,T,H,64] tensor (SPLIT: the schedule's jobs are k per head)
    const uint32_t tbytes = (uint32_t)((long)(SPLIT ? sp.BH : sc.J) * Tn * NK * 2);
    // stream position (cursor) -> byte offset of the chunk's first row, its valid length
    // (SPLIT: job j is segment j / BH of head j % BH, whose steps start at seg_first)
    auto chunk_off = [&](const Cursor& cu) {
        if (!SPLIT) return (uint32_t)(((long)(cu.bb * Tn + cu.step * CH) * H + cu.h) * NK * 2);
        const int sg = cu.j / sp.BH, head = cu.j - sg * sp.BH, b2 = head / H, h2 = head - b2 * H;
        return (uint32_t)(((long)(b2 * Tn + (cu.step + seg_first(sg)) * CH) * H + h2) * NK * 2);
    };
    auto chunk_len = [&](const Cursor& cu) {
        return min(CH, Tn - (cu.step + (SPLIT ? seg_first(cu.j / sp.BH) : 0)) * CH);
    };

    // ---------------- producer state ----------------
    uint32_t voff[2];  // this lane's LDS DMA offsets
    dma_lane_offsets(voff, rstride, lane);
    const bf16_t* const src5[5] = {r, w, k, a, b};
    // this producer's current chunk (stream index x = pw mod 4) and its next
    Cursor cx = cursor_at(sc, m, pw, H), cy = cursor_at(sc, m, pw + NPROD, H);
    Pk pTiT, pB;  // Ti^T, Brb^T packed (phase 2 -> 3)

    // scaled operands of one key half from the staged inputs and g: written to
    // the slot (P <- A~, P2 <- R~, B^, K^, e^{gL}); B- and K- (hi, lo) go to the
    // same half of the staging planes just read (r, k, a, b), for phase 2
    auto operands = [&](Slot& S, Plane* raw, const float (&g)[8], int hf) {
        const int c8 = 32 * hf + 8 * q;
        const uint4 rr = ld16_sw<SwDma>(raw[0], r16, c8), kk = ld16_sw<SwDma>(raw[2], r16, c8);
        const uint4 aa = ld16_sw<SwDma>(raw[3], r16, c8), bv = ld16_sw<SwDma>(raw[4], r16, c8);
        float at[8], rt[8], bbv[8], kbv[8], bhv[8], khv[8], el[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float eg = __expf(g[e]), eng = __expf(-g[e]);
            el[e] = row_last(eg);
            at[e] = bf_el8(aa, e) * row_prev(eg, 1.f);
            rt[e] = bf_el8(rr, e) * eg;
            bbv[e] = bf_el8(bv, e) * eng;
            kbv[e] = bf_el8(kk, e) * eng;
            bhv[e] = bbv[e] * el[e];
            khv[e] = kbv[e] * el[e];
        }
        uint4 hh, ll;
        pack8(at, hh, ll);
        st16_sw<SwLane>(S.P[0], r16, c8, hh);
        st16_sw<SwLane>(S.P[1], r16, c8, ll);
        pack8(rt, hh, ll);
        st16_sw<SwLane>(S.P2[0], r16, c8, hh);
        st16_sw<SwLane>(S.P2[1], r16, c8, ll);
        pack8(bbv, hh, ll);
        st16_sw<SwDma>(raw[0], r16, c8, hh);
        st16_sw<SwDma>(raw[2], r16, c8, ll);
        pack8(kbv, hh, ll);
        st16_sw<SwDma>(raw[3], r16, c8, hh);
        st16_sw<SwDma>(raw[4], r16, c8, ll);
        pack8(bhv, hh, ll);
        st16_sw<SwLane>(S.Bh[0], r16, c8, hh);
        st16_sw<SwLane>(S.Bh[1], r16, c8, ll);
        pack8(khv, hh, ll);
        st16_sw<SwLane>(S.Kh[0], r16, c8, hh);
        st16_sw<SwLane>(S.Kh[1], r16, c8, ll);
        if (r16 == 0) {
            *reinterpret_cast<float4*>(&S.egL[c8]) = make_float4(el[0], el[1], el[2], el[3]);
            *reinterpret_cast<float4*>(&S.egL[c8 + 4]) = make_float4(el[4], el[5], el[6], el[7]);
        }
    };
    // P = Ti A~ for 16-key tiles [tj0, tj1): tile tj of A~ (read transposed) is
    // replaced by tile tj of P
    auto p_tiles = [&](Slot& S, int tj0, int tj1) {
#pragma unroll
        for (int tj = tj0; tj < tj1; tj++) {
            const Pk pa = {ldtr_sw<SwLane>(S.P[0], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.P[1], 0, 16 * tj, lane)};
            const Pk pp = pk(mm16s(pa, pTiT));  // lane: P[t = r16][16tj + 4q + e]
            st8_sw<SwLane>(S.P[0], r16, 16 * tj + 4 * q, pp.h);
            st8_sw<SwLane>(S.P[1], r16, 16 * tj + 4 * q, pp.l);
        }
    };

    // ---------------- consumer state: S^T tiles St[tj][e] = S[i_own][16tj + 4q + e] ----------------
    const int i_own = 16 * cw + r16;
    f32x4_t St[4], Sp[4];  // (Sp: SPLIT's identity run)
    if (producer) {
        // this producer's first chunk
        if (pw < nstream) {
#pragma unroll
            for (int ts = 0; ts < 5; ts++)
                stage_plane(sm.raw[pw][ts], dma_rsrc(src5[ts], tbytes), src5[ts], chunk_off(cx), voff, rstride,
                            chunk_len(cx), lane);
        }
    }

    // The two roles run separate tick loops with the same barriers, so that
    // registers and memory-counter waits are allocated per role.
    if (producer) {
        // Producer pw's chunks are x = pw, pw + 4, ...; phase ph of chunk x runs at tick
        // x - 4 + ph, so each iteration below is four consecutive ticks.
        int n = -NPROD;
        for (; n < pw - NPROD; n++) lds_barrier();  // (ticks before this producer's first chunk)
        for (int x = pw; x < nstream; x += NPROD, n += NPROD) {
            if (x > pw) {  // on to the next chunk
                cx = cy;
                cursor_advance(cy, sc, m, NPROD, H);
            }
            Slot& S = sm.slot[x % NSLOT];
            Plane* raw = sm.raw[pw];
            const int L = chunk_len(cx);
            // cumulative log-decay of keys 32 hf + 8q + e (lane: token r16)
            auto decay_scan = [&](int hf, float (&g)[8]) {
                const uint4 wr = ld16_sw<SwDma>(raw[1], r16, 32 * hf + 8 * q);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float ld = log_decay(bf_el8(wr, e));
                    if (L < CH) ld = r16 < L ? ld : 0.f;  // padded steps keep the state
                    g[e] = row_prefix_sum(ld);
                }
            };
            {   // ---- phase 0: V by LDS DMA; keys 0-31: decays and operands ----
                vm_wait0();  // this chunk's inputs (LDS DMA issued in the previous chunk's phase 2)
                stage_plane(S.V, dma_rsrc(v, tbytes), v, chunk_off(cx), voff, rstride, L, lane);
                float g0[8];
                decay_scan(0, g0);
                operands(S, raw, g0, 0);
            }
            lds_barrier();
            {   // ---- phase 1: keys 32-63: decays and operands ----
                float g1[8];
                decay_scan(1, g1);
                operands(S, raw, g1, 1);
            }
            lds_barrier();
            f32x4_t Aak, BrkT;  // phase 2 -> 3
            {   // ---- phase 2: the chunk matrices over the keys, triangular inverse; then
                //      this producer's next chunk by LDS DMA ----
                f32x4_t Aab, AabT, BrbT;
                {
                    uint4 ath[2], atl[2], rth[2], rtl[2], bbh[2], bbl[2], kbh[2], kbl[2];
#pragma unroll
                    for (int hf = 0; hf < 2; hf++) {
                        const int c8 = 32 * hf + 8 * q;
                        ath[hf] = ld16_sw<SwLane>(S.P[0], r16, c8);
                        atl[hf] = ld16_sw<SwLane>(S.P[1], r16, c8);
                        rth[hf] = ld16_sw<SwLane>(S.P2[0], r16, c8);
                        rtl[hf] = ld16_sw<SwLane>(S.P2[1], r16, c8);
                        bbh[hf] = ld16_sw<SwDma>(raw[0], r16, c8);
                        bbl[hf] = ld16_sw<SwDma>(raw[2], r16, c8);
                        kbh[hf] = ld16_sw<SwDma>(raw[3], r16, c8);
                        kbl[hf] = ld16_sw<SwDma>(raw[4], r16, c8);
                    }
                    Aab = mm_keys8(ath, atl, bbh, bbl);
                    AabT = mm_keys8(bbh, bbl, ath, atl);
                    Aak = mm_keys8(ath, atl, kbh, kbl);
                    BrbT = mm_keys8(bbh, bbl, rth, rtl);
                    BrkT = mm_keys8(kbh, kbl, rth, rtl);
                }
                wave_lds_fence();  // staging reads done before the DMA overwrites them
                if (x + NPROD < nstream) {
#pragma unroll
                    for (int ts = 0; ts < 5; ts++)
                        stage_plane(sm.raw[pw][ts], dma_rsrc(src5[ts], tbytes), src5[ts], chunk_off(cy), voff,
                                    rstride, chunk_len(cy), lane);
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {  // D layout: row 4q+e, column r16
                    const int rw = 4 * q + e;
                    if (r16 >= rw) Aab[e] = 0.f, Aak[e] = 0.f;   // [t][s]: s < t
                    if (rw >= r16) AabT[e] = 0.f;                // [s][t]: s < t
                    if (rw > r16) BrbT[e] = 0.f, BrkT[e] = 0.f;  // [s][t]: s <= t
                }
                f32x4_t Ti, TiT;
                tri_inverse(Aab, AabT, lane, Ti, TiT);
                pTiT = pk(TiT);
                pB = pk(BrbT);
            }
            lds_barrier();
            {   // ---- phase 3: Q' = Ti Aak, Q2; P = Ti A~, P2^T = R~^T + P^T Brb^T (R~ read
                //      from the P2 plane first); then V has landed ----
                // Q' (D layout [t][s]) stored as Q'^T [s][t]
                const Pk pq1 = pk(mm16s(pTiT, pk(Aak)));
                st8(&S.Q1T[0][pl16(r16, 4 * q)], pq1.h);
                st8(&S.Q1T[1][pl16(r16, 4 * q)], pq1.l);
                // Q2^T = Brk^T + Q'^T Brb^T  (lane: Q2[t = r16][s = 4q + e])
                const Pk q2 = pk(BrkT + mm16s(pq1, pB));
                st8(&S.Q2[0][pl16(r16, 4 * q)], q2.h);
                st8(&S.Q2[1][pl16(r16, 4 * q)], q2.l);
                p_tiles(S, 0, 4);
#pragma unroll
                for (int tj = 0; tj < 4; tj++) {
                    const uint2 hh = ld8_sw<SwLane>(S.P2[0], r16, 16 * tj + 4 * q);
                    const uint2 ll = ld8_sw<SwLane>(S.P2[1], r16, 16 * tj + 4 * q);
                    f32x4_t rt;
#pragma unroll
                    for (int e = 0; e < 4; e++) rt[e] = bf_el(hh, e) + bf_el(ll, e);
                    const Pk pp = {ldtr_sw<SwLane>(S.P[0], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.P[1], 0, 16 * tj, lane)};
                    const Pk p2 = pk(rt + mm16s(pp, pB));
                    st8_sw<SwLane>(S.P2[0], r16, 16 * tj + 4 * q, p2.h);
                    st8_sw<SwLane>(S.P2[1], r16, 16 * tj + 4 * q, p2.l);
                }
                // V (phase 0) was followed only by the 10 staging DMA ops of phase 2
                if (x + NPROD < nstream) vm_wait10();
                else vm_wait0();
            }
            lds_barrier();
        }
        for (; n < nstream; n++) lds_barrier();  // (ticks after its last chunk)
    } else {
        for (int n = -NPROD; n < 0; n++) lds_barrier();
        // one segment (a head's piece) after another; tick n counts the stream
        const int jlast = (m * sc.L + nstream - 1) / sc.n;
        int n = 0;
        // y of tick nb, written to yq by all four consumer waves before that tick's
        // barrier: wave cw stores its rows 4cw .. 4cw+3, 16 lanes of 8 bytes per row
        uint32_t yrow0 = 0;  // byte offset of that tile's first row, and its valid rows
        int yL = 0;
        const uint32_t ystride = (uint32_t)(H * NK * 2);
        auto y_rows = [&](int nb) {
            const int t = 4 * cw + (lane >> 4), i4 = 4 * (lane & 15);
            const uint2 v = *reinterpret_cast<const uint2*>(&sm.yq[nb & 1][t * NK + i4]);
            store8(y, tbytes, t < yL ? yrow0 + t * ystride + i4 * 2 : OUT_OF_RANGE, v);
        };
        for (int j = m * sc.L / sc.n; j <= jlast; j++) {
          const Seg sg = seg_of(sc, m, j);
          const int sgm = SPLIT ? j / sp.BH : 0;          // (SPLIT: the job's segment and head)
          const int head = SPLIT ? j - sgm * sp.BH : j;
          const int bb = head / H, h = head - bb * H;
          const long bh = head;
          const int c_seg = SPLIT ? seg_first(sgm) : 0;    // the segment's first chunk
          const bool dual = SPLIT && sgm > 0;              // the zero and identity runs
          if (sg.fresh) {  // the initial state: s0 at the head's start ...
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const long off = (long)i_own * NK + 16 * tj + 4 * q;
                float4 x;
                if (!dual) {
                    x = *reinterpret_cast<const float4*>(s0 + bh * NN + off);
                } else {  // zero, and the identity in Sp
                    const int c0 = 16 * tj + 4 * q;
                    x = make_float4(0.f, 0.f, 0.f, 0.f);
                    Sp[tj] = f32x4_t{i_own == c0 ? 1.f : 0.f, i_own == c0 + 1 ? 1.f : 0.f,
                                     i_own == c0 + 2 ? 1.f : 0.f, i_own == c0 + 3 ? 1.f : 0.f};
                }
                St[tj] = f32x4_t{x.x, x.y, x.z, x.w};
            }
          } else {  // ... else the handoff of boundary m + 1
            const float bad = handoff_wait(flags + m + 1, 4) ? 1.f : __builtin_nanf("");
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const float4 x = handoff_get4(hand + (m + 1) * NN + (long)i_own * NK + 16 * tj + 4 * q);
                St[tj] = f32x4_t{x.x, x.y, x.z, x.w} * bad;
            }
          }
          for (int kk = 0; kk < (SPLIT ? nstream : sg.count); kk++, n++) {
            // ---------------- consumer: rows i_own through chunk c of head j ----------------
            const Slot& S = sm.slot[n % NSLOT];
            const int c = sg.step0 + kk + c_seg;
            const int t0 = c * CH, L = min(CH, Tn - t0);
            if (n > 0 && !dual) y_rows(n - 1);  // the previous tick's y
            f32x4_t sa = zero4(), yy = zero4(), sa2 = zero4(), yy2 = zero4();
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
                const uint4 pah = fragp_sw<SwLane>(S.P[0], r16, 32 * s, lane), pal = fragp_sw<SwLane>(S.P[1], r16, 32 * s, lane);
                const uint4 p2h = fragp_sw<SwLane>(S.P2[0], r16, 32 * s, lane), p2l = fragp_sw<SwLane>(S.P2[1], r16, 32 * s, lane);
                sa = mma32(sa, pah, sh);
                sa = mma32(sa, pah, sl);
                sa = mma32(sa, pal, sh);
                yy = mma32(yy, p2h, sh);
                yy = mma32(yy, p2h, sl);
                yy = mma32(yy, p2l, sh);
                if (CKPT && s == 0) {
                    // S_c, the state this tick starts from, saved while these products run,
                    // straight from the registers in the tiled order (one whole KB per
                    // store): 0.327 -> 0.300 ms at config 2 against saving S_{c+1} after
                    // the update through the row regrouping
                    __builtin_amdgcn_sched_barrier(0);
                    float* const dst = ckpt + (bh * ncp + c) * NN + (long)(16 * cw) * NK;
#pragma unroll
                    for (int tj = 0; tj < 4; tj++)
                        *reinterpret_cast<float4*>(dst + (tj * 64 + lane) * 4) =
                            make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (dual) {  // the identity run on the same operand fragments
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        sv[e] = Sp[2 * s][e];
                        sv[4 + e] = Sp[2 * s + 1][e];
                    }
                    pack8(sv, sh, sl);
                    sa2 = mma32(sa2, pah, sh);
                    sa2 = mma32(sa2, pah, sl);
                    sa2 = mma32(sa2, pal, sh);
                    yy2 = mma32(yy2, p2h, sh);
                    yy2 = mma32(yy2, p2h, sl);
                    yy2 = mma32(yy2, p2l, sh);
                }
            }
            // V parts on the K=16 instruction, in their own accumulators
            const uint2 vfr = ldtr_sw<SwDma>(S.V, 0, 16 * cw, lane);  // V[s = 4q+e][i_own]
            {
                f32x4_t sv = mma16(zero4(), ldtr16(S.Q1T[0], 0, lane), vfr);
                sv = mma16(sv, ldtr16(S.Q1T[1], 0, lane), vfr);
                f32x4_t yv = mma16(zero4(), ld8(&S.Q2[0][pl16(r16, 4 * q)]), vfr);
                yv = mma16(yv, ld8(&S.Q2[1][pl16(r16, 4 * q)]), vfr);
                sa += sv;
                yy += yv;
            }
            // S_new^T = S^T diag(e^{gL}) + [B^^T K^^T] [SA; V]   (K = 32: SA rows, then V rows;
            // the identity run has no V rows)
            uint2 sah, sal, sah2, sal2;
            pack4(sa, sah, sal);
            if (dual) pack4(sa2, sah2, sal2);
            const uint4 bhi = cat(sah, vfr), blo = cat(sal, make_uint2(0, 0));
            const uint4 bhi2 = cat(sah2, make_uint2(0, 0)), blo2 = cat(sal2, make_uint2(0, 0));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const uint4 ah = cat(ldtr_sw<SwLane>(S.Bh[0], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Kh[0], 0, 16 * tj, lane));
                const uint4 al = cat(ldtr_sw<SwLane>(S.Bh[1], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Kh[1], 0, 16 * tj, lane));
                const float4 el = *reinterpret_cast<const float4*>(&S.egL[16 * tj + 4 * q]);
                const f32x4_t e4 = {el.x, el.y, el.z, el.w};
                St[tj] = mma32(mma32(mma32(St[tj] * e4, ah, bhi), ah, blo), al, bhi);
                if (dual) Sp[tj] = mma32(mma32(mma32(Sp[tj] * e4, ah, bhi2), ah, blo2), al, bhi2);
            }
            if (!dual) {
                // this tick's y into yq (lane (q, 4m + jj): row 4q + jj, values 16cw + 4m .. +3)
                *reinterpret_cast<uint2*>(&sm.yq[n & 1][(4 * q + (lane & 3)) * NK + 16 * cw + 4 * (r16 >> 2)]) =
                    quad_rows_bf16(yy, lane);
                yrow0 = (uint32_t)(((long)(bb * Tn + t0) * H + h) * NK * 2);
                yL = L;
            } else {  // float32 tiles for split_fixup in the register layout,
                      // [segment - 1][head][chunk in segment][wave][lane][e] = Y[4q + e][i_own]
                const long o = (((((long)(sgm - 1) * sp.BH + head) * sp.m + (c - c_seg)) * 4 + cw) * 64 + lane) * 4;
                *reinterpret_cast<float4*>(sp.y0 + o) = make_float4(yy[0], yy[1], yy[2], yy[3]);
                *reinterpret_cast<float4*>(sp.z + o) = make_float4(yy2[0], yy2[1], yy2[2], yy2[3]);
                yL = 0;  // (nothing for y_rows)
            }
            lds_barrier();
          }
          // the final state, or the handoff at boundary m (its saved state is then made by
          // the workgroup that continues the head, in its first tick)
          if (CKPT && !sg.handoff) FWD_SAVE_STATE(sg.step0 + sg.count);
#pragma unroll
          for (int tj = 0; tj < 4; tj++) {
              const long off = (long)i_own * NK + 16 * tj + 4 * q;
              float* const dst = !SPLIT ? sT : dual ? sp.uend + (long)(sgm - 1) * sp.BH * NN : sp.send0;
              if (sg.handoff) handoff_put4(hand + m * NN + off, St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
              else *reinterpret_cast<float4*>(dst + bh * NN + off) = make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
              if (dual)
                  *reinterpret_cast<float4*>(sp.phi + ((long)(sgm - 1) * sp.BH + bh) * NN + off) =
                      make_float4(Sp[tj][0], Sp[tj][1], Sp[tj][2], Sp[tj][3]);
          }
          if (sg.handoff) handoff_signal(flags + m);
        }
        if (n > 0) y_rows(n - 1);  // the last tick's y (its barrier has passed)
    }
}

int chunk_forward_wait_timeouts(uint32_t* out, int reset) { return wait_timeouts_read(out, reset != 0); }
int chunk_forward_waits(int on) { return wait_switch(on); }

size_t chunk_forward_workspace(int B, int T, int H, int cus) {
    return sched_workspace(plan_schedule(B * H, (T + CH - 1) / CH, cus), NK * NK);
}
void launch_chunk_forward(const Fwd& p, int cus) {
    const Sched sc = plan_schedule(p.B * p.H, (p.T + CH - 1) / CH, cus);
    uint32_t* flags = nullptr;
    float* hand = nullptr;
    if (sched_cuts(sc)) {
        flags = static_cast<uint32_t*>(p.ws);
        hand = reinterpret_cast<float*>(static_cast<char*>(p.ws) + sched_flag_bytes(sc));
        hipLaunchKernelGGL(clear_words, dim3(1), dim3(256), 0, p.stream, flags, sc.G);
    }
    const auto kern = p.ckpt ? chunk_forward_bf16<false, true> : chunk_forward_bf16<false, false>;
    hipLaunchKernelGGL(kern, dim3(sc.G), dim3(512), 0, p.stream, sc, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.s0, (bf16_t*)p.y, p.sT, p.ckpt, flags, hand,
                       SplitArgs{});
}

// ---------------------------------------------------------------------------
// Time-split forward without saved states (few heads): one launch of the k*B*H jobs (one
// workgroup each: the caller checks k*B*H <= CUs), then the fix-up.
// ---------------------------------------------------------------------------
namespace {
constexpr int FXG = 4;       // chunks per split_fixup workgroup (one per wave)
constexpr int FXR = NK + 4;  // padded LDS row (floats)
// Workgroup (group, head), 4 waves, on the matrix cores with split-bf16 operands (hi*hi +
// hi*lo + lo*hi, as in the chunk kernels).  First the state at the start of the group's
// segment s, S_s, is chained in LDS from S_1 = send0: S_{u+1} = S_u Phi_u + U_u, wave w
// forming rows 16w .. 16w+15.  The last group stores S_k as sT.  The others: wave w takes
// chunk 4 (group mod groups per segment) + w of segment s and forms
// Y[t][i] = y0[t][i] + sum_j z[t][j] S_s[i][j]: its z tile turned into rows through the
// wave's LDS, y0 read straight in the accumulator layout, y out in whole 128-byte rows.
__global__ __launch_bounds__(256) void split_fixup(int Tn, int H, SplitArgs sp, bf16_t* __restrict__ y,
                                                   float* __restrict__ sT) {
    __shared__ float st[NK * FXR];           // S_s [i][j]
    __shared__ float zt[FXG][CH * FXR];      // per wave: its z tile as rows [t][j]
    __shared__ uint16_t yt[FXG][CH * NK];    // per wave: its y tile [t][i]
    const int ngm = (sp.m + FXG - 1) / FXG;  // chunk groups per segment
    const int grp = blockIdx.x, head = blockIdx.y, bb = head / H, h = head - bb * H;
    const bool last = grp == (sp.k - 1) * ngm;
    const int sgm = last ? sp.k : 1 + grp / ngm;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, r16 = lane & 15;
    const long NN = NK * NK;
    // 8 consecutive floats as split-bf16 operand halves
    auto op8 = [](const float* p, uint4& hi, uint4& lo) {
        const float4 x0 = *reinterpret_cast<const float4*>(p), x1 = *reinterpret_cast<const float4*>(p + 4);
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        pack8(v, hi, lo);
    };
    // rows 16w .. 16w+15 of S_1 (float4 number u*64 + lane of the strip)
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int f = 4 * (u * 64 + lane), r = 16 * w + f / NK, c = f % NK;
        *reinterpret_cast<float4*>(&st[r * FXR + c]) =
            *reinterpret_cast<const float4*>(sp.send0 + head * NN + r * NK + c);
    }
    wave_lds_fence();
    for (int u = 1; u < sgm; u++) {  // S_{u+1} = S_u Phi_u + U_u, this wave's rows
        const long o = ((long)(u - 1) * sp.BH + head) * NN;
        uint4 ah[2], al[2];  // A operand S_u: lane (q, r16) holds S_u[16w + r16][32t + 8q .. +7]
#pragma unroll
        for (int t = 0; t < 2; t++) op8(&st[(16 * w + r16) * FXR + 32 * t + 8 * q], ah[t], al[t]);
        wave_lds_fence();  // (the strip is overwritten below)
#pragma unroll
        for (int n = 0; n < 4; n++) {
            f32x4_t acc;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = sp.uend[o + (16 * w + 4 * q + e) * NK + 16 * n + r16];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                float v[8];  // B operand Phi_u: lane (q, r16) holds Phi_u[32t + 8q .. +7][16n + r16]
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = sp.phi[o + (32 * t + 8 * q + e) * NK + 16 * n + r16];
                uint4 bh, bl;
                pack8(v, bh, bl);
                acc = mma32(acc, ah[t], bh);
                acc = mma32(acc, ah[t], bl);
                acc = mma32(acc, al[t], bh);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) st[(16 * w + 4 * q + e) * FXR + 16 * n + r16] = acc[e];
        }
        wave_lds_fence();
    }
    if (last) {  // sT = S_k, this wave's rows
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int f = 4 * (u * 64 + lane), r = 16 * w + f / NK, c = f % NK;
            *reinterpret_cast<float4*>(sT + head * NN + r * NK + c) = *reinterpret_cast<const float4*>(&st[r * FXR + c]);
        }
        return;
    }
    __syncthreads();  // all of S_s
    const int c = (grp % ngm) * FXG + w;  // chunk within segment sgm (wave-uniform)
    const int cfirst = sp.m0 + (sgm - 1) * sp.m;  // the segment's first chunk
    if (c >= sp.m || CH * (cfirst + c) >= Tn) return;
    // B operand S_s^T: lane (q, r16) of tile n, K step t holds S_s[16n + r16][32t + 8q .. +7]
    uint4 bh[4][2], bl[4][2];
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
        for (int t = 0; t < 2; t++) op8(&st[(16 * n + r16) * FXR + 32 * t + 8 * q], bh[n][t], bl[n][t]);
    // the z tile (float4 u*64 + lane holds Z[4q + e][16u + r16]) into rows
    const long tile = (((long)(sgm - 1) * sp.BH + head) * sp.m + c) * 256;  // float4 index of the chunk's tile
    float* const zw = zt[w];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const float4 x = reinterpret_cast<const float4*>(sp.z)[tile + u * 64 + lane];
        float* const d = zw + 4 * q * FXR + 16 * u + r16;
        d[0] = x.x, d[FXR] = x.y, d[2 * FXR] = x.z, d[3 * FXR] = x.w;
    }
    wave_lds_fence();
    uint4 ah[2], al[2];  // A operand Z: lane (q, r16) holds Z[r16][32t + 8q .. +7]
#pragma unroll
    for (int t = 0; t < 2; t++) op8(zw + r16 * FXR + 32 * t + 8 * q, ah[t], al[t]);
    uint16_t* const yw = yt[w];
#pragma unroll
    for (int n = 0; n < 4; n++) {
        const float4 x = reinterpret_cast<const float4*>(sp.y0)[tile + n * 64 + lane];  // y0[4q + e][16n + r16]
        f32x4_t acc = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int t = 0; t < 2; t++) {
            acc = mma32(acc, ah[t], bh[n][t]);
            acc = mma32(acc, ah[t], bl[n][t]);
            acc = mma32(acc, al[t], bh[n][t]);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) yw[(4 * q + e) * NK + 16 * n + r16] = f32_to_bf16(acc[e]);
    }
    wave_lds_fence();
    // 16 rows of 128 bytes: 8 lanes per row, two rows per lane
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        const int rr = 8 * hf + (lane >> 3), pc = lane & 7, tabs = CH * (cfirst + c) + rr;
        if (tabs < Tn)
            *reinterpret_cast<uint4*>(y + ((long)(bb * Tn + tabs) * H + h) * NK + 8 * pc) =
                *reinterpret_cast<const uint4*>(&yw[rr * NK + 8 * pc]);
    }
}

// Lengths of k segments over n chunks: segment 0 (one state per consumer wave) ticks about
// 1.2x faster than the others (two states; measured per workgroup at T=4096: 1.59 against
// 1.90 us with 80 heads, 1.45 against 1.71 with 16), so m0 = n - (k-1) m chunks go to it
// with m minimising max(5 m0, 6 m); every segment holds at least one chunk and none runs
// past the end.
void split_lengths(int n, int k, int& m0, int& m) {
    int best = 1 << 30;
    m0 = n, m = 0;
    for (int mm = 1; n - (k - 1) * mm >= 1; mm++) {
        const int r = n - (k - 1) * mm, cost = max(5 * r, 6 * mm);
        if (cost < best) best = cost, m0 = r, m = mm;
    }
}
}  // namespace

// Segments of the time-split forward for B*H heads of n chunks on `cus` CUs: as many as fit
// one job per CU, at most 4 (the fix-up chains the segments' transitions one after another),
// each with at least one valid chunk; 1 = no split.
int chunk_forward_split_segments(int BH, int T, int cus) {
    const int n = (T + CH - 1) / CH;
    const int k = BH > 0 ? min(4, cus / BH) : 1;
    return max(1, min(k, n));
}
size_t chunk_forward_split_workspace(int B, int T, int H, int cus) {
    const int BH = B * H, k = chunk_forward_split_segments(BH, T, cus);
    if (k < 2) return 0;
    int m0, m;
    split_lengths((T + CH - 1) / CH, k, m0, m);
    return (size_t)BH * ((2 * k - 1) * (size_t)NK * NK + 2 * (k - 1) * (size_t)m * CH * NK) * sizeof(float);
}
void launch_chunk_forward_split(const Fwd& p, int cus) {
    SplitArgs sp;
    sp.BH = p.B * p.H, sp.k = chunk_forward_split_segments(sp.BH, p.T, cus);
    split_lengths((p.T + CH - 1) / CH, sp.k, sp.m0, sp.m);
    const size_t NN = (size_t)NK * NK, per = (size_t)(sp.k - 1) * sp.BH;
    float* const base = static_cast<float*>(p.ws);
    sp.send0 = base, sp.uend = base + sp.BH * NN, sp.phi = sp.uend + per * NN;
    sp.y0 = sp.phi + per * NN, sp.z = sp.y0 + per * sp.m * CH * NK;
    // one job per workgroup, no cuts (jobs planned at the longest segment; each runs its own)
    const Sched sc = plan_schedule(sp.k * sp.BH, max(sp.m0, sp.m), cus);
    hipLaunchKernelGGL((chunk_forward_bf16<true, false>), dim3(sc.G), dim3(512), 0, p.stream, sc, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.s0, (bf16_t*)p.y, p.sT, nullptr, nullptr,
                       nullptr, sp);
    // chunk groups of segments 1 .. k-1, then one for the final state; heads along y
    hipLaunchKernelGGL(split_fixup, dim3((sp.k - 1) * ((sp.m + FXG - 1) / FXG) + 1, sp.BH), dim3(256), 0,
                       p.stream, p.T, p.H, sp, (bf16_t*)p.y, p.sT);
}

}  // namespace wkv7
