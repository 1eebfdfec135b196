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
//    chunk x-5).  Their outputs leave in whole 128-byte rows: y through LDS,
//    stored a tick late by all four waves, and each wave's saved-state rows
//    regrouped eight at a time.
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
// Outputs leave in whole rows: a wave's own pieces are 32-byte (y) and 64-byte (saved
// states) parts of 128-byte lines, and stores of such parts cost far more than their
// bytes (measured: the forward ran 7 % and 6 % faster with each regrouped).
constexpr int LDR = NK + 4;  // padded row (floats) of the saved-state regrouping planes
struct FwdLds {
    Slot slot[NSLOT];
    Plane raw[NPROD][5];     // producer input staging: r, w, k, a, b (SwDma)
    uint16_t yq[2][CH * NK]; // y tiles of the last two ticks [t][i], stored a tick late
    float sq[4][8 * LDR];    // per consumer wave: 8 of its 16 saved-state rows at a time
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
// it, so with few heads each head's chunks are halved and the halves run at once, as
// three jobs per head: run 0 = chunks [0, m) from s0; run 1 = chunks [m, 2m) from a zero
// state; run 2 = chunks [m, 2m) from the identity with v = 0, whose "y" is z_t = Phi_t r_t
// and whose final state is the transition Phi of the second half.  split_fixup then
// forms y_t = y0_t + S_m z_t and sT = S_m Phi + S0_end (wkv7_capi.cpp decides when).
struct SplitArgs {
    int BH = 0, m = 0;
    float* sm = nullptr;     // run 0's final states [BH][64][64]
    float* s0end = nullptr;  // run 1's final states
    float* phi = nullptr;    // run 2's final states
    float* y0 = nullptr;     // run 1's y tiles [BH][m][4 waves][64 lanes][4] float32
    float* z = nullptr;      // run 2's y tiles, the same layout
};

template <bool SPLIT>
__global__ __launch_bounds__(512) void chunk_forward_bf16(
    Sched sc, int Tn, int H, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
    const bf16_t* __restrict__ b, const float* __restrict__ s0, bf16_t* __restrict__ y,
    float* __restrict__ sT, float* __restrict__ ckpt, uint32_t* __restrict__ flags, float* __restrict__ hand,
    SplitArgs sp) {
    __shared__ FwdLds sm;
    const int m = machine_of_block(sc), nstream = stream_len(sc, m);
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int lane = tid & 63, q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    const long ncp = ckpt_count(Tn);
    const bool producer = wv < NPROD;
    const int pw = wv, cw = wv - NPROD;
    const long rstride = (long)H * NK;                              // between consecutive tokens of one head
    // bytes of one [B,T,H,64] tensor (SPLIT: the schedule's jobs are three per head)
    const uint32_t tbytes = (uint32_t)((long)(SPLIT ? sp.BH : sc.J) * Tn * NK * 2);
    // stream position (cursor) -> byte offset of the chunk's first row, its valid length
    // (SPLIT: job j is run j / BH of head j % BH; runs 1 and 2 start at chunk m)
    auto run_of = [&](int j) { return SPLIT ? j / sp.BH : 0; };
    auto chunk_off = [&](const Cursor& cu) {
        if (!SPLIT) return (uint32_t)(((long)(cu.bb * Tn + cu.step * CH) * H + cu.h) * NK * 2);
        const int run = run_of(cu.j), head = cu.j - run * sp.BH, b2 = head / H, h2 = head - b2 * H;
        return (uint32_t)(((long)(b2 * Tn + (cu.step + (run ? sp.m : 0)) * CH) * H + h2) * NK * 2);
    };
    auto chunk_len = [&](const Cursor& cu) {
        return min(CH, Tn - (cu.step + (SPLIT && run_of(cu.j) ? sp.m : 0)) * CH);
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
    f32x4_t St[4];
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
                // (run 2 of the time split: v = 0)
                stage_plane(S.V, dma_rsrc(v, tbytes), v, chunk_off(cx), voff, rstride,
                            SPLIT && run_of(cx.j) == 2 ? 0 : L, lane);
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
          const int run = SPLIT ? j / sp.BH : 0;           // (SPLIT: the job's run and head)
          const int head = SPLIT ? j - run * sp.BH : j;
          const int bb = head / H, h = head - bb * H;
          const long bh = head;
          const int c_run = SPLIT && run ? sp.m : 0;      // the run's first chunk
          if (sg.fresh) {  // the initial state: s0 at the head's start ...
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const long off = (long)i_own * NK + 16 * tj + 4 * q;
                float4 x;
                if (!SPLIT || run == 0) {
                    x = *reinterpret_cast<const float4*>(s0 + bh * NN + off);
                } else {  // run 1: zero; run 2: the identity
                    const int c0 = 16 * tj + 4 * q;
                    const float one = run == 2 ? 1.f : 0.f;
                    x = make_float4(i_own == c0 ? one : 0.f, i_own == c0 + 1 ? one : 0.f,
                                    i_own == c0 + 2 ? one : 0.f, i_own == c0 + 3 ? one : 0.f);
                }
                St[tj] = f32x4_t{x.x, x.y, x.z, x.w};
                if (ckpt) *reinterpret_cast<float4*>(ckpt + bh * ncp * NN + off) = x;
            }
          } else {  // ... else the handoff of boundary m + 1
            const float bad = handoff_wait(flags + m + 1, 4) ? 1.f : __builtin_nanf("");
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const float4 x = handoff_get4(hand + (m + 1) * NN + (long)i_own * NK + 16 * tj + 4 * q);
                St[tj] = f32x4_t{x.x, x.y, x.z, x.w} * bad;
            }
          }
          for (int kk = 0; kk < sg.count; kk++, n++) {
            // ---------------- consumer: rows i_own through chunk c of head j ----------------
            const Slot& S = sm.slot[n % NSLOT];
            const int c = sg.step0 + kk + c_run;
            const int t0 = c * CH, L = min(CH, Tn - t0);
            if (n > 0) y_rows(n - 1);  // the previous tick's y
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
                const uint4 pah = fragp_sw<SwLane>(S.P[0], r16, 32 * s, lane), pal = fragp_sw<SwLane>(S.P[1], r16, 32 * s, lane);
                const uint4 p2h = fragp_sw<SwLane>(S.P2[0], r16, 32 * s, lane), p2l = fragp_sw<SwLane>(S.P2[1], r16, 32 * s, lane);
                sa = mma32(sa, pah, sh);
                sa = mma32(sa, pah, sl);
                sa = mma32(sa, pal, sh);
                yy = mma32(yy, p2h, sh);
                yy = mma32(yy, p2h, sl);
                yy = mma32(yy, p2l, sh);
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
            // S_new^T = S^T diag(e^{gL}) + [B^^T K^^T] [SA; V]   (K = 32: SA rows, then V rows)
            uint2 sah, sal;
            pack4(sa, sah, sal);
            const uint4 bhi = cat(sah, vfr), blo = cat(sal, make_uint2(0, 0));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const uint4 ah = cat(ldtr_sw<SwLane>(S.Bh[0], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Kh[0], 0, 16 * tj, lane));
                const uint4 al = cat(ldtr_sw<SwLane>(S.Bh[1], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Kh[1], 0, 16 * tj, lane));
                const float4 el = *reinterpret_cast<const float4*>(&S.egL[16 * tj + 4 * q]);
                St[tj] = mma32(mma32(mma32(St[tj] * f32x4_t{el.x, el.y, el.z, el.w}, ah, bhi), ah, blo), al, bhi);
            }
            if (!SPLIT || run == 0) {
                // this tick's y into yq (lane (q, 4m + jj): row 4q + jj, values 16cw + 4m .. +3)
                *reinterpret_cast<uint2*>(&sm.yq[n & 1][(4 * q + (lane & 3)) * NK + 16 * cw + 4 * (r16 >> 2)]) =
                    quad_rows_bf16(yy, lane);
                yrow0 = (uint32_t)(((long)(bb * Tn + t0) * H + h) * NK * 2);
                yL = L;
            } else {  // runs 1 and 2: float32 tiles for split_fixup in the register layout,
                      // [head][chunk - m][wave][lane][e] = Y[4q + e][i_own] (1 KB per wave)
                float* const yd = (run == 1 ? sp.y0 : sp.z) + ((((long)head * sp.m + (c - sp.m)) * 4 + cw) * 64 + lane) * 4;
                *reinterpret_cast<float4*>(yd) = make_float4(yy[0], yy[1], yy[2], yy[3]);
                yL = 0;  // (nothing for y_rows)
            }
            if (ckpt) {  // S_{c+1}: this wave's rows, 8 at a time through sq, 4 whole rows per store
                float* const sq = sm.sq[cw];
                float* const dst = ckpt + (bh * ncp + c + 1) * NN + (long)(16 * cw) * NK;
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    if ((r16 >> 3) == p) {
#pragma unroll
                        for (int tj = 0; tj < 4; tj++)
                            *reinterpret_cast<float4*>(sq + (r16 & 7) * LDR + 16 * tj + 4 * q) =
                                make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
                    }
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        const int rr = 4 * u + (lane >> 4), cc = 4 * (lane & 15);
                        *reinterpret_cast<float4*>(dst + (8 * p + rr) * NK + cc) = *reinterpret_cast<const float4*>(sq + rr * LDR + cc);
                    }
                }
            }
            lds_barrier();
          }
          // the final state, or the handoff at boundary m
#pragma unroll
          for (int tj = 0; tj < 4; tj++) {
              const long off = (long)i_own * NK + 16 * tj + 4 * q;
              float* const dst = !SPLIT || run == 0 ? (SPLIT ? sp.sm : sT) : run == 1 ? sp.s0end : sp.phi;
              if (sg.handoff) handoff_put4(hand + m * NN + off, St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
              else *reinterpret_cast<float4*>(dst + bh * NN + off) = make_float4(St[tj][0], St[tj][1], St[tj][2], St[tj][3]);
          }
          if (sg.handoff) handoff_signal(flags + m);
        }
        if (n > 0) y_rows(n - 1);  // the last tick's y (its barrier has passed)
    }
}

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
    hipLaunchKernelGGL(chunk_forward_bf16<false>, dim3(sc.G), dim3(512), 0, p.stream, sc, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.s0, (bf16_t*)p.y, p.sT, p.ckpt, flags, hand,
                       SplitArgs{});
}

// ---------------------------------------------------------------------------
// Time-split forward without saved states (few heads): one launch of the three runs
// (3 B*H jobs, one workgroup each: the caller checks 3 B*H <= CUs), then the fix-up.
// Workspace: S_m, S0_end, Phi ([B*H][64][64] each), y0 and z ([B*H][m][16 * 64]).
// ---------------------------------------------------------------------------
namespace {
constexpr int FXG = 4;       // chunks per split_fixup workgroup (one per wave)
constexpr int FXR = NK + 4;  // padded LDS row (floats)
// y_t = bf16(y0_t + S_m z_t) over the second half's steps, and sT = S_m Phi + S0_end, on
// the matrix cores with split-bf16 operands (hi*hi + hi*lo + lo*hi, as in the chunk
// kernels).  Workgroup (group, head), 4 waves.  Groups below the last: wave w takes
// chunk 4 group + w: Y[t][i] = y0 + sum_k Z[t][k] S_m[i][k], its z tile turned into rows
// through the wave's LDS, y0 read straight in the accumulator layout, y out in whole
// 128-byte rows through LDS.  The last group: wave w takes final-state rows 16w .. 16w+15.
__global__ __launch_bounds__(256) void split_fixup(int Tn, int H, int m, const float* __restrict__ sm,
                                                   const float* __restrict__ s0end, const float* __restrict__ phi,
                                                   const float* __restrict__ y0, const float* __restrict__ z,
                                                   bf16_t* __restrict__ y, float* __restrict__ sT) {
    __shared__ float zt[FXG][CH * FXR];      // per wave: its z tile as rows [t][k]
    __shared__ uint16_t yt[FXG][CH * NK];    // per wave: its y tile [t][i]
    const int grp = blockIdx.x, ngrp = gridDim.x - 1, head = blockIdx.y, bb = head / H, h = head - bb * H;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, r16 = lane & 15;
    const long NN = NK * NK;
    const float* const S = sm + head * NN;
    // 8 consecutive floats as split-bf16 operand halves
    auto op8 = [](const float* p, uint4& hi, uint4& lo) {
        const float4 x0 = *reinterpret_cast<const float4*>(p), x1 = *reinterpret_cast<const float4*>(p + 4);
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        pack8(v, hi, lo);
    };
    if (grp < ngrp) {
        const int c = grp * FXG + w;  // chunk of the second half (wave-uniform)
        if (c >= m) return;
        // B operand S_m^T: lane (q, r16) of tile n, K step s holds S_m[16n + r16][32s + 8q .. +7]
        uint4 bh[4][2], bl[4][2];
#pragma unroll
        for (int n = 0; n < 4; n++)
#pragma unroll
            for (int s = 0; s < 2; s++) op8(S + (16 * n + r16) * NK + 32 * s + 8 * q, bh[n][s], bl[n][s]);
        // the z tile (float4 u*64 + lane holds Z[4q + e][16u + r16]) into rows
        const long tile = ((long)head * m + c) * 256;  // float4 index of the chunk's tile
        float* const zw = zt[w];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float4 x = reinterpret_cast<const float4*>(z)[tile + u * 64 + lane];
            float* const d = zw + 4 * q * FXR + 16 * u + r16;
            d[0] = x.x, d[FXR] = x.y, d[2 * FXR] = x.z, d[3 * FXR] = x.w;
        }
        wave_lds_fence();
        uint4 ah[2], al[2];  // A operand Z: lane (q, r16) holds Z[r16][32s + 8q .. +7]
#pragma unroll
        for (int s = 0; s < 2; s++) op8(zw + r16 * FXR + 32 * s + 8 * q, ah[s], al[s]);
        uint16_t* const yw = yt[w];
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const float4 x = reinterpret_cast<const float4*>(y0)[tile + n * 64 + lane];  // y0[4q + e][16n + r16]
            f32x4_t acc = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int s = 0; s < 2; s++) {
                acc = mma32(acc, ah[s], bh[n][s]);
                acc = mma32(acc, ah[s], bl[n][s]);
                acc = mma32(acc, al[s], bh[n][s]);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) yw[(4 * q + e) * NK + 16 * n + r16] = f32_to_bf16(acc[e]);
        }
        wave_lds_fence();
        // 16 rows of 128 bytes: 8 lanes per row, two rows per lane
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            const int rr = 8 * hf + (lane >> 3), pc = lane & 7, tabs = CH * (m + c) + rr;
            if (tabs < Tn)
                *reinterpret_cast<uint4*>(y + ((long)(bb * Tn + tabs) * H + h) * NK + 8 * pc) =
                    *reinterpret_cast<const uint4*>(&yw[rr * NK + 8 * pc]);
        }
    } else {
        // rows i = 16w + 4q + e, columns j = 16n + r16:  sT = S0_end + S_m Phi
        uint4 ah[2], al[2];  // A operand S_m: lane (q, r16) holds S_m[16w + r16][32s + 8q .. +7]
#pragma unroll
        for (int s = 0; s < 2; s++) op8(S + (16 * w + r16) * NK + 32 * s + 8 * q, ah[s], al[s]);
        const float* const P = phi + head * NN;
#pragma unroll
        for (int n = 0; n < 4; n++) {
            f32x4_t acc;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = s0end[head * NN + (16 * w + 4 * q + e) * NK + 16 * n + r16];
#pragma unroll
            for (int s = 0; s < 2; s++) {
                float v[8];  // B operand Phi: lane (q, r16) holds Phi[32s + 8q .. +7][16n + r16]
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = P[(32 * s + 8 * q + e) * NK + 16 * n + r16];
                uint4 bh, bl;
                pack8(v, bh, bl);
                acc = mma32(acc, ah[s], bh);
                acc = mma32(acc, ah[s], bl);
                acc = mma32(acc, al[s], bh);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) sT[head * NN + (16 * w + 4 * q + e) * NK + 16 * n + r16] = acc[e];
        }
    }
}
}  // namespace

// m = ceil(chunks / 2): runs 1 and 2 end with an empty chunk when the count is odd
// (its steps are padding, which keeps the state)
size_t chunk_forward_split_workspace(int B, int T, int H) {
    const size_t BH = (size_t)B * H, m = ((size_t)(T + CH - 1) / CH + 1) / 2;
    return BH * (3 * NK * NK + 2 * 16 * m * NK) * sizeof(float);
}
void launch_chunk_forward_split(const Fwd& p, int cus) {
    const int BH = p.B * p.H, m = ((p.T + CH - 1) / CH + 1) / 2;
    float* const base = static_cast<float*>(p.ws);
    SplitArgs sp;
    sp.BH = BH, sp.m = m;
    sp.sm = base, sp.s0end = base + (size_t)BH * NK * NK, sp.phi = base + 2 * (size_t)BH * NK * NK;
    sp.y0 = base + 3 * (size_t)BH * NK * NK, sp.z = sp.y0 + (size_t)BH * 16 * m * NK;
    const Sched sc = plan_schedule(3 * BH, m, cus);  // 3 B*H <= cus: one job per workgroup, no cuts
    hipLaunchKernelGGL(chunk_forward_bf16<true>, dim3(sc.G), dim3(512), 0, p.stream, sc, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.s0, (bf16_t*)p.y, p.sT, nullptr, nullptr,
                       nullptr, sp);
    // groups of FXG chunks, then one for the final state; heads along y (at most cus / 3)
    hipLaunchKernelGGL(split_fixup, dim3((m + FXG - 1) / FXG + 1, BH), dim3(256), 0, p.stream, p.T, p.H, m, sp.sm,
                       sp.s0end, sp.phi, sp.y0, sp.z, (bf16_t*)p.y, p.sT);
}

}  // namespace wkv7
