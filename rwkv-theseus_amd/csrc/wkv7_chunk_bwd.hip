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
// Mapping: 704-lane workgroups, one per CU, each running a stream of chunks
// (b,h heads one after another, chunks of a head in reverse; the first and last
// pieces of a head may be shared with another workgroup: wkv7_sched.h), in
// lock-step ticks that end in one LDS barrier (no global-memory fence).
//  * Producers (waves 8-10) build everything that depends only on a chunk's
//    inputs -- A~, R~, B-, K-, g, e^{gL}, Ti, Aak, Brb, Brk, triu(V dY^T) -- one
//    chunk each, in three phases over the three ticks before it is consumed,
//    into a 3-slot LDS ring.  Their inputs arrive by LDS DMA two ticks ahead, so
//    no prefetch registers are held across ticks.  Each producer runs one
//    chunk's three phases in sequence; phase 0 may not write the slot (the
//    consumers still read it in that tick), so the operands of the first 32
//    keys it computes wait in registers until phase 1.
//  * Consumers, 8 waves in two sides.  The H side (waves 0-3: wave c owns value
//    rows 16c..16c+15 of H = dL/dS in registers) forms H', Q and the first part
//    of dV in stage B and publishes H' and Q^T rows; the S side (waves 4-7, the
//    same rows of the saved state S0, loaded a tick ahead) forms SA and
//    publishes SA^T rows.  The eight meet on an LDS counter (the producers do
//    not take part); in stage C wave c of each side produces key strip
//    16c..16c+15 of its gradients (H side dK, dB; S side dR, dA, dw) contracting
//    over all value rows in a fixed order (deterministic; the reference
//    accumulates with fp32 atomics, cu:68-72), reading the other orientation of
//    each exchanged matrix with ds_read_b64_tr_b16; the H side also finishes dV
//    and advances H to the previous chunk.
#include "wkv7_launch.h"
#include "wkv7_io.h"
#include "wkv7_sched.h"

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
// The consumers' exchange planes come first: LDS instructions reach 64 KB past
// their address register, so planes at fixed offsets below that share one
// lane-offset register per access pattern (and the slots are addressed from a
// per-tick base).
struct BwdLds {
    uint16_t Hx[2][NK * NK];                     // H' [i][j] (swizzled)
    uint16_t QT[2][NK * LDQ], SAT[2][NK * LDQ];  // Q^T, SA^T [i][t]
    float dlp[2][4][64 * 4];                     // H side's dlogd terms z_t of a chunk, per key strip
    Mat Mq[3];                                   // a tick's masked XM, M1^T and N1 (split), formed once
    Slot slot[NPROD];
    Plane raw[NPROD][5];                         // producer input staging: r, w, k, a, b
    uint32_t csync;                              // consumers' mid-tick rendezvous counter
};
static_assert(sizeof(BwdLds) <= 160 * 1024, "backward LDS budget");
// 16-byte LDS accesses and DMA rows need 16-byte aligned planes
static_assert(offsetof(BwdLds, slot) % 256 == 0 && sizeof(Slot) % 16 == 0 && offsetof(BwdLds, raw) % 16 == 0 &&
                  offsetof(Slot, g) % 16 == 0 && offsetof(Slot, egL) % 16 == 0 && offsetof(BwdLds, dlp) % 16 == 0,
              "backward LDS alignment");

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
// The consumer waves' mid-tick rendezvous (their exchange planes written before,
// read after): each of the 8 counts itself in on an LDS counter and waits for the
// tick's total.  The producers do not take part, so their work is not cut in two
// by it.  The wait is bounded (a wave that never arrives cannot hang the kernel);
// it returns false on time-out, and the waves then write NaN in place of every
// gradient from that tick on (the `bad` flag below), so a broken rendezvous can
// never pass for a result.  The count is read through readfirstlane, so the
// outcome is wave-uniform and the poisoning is a scalar branch.
constexpr int NCONS = 8;
// `lim` is the spin bound, wait_bound(1 << 22) read once per kernel.
__device__ __forceinline__ bool consumer_sync(uint32_t* cnt, uint32_t target, int lim) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS writes are done
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    bool ok = false;
    for (int i = 0; i < lim; i++) {
        if (__builtin_amdgcn_readfirstlane(
                __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) >= target) {
            ok = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
    if (!ok) note_timeout();
    return ok;
}
__device__ __forceinline__ f32x4_t nan4() {
    const float x = __builtin_nanf("");
    return f32x4_t{x, x, x, x};
}
// split-precision K=32 product (both operands split)
__device__ __forceinline__ f32x4_t mm32s(uint4 ah, uint4 al, uint4 bh, uint4 bl) {
    // one accumulator chain: no VALU adds (the VALU, not the matrix pipe, is the busier)
    return mma32(mma32(mma32(zero4(), ah, bh), ah, bl), al, bh);
}
// acc + A B for packed tiles (split precision), one accumulator chain
__device__ __forceinline__ f32x4_t mm16s_acc(f32x4_t acc, const Pk& A, const Pk& B) {
    return mma16(mma16(mma16(acc, A.h, B.h), A.h, B.l), A.l, B.h);
}
// X Y^T over 64 keys, both in the K=32 operand layout (x[hf] = X[t][32hf + 8q ..])
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

__global__ __launch_bounds__(704) void chunk_backward_bf16(
    Sched sc, int Tn, int H, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ a,
    const bf16_t* __restrict__ b, const float* __restrict__ ckpt, const bf16_t* __restrict__ dy,
    const float* __restrict__ dsT, bf16_t* __restrict__ dr, bf16_t* __restrict__ dw,
    bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, bf16_t* __restrict__ da,
    bf16_t* __restrict__ db, float* __restrict__ ds0, uint32_t* __restrict__ flags, float* __restrict__ hand) {
    __shared__ BwdLds sm;
    const int m = machine_of_block(sc), nstream = stream_len(sc, m);
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    int lane = tid & 63, q = lane >> 4, r16 = lane & 15;
    const long NN = (long)NK * NK;
    const long NH = NN + NK;  // handoff per boundary: H (dL/dS), then the dlogd carry
    const long ncp = ckpt_count(Tn);
    const int nchunk = sc.n;
    const bool consumer = wv < 8;
    const bool hside = wv < 4;  // consumer: owner of H (else the S0 side)
    const int cw = wv & 3;      // consumer: value-row block / key strip
    const int pw = wv - 8;      // producer index
    int i_own = 16 * cw + r16;
    int j_own = 16 * cw + r16;
    const int lane0 = lane;
    const long rstride = (long)H * NK;  // between consecutive tokens of one head

    // stream index x -> (head, chunk): step s of a head is its chunk nchunk-1-s
    auto chunk_at = [&](int x) {
        const int2 js = stream_at(sc, m, x);
        return make_int2(js.x, nchunk - 1 - js.y);
    };
    // stream position (cursor) -> byte offset of the chunk's first row, its valid length
    auto chunk_off = [&](const Cursor& cu) {
        return (uint32_t)(((long)(cu.bb * Tn + (nchunk - 1 - cu.step) * CH) * H + cu.h) * NK * 2);
    };
    auto chunk_len = [&](const Cursor& cu) { return min(CH, Tn - (nchunk - 1 - cu.step) * CH); };
    const uint32_t tbytes = (uint32_t)((long)sc.J * Tn * NK * 2);  // bytes of one [B,T,H,64] tensor
    // byte offset for the 8-byte row piece of a D-layout tile of chunk cc of head (bb, h):
    // lane (q, 4m + jj) stores row 4q + jj, columns 16 cw + 4m .. +3 (rows past the end: dropped)
    auto piece_off = [&](int bb, int h, int cc) {
        const int tr = 4 * q + (lane & 3);
        return tr < min(CH, Tn - cc * CH)
                   ? (uint32_t)((((long)(bb * Tn + cc * CH + tr) * H + h) * NK + 16 * cw + 4 * (r16 >> 2)) * 2)
                   : OUT_OF_RANGE;
    };
    // dw of a chunk: dlogd_t = carry + sum_{s>=t} z_s + sum_{s>t} t2_s over the chunk
    // (t = 4q + e), times fw_t = d w_t / d logd_t; the carry moves on to the chunk before
    auto dlogd_part = [&](const float (&z)[4], const float (&t2)[4], const float (&fw)[4], float& carry, float (&gw)[4]) {
        float tot = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) tot += z[e] + t2[e];
        // the other lane groups' totals s_q' (same column) by row swaps in the VALU (gfx950
        // permlane16/32_swap, layout checked with an in-bounds probe): od = s of the odd row
        // of this lane's row pair, lo / hi = s0 + s1 / s2 + s3 in every lane
        const uint32_t tb = __float_as_uint(tot);
        const auto p16 = __builtin_amdgcn_permlane16_swap(tb, tb, false, false);
        const float ev = __uint_as_float(p16[0]), od = __uint_as_float(p16[1]);
        const uint32_t pb = __float_as_uint(ev + od);
        const auto p32 = __builtin_amdgcn_permlane32_swap(pb, pb, false, false);
        const float lo = __uint_as_float(p32[0]), hi = __uint_as_float(p32[1]);
        float run = carry + ((q & 1) ? 0.f : od) + (q < 2 ? hi : 0.f);  // + sum over groups after q
#pragma unroll
        for (int e = 3; e >= 0; e--) {
            run += z[e];
            gw[e] = run * fw[e];
            run += t2[e];
        }
        carry += lo + hi;
    };
    // the per-lane quantities of stage C that depend on the slot only:
    // [A~; R~] and [B-; K-] strips as K=32 B operands, g_t (t = 4q + e); the S side
    // also needs g_{t-1} and fw_t = d w_t / d logd_t (strip_fw)
    struct Strip {
        uint4 arh, arl, bkh, bkl;
        float gv[4], gp[4], fw[4];
    };
    auto strip = [&](const Slot& S) {
        Strip st;
        st.arh = cat(ldtr_sw<SwLane>(S.At[0], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Rt[0], 0, 16 * cw, lane));
        st.arl = cat(ldtr_sw<SwLane>(S.At[1], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Rt[1], 0, 16 * cw, lane));
        st.bkh = cat(ldtr_sw<SwLane>(S.Bb[0], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Kb[0], 0, 16 * cw, lane));
        st.bkl = cat(ldtr_sw<SwLane>(S.Bb[1], 0, 16 * cw, lane), ldtr_sw<SwLane>(S.Kb[1], 0, 16 * cw, lane));
#pragma unroll
        for (int e = 0; e < 4; e++) st.gv[e] = S.g[(4 * q + e) * LDG + j_own];
        return st;
    };
    auto strip_fw = [&](const Slot& S, Strip& st) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 4 * q + e;
            st.gp[e] = t > 0 ? S.g[(t - 1) * LDG + j_own] : 0.f;
            const float sg = (st.gp[e] - st.gv[e]) * (1.f / DECAY_SCALE);  // sigmoid(w_t)
            st.fw[e] = -DECAY_SCALE * sg * (1.f - sg);
        }
    };
    auto new_tick = [&]() {  // lane-derived values, recomputed so they are not held across the loop
        lane = opaque(lane0);
        q = lane >> 4;
        r16 = lane & 15;
        i_own = 16 * cw + r16;
        j_own = i_own;
    };

    if (tid == 0) sm.csync = 0;  // (visible after the prologue's barriers)

    // The three roles run separate tick loops with the same barriers (one per tick;
    // the consumers also meet mid-tick on csync), so that registers and
    // memory-counter waits are allocated per role.
    if (!consumer) {
        // ======================= producers (lane: token r16, keys 32 hf + 8q + e) =======================
        float gq[2][8];  // cumulative log-decay, phase 0 -> 1
        // scaled operands of one key half (lane: token r16, keys 32 hf + 8q + e), split
        auto operands = [&](const Plane* raw, const float (&g)[8], int hf, uint4 (&o)[8]) {
            const int c8 = 32 * hf + 8 * q;
            const uint4 rr = ld16_sw<SwDma>(raw[0], r16, c8), kk = ld16_sw<SwDma>(raw[2], r16, c8);
            const uint4 aa = ld16_sw<SwDma>(raw[3], r16, c8), bv = ld16_sw<SwDma>(raw[4], r16, c8);
            float at[8], rt[8], bbv[8], kbv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float eg = __expf(g[e]), eng = __expf(-g[e]);
                at[e] = bf_el8(aa, e) * row_prev(eg, 1.f);
                rt[e] = bf_el8(rr, e) * eg;
                bbv[e] = bf_el8(bv, e) * eng;
                kbv[e] = bf_el8(kk, e) * eng;
            }
            pack8(at, o[0], o[1]);
            pack8(rt, o[2], o[3]);
            pack8(bbv, o[4], o[5]);
            pack8(kbv, o[6], o[7]);
        };
        auto put_operands = [&](Slot& S, int hf, const uint4 (&o)[8]) {
            const int c8 = 32 * hf + 8 * q;
            st16_sw<SwLane>(S.At[0], r16, c8, o[0]);
            st16_sw<SwLane>(S.At[1], r16, c8, o[1]);
            st16_sw<SwLane>(S.Rt[0], r16, c8, o[2]);
            st16_sw<SwLane>(S.Rt[1], r16, c8, o[3]);
            st16_sw<SwLane>(S.Bb[0], r16, c8, o[4]);
            st16_sw<SwLane>(S.Bb[1], r16, c8, o[5]);
            st16_sw<SwLane>(S.Kb[0], r16, c8, o[6]);
            st16_sw<SwLane>(S.Kb[1], r16, c8, o[7]);
            float* gp_ = &S.g[r16 * LDG + c8];
            const float* g = gq[hf];
            *reinterpret_cast<float4*>(gp_) = make_float4(g[0], g[1], g[2], g[3]);
            *reinterpret_cast<float4*>(gp_ + 4) = make_float4(g[4], g[5], g[6], g[7]);
            if (r16 == CH - 1) {  // e^{gL}: the last token's e^{g} (padded steps repeat g_L)
                *reinterpret_cast<float4*>(&S.egL[c8]) = make_float4(__expf(g[0]), __expf(g[1]), __expf(g[2]), __expf(g[3]));
                *reinterpret_cast<float4*>(&S.egL[c8 + 4]) = make_float4(__expf(g[4]), __expf(g[5]), __expf(g[6]), __expf(g[7]));
            }
        };
        uint32_t voff[2];  // this lane's LDS DMA offsets
        dma_lane_offsets(voff, rstride, lane);
        const bf16_t* const rsrc_src[5] = {r, w, k, a, b};
        // this producer's current chunk (stream index x = pw mod 3) and its next
        Cursor cx = cursor_at(sc, m, pw, H), cy = cursor_at(sc, m, pw + NPROD, H);
        if (pw < nstream) {
            // the first chunk of each producer; stream index 0's V, dY go into its slot here too
#pragma unroll
            for (int ts = 0; ts < 5; ts++)
                stage_plane(sm.raw[pw][ts], dma_rsrc(rsrc_src[ts], tbytes), rsrc_src[ts], chunk_off(cx), voff, rstride,
                            chunk_len(cx), lane);
            if (pw == 0) {
                stage_plane(sm.slot[0].V, dma_rsrc(v, tbytes), v, chunk_off(cx), voff, rstride, chunk_len(cx), lane);
                stage_plane(sm.slot[0].dY, dma_rsrc(dy, tbytes), dy, chunk_off(cx), voff, rstride, chunk_len(cx), lane);
            }
        }
        lds_barrier();
        lds_barrier();
        // Producer pw's chunks are x = pw, pw + 3, ... (slot x % 3 = pw is its own); phase
        // ph of chunk x runs at tick x - 3 + ph, while the consumers work on chunk x - 3 + ph.
        // Phase 0 may not write the slot (the consumers read it at that tick), so the
        // first key half's operands wait in registers until phase 1.
        auto phase0 = [&](uint4 (&o0)[8]) {
            // ---- log-decays, their cumulative sum; key half 0's operands ----
            vm_wait0();  // this chunk's inputs (LDS DMA issued in the previous chunk's phase 1)
            const Plane* raw = sm.raw[pw];
            const int L = chunk_len(cx);
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
            operands(raw, gq[0], 0, o0);
        };
        auto phase1 = [&](int x, const uint4 (&o0)[8]) {
            // ---- the slot's A~, R~, B-, K-, g and e^{gL}; then V, dY of this chunk and the
            //      inputs of this producer's next chunk by LDS DMA ----
            Slot& S = sm.slot[pw];
            const Plane* raw = sm.raw[pw];
            put_operands(S, 0, o0);
            uint4 o[8];
            operands(raw, gq[1], 1, o);
            put_operands(S, 1, o);
            dma_lane_offsets(voff, rstride, lane);
            if (x > 0) {  // (stream index 0's V, dY were staged before the loop)
                const uint32_t off = chunk_off(cx);
                const int L = chunk_len(cx);
                stage_plane(S.V, dma_rsrc(v, tbytes), v, off, voff, rstride, L, lane);
                stage_plane(S.dY, dma_rsrc(dy, tbytes), dy, off, voff, rstride, L, lane);
            }
            wave_lds_fence();  // staging reads done before the DMA overwrites it
            if (x + NPROD < nstream) {
                const uint32_t off = chunk_off(cy);
                const int L = chunk_len(cy);
#pragma unroll
                for (int ts = 0; ts < 5; ts++)
                    stage_plane(sm.raw[pw][ts], dma_rsrc(rsrc_src[ts], tbytes), rsrc_src[ts], off, voff, rstride, L, lane);
            }
        };
        auto phase2 = [&](int x) {
            // ---- chunk matrices over keys / value rows, triangular inverse ----
            Slot& S = sm.slot[pw];
            // V, dY of this chunk: the 10 staging DMA ops issued after them may still run
            if (x + NPROD < nstream) vm_wait10();
            else vm_wait0();
            auto rd = [&](const Plane (&pl2)[2], uint4 (&xh)[2], uint4 (&xl)[2]) {
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    xh[hf] = ld16_sw<SwLane>(pl2[0], r16, 32 * hf + 8 * q);
                    xl[hf] = ld16_sw<SwLane>(pl2[1], r16, 32 * hf + 8 * q);
                }
            };
            f32x4_t Aab, AabT, Aak, Brb, Brk, M2;
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
        };

        int n = -NPROD;
        for (; n < pw - NPROD; n++) lds_barrier();  // (ticks before this producer's first chunk)
        for (int x = pw; x < nstream; x += NPROD, n += NPROD) {
            if (x > pw) {  // on to the next chunk
                cx = cy;
                cursor_advance(cy, sc, m, NPROD, H);
            }
            uint4 o0[8];
            new_tick();
            phase0(o0);
            lds_barrier();
            new_tick();
            phase1(x, o0);
            lds_barrier();
            new_tick();
            phase2(x);
            lds_barrier();
        }
        for (; n < nstream; n++) lds_barrier();  // (ticks after its last chunk)
    } else if (hside) {
        // ======================= H side: rows i_own of H and dV; key strip j_own: dK, dB =======================
        f32x4_t Ht[4];  // H^T tiles Ht[tj][e] = H[i_own][16tj + 4q + e] (H' within a tick)
        bool bad = false;  // a rendezvous timed out: every later output is NaN
        const int slim = wait_bound(1 << 22);
        lds_barrier();
        lds_barrier();
        for (int n = -NPROD; n < 0; n++) lds_barrier();
        // one piece (a head's chunks on this workgroup) after another; tick n counts the stream
        const int jlast = (m * sc.L + nstream - 1) / sc.n;
        int n = 0;
        for (int j = m * sc.L / sc.n; j <= jlast; j++) {
          const Seg sg = seg_of(sc, m, j);
          const int bb = j / H, h = j - bb * H;
          {  // H at the piece's start: dsT (zero if absent) at the head's end, else the handoff
             // of boundary m + 1.  (Lane offsets at piece boundaries come from an opaque
             // lane, so that they are not kept in registers across the tick loop.)
            const int ln = opaque(lane0), row = 16 * cw + (ln & 15), col = 4 * (ln >> 4);
            if (sg.fresh) {
#pragma unroll
                for (int tj = 0; tj < 4; tj++) {
                    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (dsT) x = *reinterpret_cast<const float4*>(dsT + (long)j * NN + row * NK + 16 * tj + col);
                    Ht[tj] = f32x4_t{x.x, x.y, x.z, x.w};
                }
            } else {
                const float hw = handoff_wait(flags + m + 1, NCONS) ? 1.f : __builtin_nanf("");  // NaN: time-out
                const float* src = hand + (m + 1) * NH;
#pragma unroll
                for (int tj = 0; tj < 4; tj++) {
                    const float4 x = handoff_get4(src + row * NK + 16 * tj + col);
                    Ht[tj] = f32x4_t{x.x, x.y, x.z, x.w} * hw;
                }
            }
          }
          for (int kk = 0; kk < sg.count; kk++, n++) {
            // (lane-derived addresses may stay in registers on this side)
            Slot& S = sm.slot[n % NPROD];
            const int c = nchunk - 1 - (sg.step0 + kk);
            // ---- stage B: X2 = B- H'^T + Brb^T dY ; Q = Ti^T X2 ; publish H' and Q^T rows ----
            const uint2 dyf = ldtr_sw<SwDma>(S.dY, 0, 16 * cw, lane);  // dY[s = 4q+e][i_own]
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const float4 el = *reinterpret_cast<const float4*>(&S.egL[16 * tj + 4 * q]);
                Ht[tj] = Ht[tj] * f32x4_t{el.x, el.y, el.z, el.w};  // H' = H diag(e^{gL})
            }
            f32x4_t x2 = zero4(), dv0 = zero4();  // dv0 = K- H'^T (the rest of dV in stage C)
#pragma unroll
            for (int s = 0; s < 2; s++) {
                float hv[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    hv[e] = Ht[2 * s][e];
                    hv[4 + e] = Ht[2 * s + 1][e];
                }
                uint4 hbh, hbl;
                pack8(hv, hbh, hbl);
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int col = 16 * (2 * s + u) + 4 * q;
                    st8_sw<SwLane>(sm.Hx[0], i_own, col, u ? make_uint2(hbh.z, hbh.w) : make_uint2(hbh.x, hbh.y));
                    st8_sw<SwLane>(sm.Hx[1], i_own, col, u ? make_uint2(hbl.z, hbl.w) : make_uint2(hbl.x, hbl.y));
                }
                const uint4 bh_ = fragp_sw<SwLane>(S.Bb[0], r16, 32 * s, lane), bl_ = fragp_sw<SwLane>(S.Bb[1], r16, 32 * s, lane);
                x2 = mma32(x2, bh_, hbh);
                x2 = mma32(x2, bh_, hbl);
                x2 = mma32(x2, bl_, hbh);
                const uint4 kh = fragp_sw<SwLane>(S.Kb[0], r16, 32 * s, lane), kl = fragp_sw<SwLane>(S.Kb[1], r16, 32 * s, lane);
                dv0 = mma32(dv0, kh, hbh);
                dv0 = mma32(dv0, kh, hbl);
                dv0 = mma32(dv0, kl, hbh);
            }
            Pk pq;  // Q for rows i_own, as the B operand [t][i]
            {
                const Pk brbT = mat_t(S.Brb, lane);
                f32x4_t c2 = mma16(zero4(), brbT.h, dyf);
                c2 = mma16(c2, brbT.l, dyf);
                pq = pk(mm16s_acc(zero4(), mat_t(S.Ti, lane), pk(x2 + c2)));  // Q = Ti^T X2
                st8(&sm.QT[0][pl16(i_own, 4 * q)], pq.h);
                st8(&sm.QT[1][pl16(i_own, 4 * q)], pq.l);
            }
            bad |= !consumer_sync(&sm.csync, NCONS * (2 * n + 1), slim);
            // ---- stage C: key strip j_own of dK, dB (all value rows, fixed order); dV rows i_own; new H ----
            const Strip st = strip(S);
            // The masked 16x16 products XM = dY SA^T (keep s <= t), M1^T = Q V^T and N1 = SA Q^T
            // (keep s > t) are the same for all eight consumer waves: one wave forms each (this
            // side's waves 3 and 1, the S side's wave 2), publishes it split (Mq), and every
            // wave reads it back, in the orientation it needs, after a second rendezvous.
            if (cw == 3) {
                f32x4_t xm = zero4();
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const uint4 ya = fragp_sw<SwDma>(S.dY, r16, 32 * s, lane);  // dY[t][i], exact
                    const uint4 sh = rows_tr(sm.SAT[0], s, lane), sl = rows_tr(sm.SAT[1], s, lane);
                    xm = mma32(xm, ya, sh);  // dY SA^T        [t][s]
                    xm = mma32(xm, ya, sl);
                }
#pragma unroll
                for (int e = 0; e < 4; e++)  // D layout: row 4q+e, column r16
                    if (r16 > 4 * q + e) xm[e] = 0.f;  // XM[t][s]: keep s <= t
                put_mat(sm.Mq[0], xm, lane);
            } else if (cw == 1) {
                f32x4_t m1T = zero4();
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const uint4 va = fragp_sw<SwDma>(S.V, r16, 32 * s, lane);  // V[t][i], exact
                    const uint4 qh = rows_tr(sm.QT[0], s, lane), ql = rows_tr(sm.QT[1], s, lane);
                    m1T = mma32(m1T, qh, va);  // Q V^T = M1^T  [s][t]
                    m1T = mma32(m1T, ql, va);
                }
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (4 * q + e <= r16) m1T[e] = 0.f;  // M1^T[s][t]: keep s > t
                put_mat(sm.Mq[1], m1T, lane);
            }
            f32x4_t gK = zero4(), gB = zero4();
            {
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const uint4 va = fragp_sw<SwDma>(S.V, r16, 32 * s, lane);   // V[t][i], exact
                    const uint4 sh = rows_tr(sm.SAT[0], s, lane), sl = rows_tr(sm.SAT[1], s, lane);
                    const uint4 hh = rows_tr_sw(sm.Hx[0], s, 16 * cw, lane), hl = rows_tr_sw(sm.Hx[1], s, 16 * cw, lane);
                    gK = mma32(gK, va, hh);  // V H'
                    gK = mma32(gK, va, hl);
                    gB = mma32(gB, sh, hh);  // SA H'
                    gB = mma32(gB, sh, hl);
                    gB = mma32(gB, sl, hh);
                }
            }
            bad |= !consumer_sync(&sm.csync, NCONS * (2 * n + 2), slim);
            // (put_mat of a D tile of M: mat_t reads the A operand of M^T, mat_n that of M)
            const Pk m2n = mat_n(S.M2, lane), pm1 = mat_t(sm.Mq[1], lane), pn1 = mat_n(sm.Mq[2], lane),
                     pxm = mat_t(sm.Mq[0], lane);
            const f32x4_t cK = mm32s(cat(pm1.h, m2n.h), cat(pm1.l, m2n.l), st.arh, st.arl);  // [triu_s(M1) | triu(M2)]
            const f32x4_t cB = mm32s(cat(pn1.h, pxm.h), cat(pn1.l, pxm.l), st.arh, st.arl);  // [triu_s(N1) | triu(SA dY^T)]
            float gk_[4], gb_[4], z[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float uK = gK[e] + cK[e], uB = gB[e] + cB[e];
                const float eng = __expf(-st.gv[e]);
                gk_[e] = eng * uK;
                gb_[e] = eng * uB;
                const float Bb_ = bf_el8(st.bkh, e) + bf_el8(st.bkl, e);
                const float Kb_ = bf_el8(st.bkh, 4 + e) + bf_el8(st.bkl, 4 + e);
                z[e] = -(Bb_ * uB + Kb_ * uK);  // -(b dB + k dK) before e^{-g}: this side's dlogd terms
            }
            if (__builtin_expect(bad, false)) {
#pragma unroll
                for (int e = 0; e < 4; e++) gk_[e] = gb_[e] = z[e] = __builtin_nanf("");
            }
            const uint32_t o = piece_off(bb, h, c);
            store8(dk, tbytes, o, quad_rows_bf16(f32x4_t{gk_[0], gk_[1], gk_[2], gk_[3]}, lane));
            store8(db, tbytes, o, quad_rows_bf16(f32x4_t{gb_[0], gb_[1], gb_[2], gb_[3]}, lane));
            // (the S side forms dw from both sides' terms a tick later)
            *reinterpret_cast<float4*>(&sm.dlp[n & 1][cw][4 * lane]) = make_float4(z[0], z[1], z[2], z[3]);
            {  // dV = K- H'^T + Brk^T dY + Aak^T Q
                const Pk brkT = mat_t(S.Brk, lane);
                const f32x4_t c3 = mm16s_acc(mma16(mma16(zero4(), brkT.h, dyf), brkT.l, dyf), mat_t(S.Aak, lane), pq);
                const f32x4_t dvv = __builtin_expect(bad, false) ? nan4() : dv0 + c3;
                store8(dv, tbytes, o, quad_rows_bf16(dvv, lane));
            }
            // H_0^T = H'^T + [A~^T R~^T] [Q; dY]
            const uint4 bhi = cat(pq.h, dyf), blo = cat(pq.l, make_uint2(0, 0));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                const uint4 ah = cat(ldtr_sw<SwLane>(S.At[0], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Rt[0], 0, 16 * tj, lane));
                const uint4 al = cat(ldtr_sw<SwLane>(S.At[1], 0, 16 * tj, lane), ldtr_sw<SwLane>(S.Rt[1], 0, 16 * tj, lane));
                Ht[tj] = mma32(mma32(mma32(Ht[tj], ah, bhi), ah, blo), al, bhi);
            }
            if (__builtin_expect(bad, false)) {
#pragma unroll
                for (int tj = 0; tj < 4; tj++) Ht[tj] = nan4();
            }
            lds_barrier();
          }
          {  // ds0 at the head's start, or the handoff of H at boundary m
            const int ln = opaque(lane0), row = 16 * cw + (ln & 15), col = 4 * (ln >> 4);
            if (sg.handoff) {
                float* const dst = hand + m * NH;
#pragma unroll
                for (int tj = 0; tj < 4; tj++)
                    handoff_put4(dst + row * NK + 16 * tj + col, Ht[tj][0], Ht[tj][1], Ht[tj][2], Ht[tj][3]);
                handoff_signal(flags + m);
            } else {
#pragma unroll
                for (int tj = 0; tj < 4; tj++)
                    *reinterpret_cast<float4*>(ds0 + (long)j * NN + row * NK + 16 * tj + col) =
                        make_float4(Ht[tj][0], Ht[tj][1], Ht[tj][2], Ht[tj][3]);
            }
          }
        }
    } else {
        // ======================= S side: rows i_own of S0; key strip j_own: dR, dA, dw =======================
        // the next chunk's saved state as rows (same layout as Ht) and as the key strip,
        // S0s[m] = S0[32(m/8) + 16((m/4)%2) + 4q + m%4][j_own], loaded a tick ahead
        f32x4_t S0n[4];
        float S0s[16];
        float carry = 0.f;  // the dlogd carry for key j_own
        bool bad = false;   // a rendezvous timed out: every later output is NaN
        const int slim = wait_bound(1 << 22);
        // buffer loads from a head's saved states: one lane offset, the rest in
        // scalar and immediate offsets (no per-load address arithmetic)
        auto ck_rsrc = [&](int j) { return make_rsrc(ckpt + (long)j * ncp * NN, (uint32_t)(ncp * NN * 4)); };
        // (saved states before the last are in the forward's tiled order: S[i][j] at float
        // ((i/16 * 4 + j/16) * 64 + 16 * (j%16/4) + i%16) * 4 + j%4, wkv7_chunk_fwd.hip)
        auto load_rows = [&](__amdgpu_buffer_rsrc_t ckr, int cc) {  // rows i_own: one whole KB per load
            const uint32_t vo = (uint32_t)((cw * 1024 + 4 * lane) * 4), so = (uint32_t)(cc * NN * 4);
#pragma unroll
            for (int tj = 0; tj < 4; tj++)
                S0n[tj] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ckr, vo + 1024 * tj, so, 0));
        };
        auto load_strip = [&](__amdgpu_buffer_rsrc_t ckr, int cc) {  // key j_own = 16 cw + r16
            const uint32_t vo = (uint32_t)((cw * 256 + 64 * (r16 >> 2) + 16 * q + (r16 & 3)) * 4);
#pragma unroll
            for (int m = 0; m < 16; m++)
                S0s[m] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    ckr, vo + (m & 3) * 16, (uint32_t)((cc * NN + (32 * (m >> 3) + 16 * ((m >> 2) & 1)) * NK) * 4), 0));
        };
        // The previous tick's chunk (stream index np) is completed a tick late, once the H
        // side's dlogd terms of it are published: this side's terms zp, tp, its fw and its
        // piece offset are held over, the carry then moves on to it.
        float zp[4], tp[4], fwp[4];
        uint32_t o_prev = OUT_OF_RANGE;
        auto flush = [&](int np) {
            const float4 zh = *reinterpret_cast<const float4*>(&sm.dlp[np & 1][cw][4 * lane]);
            const float zz[4] = {zp[0] + zh.x, zp[1] + zh.y, zp[2] + zh.z, zp[3] + zh.w};
            float gw[4];
            dlogd_part(zz, tp, fwp, carry, gw);
            store8(dw, tbytes, o_prev, quad_rows_bf16(f32x4_t{gw[0], gw[1], gw[2], gw[3]}, lane));
        };
        auto hand_carry = [&]() {  // the carry at boundary m (after the start piece's last chunk)
            const int ln = opaque(lane0);
            if (ln < 16) handoff_put(hand + m * NH + NN + 16 * cw + ln, carry);
            handoff_signal(flags + m);
        };
        {
            const int2 jc = chunk_at(0);
            load_rows(ck_rsrc(jc.x), jc.y);
            load_strip(ck_rsrc(jc.x), jc.y);
        }
        vm_wait0();
        lds_barrier();
        lds_barrier();
        for (int n = -NPROD; n < 0; n++) lds_barrier();
        const int jlast = (m * sc.L + nstream - 1) / sc.n;
        int n = 0;
        bool hand_prev = false;  // the previous piece hands its carry over at boundary m
        for (int j = m * sc.L / sc.n; j <= jlast; j++) {
          const Seg sg = seg_of(sc, m, j);
          const int bb = j / H, h = j - bb * H;
          if (n > 0) {  // the previous piece's last chunk, with that piece's carry
              flush(n - 1);
              if (hand_prev) hand_carry();
          }
          hand_prev = sg.handoff;
          {  // (lane offsets at piece boundaries from an opaque lane: none held across the tick loop)
            const int ln = opaque(lane0), key = 16 * cw + (ln & 15);
            if (sg.fresh) {
                // the head's carry starts at colsum(dsT o S_T) (key j_own): 16 rows per lane group
                float p = 0.f;
                if (dsT) {
                    const float* d = dsT + (long)j * NN + key;
                    const float* st = ckpt + ((long)j * ncp + ncp - 1) * NN + key;
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        const int row = 16 * (u >> 2) + 4 * (ln >> 4) + (u & 3);
                        p += d[row * NK] * st[row * NK];
                    }
                    p += __shfl_xor(p, 16);
                    p += __shfl_xor(p, 32);
                }
                carry = p;
            } else {  // the carry from the handoff of boundary m + 1
                const float hw = handoff_wait(flags + m + 1, NCONS) ? 1.f : __builtin_nanf("");  // NaN: time-out
                carry = handoff_get(hand + (m + 1) * NH + NN + key) * hw;
            }
          }
          // the chunk after this piece's last: the next piece's first (or a repeat at the end)
          const int jn = j < jlast ? j + 1 : j;
          const int cn = j < jlast ? nchunk - 1 - seg_of(sc, m, j + 1).step0 : nchunk - 1 - (sg.step0 + sg.count - 1);
          for (int kk = 0; kk < sg.count; kk++, n++) {
            // (lane-derived addresses may stay in registers on this side)
            Slot& S = sm.slot[n % NPROD];
            const int c = nchunk - 1 - (sg.step0 + kk);
            // ---- stage B: X1 = A~ S0^T + Aak V ; SA = Ti X1 ; publish SA^T rows ----
            {
                const uint2 vfr = ldtr_sw<SwDma>(S.V, 0, 16 * cw, lane);  // V[s = 4q+e][i_own]
                f32x4_t x1 = zero4();
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    float sv[8];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        sv[e] = S0n[2 * s][e];
                        sv[4 + e] = S0n[2 * s + 1][e];
                    }
                    uint4 sbh, sbl;
                    pack8(sv, sbh, sbl);
                    const uint4 ah = fragp_sw<SwLane>(S.At[0], r16, 32 * s, lane), al = fragp_sw<SwLane>(S.At[1], r16, 32 * s, lane);
                    x1 = mma32(x1, ah, sbh);
                    x1 = mma32(x1, ah, sbl);
                    x1 = mma32(x1, al, sbh);
                }
                const Pk aak = mat_n(S.Aak, lane);
                f32x4_t c1 = mma16(zero4(), aak.h, vfr);
                c1 = mma16(c1, aak.l, vfr);
                const Pk psa = pk(mm16s_acc(zero4(), mat_n(S.Ti, lane), pk(x1 + c1)));  // SA = Ti X1
                st8(&sm.SAT[0][pl16(i_own, 4 * q)], psa.h);
                st8(&sm.SAT[1][pl16(i_own, 4 * q)], psa.l);
            }
            // ---- still before the rendezvous (this side's stage B is the shorter): the work
            //      of stage C that needs nothing published this tick ----
            if (kk > 0) flush(n - 1);  // the previous chunk of this piece (same carry)
            Strip st = strip(S);
            strip_fw(S, st);
            uint4 oh[2], ol[2];  // this chunk's saved-state strip (loaded a tick ago)
#pragma unroll
            for (int s = 0; s < 2; s++) pack8(&S0s[8 * s], oh[s], ol[s]);
            // the next chunk's state, a tick ahead: strip, then rows.  The memory counter is
            // in order, so this strip must be consumed before they are issued (or using it
            // would wait for them too): the asm pins that order.
            asm volatile("" ::"v"(__builtin_bit_cast(i32x4_t, oh[0])), "v"(__builtin_bit_cast(i32x4_t, oh[1])),
                         "v"(__builtin_bit_cast(i32x4_t, ol[0])), "v"(__builtin_bit_cast(i32x4_t, ol[1]))
                         : "memory");
            {  // (unconditional, like every memory operation of the loop, so the compiler's
               // waits count a fixed sequence)
                const bool last = kk + 1 == sg.count;
                const __amdgpu_buffer_rsrc_t ckr = ck_rsrc(last ? jn : j);
                load_strip(ckr, last ? cn : c - 1);
                load_rows(ckr, last ? cn : c - 1);
            }
            f32x4_t gR = zero4();
#pragma unroll
            for (int s = 0; s < 2; s++) {  // dY S0
                const uint4 ya = fragp_sw<SwDma>(S.dY, r16, 32 * s, lane);
                gR = mma32(mma32(gR, ya, oh[s]), ya, ol[s]);
            }
            bad |= !consumer_sync(&sm.csync, NCONS * (2 * n + 1), slim);
            // ---- stage C: key strip j_own of dR, dA and this chunk's dlogd terms (this side's
            //      wave 2 forms N1 for all eight consumer waves; XM and M1^T come from the H side) ----
            if (cw == 2) {
                f32x4_t n1 = zero4();
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const uint4 qh = rows_tr(sm.QT[0], s, lane), ql = rows_tr(sm.QT[1], s, lane);
                    const uint4 sh = rows_tr(sm.SAT[0], s, lane), sl = rows_tr(sm.SAT[1], s, lane);
                    n1 = mma32(n1, sh, qh);  // SA Q^T = N1    [t][s]
                    n1 = mma32(n1, sh, ql);
                    n1 = mma32(n1, sl, qh);
                }
#pragma unroll
                for (int e = 0; e < 4; e++)  // D layout: row 4q+e, column r16
                    if (r16 <= 4 * q + e) n1[e] = 0.f;  // N1[t][s]: keep s > t
                put_mat(sm.Mq[2], n1, lane);
            }
            f32x4_t gA = zero4();
            {
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const uint4 qh = rows_tr(sm.QT[0], s, lane), ql = rows_tr(sm.QT[1], s, lane);
                    gA = mma32(gA, qh, oh[s]);  // Q S0
                    gA = mma32(gA, qh, ol[s]);
                    gA = mma32(gA, ql, oh[s]);
                }
            }
            bad |= !consumer_sync(&sm.csync, NCONS * (2 * n + 2), slim);
            const Pk m2t = mat_t(S.M2, lane), pm1 = mat_n(sm.Mq[1], lane), pn1 = mat_t(sm.Mq[2], lane),
                     pxm = mat_n(sm.Mq[0], lane);
            const f32x4_t cR = mm32s(cat(pxm.h, m2t.h), cat(pxm.l, m2t.l), st.bkh, st.bkl);  // [tril(dY SA^T) | tril(dY V^T)]
            const f32x4_t cA = mm32s(cat(pn1.h, pm1.h), cat(pn1.l, pm1.l), st.bkh, st.bkl);  // [tril_s(Q SA^T) | tril_s(Q V^T)]
            float gr_[4], ga_[4], z[4], t2[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float uR = gR[e] + cR[e], uA = gA[e] + cA[e];
                gr_[e] = __expf(st.gv[e]) * uR;
                ga_[e] = __expf(st.gp[e]) * uA;
                const float At_ = bf_el8(st.arh, e) + bf_el8(st.arl, e);
                const float Rt_ = bf_el8(st.arh, 4 + e) + bf_el8(st.arl, 4 + e);
                z[e] = Rt_ * uR;
                t2[e] = At_ * uA;
            }
            if (__builtin_expect(bad, false)) {
#pragma unroll
                for (int e = 0; e < 4; e++) gr_[e] = ga_[e] = z[e] = t2[e] = __builtin_nanf("");
            }
            const uint32_t o = piece_off(bb, h, c);
            store8(dr, tbytes, o, quad_rows_bf16(f32x4_t{gr_[0], gr_[1], gr_[2], gr_[3]}, lane));
            store8(da, tbytes, o, quad_rows_bf16(f32x4_t{ga_[0], ga_[1], ga_[2], ga_[3]}, lane));
#pragma unroll
            for (int e = 0; e < 4; e++) zp[e] = z[e], tp[e] = t2[e], fwp[e] = st.fw[e];
            o_prev = o;
            lds_barrier();
          }
        }
        // the last chunk (a machine's last piece never hands over; a lone start piece does)
        flush(nstream - 1);
        if (hand_prev) hand_carry();
    }
}

int chunk_backward_wait_timeouts(uint32_t* out, int reset) { return wait_timeouts_read(out, reset != 0); }
int chunk_backward_waits(int on) { return wait_switch(on); }

size_t chunk_backward_workspace(int B, int T, int H, int cus) {
    return sched_workspace(plan_schedule(B * H, (T + CH - 1) / CH, cus), NK * NK + NK);
}
void launch_chunk_backward(const Bwd& p, int cus) {
    const Sched sc = plan_schedule(p.B * p.H, (p.T + CH - 1) / CH, cus);
    uint32_t* flags = nullptr;
    float* hand = nullptr;
    if (sched_cuts(sc)) {
        flags = static_cast<uint32_t*>(p.ws);
        hand = reinterpret_cast<float*>(static_cast<char*>(p.ws) + sched_flag_bytes(sc));
        hipLaunchKernelGGL(clear_words, dim3(1), dim3(256), 0, p.stream, flags, sc.G);
    }
    hipLaunchKernelGGL(chunk_backward_bf16, dim3(sc.G), dim3(704), 0, p.stream, sc, p.T, p.H,
                       (const bf16_t*)p.r, (const bf16_t*)p.w, (const bf16_t*)p.k, (const bf16_t*)p.v,
                       (const bf16_t*)p.a, (const bf16_t*)p.b, p.ckpt, (const bf16_t*)p.dy, p.dsT,
                       (bf16_t*)p.dr, (bf16_t*)p.dw, (bf16_t*)p.dk, (bf16_t*)p.dv, (bf16_t*)p.da,
                       (bf16_t*)p.db, p.ds0, flags, hand);
}

}  // namespace wkv7
