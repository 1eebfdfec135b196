// WKV7 backward for head size 128 (bf16) on the matrix cores, every chunk at once.
//
// The chunk form of the recurrence (kernels/wkv7_state.cu:12-79; operands A~, R~, B-, K-,
// B^, K^, Aab, Aak, Brb, Brk, Ti, P, P2 as in wkv7_chunk_fwd.hip, decays per key) gives,
// with H = dL/dS at a chunk's end, H' = H diag(e^{gL}), S0 the state at its start (a
// saved state) and dY its output gradient,
//   SA = Ti (A~ S0^T + Aak V),  Q = Ti^T (B^ H^T + Brb^T dY)
//   dV = K^ H^T + Aak^T Q + Brk^T dY
//   dK = e^{-g} o [V H' + triu_s(V Q^T) A~ + triu(V dY^T) R~]
//   dB = e^{-g} o [SA H' + triu_s(SA Q^T) A~ + triu(SA dY^T) R~]
//   dR = e^{g}  o [dY S0 + tril(dY SA^T) B- + tril(dY V^T) K-]
//   dA = e^{gp} o [Q S0 + tril_s(Q SA^T) B- + tril_s(Q V^T) K-]
//   H at the chunk's start = H diag(e^{gL}) + (H B^^T) P + dY^T P2
// and the log-decay gradient dlogd_t = sum_{s>=t} (r dR - b dB - k dK)_s +
// sum_{s>t} (a dA)_s + colsum(H_end o S_end) over the chunk's own steps: the gradients of
// the steps up to a boundary are those of the sequence cut there with dL/dS_end = H_end,
// so the carry from every later step is the column sum of H_end o S_end at the chunk's
// end (S_end: the next saved state).  dw = dlogd * (-e^{-1/2}) sig(w) (1 - sig(w)).
// (Checked in float64 against the oracle's step adjoint before the kernels.)
//
// Three kernels.  wkv7_bwd_prep (one wave per chunk, all at once) writes each chunk's
// record for the scan: B^ as the K=32 A operand over the keys, [P | P2] per 16-key tile
// as the A operand of the K=32 update, e^{gL} per key.  wkv7_bwd_scan walks each head's
// chunks backwards (one workgroup per 64 value rows of H, fp32 in registers, records
// double-buffered in LDS by DMA as gdn_scan's), storing H at every chunk's end in the
// workspace and the first chunk's start as ds0.  wkv7_bwd_chunk then forms every
// chunk's gradients independently (eight waves; wave w owns value rows 16w..16w+15 for
// SA, Q, dV and keys 16w..16w+15 for dK, dB, dR, dA, dw).
#include "wkv7_io.h"
#include "wkv7_launch.h"

namespace wkv7 {
namespace {

constexpr int BC = 16;        // chunk length
constexpr int BNK = 128;      // head size
constexpr int BKS = BNK / 32, BTJ = BNK / 16;
constexpr long BNN = (long)BNK * BNK;

// One chunk's record for the scan (byte offsets).
struct BwdRec {
    static constexpr size_t BF = 0;                                // B^ [KS][hi, lo][64 lanes] uint4
    static constexpr size_t PP = BF + (size_t)BKS * 2 * 64 * 16;   // [P | P2] [TJ][hi, lo][64] uint4
    static constexpr size_t EL = PP + (size_t)BTJ * 2 * 64 * 16;   // e^{gL} [NK]
    static constexpr size_t BYTES = EL + (size_t)BNK * 4;
    static constexpr int DMA_BLOCKS = (int)((BYTES + 1023) / 1024);
};
static_assert(BwdRec::BYTES % 256 == 0, "record alignment");

__device__ __forceinline__ f32x4_t mm3(f32x4_t acc, uint4 xh, uint4 xl, uint4 yh, uint4 yl) {
    return mma32(mma32(mma32(acc, xh, yh), xh, yl), xl, yh);
}
// M^T of a D-layout tile, by the product M^T I on the K=16 instruction (I exact in bf16)
__device__ __forceinline__ f32x4_t transpose16(const f32x4_t& m, int lane) {
    f32x4_t id;
#pragma unroll
    for (int e = 0; e < 4; e++) id[e] = (4 * (lane >> 4) + e) == (lane & 15) ? 1.f : 0.f;
    const Pk pm = pk(m), pi = pk(id);
    return mma16(mma16(zero4(), pm.h, pi.h), pm.l, pi.h);
}
__device__ __forceinline__ float bf2f(const bf16_t* p, long i) { return io<bf16_t>::ld(p, i); }

// ---------------------------------------------------------------------------
// Records of chunk blockIdx.x of head blockIdx.y (one wave; lane (q4, r16): token r16's
// keys 32ks + 4q4 + e and 32ks + 16 + 4q4 + e, as wkv7_rec_prep).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void wkv7_bwd_prep(int Tn, int H, const bf16_t* __restrict__ r,
                                                    const bf16_t* __restrict__ w, const bf16_t* __restrict__ k,
                                                    const bf16_t* __restrict__ a, const bf16_t* __restrict__ b,
                                                    uint8_t* __restrict__ ws) {
    using R = BwdRec;
    constexpr int LP = BNK + 4;
    const int c = blockIdx.x, bh = blockIdx.y, nchunk = gridDim.x;
    const int bb = bh / H, h = bh - bb * H;
    const int lane = threadIdx.x, q4 = lane >> 4, r16 = lane & 15;
    const int t0 = c * BC, L = min(BC, Tn - t0);
    const bool tv = r16 < L;
    const long row = (((long)bb * Tn + t0 + (tv ? r16 : 0)) * H + h) * (long)BNK;  // (clamped: read by every lane)
    const uint32_t tm = lane_mask(tv);
    __shared__ __attribute__((aligned(16))) float pa[BC][LP], pr[BC][LP];  // A~, R~ [t][j]
    uint8_t* const rec = ws + ((size_t)bh * nchunk + c) * R::BYTES;
    auto ld8 = [&](const bf16_t* x, int c0, float (&o)[8]) {
        const float4 p = keep4(tm, ld4f(x + row + c0)), q = keep4(tm, ld4f(x + row + c0 + 16));
        o[0] = p.x, o[1] = p.y, o[2] = p.z, o[3] = p.w, o[4] = q.x, o[5] = q.y, o[6] = q.z, o[7] = q.w;
    };
    auto st8 = [&](float (*pl)[LP], int c0, const float (&x)[8]) {
        *reinterpret_cast<float4*>(&pl[r16][c0]) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(&pl[r16][c0 + 16]) = make_float4(x[4], x[5], x[6], x[7]);
    };
    f32x4_t Aab = zero4(), AabT = zero4(), BrbT = zero4();
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) {
        const int c0 = 32 * ks + 4 * q4;
        float wv[8], av[8], bv[8], rv[8];
        ld8(w, c0, wv), ld8(a, c0, av), ld8(b, c0, bv), ld8(r, c0, rv);
        float At[8], Bm[8], Rt[8], Bh[8], eL[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float g = row_prefix_sum(tv ? log_decay(wv[e]) : 0.f);
            const float gp = row_prev(g, 0.f), gL = row_last(g);
            At[e] = av[e] * __expf(gp);
            Rt[e] = rv[e] * __expf(g);
            Bm[e] = bv[e] * __expf(-g);
            Bh[e] = bv[e] * __expf(gL - g);
            eL[e] = __expf(gL);
        }
        st8(pa, c0, At), st8(pr, c0, Rt);
        if (r16 == 0) {
            float* el = reinterpret_cast<float*>(rec + R::EL);
            *reinterpret_cast<float4*>(el + c0) = make_float4(eL[0], eL[1], eL[2], eL[3]);
            *reinterpret_cast<float4*>(el + c0 + 16) = make_float4(eL[4], eL[5], eL[6], eL[7]);
        }
        uint4 ah, al, bh_, bl, rh, rl, hh, hl;
        pack8(At, ah, al), pack8(Bm, bh_, bl), pack8(Rt, rh, rl), pack8(Bh, hh, hl);
        uint4* bf = reinterpret_cast<uint4*>(rec + R::BF) + (size_t)(2 * ks) * 64 + lane;
        bf[0] = hh;
        bf[64] = hl;
        Aab = mm3(Aab, ah, al, bh_, bl);    // A~_rr . B-_cc
        AabT = mm3(AabT, bh_, bl, ah, al);  // B-_rr . A~_cc
        BrbT = mm3(BrbT, bh_, bl, rh, rl);  // B-_rr . R~_cc
    }
    const int cc = r16;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        Aab[e] = cc < rr ? Aab[e] : 0.f;
        AabT[e] = rr < cc ? AabT[e] : 0.f;
        BrbT[e] = rr <= cc ? BrbT[e] : 0.f;  // Brb[cc][rr]
    }
    f32x4_t Ti, TiT;
    tri_inverse(Aab, AabT, lane, Ti, TiT);
    const Pk pTiT = pk(TiT), pBrbT = pk(BrbT);
    __syncthreads();  // the planes
#pragma unroll
    for (int tj = 0; tj < BTJ; tj++) {
        f32x4_t at, rt;  // D layout [t][j], t = 4q4 + e, j = 16tj + r16
#pragma unroll
        for (int e = 0; e < 4; e++) at[e] = pa[4 * q4 + e][16 * tj + r16], rt[e] = pr[4 * q4 + e][16 * tj + r16];
        const f32x4_t Pt = mm16s(pTiT, pk(at));          // P = Ti A~
        const Pk pP = pk(Pt);
        const Pk pP2 = pk(rt + mm16s(pBrbT, pP));        // P2 = R~ + Brb P
        uint4* pp = reinterpret_cast<uint4*>(rec + R::PP) + (size_t)(2 * tj) * 64 + lane;
        pp[0] = cat(pP.h, pP2.h);
        pp[64] = cat(pP.l, pP2.l);
    }
}

// ---------------------------------------------------------------------------
// Each head's chunks backwards: workgroup rg * BH + bh, four waves, wave wv of group rg
// keeps value rows i_own = 16 (4 rg + wv) + r16 of H as Ht[tj][e] = H[i_own][16tj + 4q4 + e].
// Per chunk: H is stored (the chunk kernel's H_end), U^T = B^ H^T over the keys, then
// H^T <- e^{gL} o H^T + [P^T | P2^T] [U^T; dY] on the K=32 instruction.  dY of dtype TI;
// dsT (may be null) and ds0 [key][value] when kv (GDN's layout), else [value][key]; H in
// the workspace always [value][key].
// ---------------------------------------------------------------------------
template <typename TI>
__global__ __launch_bounds__(256) void wkv7_bwd_scan(int Tn, int H, int BH, int kv, const float* __restrict__ dsT,
                                                     const TI* __restrict__ dy, float* __restrict__ ds0,
                                                     float* __restrict__ hbuf, const uint8_t* __restrict__ ws) {
    using R = BwdRec;
    __shared__ __attribute__((aligned(1024))) uint8_t recs[2][R::DMA_BLOCKS * 1024];
    const int bh = blockIdx.x % BH, rg = blockIdx.x / BH, bb = bh / H, h = bh - bb * H;
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
    const int i_own = 16 * (4 * rg + wv) + r16;
    const int nchunk = (Tn + BC - 1) / BC;
    const i32x4_t rs = dma_rsrc(ws + (size_t)bh * nchunk * R::BYTES, (uint32_t)((size_t)nchunk * R::BYTES));
    auto fetch = [&](int c, int buf) {
        uint32_t so = (uint32_t)((size_t)c * R::BYTES);
        asm volatile("" : "+s"(so));
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)recs[buf];
        for (int j = wv; j < R::DMA_BLOCKS; j += 4) dma_kb(base + 1024 * j, rs, (uint32_t)(1024 * j + 16 * lane), so);
    };
    // dY[t0 + 4q4 + e][i_own], loaded a chunk ahead as raw element bits: rows past the end
    // read row t0, and the bits are widened and zeroed where they are used (dy_of), so
    // nothing waits on the loads until the chunk's closing wait
    auto load_dy = [&](int c, uint32_t (&o)[4]) {
        const int t0 = c * BC, L = min(BC, Tn - t0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 4 * q4 + e, tc = t < L ? t : 0;
            const long i = (((long)bb * Tn + t0 + tc) * H + h) * BNK + i_own;
            if constexpr (sizeof(TI) == 2) o[e] = reinterpret_cast<const uint16_t*>(dy)[i];
            else o[e] = reinterpret_cast<const uint32_t*>(dy)[i];
        }
    };
    auto dy_of = [&](int c, const uint32_t (&o)[4]) {
        const int L = min(BC, Tn - c * BC);
        f32x4_t d;
#pragma unroll
        for (int e = 0; e < 4; e++)
            d[e] = keep(lane_mask(4 * q4 + e < L), __uint_as_float(sizeof(TI) == 2 ? o[e] << 16 : o[e]));
        return d;
    };
    fetch(nchunk - 1, 0);
    f32x4_t Ht[BTJ];
#pragma unroll
    for (int tj = 0; tj < BTJ; tj++) {
        if (!dsT) {
            Ht[tj] = zero4();
        } else if (kv) {
#pragma unroll
            for (int e = 0; e < 4; e++) Ht[tj][e] = dsT[bh * BNN + (long)(16 * tj + 4 * q4 + e) * BNK + i_own];
        } else {
            const float4 x = *reinterpret_cast<const float4*>(dsT + bh * BNN + (long)i_own * BNK + 16 * tj + 4 * q4);
            Ht[tj] = f32x4_t{x.x, x.y, x.z, x.w};
        }
    }
    uint32_t dyn[4];
    load_dy(nchunk - 1, dyn);
    vm_wait0();
    f32x4_t dyc = dy_of(nchunk - 1, dyn);  // this chunk's dY (the next chunk's is formed after each chunk's wait)
    __syncthreads();
    for (int c = nchunk - 1, it = 0; c >= 0; c--, it++) {
        if (c > 0) fetch(c - 1, (it + 1) & 1);
        const uint8_t* const rec = recs[it & 1];
        if (c > 0) load_dy(c - 1, dyn);
        // H at the chunk's end, stored after the next record's DMA and left in flight by the
        // closing wait (vmcnt(BTJ): a vmcnt(0) there had waited for these stores every chunk)
        float* const hout = hbuf + ((long)bh * nchunk + c) * BNN + (long)i_own * BNK + 4 * q4;
#pragma unroll
        for (int tj = 0; tj < BTJ; tj++)
            *reinterpret_cast<float4*>(hout + 16 * tj) = make_float4(Ht[tj][0], Ht[tj][1], Ht[tj][2], Ht[tj][3]);
        // U^T [t][i_own] = sum_j B^[t][j] H[i_own][j]
        f32x4_t u = zero4();
#pragma unroll
        for (int ks = 0; ks < BKS; ks++) {
            const float sv[8] = {Ht[2 * ks][0], Ht[2 * ks][1], Ht[2 * ks][2], Ht[2 * ks][3],
                                 Ht[2 * ks + 1][0], Ht[2 * ks + 1][1], Ht[2 * ks + 1][2], Ht[2 * ks + 1][3]};
            uint4 sh, sl;
            pack8(sv, sh, sl);
            const uint4* bf = reinterpret_cast<const uint4*>(rec + R::BF) + (2 * ks) * 64 + lane;
            u = mm3(u, bf[0], bf[64], sh, sl);
        }
        uint2 uh, ul, dh, dl;
        pack4(u, uh, ul);
        pack4(dyc, dh, dl);  // (bf16 dY: dl = 0)
        const uint4 bhi = cat(uh, dh), blo = cat(ul, dl);
#pragma unroll
        for (int tj = 0; tj < BTJ; tj++) {
            const uint4* pp = reinterpret_cast<const uint4*>(rec + R::PP) + (2 * tj) * 64 + lane;
            const uint4 ah = pp[0], al = pp[64];
            const f32x4_t eg = *reinterpret_cast<const f32x4_t*>(rec + R::EL + 4 * (16 * tj + 4 * q4));
            Ht[tj] = mma32(mma32(mma32(Ht[tj] * eg, ah, bhi), ah, blo), al, bhi);
        }
        vm_wait_n<BTJ>();  // the next record and the dY loads after it have landed (only the stores may not)
        // the next chunk's dY, formed here where its loads are known complete (formed at the
        // top of the loop, the compiler's own wait there, merged with the path into the loop,
        // would have waited for these stores too)
        if (c > 0) dyc = dy_of(c - 1, dyn);
        __syncthreads();
    }
#pragma unroll
    for (int tj = 0; tj < BTJ; tj++) {
        if (kv) {
#pragma unroll
            for (int e = 0; e < 4; e++) ds0[bh * BNN + (long)(16 * tj + 4 * q4 + e) * BNK + i_own] = Ht[tj][e];
        } else {
            *reinterpret_cast<float4*>(ds0 + bh * BNN + (long)i_own * BNK + 16 * tj + 4 * q4) =
                make_float4(Ht[tj][0], Ht[tj][1], Ht[tj][2], Ht[tj][3]);
        }
    }
}

// ---------------------------------------------------------------------------
// The gradients of one chunk (512 lanes).  Workgroups map to (head, chunk) so that a
// head's consecutive chunks share an XCD (chunk c's S_end is chunk c + 1's S0 in L2).
// ---------------------------------------------------------------------------
// The operands every wave reads as K=32 A/B fragments over the keys or value rows are
// split into bf16 hi/lo once, by the wave that owns their 16 columns, and kept so in LDS
// (splitting them in every reader had been most of the kernel's VALU work).
constexpr int CLB = BNK + 8;  // padded split-plane row (bf16)
struct SplitPlane {
    uint16_t h[BC][CLB], l[BC][CLB];
};
// a D-layout tile ([t][16 wv + c], rows t = 4q4 + e) into a split plane, 8-byte rows per lane
__device__ __forceinline__ void put_split(SplitPlane& P, const f32x4_t& d, int lane, int wv) {
    uint2 h, l;
    quad_rows_split(d, lane, h, l);  // (cross-lane: every lane takes part)
    const int tr = 4 * (lane >> 4) + (lane & 3), c = 16 * wv + 4 * ((lane >> 2) & 3);
    *reinterpret_cast<uint2*>(&P.h[tr][c]) = h;
    *reinterpret_cast<uint2*>(&P.l[tr][c]) = l;
}
// the K=32 fragment of row r16, columns 32ks + 4q4 .. +3 and 32ks + 16 + 4q4 .. +3
__device__ __forceinline__ void get_split(const SplitPlane& P, int lane, int ks, uint4& h, uint4& l) {
    const int r = lane & 15, c = 32 * ks + 4 * (lane >> 4);
    const uint2 a = *reinterpret_cast<const uint2*>(&P.h[r][c]), b = *reinterpret_cast<const uint2*>(&P.h[r][c + 16]);
    const uint2 x = *reinterpret_cast<const uint2*>(&P.l[r][c]), y = *reinterpret_cast<const uint2*>(&P.l[r][c + 16]);
    h = make_uint4(a.x, a.y, b.x, b.y);
    l = make_uint4(x.x, x.y, y.x, y.y);
}
// the same fragment of a bf16 row in memory (exact: no lo part), zero when !ok (the row
// is read either way: the caller passes a valid one)
__device__ __forceinline__ uint4 bf16_frag(const bf16_t* row, int ks, int q4, bool ok) {
    const uint2 a = *reinterpret_cast<const uint2*>(row + 32 * ks + 4 * q4);
    const uint2 b = *reinterpret_cast<const uint2*>(row + 32 * ks + 16 + 4 * q4);
    return keepu4(lane_mask(ok), make_uint4(a.x, a.y, b.x, b.y));
}
struct ChunkLds {
    SplitPlane At, Bm, Km, Rt, Bh, Kh;  // [t][j], written by the key owners
    SplitPlane SA, Q;                   // [t][i], written by the value-row owners
    float csum[BTJ][BNK];  // per wave: column sums of H_end o S_end over its 16 value rows
};

__global__ __launch_bounds__(512) void wkv7_bwd_chunk(int Tn, int H, int BH, int per_xcd,
                                                      const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
                                                      const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                      const bf16_t* __restrict__ a, const bf16_t* __restrict__ b,
                                                      const bf16_t* __restrict__ dy, const float* __restrict__ ckpt,
                                                      const float* __restrict__ hbuf, bf16_t* __restrict__ dr,
                                                      bf16_t* __restrict__ dw, bf16_t* __restrict__ dk,
                                                      bf16_t* __restrict__ dv, bf16_t* __restrict__ da,
                                                      bf16_t* __restrict__ db) {
    __shared__ __attribute__((aligned(16))) ChunkLds sm;
    const int nchunk = (Tn + BC - 1) / BC;
    const int job = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    if (job >= nchunk * BH) return;  // (whole workgroup)
    const int bh = job / nchunk, c = job - bh * nchunk, bb = bh / H, h = bh - bb * H;
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
    const int t0 = c * BC, L = min(BC, Tn - t0);
    const long tok0 = (long)bb * Tn + t0;
    const int col = 16 * wv + r16;  // the lane's key (dK ...) and value column (dV ...)
    auto at_tok = [&](int t) { return ((tok0 + t) * H + h) * (long)BNK; };
    const long ncp = nchunk + 1;
    const float* const S0 = ckpt + ((long)bh * ncp + c) * BNN;
    const float* const Se = S0 + BNN;
    const float* const Hm = hbuf + ((long)bh * nchunk + c) * BNN;
    const int irow = 16 * wv + r16;  // value row of the row-strip loads

    // ---- the wave's value rows of H_end, S_end and S0 (keys 32ks + 4q4 + e, +16) ----
    float hr[BKS][8], sr[BKS][8];
    auto rows = [&](const float* M, float (&o)[BKS][8]) {
#pragma unroll
        for (int ks = 0; ks < BKS; ks++) {
            const float4 x = *reinterpret_cast<const float4*>(M + (long)irow * BNK + 32 * ks + 4 * q4);
            const float4 y = *reinterpret_cast<const float4*>(M + (long)irow * BNK + 32 * ks + 16 + 4 * q4);
            o[ks][0] = x.x, o[ks][1] = x.y, o[ks][2] = x.z, o[ks][3] = x.w;
            o[ks][4] = y.x, o[ks][5] = y.y, o[ks][6] = y.z, o[ks][7] = y.w;
        }
    };
    rows(Hm, hr);
    rows(Se, sr);

    // ---- the chunk operands of the wave's keys in D layout ([t][col], t = 4q4 + e) ----
    float xr[4], xw[4], xk[4], xa[4], xb[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = 4 * q4 + e;
        const bool ok = t < L;
        const long o = at_tok(ok ? t : 0) + col;  // (clamped: every lane loads)
        const float r_ = bf2f(r, o), w_ = bf2f(w, o), k_ = bf2f(k, o), a_ = bf2f(a, o), b_ = bf2f(b, o);
        const uint32_t m = lane_mask(ok);
        xr[e] = keep(m, r_), xw[e] = keep(m, w_), xk[e] = keep(m, k_), xa[e] = keep(m, a_), xb[e] = keep(m, b_);
    }
    float ld[4], p[4];
#pragma unroll
    for (int e = 0; e < 4; e++) ld[e] = (4 * q4 + e) < L ? log_decay(xw[e]) : 0.f;
    p[0] = ld[0], p[1] = p[0] + ld[1], p[2] = p[1] + ld[2], p[3] = p[2] + ld[3];
    // cumulative over the four lane groups (tokens 4q'..4q'+3 of the same key)
    const float T0 = __shfl(p[3], r16), T1 = __shfl(p[3], 16 + r16), T2 = __shfl(p[3], 32 + r16),
                T3 = __shfl(p[3], 48 + r16);
    const float excl = (q4 > 0 ? T0 : 0.f) + (q4 > 1 ? T1 : 0.f) + (q4 > 2 ? T2 : 0.f);
    const float eLj = __expf(T0 + T1 + T2 + T3);
    f32x4_t At, Rt, Bm, Km, eA, eR, eM;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float g = excl + p[e], gp = e ? excl + p[e - 1] : excl;
        eA[e] = __expf(gp), eR[e] = __expf(g), eM[e] = __expf(-g);
        At[e] = xa[e] * eA[e], Rt[e] = xr[e] * eR[e], Bm[e] = xb[e] * eM[e], Km[e] = xk[e] * eM[e];
    }
    put_split(sm.At, At, lane, wv), put_split(sm.Bm, Bm, lane, wv), put_split(sm.Km, Km, lane, wv);
    put_split(sm.Rt, Rt, lane, wv), put_split(sm.Bh, Bm * eLj, lane, wv), put_split(sm.Kh, Km * eLj, lane, wv);
    // the carry's partial column sums over this wave's value rows
#pragma unroll
    for (int ks = 0; ks < BKS; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float s = row_sum16(hr[ks][e] * sr[ks][e]);
            if (r16 == 0) sm.csum[wv][32 * ks + (e < 4 ? 4 * q4 + e : 16 + 4 * q4 + e - 4)] = s;
        }
    uint4 Hh[BKS], Hl[BKS], Sh[BKS], Sl[BKS];
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) pack8(hr[ks], Hh[ks], Hl[ks]);
    rows(S0, sr);
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) pack8(sr[ks], Sh[ks], Sl[ks]);
    __syncthreads();

    // ---- chunk matrices (every wave) and the wave's [t][i] products over the keys ----
    f32x4_t Aab = zero4(), AabT = zero4(), Aak = zero4(), Brb = zero4(), Brk = zero4();
    f32x4_t P1 = zero4(), P2 = zero4(), P3 = zero4();
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) {
        uint4 ah, al, bh_, bl, kh, kl, rh, rl, hh, hl, xh, xl;
        get_split(sm.At, lane, ks, ah, al), get_split(sm.Bm, lane, ks, bh_, bl);
        get_split(sm.Km, lane, ks, kh, kl), get_split(sm.Rt, lane, ks, rh, rl);
        get_split(sm.Bh, lane, ks, hh, hl), get_split(sm.Kh, lane, ks, xh, xl);
        Aab = mm3(Aab, ah, al, bh_, bl);
        AabT = mm3(AabT, bh_, bl, ah, al);
        Aak = mm3(Aak, ah, al, kh, kl);
        Brb = mm3(Brb, rh, rl, bh_, bl);   // R~_rr . B-_cc
        Brk = mm3(Brk, rh, rl, kh, kl);    // R~_rr . K-_cc
        P1 = mm3(P1, ah, al, Sh[ks], Sl[ks]);  // A~ S0^T
        P2 = mm3(P2, hh, hl, Hh[ks], Hl[ks]);  // B^ H^T
        P3 = mm3(P3, xh, xl, Hh[ks], Hl[ks]);  // K^ H^T
    }
    const int cc = r16;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        Aab[e] = cc < rr ? Aab[e] : 0.f;
        AabT[e] = rr < cc ? AabT[e] : 0.f;
        Aak[e] = cc < rr ? Aak[e] : 0.f;
        Brb[e] = cc <= rr ? Brb[e] : 0.f;
        Brk[e] = cc <= rr ? Brk[e] : 0.f;
    }
    f32x4_t Ti, TiT;
    tri_inverse(Aab, AabT, lane, Ti, TiT);
    const Pk pAak = pk(Aak), pBrb = pk(Brb), pBrk = pk(Brk), pTi = pk(Ti), pTiT = pk(TiT);
    const Pk pAakT = pk(transpose16(Aak, lane));

    // ---- SA, Q, dV for the wave's value columns ----
    f32x4_t vD, dyD;  // [t][col]
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = 4 * q4 + e;
        const long o = at_tok(t < L ? t : 0) + col;
        const float v_ = bf2f(v, o), y_ = bf2f(dy, o);
        vD[e] = keep(lane_mask(t < L), v_);
        dyD[e] = keep(lane_mask(t < L), y_);
    }
    const Pk pV = pk(vD), pdY = pk(dyD);
    const f32x4_t SA = mm16s(pTiT, pk(P1 + mm16s(pAakT, pV)));  // Ti (A~ S0^T + Aak V)
    const f32x4_t Q = mm16s(pTi, pk(P2 + mm16s(pBrb, pdY)));    // Ti^T (B^ H^T + Brb^T dY)
    const f32x4_t dV = P3 + mm16s(pAak, pk(Q)) + mm16s(pBrk, pdY);
    put_split(sm.SA, SA, lane, wv), put_split(sm.Q, Q, lane, wv);
    {
        const int tr = 4 * q4 + (lane & 3);  // the row quad_rows_bf16 gives this lane
        const uint2 q = quad_rows_bf16(dV, lane);  // (cross-lane: every lane takes part)
        if (tr < L) *reinterpret_cast<uint2*>(dv + at_tok(tr) + 16 * wv + 4 * ((lane >> 2) & 3)) = q;
    }
    // the key columns of H_end and S0 (value rows 32ks + 4q4 + e, +16) for the products over
    // the value rows
#pragma unroll
    for (int ks = 0; ks < BKS; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int i = 32 * ks + (e < 4 ? 4 * q4 + e : 16 + 4 * q4 + e - 4);
            hr[ks][e] = Hm[(long)i * BNK + col];
            sr[ks][e] = S0[(long)i * BNK + col];
        }
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) pack8(hr[ks], Hh[ks], Hl[ks]), pack8(sr[ks], Sh[ks], Sl[ks]);
    __syncthreads();  // SA, Q, csum

    // ---- dK, dB, dR, dA, dw for the wave's keys ----
    f32x4_t VH = zero4(), SAH = zero4(), dYS = zero4(), QS = zero4();
    f32x4_t Gqv = zero4(), Gyv = zero4(), Gqs = zero4(), Gys = zero4();  // Gram matrices over the value rows
    const bool tv = r16 < L;
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) {
        uint4 sh, sl, qh, ql;
        get_split(sm.SA, lane, ks, sh, sl), get_split(sm.Q, lane, ks, qh, ql);
        const long o = at_tok(tv ? r16 : 0);
        const uint4 vh = bf16_frag(v + o, ks, q4, tv), yh = bf16_frag(dy + o, ks, q4, tv);  // (exact in bf16)
        VH = mma32(mma32(VH, vh, Hh[ks]), vh, Hl[ks]);
        SAH = mm3(SAH, sh, sl, Hh[ks], Hl[ks]);
        dYS = mma32(mma32(dYS, yh, Sh[ks]), yh, Sl[ks]);
        QS = mm3(QS, qh, ql, Sh[ks], Sl[ks]);
        Gqv = mma32(mma32(Gqv, qh, vh), ql, vh);   // Q_rr . V_cc
        Gyv = mma32(Gyv, yh, vh);                  // dY_rr . V_cc
        Gqs = mm3(Gqs, qh, ql, sh, sl);            // Q_rr . SA_cc
        Gys = mma32(mma32(Gys, yh, sh), yh, sl);   // dY_rr . SA_cc
    }
    const f32x4_t Gvq = transpose16(Gqv, lane), Gvy = transpose16(Gyv, lane);
    const f32x4_t Gsq = transpose16(Gqs, lane), Gsy = transpose16(Gys, lane);
    // masked transposes of the intra-chunk matrices, element [rr][cc] (rr = 4q4 + e, cc = r16)
    f32x4_t M1, M2, M3, M4, M5, M6, M7, M8;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        M1[e] = rr > cc ? Gqv[e] : 0.f;   // triu_s(V Q^T)^T
        M2[e] = rr >= cc ? Gyv[e] : 0.f;  // triu(V dY^T)^T
        M3[e] = rr > cc ? Gqs[e] : 0.f;   // triu_s(SA Q^T)^T
        M4[e] = rr >= cc ? Gys[e] : 0.f;  // triu(SA dY^T)^T
        M5[e] = rr <= cc ? Gsy[e] : 0.f;  // tril(dY SA^T)^T
        M6[e] = rr <= cc ? Gvy[e] : 0.f;  // tril(dY V^T)^T
        M7[e] = rr < cc ? Gsq[e] : 0.f;   // tril_s(Q SA^T)^T
        M8[e] = rr < cc ? Gvq[e] : 0.f;   // tril_s(Q V^T)^T
    }
    const Pk pAt = pk(At), pRt = pk(Rt), pBm = pk(Bm), pKm = pk(Km);
    const f32x4_t gK = eM * (VH * eLj + mm16s(pk(M1), pAt) + mm16s(pk(M2), pRt));
    const f32x4_t gB = eM * (SAH * eLj + mm16s(pk(M3), pAt) + mm16s(pk(M4), pRt));
    const f32x4_t gR = eR * (dYS + mm16s(pk(M5), pBm) + mm16s(pk(M6), pKm));
    const f32x4_t gA = eA * (QS + mm16s(pk(M7), pBm) + mm16s(pk(M8), pKm));
    // dlogd_t = sum_{s>=t} (r dR - b dB - k dK)_s + sum_{s>t} (a dA)_s + carry
    float sx[4], sy[4];
    {
        float x[4], y[4];
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = xr[e] * gR[e] - xb[e] * gB[e] - xk[e] * gK[e], y[e] = xa[e] * gA[e];
        sx[3] = x[3], sy[3] = 0.f;
#pragma unroll
        for (int e = 2; e >= 0; e--) sx[e] = sx[e + 1] + x[e], sy[e] = sy[e + 1] + y[e + 1];
        const float ytot = sy[0] + y[0];
        const float X1 = __shfl(sx[0], 16 + r16), X2 = __shfl(sx[0], 32 + r16), X3 = __shfl(sx[0], 48 + r16);
        const float Y1 = __shfl(ytot, 16 + r16), Y2 = __shfl(ytot, 32 + r16), Y3 = __shfl(ytot, 48 + r16);
        const float xa_ = (q4 < 1 ? X1 : 0.f) + (q4 < 2 ? X2 : 0.f) + (q4 < 3 ? X3 : 0.f);
        const float ya_ = (q4 < 1 ? Y1 : 0.f) + (q4 < 2 ? Y2 : 0.f) + (q4 < 3 ? Y3 : 0.f);
        float carry = 0.f;
#pragma unroll
        for (int u = 0; u < BTJ; u++) carry += sm.csum[u][col];
#pragma unroll
        for (int e = 0; e < 4; e++) sx[e] += xa_ + carry, sy[e] += ya_;
    }
    f32x4_t gW;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float s = sigmoidf_(xw[e]);
        gW[e] = (sx[e] + sy[e]) * (-DECAY_SCALE) * s * (1.f - s);
    }
    const int tr = 4 * q4 + (lane & 3);
    const uint2 qk = quad_rows_bf16(gK, lane), qb = quad_rows_bf16(gB, lane), qr = quad_rows_bf16(gR, lane),
                qa = quad_rows_bf16(gA, lane), qw = quad_rows_bf16(gW, lane);
    if (tr < L) {
        const long o = at_tok(tr) + 16 * wv + 4 * ((lane >> 2) & 3);
        *reinterpret_cast<uint2*>(dk + o) = qk;
        *reinterpret_cast<uint2*>(db + o) = qb;
        *reinterpret_cast<uint2*>(dr + o) = qr;
        *reinterpret_cast<uint2*>(da + o) = qa;
        *reinterpret_cast<uint2*>(dw + o) = qw;
    }
}


// ---------------------------------------------------------------------------
// The gated delta rule's backward (GDN layers: one decay e^{g_t} per token and head,
// r = q/sqrt(N), a = k, b = -e^{g} beta k, v' = beta v; q and k as the forward used them).
// With gamma the chunk's inclusive cumulative g, the per-key factors above become 16x16
// decay-ratio masks, every one of them e^{(a later gamma) - (an earlier one)} <= 1, so
// nothing overflows for any decay (as gdn_prep in the forward):
//   Aab[t][s] = -beta_s (k_t.k_s) e^{gm1_t - gm1_s} (s < t)   Aak = (k_t.k_s) e^{gm1_t - gam_s}
//   Brb[t][s] = -beta_s (r_t.k_s) e^{gam_t - gm1_s} (s <= t)  Brk = (r_t.k_s) e^{gam_t - gam_s}
//   A~ S0^T = e^{gm1_t} (k S0^T),  B^ H^T = -beta_t e^{gL - gm1_t} (k H^T),  K^ H^T = e^{gL - gam_t} (k H^T)
//   dK = e^{gL - gam_t} V'H + M1 k + M2 r,   dB = e^{gL - gam_t} SA H + M3 k + M4 r
//   dR = e^{gam_t} dY S0 + (M5 + M6) k,      dA = e^{gm1_t} Q S0 + (M7 + M8) k
// with M1 = triu_s(V'Q^T) e^{gm1_s - gam_t}, M2 = triu(V'dY^T) e^{gam_s - gam_t}, M3, M4 the
// same for SA, M5 = tril(dY SA^T) (-beta_s) e^{gam_t - gm1_s}, M6 = tril(dY V'^T)
// e^{gam_t - gam_s}, M7 = tril_s(Q SA^T) (-beta_s) e^{gm1_t - gm1_s}, M8 = tril_s(Q V'^T)
// e^{gm1_t - gam_s}; then dq = dR/sqrt(N), dk = dK + dA - e^{g} beta dB, dv = beta dV',
// dbeta = sum_i v dV' - e^{g} sum_j k dB, dg = sum_j dlogd - e^{g} beta sum_j k dB.
// (Checked in float64 against the oracle's exp-mode step adjoint, strong decays included,
// before the kernels.)  The reverse scan's records are the WKV7 ones (e^{gL} repeated
// per key), so wkv7_bwd_scan runs them unchanged.
// ---------------------------------------------------------------------------
template <typename TI>
__global__ __launch_bounds__(64) void gdn_bwd_prep(int Tn, int H, const TI* __restrict__ q, const TI* __restrict__ k,
                                                   const float* __restrict__ g, const float* __restrict__ beta,
                                                   uint8_t* __restrict__ ws) {
    using R = BwdRec;
    const int c = blockIdx.x, bh = blockIdx.y, nchunk = gridDim.x;
    const int bb = bh / H, h = bh - bb * H;
    const int lane = threadIdx.x, q4 = lane >> 4, r16 = lane & 15;
    const int t0 = c * BC, L = min(BC, Tn - t0);
    const long tok0 = (long)bb * Tn + t0;
    auto row = [&](int t) { return ((tok0 + t) * H + h) * (long)BNK; };
    const float rs = 1.f / __builtin_sqrtf((float)BNK);
    __shared__ float gsh[3][BC];  // gamma_t, gamma_{t-1}, beta_t (past the end: 0)
    const bool tv = r16 < L;
    const int tl = tv ? r16 : 0;  // (clamped: every lane loads)
    const float g_ = g[(tok0 + tl) * H + h], b_ = beta[(tok0 + tl) * H + h];
    const uint32_t tm = lane_mask(tv);
    const float gt = keep(tm, g_), bt = keep(tm, b_);
    const float gam = row_prefix_sum(gt), gm1 = row_prev(gam, 0.f), gL = row_last(gam);
    if (q4 == 0) gsh[0][r16] = gam, gsh[1][r16] = gm1, gsh[2][r16] = bt;
    uint8_t* const rec = ws + ((size_t)bh * nchunk + c) * R::BYTES;
    const float sb = -bt * __expf(gL - gm1);  // B^ = sb k for the lane's token
    f32x4_t KK = zero4(), KR = zero4();
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) {
        const int c0 = 32 * ks + 4 * q4;
        const float4 ka = keep4(tm, ld4f(k + row(tl) + c0)), kb = keep4(tm, ld4f(k + row(tl) + c0 + 16));
        const float4 qa = keep4(tm, ld4f(q + row(tl) + c0)), qb = keep4(tm, ld4f(q + row(tl) + c0 + 16));
        const float kr[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
        const float qr[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float br8[8];
#pragma unroll
        for (int e = 0; e < 8; e++) br8[e] = kr[e] * sb;
        uint4 kh, kl, qh, ql, bh_, bl;
        pack8(kr, kh, kl), pack8(qr, qh, ql), pack8(br8, bh_, bl);
        uint4* bf = reinterpret_cast<uint4*>(rec + R::BF) + (size_t)(2 * ks) * 64 + lane;
        bf[0] = bh_;
        bf[64] = bl;
        KK = mm3(KK, kh, kl, kh, kl);  // k_rr . k_cc
        KR = mm3(KR, kh, kl, qh, ql);  // k_rr . q_cc
    }
    __syncthreads();  // gsh
    const int cc = r16;
    f32x4_t Aab, AabT, BrbT;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        const float gm1r = gsh[1][rr], br = gsh[2][rr];
        const float kk = KK[e], kq = KR[e] * rs;  // k_rr.k_cc, k_rr.r_cc
        Aab[e] = cc < rr ? -bt * kk * __expf(gm1r - gm1) : 0.f;    // Aab[rr][cc]
        AabT[e] = rr < cc ? -br * kk * __expf(gm1 - gm1r) : 0.f;   // Aab[cc][rr]
        BrbT[e] = rr <= cc ? -br * kq * __expf(gam - gm1r) : 0.f;  // Brb[cc][rr]
    }
    f32x4_t Ti, TiT;
    tri_inverse(Aab, AabT, lane, Ti, TiT);
    const Pk pTiT = pk(TiT), pBrbT = pk(BrbT);
    float ea[4], er[4];
    const TI *krow[4], *qrow[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = 4 * q4 + e;
        krow[e] = k + row(t < L ? t : 0) + r16;
        qrow[e] = q + row(t < L ? t : 0) + r16;
        ea[e] = t < L ? __expf(gsh[1][t]) : 0.f;
        er[e] = t < L ? rs * __expf(gsh[0][t]) : 0.f;
    }
#pragma unroll
    for (int tj = 0; tj < BTJ; tj++) {
        f32x4_t at, rt;  // A~, R~ in D layout [t][j], j = 16tj + r16
#pragma unroll
        for (int e = 0; e < 4; e++) at[e] = io<TI>::ld(krow[e], 16 * tj) * ea[e], rt[e] = io<TI>::ld(qrow[e], 16 * tj) * er[e];
        const f32x4_t Pt = mm16s(pTiT, pk(at));
        const Pk pP = pk(Pt);
        const Pk pP2 = pk(rt + mm16s(pBrbT, pP));
        uint4* pp = reinterpret_cast<uint4*>(rec + R::PP) + (size_t)(2 * tj) * 64 + lane;
        pp[0] = cat(pP.h, pP2.h);
        pp[64] = cat(pP.l, pP2.l);
    }
    if (lane < BNK / 4) {
        const float egL = __expf(gL);
        reinterpret_cast<float4*>(rec + R::EL)[lane] = make_float4(egL, egL, egL, egL);
    }
}

struct GdnChunkLds {
    SplitPlane K, R;   // k, r = q / sqrt(N) [t][j], written by the key owners
    SplitPlane SA, Q;  // [t][i], written by the value-row owners
    float gam[BC], gm1[BC], beta[BC];
    float csum[BTJ][BNK];
    float pv[BTJ][BC], pd[BTJ][BC], pk[BTJ][BC];  // per wave and token: sum v dV', sum dlogd, sum k dB
};

template <typename TI>
__global__ __launch_bounds__(512) void gdn_bwd_chunk(int Tn, int H, int BH, int per_xcd, const TI* __restrict__ q,
                                                     const TI* __restrict__ k, const TI* __restrict__ v,
                                                     const float* __restrict__ g, const float* __restrict__ beta,
                                                     const TI* __restrict__ dy, const float* __restrict__ ckpt,
                                                     const float* __restrict__ hbuf, TI* __restrict__ dq,
                                                     TI* __restrict__ dk, TI* __restrict__ dv, float* __restrict__ dg,
                                                     float* __restrict__ dbeta) {
    __shared__ __attribute__((aligned(16))) GdnChunkLds sm;
    const int nchunk = (Tn + BC - 1) / BC;
    const int job = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    if (job >= nchunk * BH) return;  // (whole workgroup)
    const int bh = job / nchunk, c = job - bh * nchunk, bb = bh / H, h = bh - bb * H;
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
    const int t0 = c * BC, L = min(BC, Tn - t0);
    const long tok0 = (long)bb * Tn + t0;
    const int col = 16 * wv + r16;
    const float rs = 1.f / __builtin_sqrtf((float)BNK);
    auto at_tok = [&](int t) { return ((tok0 + t) * H + h) * (long)BNK; };
    const long ncp = nchunk + 1;
    const float* const S0 = ckpt + ((long)bh * ncp + c) * BNN;
    const float* const Se = S0 + BNN;
    const float* const Hm = hbuf + ((long)bh * nchunk + c) * BNN;
    const int irow = 16 * wv + r16;
    // the token scalars (wave 0)
    if (wv == 0) {
        const bool tv = r16 < L;
        const int tl = tv ? r16 : 0;  // (clamped: every lane loads)
        const float g_ = g[(tok0 + tl) * H + h], b_ = beta[(tok0 + tl) * H + h];
        const float gt = keep(lane_mask(tv), g_), bt = keep(lane_mask(tv), b_);
        const float gam = row_prefix_sum(gt), gm1 = row_prev(gam, 0.f);
        if (q4 == 0) sm.gam[r16] = gam, sm.gm1[r16] = gm1, sm.beta[r16] = bt;
    }
    float hr[BKS][8], sr[BKS][8];
    auto rows = [&](const float* M, float (&o)[BKS][8]) {
#pragma unroll
        for (int ks = 0; ks < BKS; ks++) {
            const float4 x = *reinterpret_cast<const float4*>(M + (long)irow * BNK + 32 * ks + 4 * q4);
            const float4 y = *reinterpret_cast<const float4*>(M + (long)irow * BNK + 32 * ks + 16 + 4 * q4);
            o[ks][0] = x.x, o[ks][1] = x.y, o[ks][2] = x.z, o[ks][3] = x.w;
            o[ks][4] = y.x, o[ks][5] = y.y, o[ks][6] = y.z, o[ks][7] = y.w;
        }
    };
    rows(Hm, hr);
    rows(Se, sr);
    // k and r of the wave's keys in D layout ([t][col], t = 4q4 + e)
    f32x4_t kD, rD;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = 4 * q4 + e;
        const bool ok = t < L;
        const long o = at_tok(ok ? t : 0) + col;  // (clamped: every lane loads)
        const float k_ = io<TI>::ld(k, o), q_ = io<TI>::ld(q, o);
        kD[e] = keep(lane_mask(ok), k_);
        rD[e] = keep(lane_mask(ok), q_) * rs;
    }
    put_split(sm.K, kD, lane, wv), put_split(sm.R, rD, lane, wv);
#pragma unroll
    for (int ks = 0; ks < BKS; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float s = row_sum16(hr[ks][e] * sr[ks][e]);
            if (r16 == 0) sm.csum[wv][32 * ks + (e < 4 ? 4 * q4 + e : 16 + 4 * q4 + e - 4)] = s;
        }
    uint4 Hh[BKS], Hl[BKS], Sh[BKS], Sl[BKS];
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) pack8(hr[ks], Hh[ks], Hl[ks]);
    rows(S0, sr);
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) pack8(sr[ks], Sh[ks], Sl[ks]);
    __syncthreads();

    // token scalars: rows rr = 4q4 + e, column token cc = r16
    const int cc = r16;
    float gr[4], gm1r[4], br[4];
#pragma unroll
    for (int e = 0; e < 4; e++) gr[e] = sm.gam[4 * q4 + e], gm1r[e] = sm.gm1[4 * q4 + e], br[e] = sm.beta[4 * q4 + e];
    const float gc = sm.gam[cc], gm1c = sm.gm1[cc], bc = sm.beta[cc], gL = sm.gam[BC - 1];
    // Gram matrices over the keys and the wave's products k S0^T, k H^T
    f32x4_t KK = zero4(), RK = zero4(), kS = zero4(), kH = zero4();
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) {
        uint4 kh, kl, rh, rl;
        get_split(sm.K, lane, ks, kh, kl), get_split(sm.R, lane, ks, rh, rl);
        KK = mm3(KK, kh, kl, kh, kl);
        RK = mm3(RK, rh, rl, kh, kl);  // r_rr . k_cc
        kS = mm3(kS, kh, kl, Sh[ks], Sl[ks]);
        kH = mm3(kH, kh, kl, Hh[ks], Hl[ks]);
    }
    f32x4_t Aab, AabT, Aak, Brb, Brk, P1, P2, P3;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        Aab[e] = cc < rr ? -bc * KK[e] * __expf(gm1r[e] - gm1c) : 0.f;
        AabT[e] = rr < cc ? -br[e] * KK[e] * __expf(gm1c - gm1r[e]) : 0.f;
        Aak[e] = cc < rr ? KK[e] * __expf(gm1r[e] - gc) : 0.f;
        Brb[e] = cc <= rr ? -bc * RK[e] * __expf(gr[e] - gm1c) : 0.f;
        Brk[e] = cc <= rr ? RK[e] * __expf(gr[e] - gc) : 0.f;
        P1[e] = kS[e] * __expf(gm1r[e]);
        P2[e] = kH[e] * (-br[e] * __expf(gL - gm1r[e]));
        P3[e] = kH[e] * __expf(gL - gr[e]);
    }
    f32x4_t Ti, TiT;
    tri_inverse(Aab, AabT, lane, Ti, TiT);
    const Pk pAak = pk(Aak), pBrb = pk(Brb), pBrk = pk(Brk), pTi = pk(Ti), pTiT = pk(TiT);
    const Pk pAakT = pk(transpose16(Aak, lane));

    auto put = [&](TI* dst, const f32x4_t& x) {
        if constexpr (sizeof(TI) == 2) {
            const int tr = 4 * q4 + (lane & 3);
            const uint2 qv = quad_rows_bf16(x, lane);  // (cross-lane: every lane takes part)
            if (tr < L) *reinterpret_cast<uint2*>(dst + at_tok(tr) + 16 * wv + 4 * ((lane >> 2) & 3)) = qv;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (4 * q4 + e < L) dst[at_tok(4 * q4 + e) + col] = x[e];
        }
    };
    // ---- SA, Q, dV' for the wave's value columns ----
    f32x4_t vraw, vD, dyD;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = 4 * q4 + e;
        const long o = at_tok(t < L ? t : 0) + col;
        const float v_ = io<TI>::ld(v, o), y_ = io<TI>::ld(dy, o);
        vraw[e] = keep(lane_mask(t < L), v_);
        vD[e] = br[e] * vraw[e];
        dyD[e] = keep(lane_mask(t < L), y_);
    }
    const Pk pV = pk(vD), pdY = pk(dyD);
    const f32x4_t SA = mm16s(pTiT, pk(P1 + mm16s(pAakT, pV)));
    const f32x4_t Q = mm16s(pTi, pk(P2 + mm16s(pBrb, pdY)));
    const f32x4_t dVp = P3 + mm16s(pAak, pk(Q)) + mm16s(pBrk, pdY);
    put_split(sm.SA, SA, lane, wv), put_split(sm.Q, Q, lane, wv);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float s = row_sum16(vraw[e] * dVp[e]);
        if (r16 == 0) sm.pv[wv][4 * q4 + e] = s;
    }
    put(dv, f32x4_t{br[0] * dVp[0], br[1] * dVp[1], br[2] * dVp[2], br[3] * dVp[3]});
#pragma unroll
    for (int ks = 0; ks < BKS; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int i = 32 * ks + (e < 4 ? 4 * q4 + e : 16 + 4 * q4 + e - 4);
            hr[ks][e] = Hm[(long)i * BNK + col];
            sr[ks][e] = S0[(long)i * BNK + col];
        }
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) pack8(hr[ks], Hh[ks], Hl[ks]), pack8(sr[ks], Sh[ks], Sl[ks]);
    __syncthreads();  // SA, Q, csum, pv

    // ---- dq, dk and the token sums for the wave's keys ----
    f32x4_t VH = zero4(), SAH = zero4(), dYS = zero4(), QS = zero4();
    f32x4_t Gqv = zero4(), Gyv = zero4(), Gqs = zero4(), Gys = zero4();
    const bool tv = r16 < L;
#pragma unroll
    for (int ks = 0; ks < BKS; ks++) {
        float fv[8], fy[8];
        {
            const long o = at_tok(tv ? r16 : 0) + 32 * ks + 4 * q4;
            const uint32_t m = lane_mask(tv);
            const float4 v0 = keep4(m, ld4f(v + o)), v1 = keep4(m, ld4f(v + o + 16));
            const float4 y0 = keep4(m, ld4f(dy + o)), y1 = keep4(m, ld4f(dy + o + 16));
            fv[0] = v0.x, fv[1] = v0.y, fv[2] = v0.z, fv[3] = v0.w, fv[4] = v1.x, fv[5] = v1.y, fv[6] = v1.z, fv[7] = v1.w;
            fy[0] = y0.x, fy[1] = y0.y, fy[2] = y0.z, fy[3] = y0.w, fy[4] = y1.x, fy[5] = y1.y, fy[6] = y1.z, fy[7] = y1.w;
#pragma unroll
            for (int e = 0; e < 8; e++) fv[e] *= bc;  // V' = beta v (the lane's token r16)
        }
        uint4 sh, sl, qh, ql, vh, vl, yh, yl;
        get_split(sm.SA, lane, ks, sh, sl), get_split(sm.Q, lane, ks, qh, ql);
        pack8(fv, vh, vl), pack8(fy, yh, yl);
        VH = mm3(VH, vh, vl, Hh[ks], Hl[ks]);
        SAH = mm3(SAH, sh, sl, Hh[ks], Hl[ks]);
        dYS = mm3(dYS, yh, yl, Sh[ks], Sl[ks]);
        QS = mm3(QS, qh, ql, Sh[ks], Sl[ks]);
        Gqv = mm3(Gqv, qh, ql, vh, vl);  // Q_rr . V'_cc
        Gyv = mm3(Gyv, yh, yl, vh, vl);  // dY_rr . V'_cc
        Gqs = mm3(Gqs, qh, ql, sh, sl);  // Q_rr . SA_cc
        Gys = mm3(Gys, yh, yl, sh, sl);  // dY_rr . SA_cc
    }
    const f32x4_t Gvq = transpose16(Gqv, lane), Gvy = transpose16(Gyv, lane);
    const f32x4_t Gsq = transpose16(Gqs, lane), Gsy = transpose16(Gys, lane);
    f32x4_t M1, M2, M3, M4, M56, M78;  // transposes, element [rr][cc]
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = 4 * q4 + e;
        M1[e] = rr > cc ? Gqv[e] * __expf(gm1r[e] - gc) : 0.f;
        M2[e] = rr >= cc ? Gyv[e] * __expf(gr[e] - gc) : 0.f;
        M3[e] = rr > cc ? Gqs[e] * __expf(gm1r[e] - gc) : 0.f;
        M4[e] = rr >= cc ? Gys[e] * __expf(gr[e] - gc) : 0.f;
        M56[e] = rr <= cc ? -br[e] * Gsy[e] * __expf(gc - gm1r[e]) + Gvy[e] * __expf(gc - gr[e]) : 0.f;
        M78[e] = rr < cc ? -br[e] * Gsq[e] * __expf(gm1c - gm1r[e]) + Gvq[e] * __expf(gm1c - gr[e]) : 0.f;
    }
    const Pk pkD = pk(kD), prD = pk(rD);
    const f32x4_t tK = mm16s(pk(M1), pkD) + mm16s(pk(M2), prD);
    const f32x4_t tB = mm16s(pk(M3), pkD) + mm16s(pk(M4), prD);
    const f32x4_t tR = mm16s(pk(M56), pkD), tA = mm16s(pk(M78), pkD);
    f32x4_t gK, gB, gR, gA, egb;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float fL = __expf(gL - gr[e]);
        gK[e] = fL * VH[e] + tK[e];
        gB[e] = fL * SAH[e] + tB[e];
        gR[e] = __expf(gr[e]) * dYS[e] + tR[e];
        gA[e] = __expf(gm1r[e]) * QS[e] + tA[e];
        egb[e] = __expf(gr[e] - gm1r[e]) * br[e];  // e^{g_t} beta_t
    }
    float sx[4], sy[4];
    {
        float x[4], y[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            x[e] = rD[e] * gR[e] + egb[e] * kD[e] * gB[e] - kD[e] * gK[e], y[e] = kD[e] * gA[e];
        sx[3] = x[3], sy[3] = 0.f;
#pragma unroll
        for (int e = 2; e >= 0; e--) sx[e] = sx[e + 1] + x[e], sy[e] = sy[e + 1] + y[e + 1];
        const float ytot = sy[0] + y[0];
        const float X1 = __shfl(sx[0], 16 + r16), X2 = __shfl(sx[0], 32 + r16), X3 = __shfl(sx[0], 48 + r16);
        const float Y1 = __shfl(ytot, 16 + r16), Y2 = __shfl(ytot, 32 + r16), Y3 = __shfl(ytot, 48 + r16);
        const float xa_ = (q4 < 1 ? X1 : 0.f) + (q4 < 2 ? X2 : 0.f) + (q4 < 3 ? X3 : 0.f);
        const float ya_ = (q4 < 1 ? Y1 : 0.f) + (q4 < 2 ? Y2 : 0.f) + (q4 < 3 ? Y3 : 0.f);
        float carry = 0.f;
#pragma unroll
        for (int u = 0; u < BTJ; u++) carry += sm.csum[u][col];
#pragma unroll
        for (int e = 0; e < 4; e++) sx[e] += xa_ + carry, sy[e] += ya_;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float sd = row_sum16(sx[e] + sy[e]), skb = row_sum16(kD[e] * gB[e]);
        if (r16 == 0) sm.pd[wv][4 * q4 + e] = sd, sm.pk[wv][4 * q4 + e] = skb;
    }
    put(dq, gR * rs);
    put(dk, gK + gA - egb * gB);
    __syncthreads();  // pd, pk
    if (wv == 0 && lane < L) {
        float spv = 0.f, spd = 0.f, spk = 0.f;
#pragma unroll
        for (int u = 0; u < BTJ; u++) spv += sm.pv[u][lane], spd += sm.pd[u][lane], spk += sm.pk[u][lane];
        const float eg = __expf(sm.gam[lane] - sm.gm1[lane]);
        const long o = (tok0 + lane) * H + h;
        dg[o] = spd - eg * sm.beta[lane] * spk;
        dbeta[o] = spv - eg * spk;
    }
}

}  // namespace

size_t wkv7_rec_bwd_workspace(int B, int T, int H) {
    const size_t n = (size_t)B * H * ((T + BC - 1) / BC);
    return (n * BwdRec::BYTES + 255) / 256 * 256 + n * BNN * sizeof(float);
}

void launch_wkv7_rec_backward(const Bwd& p) {
    const int nchunk = (p.T + BC - 1) / BC, BH = p.B * p.H;
    uint8_t* const recs = static_cast<uint8_t*>(p.ws);
    float* const hbuf = reinterpret_cast<float*>(recs + ((size_t)BH * nchunk * BwdRec::BYTES + 255) / 256 * 256);
    const bf16_t *r = static_cast<const bf16_t*>(p.r), *w = static_cast<const bf16_t*>(p.w),
                 *k = static_cast<const bf16_t*>(p.k), *v = static_cast<const bf16_t*>(p.v),
                 *a = static_cast<const bf16_t*>(p.a), *b = static_cast<const bf16_t*>(p.b),
                 *dy = static_cast<const bf16_t*>(p.dy);
    hipLaunchKernelGGL(wkv7_bwd_prep, dim3(nchunk, BH), dim3(64), 0, p.stream, p.T, p.H, r, w, k, a, b, recs);
    hipLaunchKernelGGL(wkv7_bwd_scan<bf16_t>, dim3(BH * (BNK / 64)), dim3(256), 0, p.stream, p.T, p.H, BH, 0, p.dsT,
                       dy, p.ds0, hbuf, recs);
    const int jobs = nchunk * BH, per_xcd = (jobs + 7) / 8;
    hipLaunchKernelGGL(wkv7_bwd_chunk, dim3(8 * per_xcd), dim3(512), 0, p.stream, p.T, p.H, BH, per_xcd, r, w, k, v,
                       a, b, dy, p.ckpt, hbuf, static_cast<bf16_t*>(p.dr), static_cast<bf16_t*>(p.dw),
                       static_cast<bf16_t*>(p.dk), static_cast<bf16_t*>(p.dv), static_cast<bf16_t*>(p.da),
                       static_cast<bf16_t*>(p.db));
}

size_t gdn_backward_workspace(int B, int T, int H) { return wkv7_rec_bwd_workspace(B, T, H); }

template <typename TI>
static void launch_gdn_bwd(const GdnBwd& p) {
    const int nchunk = (p.T + BC - 1) / BC, BH = p.B * p.H;
    uint8_t* const recs = static_cast<uint8_t*>(p.ws);
    float* const hbuf = reinterpret_cast<float*>(recs + ((size_t)BH * nchunk * BwdRec::BYTES + 255) / 256 * 256);
    const TI *q = static_cast<const TI*>(p.q), *k = static_cast<const TI*>(p.k), *v = static_cast<const TI*>(p.v),
             *dout = static_cast<const TI*>(p.dout);
    hipLaunchKernelGGL(gdn_bwd_prep<TI>, dim3(nchunk, BH), dim3(64), 0, p.stream, p.T, p.H, q, k, p.g, p.beta, recs);
    hipLaunchKernelGGL(wkv7_bwd_scan<TI>, dim3(BH * (BNK / 64)), dim3(256), 0, p.stream, p.T, p.H, BH, 1, p.dsT, dout,
                       p.ds0, hbuf, recs);
    const int jobs = nchunk * BH, per_xcd = (jobs + 7) / 8;
    hipLaunchKernelGGL(gdn_bwd_chunk<TI>, dim3(8 * per_xcd), dim3(512), 0, p.stream, p.T, p.H, BH, per_xcd, q, k, v,
                       p.g, p.beta, dout, p.ckpt, hbuf, static_cast<TI*>(p.dq), static_cast<TI*>(p.dk),
                       static_cast<TI*>(p.dv), p.dg, p.dbeta);
}
void launch_gdn_backward(const GdnBwd& p) {
    if (p.dtype == 0) launch_gdn_bwd<bf16_t>(p);
    else launch_gdn_bwd<float>(p);
}

}  // namespace wkv7
