// MFMA building blocks for the chunked WKV7 kernels (gfx950, wave64).
//
// Matrices that feed the matrix cores live in LDS as bfloat16 pairs (hi, lo)
// with x = hi + lo to ~2^-16 relative precision; a product of two such
// operands is formed from three bf16 MFMAs (hi*hi + hi*lo + lo*hi), which
// keeps float32-level accuracy on the bf16 matrix pipe.
//
// Fragment layouts, verified on gfx950 (lane l, q = l / 16, e = element):
//   v_mfma_f32_16x16x32_bf16: A[row = l%16][k = 8q+e], B[k = 8q+e][col = l%16]
//   v_mfma_f32_16x16x16_bf16: A[row = l%16][k = 4q+e], B[k = 4q+e][col = l%16]
//   accumulator (both):       D[row = 4q+e][col = l%16], e = 0..3
// Every operand array is therefore stored "[outer][k]" with k contiguous:
// A operands row-major, B operands as B^T.  Row strides are padded to
// K + 8 elements so a 16-lane group reading 16-byte fragments hits every
// LDS bank group exactly twice.
#pragma once

#include "wkv7_common.h"

namespace wkv7 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t zero4() { return f32x4_t{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ f32x4_t mma32(f32x4_t acc, uint4 a, uint4 b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mma16(f32x4_t acc, uint2 a, uint2 b) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, a),
                                                     __builtin_bit_cast(i16x4_t, b), acc, 0, 0, 0);
}

// hi = truncation of x to bf16 (exact remainder), lo = RNE(x - hi).
__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
    const uint32_t u = __float_as_uint(x);
    hi = static_cast<uint16_t>(u >> 16);
    lo = f32_to_bf16(x - __uint_as_float(u & 0xffff0000u));
}
// Split two floats at once into packed (hi, lo) bf16 pairs.
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    const uint32_t u0 = __float_as_uint(x0), u1 = __float_as_uint(x1);
    hi = (u0 >> 16) | (u1 & 0xffff0000u);
    lo = f32x2_to_bf16x2(x0 - __uint_as_float(u0 & 0xffff0000u), x1 - __uint_as_float(u1 & 0xffff0000u));
}
__device__ __forceinline__ float join_bf16(uint16_t hi, uint16_t lo) {
    return bf16_to_f32(hi) + bf16_to_f32(lo);
}

// An LDS operand: hi and lo planes, row stride ld (elements).
struct Op {
    uint16_t* hi;
    uint16_t* lo;
    int ld;
    __device__ __forceinline__ void put(int x, int k, float v) const {
        uint16_t h, l;
        split_bf16(v, h, l);
        hi[x * ld + k] = h;
        lo[x * ld + k] = l;
    }
    __device__ __forceinline__ float get(int x, int k) const { return join_bf16(hi[x * ld + k], lo[x * ld + k]); }
};

// 16x32 (A) / 32x16 (B) fragment: outer index x0 + l%16, k = k0 + 8q .. +7.
__device__ __forceinline__ uint4 frag32(const uint16_t* p, int ld, int x0, int k0, int lane) {
    return *reinterpret_cast<const uint4*>(p + (x0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
}
// 16x16 (A) / 16x16 (B) fragment for the K=16 instruction: k = k0 + 4q .. +3.
__device__ __forceinline__ uint2 frag16(const uint16_t* p, int ld, int x0, int k0, int lane) {
    return *reinterpret_cast<const uint2*>(p + (x0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4));
}

// acc += A[a_x0.., k0..k0+K) * B[k0..k0+K, b_x0..] for K = 32*nk (split precision).
// lo_a / lo_b: false when that operand is exact in bf16 (its lo plane is zero).
// NOTE: an accumulator produced by one MFMA shape is never fed straight into
// the SrcC of another shape (16x16x32 <-> 16x16x16): such back-to-back chains
// returned stale accumulator elements on gfx950.  Mixed-shape sums go through
// separate accumulators that are added with VALU instructions.
template <int NK, bool LO_A = true, bool LO_B = true>
__device__ __forceinline__ f32x4_t mma_k32(f32x4_t acc, const Op& A, int a_x0, const Op& B, int b_x0,
                                           int k0, int lane) {
    f32x4_t c1 = zero4(), c2 = zero4();
#pragma unroll
    for (int s = 0; s < NK; s++) {
        const int k = k0 + 32 * s;
        const uint4 ah = frag32(A.hi, A.ld, a_x0, k, lane);
        const uint4 bh = frag32(B.hi, B.ld, b_x0, k, lane);
        acc = mma32(acc, ah, bh);
        if (LO_B) c1 = mma32(c1, ah, frag32(B.lo, B.ld, b_x0, k, lane));
        if (LO_A) c2 = mma32(c2, frag32(A.lo, A.ld, a_x0, k, lane), bh);
    }
    return acc + c1 + c2;
}

// Same for one K=16 step.
template <bool LO_A = true, bool LO_B = true>
__device__ __forceinline__ f32x4_t mma_k16(f32x4_t acc, const Op& A, int a_x0, const Op& B, int b_x0,
                                           int k0, int lane) {
    const uint2 ah = frag16(A.hi, A.ld, a_x0, k0, lane);
    const uint2 bh = frag16(B.hi, B.ld, b_x0, k0, lane);
    acc = mma16(acc, ah, bh);
    f32x4_t c = zero4();
    if (LO_B) c = mma16(c, ah, frag16(B.lo, B.ld, b_x0, k0, lane));
    if (LO_A) c = mma16(c, frag16(A.lo, A.ld, a_x0, k0, lane), bh);
    return acc + c;
}

// 8 floats -> (hi, lo) bf16x8 fragments (element e in slot e).
__device__ __forceinline__ void pack8(const float* x, uint4& hi, uint4& lo) {
    split2(x[0], x[1], hi.x, lo.x);
    split2(x[2], x[3], hi.y, lo.y);
    split2(x[4], x[5], hi.z, lo.z);
    split2(x[6], x[7], hi.w, lo.w);
}
// accumulator (4 floats) -> (hi, lo) bf16x4 fragments: a D-layout tile used as
// the B operand of the K=16 instruction (its rows are the contraction index).
__device__ __forceinline__ void pack4(const f32x4_t& x, uint2& hi, uint2& lo) {
    split2(x[0], x[1], hi.x, lo.x);
    split2(x[2], x[3], hi.y, lo.y);
}
// Two 4-element fragments as one 8-element fragment: slots 0-3 = a, 4-7 = b.
// Used for K=32 steps whose k index is permuted (slot e <-> k0+4q+e,
// slot 4+e <-> k0+16+4q+e) so that two accumulator tiles form one B operand.
__device__ __forceinline__ uint4 cat(uint2 a, uint2 b) { return make_uint4(a.x, a.y, b.x, b.y); }
__device__ __forceinline__ uint2 ld8B(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }
// A-operand fragment of a [row][k] plane in the permuted K=32 order above.
__device__ __forceinline__ uint4 fragp(const uint16_t* p, int ld, int row, int k0, int lane) {
    const uint16_t* base = p + row * ld + k0 + 4 * (lane >> 4);
    return cat(ld8B(base), ld8B(base + 16));
}

// ---------------------------------------------------------------------------
// LDS transpose read (gfx950 ds_read_b64_tr_b16).  For a row-major bf16
// matrix X in LDS (row stride ld elements, 8-byte aligned rows), lane (q, r16)
// supplies &X[4q + r16/4][4*(r16%4)] and receives X[4q + e][r16], e = 0..3
// (layout verified with an in-bounds probe).  That is the B operand of the
// K=16 instruction for X, the A operand for X^T, and the D layout of X, read
// from memory whose rows run along the other index.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
__device__ __forceinline__ uint2 ldtr(const uint16_t* x, int ld, int lane) {
    const uint16_t* p = x + (4 * (lane >> 4) + ((lane & 15) >> 2)) * ld + 4 * (lane & 3);
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(uint16_t*)p));
}
// Row-swizzled bf16 planes without padding (gfx950 LDS, measured: 8-byte
// reads serve 32 lanes per cycle over 64 banks, 8-byte writes 16 lanes per
// cycle over 32 banks; 16-byte reads run at half the bandwidth of two 8-byte
// reads, so operands are read 8 bytes at a time).
//  * [rows][64] planes, 8-byte chunk c of row p stored at chunk c ^ swz(p):
//    SwLane = 4((p>>1)&3) + 2((p>>3)&1) + (p&1), conflict-free for 8-byte writes
//    down 16 rows, 8-byte reads down 16 rows and transpose reads;
//    SwDma  = the same without the last term, which keeps 16-byte pairs together
//    for planes filled by LDS DMA (8-byte writes down 16 rows then meet 2-way).
//  * [rows][16] planes (32-byte rows), chunk c of row p at c ^ ((p>>2)&3):
//    conflict-free for 8-byte writes and reads down 16 rows and transpose reads.
enum Sw { SwLane, SwDma };
template <Sw S> __device__ __forceinline__ int swz(int row) {
    return 4 * ((row >> 1) & 3) + 2 * ((row >> 3) & 1) + (S == SwLane ? (row & 1) : 0);
}
// element offset of (row, col) in a [rows][64] plane, col a multiple of 4
template <Sw S> __device__ __forceinline__ int pl(int row, int col) { return row * 64 + (((col >> 2) ^ swz<S>(row)) << 2); }
// element offset of (row, col) in a [rows][16] plane, col a multiple of 4
__device__ __forceinline__ int pl16(int row, int col) { return row * 16 + (((col >> 2) ^ ((row >> 2) & 3)) << 2); }
__device__ __forceinline__ uint2 tr_at(const uint16_t* p) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(uint16_t*)p));
}
// transpose read: lane gets X[row0 + 4q + e][col0 + l%16]
template <Sw S> __device__ __forceinline__ uint2 ldtr_sw(const uint16_t* x, int row0, int col0, int lane) {
    return tr_at(x + pl<S>(row0 + 4 * (lane >> 4) + ((lane & 15) >> 2), col0 + 4 * (lane & 3)));
}
__device__ __forceinline__ uint2 ldtr16(const uint16_t* x, int row0, int lane) {  // [rows][16] plane
    return tr_at(x + pl16(row0 + 4 * (lane >> 4) + ((lane & 15) >> 2), 4 * (lane & 3)));
}
template <Sw S> __device__ __forceinline__ uint2 ld8_sw(const uint16_t* x, int row, int col) {
    return *reinterpret_cast<const uint2*>(x + pl<S>(row, col));
}
template <Sw S> __device__ __forceinline__ void st8_sw(uint16_t* x, int row, int col, uint2 v) {
    *reinterpret_cast<uint2*>(x + pl<S>(row, col)) = v;
}
// 8 consecutive elements (two 8-byte reads / writes)
template <Sw S> __device__ __forceinline__ uint4 ld16_sw(const uint16_t* x, int row, int col) {
    return cat(ld8_sw<S>(x, row, col), ld8_sw<S>(x, row, col + 4));
}
template <Sw S> __device__ __forceinline__ void st16_sw(uint16_t* x, int row, int col, uint4 v) {
    st8_sw<S>(x, row, col, make_uint2(v.x, v.y));
    st8_sw<S>(x, row, col + 4, make_uint2(v.z, v.w));
}
// permuted K=32 A-operand fragment of row `row` (k = k0 + 4q + e, k0 + 16 + 4q + e)
template <Sw S> __device__ __forceinline__ uint4 fragp_sw(const uint16_t* x, int row, int k0, int lane) {
    const int c = k0 + 4 * (lane >> 4);
    return cat(ld8_sw<S>(x, row, c), ld8_sw<S>(x, row, c + 16));
}

// Orders this wave's earlier LDS accesses before its later ones (LDS executes
// one wave's instructions in order; this also stops the compiler from moving
// loads above stores it cannot prove disjoint).
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Row operations over the 16 lanes that share q (a "row" of the wave):
// inclusive prefix sum along r16, value of lane r16-1 (lane 0: `first`), and
// the value of lane 15 broadcast to the row.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float old, float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_prefix_sum(float x) {
    x += dpp_f<0x111>(0.f, x);  // row_shr:1
    x += dpp_f<0x112>(0.f, x);  // row_shr:2
    x += dpp_f<0x114>(0.f, x);  // row_shr:4
    x += dpp_f<0x118>(0.f, x);  // row_shr:8
    return x;
}
__device__ __forceinline__ float row_prev(float x, float first) { return dpp_f<0x111>(first, x); }

// A D-layout tile (lane (q, r16) holds rows 4q..4q+3 of column r16) rounded to
// bf16 and regrouped within each quad of lanes (r16 = 4m + jj) so that lane
// (q, 4m + jj) holds row 4q + jj, columns 4m..4m+3: an 8-byte piece of a row,
// stored with one instruction instead of four 2-byte ones.  Two DPP exchanges
// (quad_perm) and byte permutes, no LDS.
// quad_regroup does the regrouping for a tile already packed as bf16 row pairs (d0: rows
// 0, 1 and d1: rows 2, 3 of the lane's column), quad_rows_split for both halves of the
// tile's split-bf16 pair (split2's hi and lo).
__device__ __forceinline__ uint2 quad_regroup(uint32_t d0, uint32_t d1, int lane) {
    const bool lo2 = (lane & 2) == 0, odd = lane & 1;
    // lanes jj, jj^2 swap halves of the column: jj < 2 keeps rows 0,1 of columns jj, jj+2,
    // jj >= 2 keeps rows 2,3 of columns jj-2, jj (a0: the even column, a1: the odd+2 one)
    const uint32_t ra = __builtin_amdgcn_update_dpp(0, lo2 ? d1 : d0, 0x4e, 0xf, 0xf, false);  // quad_perm 2,3,0,1
    const uint32_t a0 = lo2 ? d0 : ra, a1 = lo2 ? ra : d1;
    // lanes jj, jj^1 swap rows: even lanes send their second row, odd lanes their first
    const uint32_t sb = __builtin_amdgcn_perm(a1, a0, odd ? 0x05040100u : 0x07060302u);
    const uint32_t rb = __builtin_amdgcn_update_dpp(0, sb, 0xb1, 0xf, 0xf, false);  // quad_perm 1,0,3,2
    return make_uint2(__builtin_amdgcn_perm(rb, a0, odd ? 0x03020504u : 0x05040100u),
                      __builtin_amdgcn_perm(rb, a1, odd ? 0x03020706u : 0x07060100u));
}
__device__ __forceinline__ uint2 quad_rows_bf16(const f32x4_t& d, int lane) {
    return quad_regroup(f32x2_to_bf16x2(d[0], d[1]), f32x2_to_bf16x2(d[2], d[3]), lane);  // rows (0,1), (2,3)
}
__device__ __forceinline__ void quad_rows_split(const f32x4_t& d, int lane, uint2& hi, uint2& lo) {
    uint32_t h01, l01, h23, l23;
    split2(d[0], d[1], h01, l01);
    split2(d[2], d[3], h23, l23);
    hi = quad_regroup(h01, h23, lane);
    lo = quad_regroup(l01, l23, lane);
}
__device__ __forceinline__ float row_last(float x) {  // ds_swizzle, and_mask 0x10, or_mask 0x0f
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1f0));
}

// Four 16-key tiles of a [token][key] operand held by a lane as
// x[tj][e] = X[t = r16][16 tj + 4q + e], split into (hi, lo) bf16 pairs.
// As the A or B operand of the K=32 instruction (slots e <-> 32s + 4q + e,
// 4 + e <-> 32s + 16 + 4q + e) it contracts over keys.
struct Pk4 {
    uint2 h[4], l[4];
};
__device__ __forceinline__ Pk4 pk4(const f32x4_t (&x)[4]) {
    Pk4 p;
#pragma unroll
    for (int tj = 0; tj < 4; tj++) pack4(x[tj], p.h[tj], p.l[tj]);
    return p;
}
// X Y^T over the 64 keys (split precision): D[t][s] = sum_j X[t][j] Y[s][j].
__device__ __forceinline__ f32x4_t mm_keys(const Pk4& X, const Pk4& Y) {
    f32x4_t acc = zero4(), c1 = zero4(), c2 = zero4();
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint4 ah = make_uint4(X.h[2 * s].x, X.h[2 * s].y, X.h[2 * s + 1].x, X.h[2 * s + 1].y);
        const uint4 al = make_uint4(X.l[2 * s].x, X.l[2 * s].y, X.l[2 * s + 1].x, X.l[2 * s + 1].y);
        const uint4 bh = make_uint4(Y.h[2 * s].x, Y.h[2 * s].y, Y.h[2 * s + 1].x, Y.h[2 * s + 1].y);
        const uint4 bl = make_uint4(Y.l[2 * s].x, Y.l[2 * s].y, Y.l[2 * s + 1].x, Y.l[2 * s + 1].y);
        acc = mma32(acc, ah, bh);
        c1 = mma32(c1, ah, bl);
        c2 = mma32(c2, al, bh);
    }
    return acc + c1 + c2;
}

// ---------------------------------------------------------------------------
// 16x16 tile algebra entirely in accumulator registers.
// A D-layout tile X (lane (q, r16) holds X[4q+e][r16]) is the B operand of
// the K=16 instruction as it stands, and it is the A operand of X^T.  So a
// product Z = X Y needs X^T and Y in D layout, and Z^T = Y^T X^T uses the same
// two packed tiles with the roles swapped.
// ---------------------------------------------------------------------------
struct Pk {
    uint2 h, l;
};
__device__ __forceinline__ Pk pk(const f32x4_t& x) {
    Pk p;
    pack4(x, p.h, p.l);
    return p;
}
// split-precision product of packed tiles: A = packed D-layout of X^T, B = of Y
__device__ __forceinline__ f32x4_t mm16s(const Pk& A, const Pk& B) {
    // one accumulator chain: no VALU adds (per SIMD the VALU is the busier pipe)
    return mma16(mma16(mma16(zero4(), A.h, B.h), A.h, B.l), A.l, B.h);
}
// (I - L)^{-1} = (I + L)(I + L^2)(I + L^4)(I + L^8) for a strictly lower
// triangular 16x16 L (L^16 = 0), from L and L^T in D layout; returns the
// inverse and its transpose in D layout.
__device__ __forceinline__ void tri_inverse(const f32x4_t& L, const f32x4_t& LT, int lane, f32x4_t& Ti,
                                            f32x4_t& TiT) {
    const Pk pL = pk(L), pLT = pk(LT);
    const f32x4_t L2 = mm16s(pLT, pL), L2T = mm16s(pL, pLT);
    const Pk pL2 = pk(L2), pL2T = pk(L2T);
    const f32x4_t L4 = mm16s(pL2T, pL2), L4T = mm16s(pL2, pL2T);
    const Pk pL4 = pk(L4), pL4T = pk(L4T);
    const Pk pL8T = pk(mm16s(pL4, pL4T));
    f32x4_t M, MT;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float d = (4 * (lane >> 4) + e) == (lane & 15) ? 1.f : 0.f;
        M[e] = L[e] + d;
        MT[e] = LT[e] + d;
    }
    Pk pM = pk(M);
    M += mm16s(pL2T, pM);
    MT += mm16s(pM, pL2T);
    pM = pk(M);
    M += mm16s(pL4T, pM);
    MT += mm16s(pM, pL4T);
    pM = pk(M);
    Ti = M + mm16s(pL8T, pM);
    TiT = MT + mm16s(pM, pL8T);
}

}  // namespace wkv7
