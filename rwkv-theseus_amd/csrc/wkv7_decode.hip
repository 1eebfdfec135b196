// Single-step (T = 1) WKV7 update -- the serving step: the fp32 state is read
// from s_in and the new state written to s_out, which may be the same buffer
// (in place: each lane reads its state elements before it writes them, and no
// lane touches another's).  HBM-bound: per (b,h) it moves 2*N*N*4 bytes of
// state and 7*N token values.
//
// One workgroup of G 16-lane groups per (b,h); group g handles value rows
// g, g + G, ...; a lane owns VEC consecutive keys (float4 when N % 4 == 0, so
// one 16-lane group reads a 256-byte row of an N=64 state in one coalesced
// request).  Row sums (sa_i, y_i) are 16-lane butterfly reductions.  For
// N <= 64 a workgroup is one wave (G = 4, 16 rows per lane, all 16 row loads in
// flight at once), so every head of a B=64, H=80 step is resident at once; for
// larger N it is 256 lanes (G = 16).
#include "wkv7_common.h"
#include "wkv7_io.h"

namespace wkv7 {

template <typename T, int VEC, int NP, int G, int MODE>
__global__ __launch_bounds__(16 * G) void decode_step(
    int H, int N, const T* __restrict__ r, const T* __restrict__ w, const T* __restrict__ k,
    const T* __restrict__ v, const T* __restrict__ a, const T* __restrict__ b,
    const float* s_in, float* s_out, T* __restrict__ y) {
    constexpr int MM = (NP + 16 * VEC - 1) / (16 * VEC);  // key groups per lane
    // rows per lane (i = G rr + grp), handled RB at a time: all at once for the float4
    // variants, one by one for the scalar one (whose key loop is long)
    constexpr int RR = NP / G, RB = VEC == 4 ? RR : 1;
    const int bh = blockIdx.x;
    const int l16 = threadIdx.x & 15, grp = threadIdx.x >> 4;
    const long o = (long)bh * N;  // token vectors of this (b,h): T = 1
    const float* S = s_in + (long)bh * N * N;
    float* So = s_out + (long)bh * N * N;

    float kr[MM][VEC], kd[MM][VEC], kk[MM][VEC], ka[MM][VEC], kb[MM][VEC];
#pragma unroll
    for (int m = 0; m < MM; m++)
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            // keys past N read key 0 and are masked after the load (a load under a branch
            // would wait for every earlier load of the wave)
            const int j = VEC * (l16 + 16 * m) + e;
            const bool ok = j < N;
            const long jj = o + (ok ? j : 0);
            const uint32_t mk = lane_mask(ok);
            kr[m][e] = keep(mk, io<T>::ld(r, jj));
            const float dd = decay_of<MODE>(io<T>::ld(w, jj));
            kd[m][e] = __uint_as_float((__float_as_uint(dd) & mk) | (0x3f800000u & ~mk));  // 1 past N
            kk[m][e] = keep(mk, io<T>::ld(k, jj));
            ka[m][e] = keep(mk, io<T>::ld(a, jj));
            kb[m][e] = keep(mk, io<T>::ld(b, jj));
        }
    for (int r0 = 0; r0 < RR; r0 += RB) {
        // the batch's state elements are all loaded before any is stored (so the loads are
        // in flight together; s_in == s_out is safe as a lane rewrites only what it read)
        float s[RB][MM][VEC];
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const int i = G * (r0 + rr) + grp;
#pragma unroll
            for (int m = 0; m < MM; m++) {
                const int j0 = VEC * (l16 + 16 * m);
                if constexpr (VEC == 4) {
                    const bool ok = i < N && j0 < N;
                    const float4 x = keep4(lane_mask(ok), *reinterpret_cast<const float4*>(S + (ok ? (long)i * N + j0 : 0)));
                    s[rr][m][0] = x.x; s[rr][m][1] = x.y; s[rr][m][2] = x.z; s[rr][m][3] = x.w;
                } else {
#pragma unroll
                    for (int e = 0; e < VEC; e++) {
                        const bool ok = i < N && j0 + e < N;
                        s[rr][m][e] = keep(lane_mask(ok), S[ok ? (long)i * N + j0 + e : 0]);
                    }
                }
            }
        }
        float vi[RB];
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const int i = G * (r0 + rr) + grp;
            vi[rr] = keep(lane_mask(i < N), io<T>::ld(v, o + (i < N ? i : 0)));
        }

#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const int i = G * (r0 + rr) + grp;
            float sa = 0.f;
#pragma unroll
            for (int m = 0; m < MM; m++)
#pragma unroll
                for (int e = 0; e < VEC; e++) sa += s[rr][m][e] * ka[m][e];
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) sa += __shfl_xor(sa, off, 16);
            float out = 0.f;
#pragma unroll
            for (int m = 0; m < MM; m++)
#pragma unroll
                for (int e = 0; e < VEC; e++) {
                    s[rr][m][e] = s[rr][m][e] * kd[m][e] + (sa * kb[m][e] + vi[rr] * kk[m][e]);
                    out += s[rr][m][e] * kr[m][e];
                }
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) out += __shfl_xor(out, off, 16);
            if (i < N && l16 == 0) io<T>::st(y, o + i, out);
        }
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const int i = G * (r0 + rr) + grp;
#pragma unroll
            for (int m = 0; m < MM; m++) {
                const int j0 = VEC * (l16 + 16 * m);
                if constexpr (VEC == 4) {
                    if (i < N && j0 < N)
                        *reinterpret_cast<float4*>(So + (long)i * N + j0) =
                            make_float4(s[rr][m][0], s[rr][m][1], s[rr][m][2], s[rr][m][3]);
                } else {
#pragma unroll
                    for (int e = 0; e < VEC; e++)
                        if (i < N && j0 + e < N) So[(long)i * N + j0 + e] = s[rr][m][e];
                }
            }
        }
    }
}

// N = 64 exactly (the chunked kernels' head size): one wave per (b,h), no
// bounds checks.  Lane group g = lane / 16 owns rows g, g + 4, ..., g + 60 and
// lane l16 keys 4 l16 .. 4 l16 + 3; all 16 rows of a lane are loaded before any
// is stored (s_in == s_out is safe: a lane rewrites only what it read); row sums
// are DPP reductions; lane l16 of group g writes y[4 l16 + g], so the wave's y
// store is one 128-byte row.
template <typename T> __device__ __forceinline__ void ld4(const T* p, float (&x)[4]);
template <> __device__ __forceinline__ void ld4<float>(const float* p, float (&x)[4]) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    x[0] = u.x, x[1] = u.y, x[2] = u.z, x[3] = u.w;
}
template <> __device__ __forceinline__ void ld4<bf16_t>(const bf16_t* p, float (&x)[4]) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    x[0] = __uint_as_float(u.x << 16), x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16), x[3] = __uint_as_float(u.y & 0xffff0000u);
}

template <typename T, int MODE>
// (five waves per SIMD: at the compiler's 98 VGPRs only four fit, so a B=64, H=80 step's
// 5120 waves took 1.25 rounds; at 94 they all run at once, 27.5 -> 26.8 µs per step)
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(5, 8))) void decode_step64(
    const T* __restrict__ r, const T* __restrict__ w, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ a, const T* __restrict__ b, const float* s_in, float* s_out, T* __restrict__ y) {
    const int l16 = threadIdx.x & 15, grp = threadIdx.x >> 4;
    const long o = (long)blockIdx.x * 64;
    const float* S = s_in + (long)blockIdx.x * 4096 + 4 * l16;
    float* So = s_out + (long)blockIdx.x * 4096 + 4 * l16;
    float4 s[16];
#pragma unroll
    for (int rr = 0; rr < 16; rr++) s[rr] = *reinterpret_cast<const float4*>(S + (4 * rr + grp) * 64);
    float kr[4], kw[4], kk[4], ka[4], kb[4], vi[16];
    ld4(r + o + 4 * l16, kr);
    ld4(w + o + 4 * l16, kw);
    ld4(k + o + 4 * l16, kk);
    ld4(a + o + 4 * l16, ka);
    ld4(b + o + 4 * l16, kb);
#pragma unroll
    for (int rr = 0; rr < 16; rr++) vi[rr] = io<T>::ld(v, o + 4 * rr + grp);
    float kd[4];
#pragma unroll
    for (int e = 0; e < 4; e++) kd[e] = decay_of<MODE>(kw[e]);
    float yv = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; rr++) {
        float4& x = s[rr];
        const float sa = row_sum16(x.x * ka[0] + x.y * ka[1] + x.z * ka[2] + x.w * ka[3]);
        x.x = x.x * kd[0] + (sa * kb[0] + vi[rr] * kk[0]);
        x.y = x.y * kd[1] + (sa * kb[1] + vi[rr] * kk[1]);
        x.z = x.z * kd[2] + (sa * kb[2] + vi[rr] * kk[2]);
        x.w = x.w * kd[3] + (sa * kb[3] + vi[rr] * kk[3]);
        const float out = row_sum16(x.x * kr[0] + x.y * kr[1] + x.z * kr[2] + x.w * kr[3]);
        if (l16 == rr) yv = out;
    }
    io<T>::st(y, o + 4 * l16 + grp, yv);
#pragma unroll
    for (int rr = 0; rr < 16; rr++) *reinterpret_cast<float4*>(So + (4 * rr + grp) * 64) = s[rr];
}

}  // namespace wkv7

#include "wkv7_launch.h"

namespace wkv7 {

template <typename T, int VEC, int NP, int G, int MODE>
static void decode_launch(const Dec& p) {
    hipLaunchKernelGGL((decode_step<T, VEC, NP, G, MODE>), dim3(p.B * p.H), dim3(16 * G), 0, p.stream, p.H, p.N,
                       (const T*)p.r, (const T*)p.w, (const T*)p.k, (const T*)p.v, (const T*)p.a, (const T*)p.b,
                       p.state_in, p.state, (T*)p.y);
}
template <typename T, int MODE>
static void decode_t(const Dec& p) {
    if (p.N == 64) {
        hipLaunchKernelGGL((decode_step64<T, MODE>), dim3(p.B * p.H), dim3(64), 0, p.stream, (const T*)p.r,
                           (const T*)p.w, (const T*)p.k, (const T*)p.v, (const T*)p.a, (const T*)p.b, p.state_in,
                           p.state, (T*)p.y);
    } else if (p.N % 4 == 0) {
        if (p.N <= 64) decode_launch<T, 4, 64, 4, MODE>(p);
        else decode_launch<T, 4, 128, 16, MODE>(p);
    } else {
        decode_launch<T, 1, 128, 16, MODE>(p);
    }
}

// (states [value][key] only: a call with FLAG_STATE_KV runs the step-serial forward)
void launch_decode(const Dec& p) {
    const bool ex = p.flags & FLAG_DECAY_EXP;
    if (p.dtype == 0) {
        if (ex) decode_t<bf16_t, MODE_EXP>(p); else decode_t<bf16_t, MODE_RWKV>(p);
    } else {
        if (ex) decode_t<float, MODE_EXP>(p); else decode_t<float, MODE_RWKV>(p);
    }
}

}  // namespace wkv7
