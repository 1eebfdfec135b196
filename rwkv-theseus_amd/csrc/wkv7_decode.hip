// Single-step (T = 1) WKV7 update -- the serving step: the fp32 state is read
// from s_in and the new state written to s_out, which may be the same buffer
// (in place: each lane reads its state elements before it writes them, and no
// lane touches another's).  HBM-bound: per (b,h) it moves 2*N*N*4 bytes of
// state and 7*N token values.
//
// One 256-lane workgroup per (b,h).  Each value row is handled by a 16-lane
// group; a lane owns VEC consecutive keys (float4 when N % 4 == 0, so one
// 16-lane group reads a 256-byte row of an N=64 state in one coalesced
// request).  Row sums (sa_i, y_i) are 16-lane butterfly reductions.
#include "wkv7_common.h"

namespace wkv7 {

template <typename T, int VEC, int NP>
__global__ __launch_bounds__(256) void decode_step(
    int H, int N, const T* __restrict__ r, const T* __restrict__ w, const T* __restrict__ k,
    const T* __restrict__ v, const T* __restrict__ a, const T* __restrict__ b,
    const float* s_in, float* s_out, T* __restrict__ y) {
    constexpr int MM = (NP + 16 * VEC - 1) / (16 * VEC);  // key groups per lane
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
            const int j = VEC * (l16 + 16 * m) + e;
            const bool ok = j < N;
            kr[m][e] = ok ? io<T>::ld(r, o + j) : 0.f;
            kd[m][e] = ok ? __expf(log_decay(io<T>::ld(w, o + j))) : 1.f;
            kk[m][e] = ok ? io<T>::ld(k, o + j) : 0.f;
            ka[m][e] = ok ? io<T>::ld(a, o + j) : 0.f;
            kb[m][e] = ok ? io<T>::ld(b, o + j) : 0.f;
        }

    for (int i0 = 0; i0 < N; i0 += 16) {
        const int i = i0 + grp;
        const bool row = i < N;
        float s[MM][VEC];
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const int j0 = VEC * (l16 + 16 * m);
            if constexpr (VEC == 4) {
                if (row && j0 < N) {
                    const float4 x = *reinterpret_cast<const float4*>(S + (long)i * N + j0);
                    s[m][0] = x.x; s[m][1] = x.y; s[m][2] = x.z; s[m][3] = x.w;
                } else {
                    s[m][0] = s[m][1] = s[m][2] = s[m][3] = 0.f;
                }
            } else {
#pragma unroll
                for (int e = 0; e < VEC; e++)
                    s[m][e] = (row && j0 + e < N) ? S[(long)i * N + j0 + e] : 0.f;
            }
        }
        float sa = 0.f;
#pragma unroll
        for (int m = 0; m < MM; m++)
#pragma unroll
            for (int e = 0; e < VEC; e++) sa += s[m][e] * ka[m][e];
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) sa += __shfl_xor(sa, off, 16);
        const float vi = row ? io<T>::ld(v, o + i) : 0.f;
        float out = 0.f;
#pragma unroll
        for (int m = 0; m < MM; m++)
#pragma unroll
            for (int e = 0; e < VEC; e++) {
                s[m][e] = s[m][e] * kd[m][e] + (sa * kb[m][e] + vi * kk[m][e]);
                out += s[m][e] * kr[m][e];
            }
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) out += __shfl_xor(out, off, 16);
        if (row && l16 == 0) io<T>::st(y, o + i, out);
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const int j0 = VEC * (l16 + 16 * m);
            if constexpr (VEC == 4) {
                if (row && j0 < N)
                    *reinterpret_cast<float4*>(So + (long)i * N + j0) =
                        make_float4(s[m][0], s[m][1], s[m][2], s[m][3]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; e++)
                    if (row && j0 + e < N) So[(long)i * N + j0 + e] = s[m][e];
            }
        }
    }
}

}  // namespace wkv7

#include "wkv7_launch.h"

namespace wkv7 {

template <typename T>
static void decode_t(const Dec& p) {
    const dim3 grid(p.B * p.H), block(256);
    if (p.N % 4 == 0) {
        if (p.N <= 64)
            hipLaunchKernelGGL((decode_step<T, 4, 64>), grid, block, 0, p.stream, p.H, p.N, (const T*)p.r,
                               (const T*)p.w, (const T*)p.k, (const T*)p.v, (const T*)p.a, (const T*)p.b, p.state_in, p.state, (T*)p.y);
        else
            hipLaunchKernelGGL((decode_step<T, 4, 128>), grid, block, 0, p.stream, p.H, p.N, (const T*)p.r,
                               (const T*)p.w, (const T*)p.k, (const T*)p.v, (const T*)p.a, (const T*)p.b, p.state_in, p.state, (T*)p.y);
    } else {
        hipLaunchKernelGGL((decode_step<T, 1, 128>), grid, block, 0, p.stream, p.H, p.N, (const T*)p.r,
                           (const T*)p.w, (const T*)p.k, (const T*)p.v, (const T*)p.a, (const T*)p.b, p.state_in, p.state, (T*)p.y);
    }
}

void launch_decode(const Dec& p) {
    if (p.dtype == 0) decode_t<bf16_t>(p); else decode_t<float>(p);
}

}  // namespace wkv7
