// Step-serial WKV7 kernels for any head size 2..128 (the generic path).
//
// One workgroup per (batch, head), one lane per value row i.  Forward keeps
// row i of the fp32 state in VGPRs; the per-step key vectors are staged
// through double-buffered LDS so each step needs a single barrier.  The
// state is written to the checkpoint buffer every CKPT steps.
//
// Backward walks the CKPT-step segments in reverse.  For each segment it
// replays the forward from the segment's checkpoint into a per-(b,h) slice of
// the caller's workspace (CKPT+1 states plus the sa vectors), then runs the
// adjoint of kernels/wkv7_state.cu:52-77 step by step in reverse.  Row sums
// (q, dv) are done by the lane that owns row i; column sums (dr, dw, dk, db,
// da) by the lane that owns column j, reading the transposed gradient state
// from LDS -- a fixed-order reduction, so results are deterministic (the
// reference uses fp32 atomicAdd, cu:68-72).
//
// MODE picks the decay (MODE_RWKV / MODE_EXP, wkv7_common.h); `kv` != 0 means the
// caller's states (s0, sT, dsT, ds0) are stored [key][value] (GDN's layout) instead of
// [value][key]: lane i then reads and writes element (j, i) at j*N + i, which is
// coalesced across lanes.  Saved states always use [value][key].
#include "wkv7_common.h"
#include "wkv7_io.h"

namespace wkv7 {

template <typename T, int NP, int MODE>
__global__ __launch_bounds__(NP) void seq_forward(
    int Tn, int H, int N, int kv, const T* __restrict__ r, const T* __restrict__ w,
    const T* __restrict__ k, const T* __restrict__ v, const T* __restrict__ a,
    const T* __restrict__ b, const float* s0, T* __restrict__ y,
    float* sT, float* __restrict__ ckpt) {
    const int bh = blockIdx.x, bb = bh / H, h = bh % H, i = threadIdx.x;
    const bool row = i < N;
    const long NN = (long)N * N;
    const long ncp = ckpt_count(Tn);
    __shared__ float vec[2][5][NP];  // r, d, k, a, b for the current / next step

    // element (i, j) of a caller state: [value][key], or [key][value] when kv
    const long ei = kv ? 1 : N, ej = kv ? N : 1;
    float st[NP];
#pragma unroll
    for (int j = 0; j < NP; j++) st[j] = (row && j < N) ? s0[bh * NN + i * ei + j * ej] : 0.f;
    if (ckpt && row) {
#pragma unroll
        for (int j = 0; j < NP; j++)
            if (j < N) ckpt[(bh * ncp) * NN + (long)i * N + j] = st[j];
    }

    auto stage = [&](int t, int buf) {
        const long o = ((long)(bb * Tn + t) * H + h) * N;
        if (row) {
            vec[buf][0][i] = io<T>::ld(r, o + i);
            vec[buf][1][i] = decay_of<MODE>(io<T>::ld(w, o + i));
            vec[buf][2][i] = io<T>::ld(k, o + i);
            vec[buf][3][i] = io<T>::ld(a, o + i);
            vec[buf][4][i] = io<T>::ld(b, o + i);
        } else {  // padded keys: zero r/k/a/b keep padded state columns at zero
            vec[buf][0][i] = 0.f; vec[buf][1][i] = 1.f;
            vec[buf][2][i] = 0.f; vec[buf][3][i] = 0.f; vec[buf][4][i] = 0.f;
        }
    };
    stage(0, 0);
    __syncthreads();
    for (int t = 0; t < Tn; t++) {
        const int buf = t & 1;
        const long o = ((long)(bb * Tn + t) * H + h) * N;
        const float vi = row ? io<T>::ld(v, o + i) : 0.f;
        if (t + 1 < Tn) stage(t + 1, buf ^ 1);
        float sa = 0.f;
#pragma unroll
        for (int j = 0; j < NP; j++) sa += st[j] * vec[buf][3][j];
        float out = 0.f;
#pragma unroll
        for (int j = 0; j < NP; j++) {
            st[j] = st[j] * vec[buf][1][j] + (sa * vec[buf][4][j] + vi * vec[buf][2][j]);
            out += st[j] * vec[buf][0][j];
        }
        if (row) io<T>::st(y, o + i, out);
        if (ckpt && row && ((t + 1) % CKPT == 0 || t + 1 == Tn)) {
            const long c = (t + CKPT) / CKPT;  // (t+1)/CKPT, or the last slot for a tail
#pragma unroll
            for (int j = 0; j < NP; j++)
                if (j < N) ckpt[(bh * ncp + c) * NN + (long)i * N + j] = st[j];
        }
        __syncthreads();
    }
    if (row) {
#pragma unroll
        for (int j = 0; j < NP; j++)
            if (j < N) sT[bh * NN + i * ei + j * ej] = st[j];
    }
}

// Workspace floats per (b,h) for seq_backward: CKPT+1 states and CKPT sa rows.
__host__ __device__ inline long seq_ws_floats(int N) { return (long)(CKPT + 1) * N * N + (long)CKPT * N; }

template <typename T, int NP, int MODE>
__global__ __launch_bounds__(NP) void seq_backward(
    int Tn, int H, int N, int kv, const T* __restrict__ r, const T* __restrict__ w,
    const T* __restrict__ k, const T* __restrict__ v, const T* __restrict__ a,
    const T* __restrict__ b, const float* __restrict__ ckpt, const T* __restrict__ dy,
    const float* __restrict__ dsT, T* __restrict__ dr, T* __restrict__ dw,
    T* __restrict__ dk, T* __restrict__ dv, T* __restrict__ da, T* __restrict__ db,
    float* __restrict__ ds0, float* __restrict__ ws) {
    const int bh = blockIdx.x, bb = bh / H, h = bh % H, tid = threadIdx.x;
    const bool lane_ok = tid < N;
    const long NN = (long)N * N;
    const long ncp = ckpt_count(Tn);
    float* wst = ws + bh * seq_ws_floats(N);     // states [CKPT+1][N][N]
    float* wsa = wst + (long)(CKPT + 1) * NN;    // sa     [CKPT][N]

    // G^T lives in LDS with a rotation swizzle: element (i,j) at [i][(i+j)%NP],
    // so both the row writes (lane i) and the column reads (lane j) are free
    // of bank conflicts.
    extern __shared__ float lds[];
    float* Gs = lds;                     // [NP][NP]
    float* vr = Gs + NP * NP;            // per-step vectors, NP each:
    float* vd = vr + NP;                 //   r, d, dlogd/dw factor, k, a, b,
    float* vf = vd + NP;                 //   dy, v, sa, q
    float* vk = vf + NP;
    float* va = vk + NP;
    float* vb = va + NP;
    float* vdy = vb + NP;
    float* vv = vdy + NP;
    float* vsa = vv + NP;
    float* vq = vsa + NP;

    // G row `tid` (gradient w.r.t. the state), kept in registers; element (i, j) of a
    // caller state at i*ei + j*ej ([value][key], or [key][value] when kv)
    const long ei = kv ? 1 : N, ej = kv ? N : 1;
    // (edge lanes and columns read element 0 and are masked after the load, here and below:
    // a load under a branch is waited for inside it, one after another)
    const int tc = lane_ok ? tid : 0;
    const uint32_t lm = lane_mask(lane_ok);
    float g[NP];
#pragma unroll
    for (int j = 0; j < NP; j++) g[j] = 0.f;
    if (dsT) {
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const bool ok = lane_ok && j < N;
            g[j] = keep(lane_mask(ok), dsT[bh * NN + (ok ? tid * ei + j * ej : 0)]);
        }
    }

    const int nseg = (Tn + CKPT - 1) / CKPT;
    for (int c = nseg - 1; c >= 0; c--) {
        const int t0 = c * CKPT;
        const int L = min(CKPT, Tn - t0);
        __syncthreads();  // the later segment's column phase is done reading ws
        // ---- replay the segment forward, storing states and sa into ws ----
        float st[NP];
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const bool ok = lane_ok && j < N;
            st[j] = keep(lane_mask(ok), ckpt[(bh * ncp + c) * NN + (ok ? (long)tid * N + j : 0)]);
        }
        if (lane_ok) {
#pragma unroll
            for (int j = 0; j < NP; j++)
                if (j < N) wst[(long)tid * N + j] = st[j];
        }
        for (int u = 0; u < L; u++) {
            const long o = ((long)(bb * Tn + t0 + u) * H + h) * N;
            const float xw = io<T>::ld(w, o + tc), xk = io<T>::ld(k, o + tc), xa = io<T>::ld(a, o + tc);
            const float xb = io<T>::ld(b, o + tc), vi = keep(lm, io<T>::ld(v, o + tc));
            __syncthreads();
            const float dd = decay_of<MODE>(xw);
            vd[tid] = __uint_as_float((__float_as_uint(dd) & lm) | (0x3f800000u & ~lm));  // (1 past N)
            vk[tid] = keep(lm, xk);
            va[tid] = keep(lm, xa);
            vb[tid] = keep(lm, xb);
            __syncthreads();
            float sa = 0.f;
#pragma unroll
            for (int j = 0; j < NP; j++) sa += st[j] * va[j];
#pragma unroll
            for (int j = 0; j < NP; j++) st[j] = st[j] * vd[j] + (sa * vb[j] + vi * vk[j]);
            if (lane_ok) {
                wsa[(long)u * N + tid] = sa;
#pragma unroll
                for (int j = 0; j < NP; j++)
                    if (j < N) wst[(long)(u + 1) * NN + (long)tid * N + j] = st[j];
            }
        }
        // ---- adjoint, reverse over the segment ----
        for (int u = L - 1; u >= 0; u--) {
            const long o = ((long)(bb * Tn + t0 + u) * H + h) * N;
            {
                const float wv = io<T>::ld(w, o + tc), xr = io<T>::ld(r, o + tc), xk = io<T>::ld(k, o + tc);
                const float xa = io<T>::ld(a, o + tc), xb = io<T>::ld(b, o + tc), xy = io<T>::ld(dy, o + tc);
                const float xv = io<T>::ld(v, o + tc), xs = wsa[(long)u * N + tc];
                const float dd = decay_of<MODE>(wv), df = dw_factor<MODE>(wv, dd);
                __syncthreads();  // previous column phase done with the vectors / G^T
                vr[tid] = keep(lm, xr);
                vd[tid] = __uint_as_float((__float_as_uint(dd) & lm) | (0x3f800000u & ~lm));  // (1 past N)
                vf[tid] = keep(lm, df);
                vk[tid] = keep(lm, xk);
                va[tid] = keep(lm, xa);
                vb[tid] = keep(lm, xb);
                vdy[tid] = keep(lm, xy);
                vv[tid] = keep(lm, xv);
                vsa[tid] = keep(lm, xs);
            }
            __syncthreads();
            // row phase (lane = value row i): G += dy_i r^T; q_i; dv_i.
            const float dyi = vdy[tid];
            float q = 0.f, dvi = 0.f;
#pragma unroll
            for (int j = 0; j < NP; j++) {
                g[j] += dyi * vr[j];
                q += g[j] * vb[j];
                dvi += g[j] * vk[j];
            }
            if (lane_ok) io<T>::st(dv, o + tid, dvi);
            vq[tid] = q;
#pragma unroll
            for (int j = 0; j < NP; j++) Gs[tid * NP + ((tid + j) & (NP - 1))] = g[j];
            __syncthreads();
            // column phase (lane = key column j).
            const int j = tid;
            const float* Sp = wst + (long)u * NN;
            const float* Sn = Sp + NN;
            float gr = 0.f, gw = 0.f, gk = 0.f, gb = 0.f, ga = 0.f;
            if (lane_ok) {
                // 16 rows' state loads in flight at a time (each a coalesced row of the
                // replayed state), not one dependent load after another
                for (int i0 = 0; i0 < N; i0 += 16) {
                    float spv[16], snv[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        const int i = i0 + u < N ? i0 + u : 0;  // (rows past N: read row 0, unused)
                        spv[u] = Sp[(long)i * N + j];
                        snv[u] = Sn[(long)i * N + j];
                    }
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        const int i = i0 + u;
                        if (i < N) {
                            const float gij = Gs[i * NP + ((i + j) & (NP - 1))];
                            gr += vdy[i] * snv[u];
                            gw += gij * spv[u];
                            gk += gij * vv[i];
                            gb += gij * vsa[i];
                            ga += vq[i] * spv[u];
                        }
                    }
                }
                io<T>::st(dr, o + j, gr);
                io<T>::st(dw, o + j, gw * vf[j]);
                io<T>::st(dk, o + j, gk);
                io<T>::st(db, o + j, gb);
                io<T>::st(da, o + j, ga);
            }
            // G <- G*d + q a^T  (row phase again, in registers)
#pragma unroll
            for (int jj = 0; jj < NP; jj++) g[jj] = g[jj] * vd[jj] + q * va[jj];
        }
    }
    if (lane_ok) {
#pragma unroll
        for (int j = 0; j < NP; j++)
            if (j < N) ds0[bh * NN + tid * ei + j * ej] = g[j];
    }
}

}  // namespace wkv7

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
#include "wkv7_launch.h"

namespace wkv7 {

template <typename T, int NP, int MODE>
static void seq_forward_t(const Fwd& p) {
    hipLaunchKernelGGL((seq_forward<T, NP, MODE>), dim3(p.B * p.H), dim3(NP), 0, p.stream, p.T, p.H, p.N,
                       (p.flags & FLAG_STATE_KV) ? 1 : 0, (const T*)p.r, (const T*)p.w, (const T*)p.k,
                       (const T*)p.v, (const T*)p.a, (const T*)p.b, p.s0, (T*)p.y, p.sT, p.ckpt);
}
template <typename T, int NP>
static void seq_forward_m(const Fwd& p) {
    if (p.flags & FLAG_DECAY_EXP) seq_forward_t<T, NP, MODE_EXP>(p);
    else seq_forward_t<T, NP, MODE_RWKV>(p);
}

void launch_seq_forward(const Fwd& p) {
    const bool bf = p.dtype == 0;
    if (p.N <= 64) {
        if (bf) seq_forward_m<bf16_t, 64>(p); else seq_forward_m<float, 64>(p);
    } else {
        if (bf) seq_forward_m<bf16_t, 128>(p); else seq_forward_m<float, 128>(p);
    }
}

size_t seq_backward_workspace(int B, int H, int N) {
    return (size_t)B * H * seq_ws_floats(N) * sizeof(float);
}

template <typename T, int NP, int MODE>
static void seq_backward_t(const Bwd& p) {
    const size_t lds = (size_t)(NP * NP + 10 * NP) * sizeof(float);
    if (lds > 65536)  // above the default dynamic-LDS cap; gfx950 has 160 KB per CU
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&seq_backward<T, NP, MODE>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((seq_backward<T, NP, MODE>), dim3(p.B * p.H), dim3(NP), lds, p.stream, p.T, p.H,
                       p.N, (p.flags & FLAG_STATE_KV) ? 1 : 0, (const T*)p.r, (const T*)p.w, (const T*)p.k,
                       (const T*)p.v, (const T*)p.a, (const T*)p.b, p.ckpt, (const T*)p.dy, p.dsT, (T*)p.dr,
                       (T*)p.dw, (T*)p.dk, (T*)p.dv, (T*)p.da, (T*)p.db, p.ds0, (float*)p.ws);
}
template <typename T, int NP>
static void seq_backward_m(const Bwd& p) {
    if (p.flags & FLAG_DECAY_EXP) seq_backward_t<T, NP, MODE_EXP>(p);
    else seq_backward_t<T, NP, MODE_RWKV>(p);
}

void launch_seq_backward(const Bwd& p) {
    const bool bf = p.dtype == 0;
    if (p.N <= 64) {
        if (bf) seq_backward_m<bf16_t, 64>(p); else seq_backward_m<float, 64>(p);
    } else {
        if (bf) seq_backward_m<bf16_t, 128>(p); else seq_backward_m<float, 128>(p);
    }
}

}  // namespace wkv7
