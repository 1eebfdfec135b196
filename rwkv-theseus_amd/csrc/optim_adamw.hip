// Fused optimizer step after backward (C ABI: include/theseus_optim.h): gradient
// scale, global L2-norm clip with a non-finite flag, and AdamW, over a list of
// float32 tensors -- the reference's train.py:202-208 (optimizer from
// theseus/stage.py:39-42) without its host synchronisations and extra passes.
//
// Work is cut into chunks of CHUNK elements, one workgroup each, numbered
// tensor after tensor.  Three launches on the caller's stream:
//   grad_sumsq:  chunk c's sum of squared gradients, in float64, -> ws[c]
//                (per-thread sums in a fixed order, then a fixed-shape
//                block reduction: the same partials on every run);
//   norm_finish: one workgroup sums ws[0..nchunks) in a fixed order, forms
//                norm = |grad_scale| sqrt(sum), the clip factor and the flag;
//   adamw:       every element's update with g = grad * (grad_scale * clip),
//                reading the factor from device memory.
// HBM per parameter: the gradient twice (4 + 4 B), param / moments read and
// written (24 B): 32 B; the update alone needs 28 B.
//
// The tensor list travels in kernel arguments (32 tensors per launch, under
// the 4 KB argument limit), so nothing is copied to the device per step and
// the sequence can be captured into a graph.
#include "../../include/theseus_optim.h"
#include "../../include/theseus_wkv7.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace optim {

constexpr int CHUNK = THESEUS_ADAMW_CHUNK;
constexpr int THREADS = 256;
constexpr int BATCH = 32;  // tensors per launch

// Streaming loads and stores marked non-temporal: every byte is touched once per pass
// (measured on MI355X at 112 M parameters: update 0.619 -> 0.593 ms, norm pass 98 -> 67 us).
typedef float vf4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt(const float4* p) {
    const vf4 t = __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void st_nt(float4* p, float4 v) {
    const vf4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<vf4*>(p));
}

struct TensorArg {
    float* p;
    const float* g;
    float* m;
    float* v;
    long long n;
    float lr, wd, step_size, bc2_sqrt;
};
struct Batch {
    int count;               // tensors in this launch
    int chunk_base;          // global index of this launch's first chunk
    int chunk0[BATCH + 1];   // first chunk of tensor i within the launch (prefix)
    TensorArg t[BATCH];
};
static_assert(sizeof(Batch) < 4096, "kernel arguments");

static long long chunks_of(long long n) { return (n + CHUNK - 1) / CHUNK; }

// the tensor of this workgroup's chunk, and the chunk's first element and length
struct Where {
    int i;
    long long start;
    int len;
};
__device__ __forceinline__ Where locate(const Batch& bt) {
    const int b = blockIdx.x;
    int i = 0;
    while (i + 1 < bt.count && bt.chunk0[i + 1] <= b) i++;
    const long long start = (long long)(b - bt.chunk0[i]) * CHUNK;
    const long long rem = bt.t[i].n - start;
    return Where{i, start, (int)(rem < CHUNK ? rem : CHUNK)};
}

__device__ __forceinline__ bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// sum over the workgroup in a fixed order: xor-butterfly within each wave, then waves 0..3
__device__ __forceinline__ double block_sum(double x, double* red) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = x;
    __syncthreads();
    double s = 0.0;
    if (threadIdx.x == 0)
        for (int k = 0; k < (int)(blockDim.x >> 6); k++) s += red[k];
    return s;  // valid in thread 0
}

__global__ __launch_bounds__(THREADS) void grad_sumsq(Batch bt, double* __restrict__ partial) {
    __shared__ double red[THREADS / 64];
    const Where w = locate(bt);
    const float* g = bt.t[w.i].g + w.start;
    double acc = 0.0;
    int e0 = 0;
    if (aligned16(g)) {
        const int nv = w.len >> 2;
        const float4* g4 = reinterpret_cast<const float4*>(g);
#pragma unroll 4
        for (int q = threadIdx.x; q < nv; q += THREADS) {
            const float4 x = ld_nt(g4 + q);
            acc += (double)x.x * x.x + (double)x.y * x.y + (double)x.z * x.z + (double)x.w * x.w;
        }
        e0 = nv * 4;
    }
    for (int e = e0 + threadIdx.x; e < w.len; e += THREADS) acc += (double)g[e] * g[e];
    const double s = block_sum(acc, red);
    if (threadIdx.x == 0) partial[bt.chunk_base + blockIdx.x] = s;
}

__global__ __launch_bounds__(1024) void norm_finish(const double* __restrict__ partial, int nchunks,
                                                    float grad_scale, float max_norm,
                                                    float* __restrict__ result) {
    __shared__ double red[1024 / 64];
    double acc = 0.0;
    for (int c = threadIdx.x; c < nchunks; c += 1024) acc += partial[c];
    const double s = block_sum(acc, red);
    if (threadIdx.x == 0) {
        if (max_norm >= 0.0f) {  // clip_grad_norm_ (torch.nn.utils.clip_grad_norm_'s formula)
            const float norm = (float)(sqrt(s) * fabs((double)grad_scale));
            const float c = max_norm / (norm + 1e-6f);
            const float clip = isnan(c) ? c : fminf(c, 1.0f);  // torch.clamp(max=1) keeps a NaN
            result[0] = norm;
            result[1] = grad_scale * clip;
            result[2] = isfinite(norm) ? 0.0f : 1.0f;
        } else {  // no norm, no clipping
            result[0] = __builtin_nanf("");
            result[1] = grad_scale;
            result[2] = 0.0f;
        }
    }
}

struct Hyper {
    float beta1, beta2, eps;
    int skip_nonfinite;
};

__device__ __forceinline__ void adamw_one(float& p, float g, float& m, float& v, const TensorArg& t,
                                          const Hyper& h) {
    p *= 1.0f - t.lr * t.wd;
    m += (1.0f - h.beta1) * (g - m);
    v = v * h.beta2 + (1.0f - h.beta2) * g * g;
    const float denom = sqrtf(v) / t.bc2_sqrt + h.eps;
    p -= t.step_size * (m / denom);
}

__global__ __launch_bounds__(THREADS) void adamw(Batch bt, Hyper h, const float* __restrict__ result) {
    if (h.skip_nonfinite && result[2] != 0.0f) return;
    const float mult = result[1];
    const Where w = locate(bt);
    const TensorArg& t = bt.t[w.i];
    float* p = t.p + w.start;
    const float* g = t.g + w.start;
    float* m = t.m + w.start;
    float* v = t.v + w.start;
    int e0 = 0;
    if (aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v)) {
        const int nv = w.len >> 2;
        float4* p4 = reinterpret_cast<float4*>(p);
        const float4* g4 = reinterpret_cast<const float4*>(g);
        float4* m4 = reinterpret_cast<float4*>(m);
        float4* v4 = reinterpret_cast<float4*>(v);
#pragma unroll 4
        for (int q = threadIdx.x; q < nv; q += THREADS) {
            float4 pp = ld_nt(p4 + q), mm = ld_nt(m4 + q), vv = ld_nt(v4 + q);
            const float4 gg = ld_nt(g4 + q);
            adamw_one(pp.x, gg.x * mult, mm.x, vv.x, t, h);
            adamw_one(pp.y, gg.y * mult, mm.y, vv.y, t, h);
            adamw_one(pp.z, gg.z * mult, mm.z, vv.z, t, h);
            adamw_one(pp.w, gg.w * mult, mm.w, vv.w, t, h);
            st_nt(p4 + q, pp), st_nt(m4 + q, mm), st_nt(v4 + q, vv);
        }
        e0 = nv * 4;
    }
    for (int e = e0 + threadIdx.x; e < w.len; e += THREADS) {
        float pp = p[e], mm = m[e], vv = v[e];
        adamw_one(pp, g[e] * mult, mm, vv, t, h);
        p[e] = pp, m[e] = mm, v[e] = vv;
    }
}

// Fill `bt` with tensors [*next, ...) up to BATCH of them and 2^31-1 chunks; skips empty ones.
static bool next_batch(const theseus_adamw_tensor* ts, int nt, int& next, long long& chunk_base, Batch& bt) {
    bt.count = 0;
    bt.chunk_base = (int)chunk_base;
    long long c = 0;
    while (next < nt && bt.count < BATCH) {
        const theseus_adamw_tensor& s = ts[next];
        const long long k = chunks_of(s.numel);
        if (k == 0) {
            next++;
            continue;
        }
        if (c + k > 0x7fffffffLL) break;
        bt.chunk0[bt.count] = (int)c;
        bt.t[bt.count] = TensorArg{s.param, s.grad, s.exp_avg, s.exp_avg_sq, s.numel, s.lr, s.weight_decay,
                                   s.step_size, s.bias_correction2_sqrt};
        bt.count++;
        c += k;
        next++;
    }
    bt.chunk0[bt.count] = (int)c;
    chunk_base += c;
    return bt.count > 0;
}

}  // namespace optim

extern "C" {

size_t theseus_adamw_workspace_size(const theseus_adamw_tensor* tensors, int ntensors) {
    if (!tensors || ntensors < 0) return 0;
    long long c = 0;
    for (int i = 0; i < ntensors; i++)
        if (tensors[i].numel > 0) c += optim::chunks_of(tensors[i].numel);
    return (size_t)c * sizeof(double);
}

int theseus_adamw_step(const theseus_adamw_tensor* tensors, int ntensors, float grad_scale, float max_norm,
                       float beta1, float beta2, float eps, int skip_nonfinite, float* result, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
    if (ntensors < 0 || (ntensors > 0 && !tensors)) return THESEUS_WKV7_ERR_SHAPE;
    if (!result) return THESEUS_WKV7_ERR_NULL;
    long long nchunks = 0;
    for (int i = 0; i < ntensors; i++) {
        const theseus_adamw_tensor& s = tensors[i];
        if (s.numel < 0) return THESEUS_WKV7_ERR_SHAPE;
        if (s.numel > 0 && (!s.param || !s.grad || !s.exp_avg || !s.exp_avg_sq)) return THESEUS_WKV7_ERR_NULL;
        nchunks += optim::chunks_of(s.numel);
    }
    if (nchunks > 0x7fffffffLL) return THESEUS_WKV7_ERR_SHAPE;
    const bool norm = max_norm >= 0.0f;
    if (norm && nchunks && (!workspace || workspace_bytes < (size_t)nchunks * sizeof(double)))
        return THESEUS_WKV7_ERR_WORKSPACE;
    double* partial = static_cast<double*>(workspace);
    optim::Batch bt;
    int next = 0;
    long long base = 0;
    while (norm && optim::next_batch(tensors, ntensors, next, base, bt))
        hipLaunchKernelGGL(optim::grad_sumsq, dim3(bt.chunk0[bt.count]), dim3(optim::THREADS), 0, stream, bt,
                           partial);
    hipLaunchKernelGGL(optim::norm_finish, dim3(1), dim3(1024), 0, stream, partial, norm ? (int)nchunks : 0,
                       grad_scale, max_norm, result);
    const optim::Hyper h{beta1, beta2, eps, skip_nonfinite};
    next = 0;
    base = 0;
    while (optim::next_batch(tensors, ntensors, next, base, bt))
        hipLaunchKernelGGL(optim::adamw, dim3(bt.chunk0[bt.count]), dim3(optim::THREADS), 0, stream, bt, h,
                           result);
    return hipGetLastError() == hipSuccess ? THESEUS_WKV7_OK : THESEUS_WKV7_ERR_LAUNCH;
}

}  // extern "C"
