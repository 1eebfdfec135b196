// Shared device helpers for the WKV7 kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wkv7 {

// e^{-1/2}; the decay is exp(-DECAY_SCALE * sigmoid(w)) (kernels/wkv7_state.cu:27).
constexpr float DECAY_SCALE = 0.6065306597126334f;
// Saved-state interval (steps) shared by every forward/backward kernel.
constexpr int CKPT = 16;

// bfloat16 stored as its raw 16 bits; conversions use round-to-nearest-even,
// the rounding torch applies when it casts float32 to bfloat16.
struct bf16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_to_f32(uint16_t u) {
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
}
// gfx950 converts in hardware (v_cvt_pk_bf16_f32, round-to-nearest-even).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// two floats -> packed bf16 pair (element 0 in the low half), one instruction
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

template <typename T> struct io;
template <> struct io<float> {
    __device__ __forceinline__ static float ld(const float* p, long i) { return p[i]; }
    __device__ __forceinline__ static void st(float* p, long i, float x) { p[i] = x; }
};
template <> struct io<bf16_t> {
    __device__ __forceinline__ static float ld(const bf16_t* p, long i) { return bf16_to_f32(p[i].bits); }
    __device__ __forceinline__ static void st(bf16_t* p, long i, float x) { p[i].bits = f32_to_bf16(x); }
};

// v_rcp_f32 (1 ulp) instead of an IEEE division sequence
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// log of the per-key decay: log d = -e^{-1/2} * sigmoid(w).
__device__ __forceinline__ float log_decay(float w) { return -DECAY_SCALE * sigmoidf_(w); }

// Decay modes (THESEUS_WKV7_DECAY_EXP of theseus_wkv7.h).  MODE_RWKV: the reference's
// d = exp(-e^{-1/2} sigmoid(w)) (kernels/wkv7_state.cu:27).  MODE_EXP: d = exp(w) with no
// clamp -- the GDN teacher's decay, w = g (convert_qwen2rwkv_lightning.py:383-384).
constexpr int MODE_RWKV = 0, MODE_EXP = 1;
template <int MODE> __device__ __forceinline__ float decay_of(float w) {
    if constexpr (MODE == MODE_EXP) return __expf(w);
    else return __expf(log_decay(w));
}
// d * d(log d)/dw: the factor that turns sum_i G_ij S_{t-1,ij} into dw_j (cu:69)
template <int MODE> __device__ __forceinline__ float dw_factor(float w, float d) {
    if constexpr (MODE == MODE_EXP) return d;
    else {
        const float s = sigmoidf_(w);
        return d * (-DECAY_SCALE) * s * (1.f - s);
    }
}

__host__ __device__ constexpr inline long ckpt_count(int T) { return (T + CKPT - 1) / CKPT + 1; }

// Sum over each 16-lane row of the wave, left in every lane of the row: DPP
// exchanges (quad_perm 1,0,3,2 and 2,3,0,1, then row_half_mirror and row_mirror),
// so the data stays in the VALU (no LDS permute).  Fixed order: deterministic.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp_move<0xb1>(x);
    x += dpp_move<0x4e>(x);
    x += dpp_move<0x141>(x);
    x += dpp_move<0x140>(x);
    return x;
}

}  // namespace wkv7
