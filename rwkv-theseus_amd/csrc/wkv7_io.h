// Global <-> LDS movement for the chunked WKV7 kernels (gfx950, wave64).
//
// Inputs reach LDS by LDS DMA (buffer_load_dwordx4 ... lds): the data goes
// from memory straight into a swizzled [16][64] plane without passing through
// registers, so nothing is held in VGPRs across the ticks between a prefetch
// and its use.  Outputs leave through raw-buffer stores whose range check drops
// rows past a chunk's end, so partial chunks need no per-lane branches.
//
// Every tensor addressed here is one [B,T,H,64] bf16 tensor of fewer than
// 2^31 bytes (the host checks this before choosing these kernels), so 32-bit
// buffer offsets cover it and OUT_OF_RANGE lies past all of them.
#pragma once

#include "wkv7_mfma.h"

namespace wkv7 {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t OUT_OF_RANGE = 0x80000000u;  // buffer offset past every tensor

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// vmcnt(0) / vmcnt(10): this wave's memory operations done / all but the last 10
__device__ __forceinline__ void vm_wait0() {
    __builtin_amdgcn_s_waitcnt(0x0f70);
    asm volatile("" ::: "memory");
}
__device__ __forceinline__ void vm_wait10() {
    __builtin_amdgcn_s_waitcnt(0x0f7a);
    asm volatile("" ::: "memory");
}
// vmcnt(N): all but this wave's last N memory operations done (gfx9 encoding: vmcnt bits
// 3:0 and 15:14, expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void vm_wait_n() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
    asm volatile("" ::: "memory");
}

// Raw-buffer descriptor for a tensor of `bytes` bytes (gfx9 word 3:
// 0x00020000).  Accesses at byte offsets >= bytes are dropped (stores) or read
// as zero (loads) by the hardware.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// The same descriptor as four scalar words, for the LDS DMA below.
__device__ __forceinline__ i32x4_t dma_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    return i32x4_t{(int)(uint32_t)p, (int)((p >> 32) & 0xffff), (int)bytes, 0x00020000};
}
// 8-byte store into a tensor of `bytes` bytes at byte offset `off` (OUT_OF_RANGE:
// dropped).  Every tick then issues the same stores, partial chunk or not.
__device__ __forceinline__ void store8(void* base, uint32_t bytes, uint32_t off, uint2 v) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{v.x, v.y}, make_rsrc(base, bytes), off, 0, 0);
}

// One LDS DMA of 16 bytes per lane (lane l fills lds + 16 l from the buffer at
// soff + voff).  It is issued from inline asm so that the compiler does not
// model it: the compiler would otherwise wait for it (vmcnt(0), which also
// waits for every pending global store of the wave) before each later LDS read
// anywhere in the kernel.  Its completion is awaited explicitly (vm_wait*)
// before its data is read.  M0 holds the LDS address; the compiler keeps
// nothing in M0 on gfx9 (LDS instructions there do not read it).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const uint16_t* lds, i32x4_t rs, uint32_t voff, uint32_t soff) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)lds;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(m0), "v"(voff), "s"(rs), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS DMA of 1 KB: lane l moves 16 bytes from the buffer at soff + voff to lds_off + 16 l
// (lds_off: byte address in LDS, made scalar for M0), issued like dma16 above.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_kb(uint32_t lds_off, i32x4_t rs, uint32_t voff, uint32_t soff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_off);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(m0), "v"(voff), "s"(rs), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop

// Rows past a chunk's valid steps are read from a clamped (valid) address and zeroed after
// the load by a lane mask, never loaded under a condition: a load inside a branch makes
// the compiler wait, before the branch joins, for every load the wave issued before it, so
// a run of such loads becomes one memory round trip after another (measured: the first
// 20 k cycles of the head-size-128 chunk-gradient kernel's 64 k).  A plain `ok ? x : 0` of
// a loaded x is no cure: the compiler turns such a select back into a branch around the
// load, so the mask is hidden from it and applied with an AND.
__device__ __forceinline__ uint32_t lane_mask(bool ok) {
    uint32_t m = ok ? 0xffffffffu : 0u;
    asm("" : "+v"(m));
    return m;
}
__device__ __forceinline__ float keep(uint32_t m, float x) { return __uint_as_float(__float_as_uint(x) & m); }
__device__ __forceinline__ float4 keep4(uint32_t m, const float4& x) {
    return make_float4(keep(m, x.x), keep(m, x.y), keep(m, x.z), keep(m, x.w));
}
__device__ __forceinline__ uint4 keepu4(uint32_t m, const uint4& x) {
    return make_uint4(x.x & m, x.y & m, x.z & m, x.w & m);
}

// four consecutive elements as float
__device__ __forceinline__ float4 ld4f(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4f(const bf16_t* p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
}

// Per-lane DMA offsets for a [16][64] SwDma plane: lane l fills physical
// 16-byte chunk l%8 of row 8m + l/8 with the logical chunk that belongs there
// (rstride = elements between consecutive tokens of one head).
__device__ __forceinline__ void dma_lane_offsets(uint32_t (&voff)[2], long rstride, int lane) {
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const int rho = 8 * m + (lane >> 3);
        voff[m] = (uint32_t)(rho * rstride * 2 + 16 * ((lane & 7) ^ (swz<SwDma>(rho) >> 1)));
    }
}
// LDS DMA of a full chunk: rows [t0, t0+16) of one head of a [B,T,H,64] bf16
// tensor (soff = byte offset of row t0) into a SwDma plane.
__device__ __forceinline__ void dma_plane(uint16_t* dst, i32x4_t rs, uint32_t soff, const uint32_t (&voff)[2]) {
#pragma unroll
    for (int m = 0; m < 2; m++) dma16(dst + 512 * m, rs, voff[m], soff);
}
// The same for a chunk of any length L: a partial chunk goes through registers
// (an ordinary load and LDS store) with zeros past the end.
__device__ __forceinline__ void stage_plane(uint16_t* dst, i32x4_t rs, const bf16_t* src, uint32_t soff,
                                            const uint32_t (&voff)[2], long rstride, int L, int lane) {
    if (L == CKPT) {
        dma_plane(dst, rs, soff, voff);
    } else {
        const int r16 = lane & 15, q = lane >> 4;
        const bf16_t* s0 = src + soff / 2;
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            uint4 x = make_uint4(0, 0, 0, 0);
            if (r16 < L) x = *reinterpret_cast<const uint4*>(s0 + r16 * rstride + 32 * hf + 8 * q);
            st16_sw<SwDma>(dst, r16, 32 * hf + 8 * q, x);
        }
    }
}

}  // namespace wkv7
