// Device helpers shared by the gfx950 kernels of kf-hip: f16 conversion, the 4-way int8 dot, wave reductions and
// the block layouts of the GGUF types the path consumes unchanged.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kf_layout.h"

#define KF_WAVE 64

// IEEE binary16 bits to f32, exact (v_cvt_f32_f16)
__device__ __forceinline__ float kf_h2f(uint32_t bits) {
    _Float16 h;
    uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// f32 rounded to the nearest binary16 value (ties to even) and widened back, as half::f16::from_f32(v).to_f32()
__device__ __forceinline__ float kf_round_f16(float v) { return (float)(_Float16)v; }

// Four signed int8 lanes of a and b multiplied and added into c (v_dot4_i32_i8)
__device__ __forceinline__ int kf_dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Sum over the 64 lanes of a wave; every lane receives the total (LDS permutes, for code off the hot path)
__device__ __forceinline__ float kf_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, KF_WAVE);
    return v;
}

// DPP lane move of a float (v_mov_b32_dpp), all rows and banks enabled
template <int CTRL>
__device__ __forceinline__ float kf_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

template <int CTRL>
__device__ __forceinline__ int kf_dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}

// Lane `lane`'s value of a float, as a wave-uniform value (v_readlane_b32)
__device__ __forceinline__ float kf_readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Lane i's value combined with lane i ^ 16 / i ^ 32 (gfx950 v_permlane16_swap / v_permlane32_swap: the two results
// hold each lane's own row or half and the partner's, in some order, so a commutative op of the pair is the same
// on every lane)
template <typename Op>
__device__ __forceinline__ uint32_t kf_xor16(uint32_t v, Op op) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return op(r[0], r[1]);
}
template <typename Op>
__device__ __forceinline__ uint32_t kf_xor32(uint32_t v, Op op) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return op(r[0], r[1]);
}

// Maximum of a float over the 64 lanes, on every lane: DPP within each row of 16, then the permlane swaps (VALU
// only, no LDS traffic)
__device__ __forceinline__ float kf_wave_max_all(float v) {
    v = fmaxf(v, kf_dpp<0xb1>(v));   // xor 1
    v = fmaxf(v, kf_dpp<0x4e>(v));   // xor 2
    v = fmaxf(v, kf_dpp<0x141>(v));  // half-row mirror: lane i and 7 - i
    v = fmaxf(v, kf_dpp<0x140>(v));  // row mirror: lane i and 15 - i
    auto fmax_u = [](uint32_t x, uint32_t y) {
        return __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, x), __builtin_bit_cast(float, y)));
    };
    uint32_t u = kf_xor16(__builtin_bit_cast(uint32_t, v), fmax_u);
    u = kf_xor32(u, fmax_u);
    return __builtin_bit_cast(float, u);
}

// Minimum of an int over the 64 lanes, on every lane
__device__ __forceinline__ int kf_wave_min_all_i(int v) {
    v = min(v, kf_dpp_i<0xb1>(v));
    v = min(v, kf_dpp_i<0x4e>(v));
    v = min(v, kf_dpp_i<0x141>(v));
    v = min(v, kf_dpp_i<0x140>(v));
    auto min_u = [](uint32_t x, uint32_t y) { return (uint32_t)min((int)x, (int)y); };
    uint32_t u = kf_xor16((uint32_t)v, min_u);
    u = kf_xor32(u, min_u);
    return (int)u;
}

// Sum over the 64 lanes of a wave through DPP within each row of 16 lanes and four lane reads across the rows; the
// result is uniform (held in a scalar register). Full-rate VALU work instead of LDS permutes.
__device__ __forceinline__ float kf_wave_sum_dpp(float v) {
    v += kf_dpp<0xb1>(v);   // quad_perm [1,0,3,2]
    v += kf_dpp<0x4e>(v);   // quad_perm [2,3,0,1]
    v += kf_dpp<0x124>(v);  // row_ror:4
    v += kf_dpp<0x128>(v);  // row_ror:8
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ int kf_wave_isum(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, KF_WAVE);
    return v;
}

// Byte window helper: bytes [s, s+4) of the 8-byte little-endian pair (hi:lo), s in 0..3 (v_alignbyte_b32)
__device__ __forceinline__ uint32_t kf_alignbyte(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}

typedef uint32_t kf_u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load of streamed data read once (non-temporal hint), p 16-byte aligned
__device__ __forceinline__ uint4 kf_load_stream_u4(const void* p) {
    const kf_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const kf_u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte load of streamed data at a 2-byte aligned address. gfx9 HSA targets run in unaligned access mode, so this
// is one global_load_dwordx4 that the memory pipeline splits across cache lines as needed.
typedef uint32_t kf_u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
__device__ __forceinline__ uint4 kf_load_stream_u4_unaligned(const void* p) {
    const kf_u32x4_a2 v = __builtin_nontemporal_load(reinterpret_cast<const kf_u32x4_a2*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// s_waitcnt immediate waiting until at most N vector memory loads are outstanding (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima so they are not waited on)
#define KF_WAITCNT_VM(N) ((((N) & 15)) | (7 << 4) | (15 << 8) | ((((N) >> 4) & 3) << 14))

typedef __attribute__((address_space(3))) void kf_lds_void;
typedef const __attribute__((address_space(1))) void kf_gbl_void;

// global_load_lds_dwordx4 / _dword (gfx950): lane l of one instruction writes its 16 (4) bytes at the instruction's
// LDS base + 16 l (4 l). lds_base must be the same for every lane of the wave.
__device__ __forceinline__ void kf_dma16(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds((kf_gbl_void*)src, (kf_lds_void*)lds_base, 16, 0, 0);
}

__device__ __forceinline__ void kf_dma4(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds((kf_gbl_void*)src, (kf_lds_void*)lds_base, 4, 0, 0);
}

// Raw buffer resource over [base, base + bytes) (stride 0, 32-bit data format word as gfx9 raw buffers need it).
// Loads through it take a per-lane 32-bit byte offset in a VGPR plus a wave-uniform one in an SGPR, so a loop that
// advances all lanes by the same amount pays no vector address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kf_rsrc(const void* base, uint64_t bytes) {
    const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

// The same DMA issued through inline assembly, for kernels whose every wait on it is explicit. The compiler's own
// waits for DMA-written LDS are conservative where it cannot tell the buffers apart (a read of one buffer waits for
// the DMA into another, which serializes a prefetch ring); assembly it does not see gets none, so such a kernel waits
// with exact vmcnt counts (loads complete in issue order) before it reads a buffer. The descriptor is the raw buffer
// kf_rsrc builds: base, stride 0, num_records bytes (reads past it return zeros), word 3 0x00020000.
typedef int kf_arsrc_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ kf_arsrc_t kf_arsrc(const void* base, uint64_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return kf_arsrc_t{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), (int)n, 0x00020000};
}

__device__ __forceinline__ uint32_t kf_lds_addr(const void* p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// lane l writes the 16 (4) bytes at voff + soff of the buffer to lds + 16 l (4 l)
__device__ __forceinline__ void kf_adma16(kf_arsrc_t r, int voff, int soff, const void* lds) {
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "s"(kf_lds_addr(lds))
                 : "memory", "m0");
}

__device__ __forceinline__ void kf_adma4(kf_arsrc_t r, int voff, int soff, const void* lds) {
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "s"(kf_lds_addr(lds))
                 : "memory", "m0");
}

// buffer_load_dwordx4 / _dword ... lds: lane l writes its 16 (4) bytes read at voff + soff to lds_base + 16 l (4 l).
__device__ __forceinline__ void kf_bdma16(__amdgpu_buffer_rsrc_t r, int voff, int soff, void* lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (kf_lds_void*)lds_base, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ void kf_bdma4(__amdgpu_buffer_rsrc_t r, int voff, int soff, void* lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (kf_lds_void*)lds_base, 4, voff, soff, 0, 0);
}
