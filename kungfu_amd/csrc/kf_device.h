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

// Sum over the 64 lanes of a wave; every lane receives the total
__device__ __forceinline__ float kf_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, KF_WAVE);
    return v;
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
