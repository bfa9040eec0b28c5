// Per-lane integer dot products on native GGUF block bytes, shared by the GEMV kernels and the block-integer check.
//
// q4_K lane unit: one pair j of sub-blocks (2j, 2j+1) of one super-block, 32 bytes of nibbles (64 weights), against
// 64 int8 activations. It yields the lane's share of the super-block integers of the reference's dot_i8
// (crates/kf-quant/src/types/q4_k.rs:10-58): isum = sc_2j * dot_2j + sc_2j+1 * dot_2j+1 and
// imin = m_2j * bsum_2j + m_2j+1 * bsum_2j+1. Summing the four lanes of a super-block gives exactly the reference's
// sumi and mins.
//
// q8_0 lane unit: one 34-byte block (only 2-byte aligned: its f16 scale, then 32 int8 weights read as two unaligned
// 16-byte loads), yielding the int32 sum of q_w * q_x (crates/kf-quant/src/types/q8_0.rs:10-29).
#pragma once
#include "kf_device.h"

// The four scale/min pairs of sub-blocks (2j, 2j+1) of a q4_K header (scale_min_k4, crates/kf-quant/src/types/mod.rs:86-94).
// hy, hz, hw are the header's scale bytes 0-3, 4-7 and 8-11. Both results come as two bytes: low byte sub-block 2j,
// next byte 2j+1.
__device__ __forceinline__ void kf_q4k_scales(uint32_t hy, uint32_t hz, uint32_t hw, int j, uint32_t& sc2, uint32_t& m2) {
    const uint32_t sh = (uint32_t)(j & 1) * 16u;
    const uint32_t pa = (hy >> sh) & 0xffffu;  // bytes 2(j&1), 2(j&1)+1 of scales[0..3]
    const uint32_t pb = (hz >> sh) & 0xffffu;  // of scales[4..7]
    const uint32_t pw = (hw >> sh) & 0xffffu;  // of scales[8..11]
    if (j < 2) {
        sc2 = pa & 0x3f3fu;
        m2 = pb & 0x3f3fu;
    } else {
        sc2 = (pw & 0x0f0fu) | ((pa >> 2) & 0x3030u);
        m2 = ((pw >> 4) & 0x0f0fu) | ((pb >> 2) & 0x3030u);
    }
}

// Integer dot of sub-block pair j: qa = nibble bytes 32j..32j+15, qb = 32j+16..32j+31; x0..x3 the 64 activation bytes
// 64j..64j+63 of the super-block as four 16-byte pieces.
__device__ __forceinline__ void kf_q4k_pair_dots(const uint4 qa, const uint4 qb, const uint4 x0, const uint4 x1, const uint4 x2,
                                                 const uint4 x3, int& dlo, int& dhi) {
    const uint32_t m4 = 0x0f0f0f0fu;
    int lo = 0, hi = 0;
    lo = kf_dot4(qa.x & m4, x0.x, lo);
    lo = kf_dot4(qa.y & m4, x0.y, lo);
    lo = kf_dot4(qa.z & m4, x0.z, lo);
    lo = kf_dot4(qa.w & m4, x0.w, lo);
    lo = kf_dot4(qb.x & m4, x1.x, lo);
    lo = kf_dot4(qb.y & m4, x1.y, lo);
    lo = kf_dot4(qb.z & m4, x1.z, lo);
    lo = kf_dot4(qb.w & m4, x1.w, lo);
    hi = kf_dot4((qa.x >> 4) & m4, x2.x, hi);
    hi = kf_dot4((qa.y >> 4) & m4, x2.y, hi);
    hi = kf_dot4((qa.z >> 4) & m4, x2.z, hi);
    hi = kf_dot4((qa.w >> 4) & m4, x2.w, hi);
    hi = kf_dot4((qb.x >> 4) & m4, x3.x, hi);
    hi = kf_dot4((qb.y >> 4) & m4, x3.y, hi);
    hi = kf_dot4((qb.z >> 4) & m4, x3.z, hi);
    hi = kf_dot4((qb.w >> 4) & m4, x3.w, hi);
    dlo = lo;
    dhi = hi;
}

// One q4_K lane unit: integer share of the super-block. bs0, bs1: integer sums of the activation sub-blocks 2j, 2j+1.
__device__ __forceinline__ void kf_q4k_lane(const uint4 hdr, const uint4 qa, const uint4 qb, int j, const uint4 x0, const uint4 x1,
                                            const uint4 x2, const uint4 x3, int bs0, int bs1, int& isum, int& imin) {
    uint32_t sc2, m2;
    kf_q4k_scales(hdr.y, hdr.z, hdr.w, j, sc2, m2);
    int dlo, dhi;
    kf_q4k_pair_dots(qa, qb, x0, x1, x2, x3, dlo, dhi);
    // 24-bit multiplies are exact here: scales and mins are 6-bit, |dot| <= 15*127*32 and |bsum| <= 128*32
    isum = __mul24((int)(sc2 & 0xffu), dlo) + __mul24((int)(sc2 >> 8), dhi);
    imin = __mul24((int)(m2 & 0xffu), bs0) + __mul24((int)(m2 >> 8), bs1);
}

__device__ __forceinline__ int kf_q8_0_dot(const uint32_t* wq, const uint4 x0, const uint4 x1) {
    int s = 0;
    s = kf_dot4(wq[0], x0.x, s);
    s = kf_dot4(wq[1], x0.y, s);
    s = kf_dot4(wq[2], x0.z, s);
    s = kf_dot4(wq[3], x0.w, s);
    s = kf_dot4(wq[4], x1.x, s);
    s = kf_dot4(wq[5], x1.y, s);
    s = kf_dot4(wq[6], x1.z, s);
    s = kf_dot4(wq[7], x1.w, s);
    return s;
}
