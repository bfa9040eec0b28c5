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

// All eight scale/min pairs of a q4_K / q5_K header at once (scale_min_k4 for every group): byte g of sc[g >> 2] and
// mn[g >> 2] is group g's 6-bit scale and min. Pair j's two bytes, as kf_q4k_scales returns them, are
// kf_pair(sc, j) and kf_pair(mn, j).
__device__ __forceinline__ void kf_q4k_scales8(uint32_t hy, uint32_t hz, uint32_t hw, uint32_t (&sc)[2], uint32_t (&mn)[2]) {
    sc[0] = hy & 0x3f3f3f3fu;
    sc[1] = (hw & 0x0f0f0f0fu) | ((hy >> 2) & 0x30303030u);
    mn[0] = hz & 0x3f3f3f3fu;
    mn[1] = ((hw >> 4) & 0x0f0f0f0fu) | ((hz >> 2) & 0x30303030u);
}

__device__ __forceinline__ uint32_t kf_pair(const uint32_t (&v)[2], int j) { return (v[j >> 1] >> (16 * (j & 1))) & 0xffffu; }

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
    // The empty asm hides what the compiler knows of sc2 and m2 (below 2^14) so that the byte masks stay in the
    // block of the products: the products are matched to 24-bit multiplies only from ranges visible there, and the
    // scale words come from another block (a full-width quarter-rate multiply otherwise)
    asm("" : "+v"(sc2), "+v"(m2));
    isum = __mul24((int)(sc2 & 0xffu), dlo) + __mul24((int)((sc2 >> 8) & 0xffu), dhi);
    imin = __mul24((int)(m2 & 0xffu), bs0) + __mul24((int)((m2 >> 8) & 0xffu), bs1);
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

// q6_K lane unit: quarter j of a super-block, i.e. half h = j >> 1 and offsets l in [16 (j & 1), +16) of the half's
// four 32-element runs: the 16-element groups g = 8h + (j & 1) + 2k (k < 4). The lane's integer is
// sum_k sc_g (dot_g - 32 bsum_g), with dot_g of the unsigned 6-bit values (0..63) and the int8 activations; the four
// lanes of a super-block add up to the reference's dot - bias (crates/kf-quant/src/types/q6_k.rs:17-59), exactly.
struct KfQ6Lane {
    uint4 a, b, h;  // ql bytes of runs k = 0, 2 (a) and 1, 3 (b), and the qh bytes, at the lane's 16 offsets
    int sc[4];      // the int8 scales of the lane's groups
    float d;

    // blk: the super-block's 210 bytes (2-byte aligned), in global memory (LDS = false) or LDS (LDS = true)
    template <bool LDS = false>
    __device__ __forceinline__ void load(const uint8_t* blk, int j) {
        const int hh = j >> 1, o = 16 * (j & 1);
        if constexpr (LDS) {
            const kf_u32x4_a2 va = *reinterpret_cast<const kf_u32x4_a2*>(blk + 64 * hh + o);
            const kf_u32x4_a2 vb = *reinterpret_cast<const kf_u32x4_a2*>(blk + 64 * hh + 32 + o);
            const kf_u32x4_a2 vh = *reinterpret_cast<const kf_u32x4_a2*>(blk + 128 + 32 * hh + o);
            a = make_uint4(va.x, va.y, va.z, va.w);
            b = make_uint4(vb.x, vb.y, vb.z, vb.w);
            h = make_uint4(vh.x, vh.y, vh.z, vh.w);
        } else {
            a = kf_load_stream_u4_unaligned(blk + 64 * hh + o);
            b = kf_load_stream_u4_unaligned(blk + 64 * hh + 32 + o);
            h = kf_load_stream_u4_unaligned(blk + 128 + 32 * hh + o);
        }
        // the eight scale bytes of the half as four 16-bit words; the lane's scales are bytes (j & 1) + 2k
        const uint16_t* s2 = reinterpret_cast<const uint16_t*>(blk + 192 + 8 * hh);
#pragma unroll
        for (int k = 0; k < 4; k++) sc[k] = (int)(int8_t)(uint8_t)(s2[k] >> (8 * (j & 1)));
        d = kf_h2f(*reinterpret_cast<const uint16_t*>(blk + 208));
    }

    // x: the super-block's 256 int8 activations (16-byte aligned); s16: its 16 per-16 integer sums
    __device__ __forceinline__ int dot(const int8_t* x, const int32_t* s16, int j) const {
        const int hh = j >> 1, o = 16 * (j & 1);
        const uint32_t m4 = 0x0f0f0f0fu, m30 = 0x30303030u;
        const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w}, hv[4] = {h.x, h.y, h.z, h.w};
        int isum = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 xv = *reinterpret_cast<const uint4*>(x + 128 * hh + 32 * k + o);
            const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
            int dt = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                uint32_t wq;
                if (k == 0) wq = (av[e] & m4) | ((hv[e] << 4) & m30);
                else if (k == 1) wq = (bv[e] & m4) | ((hv[e] << 2) & m30);
                else if (k == 2) wq = ((av[e] >> 4) & m4) | (hv[e] & m30);
                else wq = ((bv[e] >> 4) & m4) | ((hv[e] >> 2) & m30);
                dt = kf_dot4(wq, xs[e], dt);
            }
            // |dot| <= 63 * 128 * 16 and |sc| <= 128: 24-bit multiplies are exact
            isum += __mul24(sc[k], dt - 32 * s16[8 * hh + (j & 1) + 2 * k]);
        }
        return isum;
    }
};

// q5_K lane unit: pair j of sub-blocks (2j, 2j+1), q4_K's unit with the fifth bit of element l of sub-block s taken
// from bit s of qh[l] (crates/kf-quant/src/types/q5_k.rs:7-60); the four lanes' isum and imin add up to the
// super-block's sumi and mins.
struct KfQ5Lane {
    uint4 hdr, qa, qb, ha, hb;

    // blk: the super-block's 176 bytes (16-byte aligned), in global memory (LDS = false) or LDS (LDS = true)
    template <bool LDS = false>
    __device__ __forceinline__ void load(const uint8_t* blk, int j) {
        if constexpr (LDS) {
            const uint4* p = reinterpret_cast<const uint4*>(blk);
            hdr = p[0];
            ha = p[1];
            hb = p[2];
            qa = p[3 + 2 * j];
            qb = p[4 + 2 * j];
        } else {
            hdr = kf_load_stream_u4(blk);
            ha = kf_load_stream_u4(blk + 16);
            hb = kf_load_stream_u4(blk + 32);
            qa = kf_load_stream_u4(blk + 48 + 32 * j);
            qb = kf_load_stream_u4(blk + 64 + 32 * j);
        }
    }

    // x: the super-block's 256 int8 activations; s32: its 8 per-32 integer sums
    __device__ __forceinline__ void dot(const int8_t* x, const int32_t* s32, int j, int& isum, int& imin) const {
        const uint32_t m4 = 0x0f0f0f0fu, m1 = 0x01010101u;
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const uint32_t hq[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
        const uint4* xl = reinterpret_cast<const uint4*>(x + 64 * j);
        const uint4 x0 = xl[0], x1 = xl[1], x2 = xl[2], x3 = xl[3];
        const uint32_t xlo[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t xhi[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            dlo = kf_dot4((q[e] & m4) | (((hq[e] >> (2 * j)) & m1) << 4), xlo[e], dlo);
            dhi = kf_dot4(((q[e] >> 4) & m4) | (((hq[e] >> (2 * j + 1)) & m1) << 4), xhi[e], dhi);
        }
        uint32_t sc2, m2;
        kf_q4k_scales(hdr.y, hdr.z, hdr.w, j, sc2, m2);
        isum = __mul24((int)(sc2 & 0xffu), dlo) + __mul24((int)(sc2 >> 8), dhi);
        imin = __mul24((int)(m2 & 0xffu), s32[2 * j]) + __mul24((int)(m2 >> 8), s32[2 * j + 1]);
    }
};
