// The activation quantizer's arithmetic for four consecutive columns a lane, shared by the standalone quantizer
// (quant_act.hip) and the products that quantize their own activation row (gemv.hip), so both produce the same
// integers, scales and sums bit for bit.
//
// Restates crates/kf-quant/src/lib.rs:81-140 (quantize_activations):
//   kind 3 (Q8_0): per 32 columns d = amax/127, q = round-half-away(v / d) with 1/d taken from the unrounded d,
//                  d stored f16-rounded
//   kind 4 (Q8K):  per 256 columns, the first value of largest magnitude `mx`, iscale = -127/mx,
//                  q = min(round-half-even(iscale * v), 127), d = 1/iscale
// A wave of 64 lanes covers 256 columns, four consecutive columns a lane, so a Q8K block is one wave and a Q8_0 block
// eight lanes. Every lane of the wave calls it (the reductions are wave-wide).
#pragma once

#include "kf_device.h"

struct KfQa {
    uint32_t packed;  // the four int8 values, column c0 in the low byte
    float d;          // the scale of the lane's 32-column group (Q8K: of its 256 columns)
    int sum16, sum32;  // integer sums of the lane's 16- and 32-column groups
};

// v: the lane's columns c0..c0 + 3 (zeros where `in` is false, i.e. past the row's end)
__device__ __forceinline__ KfQa kf_qa_quant(const float (&v)[4], int c0, bool in, int kind) {
    // The reference rounds the f32 product v * id: with contraction, roundf's expansion (trunc, then p - trunc(p))
    // becomes fma(v, id, -trunc(p)), which sees the unrounded product and turns ties such as 58.4999999 -> 58.5 into 58.
#pragma clang fp contract(off)
    int qi[4];
    float d;
    if (kind == KF_ACT_Q8_0) {
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        // eight lanes make a block of 32: lanes xor 1, xor 2, then the mirrored half-row (lane i and 7 - i)
        amax = fmaxf(amax, kf_dpp<0xb1>(amax));
        amax = fmaxf(amax, kf_dpp<0x4e>(amax));
        amax = fmaxf(amax, kf_dpp<0x141>(amax));
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) qi[j] = (int)roundf(v[j] * id);
        d = kf_round_f16(dd);
    } else {
        // the largest magnitude over the wave, then the first column holding it and that column's signed value (the
        // reference's first-index maximum: NaN never compares, lanes past the row's end hold zeros)
        const float a4[4] = {fabsf(v[0]), fabsf(v[1]), fabsf(v[2]), fabsf(v[3])};
        const float a = kf_wave_max_all(fmaxf(fmaxf(a4[0], a4[1]), fmaxf(a4[2], a4[3])));
        int cand = 0x7fffffff;
#pragma unroll
        for (int j = 3; j >= 0; j--)
            if (in && a4[j] == a) cand = c0 + j;
        const int idx = kf_wave_min_all_i(cand);
        // the owner of column idx is lane (idx % 256) / 4 of the wave; every lane picks its own value at idx % 4
        const int jj = idx & 3;
        const float mine = jj == 0 ? v[0] : jj == 1 ? v[1] : jj == 2 ? v[2] : v[3];
        const float mx = kf_readlane_f(mine, (idx >> 2) & 63);
        if (a > 0.0f) {
            const float iscale = -127.0f / mx;
            d = 1.0f / iscale;
#pragma unroll
            for (int j = 0; j < 4; j++) qi[j] = min((int)rintf(iscale * v[j]), 127);
        } else {
            d = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) qi[j] = 0;
        }
    }
    // four lanes make a group of 16, eight a group of 32
    int sum16 = qi[0] + qi[1] + qi[2] + qi[3];
    sum16 += kf_dpp_i<0xb1>(sum16);
    sum16 += kf_dpp_i<0x4e>(sum16);
    const int sum32 = sum16 + kf_dpp_i<0x141>(sum16);
    KfQa r;
    r.packed = (uint32_t)(qi[0] & 0xff) | ((uint32_t)(qi[1] & 0xff) << 8) | ((uint32_t)(qi[2] & 0xff) << 16) | ((uint32_t)(qi[3] & 0xff) << 24);
    r.d = d;
    r.sum16 = sum16;
    r.sum32 = sum32;
    return r;
}
