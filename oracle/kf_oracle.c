/*
 * kf_oracle.c — CPU restatement of kungfu's quantized linear-layer arithmetic (the parity oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the product never links or loads this file's library; tests/, the smoke check and the
 * benchmark's CPU-baseline leg use it as the checker. Built with -ffp-contract=off so every float operation rounds
 * where the Rust source rounds (Rust never contracts a*b+c into an fma on its own).
 *
 * Third-party arithmetic restated here: f16 conversion of the `half` crate 2.7.1 (IEEE binary16, round to nearest
 * even, subnormals kept, overflow to infinity). rayon only schedules, it never changes a value, because every output
 * is computed by one closure.
 */
#include "kf_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- f16 (half 2.7.1, called at
 * crates/kf-quant/src/types/mod.rs:73-75 and crates/kf-quant/src/lib.rs:109) */

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

float kfo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return bits_f32(f32_bits(v) | sign);
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

uint16_t kfo_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        /* infinity, or NaN kept quiet with the top payload bits */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
    }
    if (ax < 0x38800000u) {
        /* below the smallest normal f16 (2^-14): a subnormal multiple of 2^-24, rounded to even. The scaling by 2^24
         * is exact in double and rint rounds half to even in the default rounding mode. */
        double v = (double)bits_f32(ax) * 16777216.0;
        return sign | (uint16_t)rint(v);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    if (e >= 31) return sign | 0x7c00u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* a carry into the exponent is the right result */
    return sign | (uint16_t)h;
}

static float f16_at(const uint8_t* p) { return kfo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ---------------------------------------------------------------- layouts
 * q8_0 (8, 32, 34): crates/kf-quant/src/types/q8_0.rs:4; q4_K (12, 256, 144): types/q4_k.rs:4;
 * q5_K (13, 256, 176): types/q5_k.rs:4; q6_K (14, 256, 210): types/q6_k.rs:4;
 * q8_K (15, 256, 292): types/q8_k.rs:4; row_bytes: crates/kf-quant/src/lib.rs:17-20 */

int kfo_type_info(uint32_t ty, int* block, int* size) {
    switch (ty) {
        case KFO_TYPE_Q8_0: *block = 32; *size = 34; return 0;
        case KFO_TYPE_Q4_K: *block = 256; *size = 144; return 0;
        case KFO_TYPE_Q5_K: *block = 256; *size = 176; return 0;
        case KFO_TYPE_Q6_K: *block = 256; *size = 210; return 0;
        case KFO_TYPE_Q8_K: *block = 256; *size = 292; return 0;
        default: return -1;
    }
}

/* act_kind: crates/kf-quant/src/lib.rs:154-163 (q8_0 -> Q8_0, the K types -> Q8K) */
int kfo_act_kind(uint32_t ty) {
    switch (ty) {
        case KFO_TYPE_Q8_0: return KFO_ACT_Q8_0;
        case KFO_TYPE_Q4_K:
        case KFO_TYPE_Q5_K:
        case KFO_TYPE_Q6_K:
        case KFO_TYPE_Q8_K: return KFO_ACT_Q8K;
        default: return -1;
    }
}

/* Rust `f32 as i8`: saturating, NaN to zero */
static int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* Rust `f32 as i32`: saturating, NaN to zero */
static int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)v;
}

/* nearest_int: crates/kf-quant/src/lib.rs:166-169, round half to even then `as i32` */
static int32_t nearest_int(float v) { return sat_i32(rintf(v)); }

/* scale_min_k4: crates/kf-quant/src/types/mod.rs:86-94 */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ---------------------------------------------------------------- q8_0::quantize_row
 * crates/kf-quant/src/types/q8_0.rs:33-42 */
void kfo_q8_0_quantize_row(const float* x, int n, uint8_t* dst) {
    for (int b = 0; b < n / 32; b++) {
        const float* blk = x + 32 * b;
        uint8_t* out = dst + 34 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(blk[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = kfo_f32_to_f16(d);
        out[0] = (uint8_t)(h & 0xff);
        out[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) {
            int32_t v = sat_i32(rintf(blk[j] * id));
            if (v < -127) v = -127;
            if (v > 127) v = 127;
            out[2 + j] = (uint8_t)(int8_t)v;
        }
    }
}

/* quads: crates/kf-quant/src/types/q6_k.rs:7-15, the signed 6-bit quant k (0..3) at offset l of a 128-element half */
static int q6_quad(const uint8_t* ql, const uint8_t* qh, int l, int k) {
    switch (k) {
        case 0: return ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
        case 1: return ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
        case 2: return ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        default: return ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
    }
}

/* ---------------------------------------------------------------- dequant_row
 * q8_0: crates/kf-quant/src/types/q8_0.rs:49-57; q4_K: types/q4_k.rs:64-85; q8_K: types/q8_k.rs:11-19 */
int kfo_dequant_row(uint32_t ty, const uint8_t* src, int n, float* dst) {
    if (ty == KFO_TYPE_Q8_0) {
        for (int b = 0; b < n / 32; b++) {
            const uint8_t* blk = src + 34 * b;
            float d = f16_at(blk);
            for (int j = 0; j < 32; j++) dst[32 * b + j] = (float)(int8_t)blk[2 + j] * d;
        }
        return 0;
    }
    if (ty == KFO_TYPE_Q4_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 144 * b;
            float d = f16_at(blk), mn = f16_at(blk + 2);
            const uint8_t* scales = blk + 4;
            float* out = dst + 256 * b;
            for (int j = 0; j < 4; j++) {
                const uint8_t* q = blk + 16 + 32 * j;
                uint8_t sc, m;
                scale_min_k4(2 * j, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = mn * (float)m;
                scale_min_k4(2 * j + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = mn * (float)m;
                for (int l = 0; l < 32; l++) {
                    out[64 * j + l] = d1 * (float)(q[l] & 0xF) - m1;
                    out[64 * j + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
                }
            }
        }
        return 0;
    }
    if (ty == KFO_TYPE_Q5_K) {  /* types/q5_k.rs:67-93 */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 176 * b;
            float d = f16_at(blk), mn = f16_at(blk + 2);
            const uint8_t* scales = blk + 4;
            const uint8_t* qh = blk + 16;
            float* out = dst + 256 * b;
            for (int j = 0; j < 4; j++) {
                const uint8_t* ql = blk + 48 + 32 * j;
                uint8_t sc, m;
                scale_min_k4(2 * j, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = mn * (float)m;
                scale_min_k4(2 * j + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = mn * (float)m;
                for (int l = 0; l < 32; l++) {
                    int h1 = (qh[l] >> (2 * j)) & 1 ? 16 : 0, h2 = (qh[l] >> (2 * j + 1)) & 1 ? 16 : 0;
                    out[64 * j + l] = d1 * (float)((ql[l] & 0xF) + h1) - m1;
                    out[64 * j + 32 + l] = d2 * (float)((ql[l] >> 4) + h2) - m2;
                }
            }
        }
        return 0;
    }
    if (ty == KFO_TYPE_Q6_K) {  /* types/q6_k.rs:74-90 */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 210 * b;
            float d = f16_at(blk + 208);
            for (int h = 0; h < 2; h++) {
                const uint8_t* ql = blk + 64 * h;
                const uint8_t* qh = blk + 128 + 32 * h;
                const uint8_t* sc = blk + 192 + 8 * h;
                float* ys = dst + 256 * b + 128 * h;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    for (int k = 0; k < 4; k++) {
                        int q = q6_quad(ql, qh, l, k);
                        ys[l + 32 * k] = d * (float)(int8_t)sc[is + 2 * k] * (float)q;
                    }
                }
            }
        }
        return 0;
    }
    if (ty == KFO_TYPE_Q8_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 292 * b;
            uint32_t u = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) | ((uint32_t)blk[3] << 24);
            float d = bits_f32(u);
            for (int j = 0; j < 256; j++) dst[256 * b + j] = d * (float)(int8_t)blk[4 + j];
        }
        return 0;
    }
    return -1;
}

/* ---------------------------------------------------------------- dot_row (float path)
 * q8_0: crates/kf-quant/src/types/q8_0.rs:58-70; q4_K: types/q4_k.rs:86-110; q8_K: types/q8_k.rs:20-31 */
float kfo_dot_row(uint32_t ty, const uint8_t* src, const float* x, int n) {
    float acc = 0.0f;
    if (ty == KFO_TYPE_Q8_0) {
        for (int b = 0; b < n / 32; b++) {
            const uint8_t* blk = src + 34 * b;
            float d = f16_at(blk);
            float s = 0.0f;
            for (int j = 0; j < 32; j++) s += (float)(int8_t)blk[2 + j] * x[32 * b + j];
            acc += s * d;
        }
    } else if (ty == KFO_TYPE_Q4_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 144 * b;
            float d = f16_at(blk), mn = f16_at(blk + 2);
            const uint8_t* scales = blk + 4;
            const float* xs = x + 256 * b;
            for (int j = 0; j < 4; j++) {
                const uint8_t* q = blk + 16 + 32 * j;
                uint8_t sc1, m1, sc2, m2;
                scale_min_k4(2 * j, scales, &sc1, &m1);
                scale_min_k4(2 * j + 1, scales, &sc2, &m2);
                const float* x1 = xs + 64 * j;
                const float* x2 = x1 + 32;
                float qx1 = 0.0f, sx1 = 0.0f, qx2 = 0.0f, sx2 = 0.0f;
                for (int l = 0; l < 32; l++) {
                    qx1 += (float)(q[l] & 0xF) * x1[l];
                    sx1 += x1[l];
                    qx2 += (float)(q[l] >> 4) * x2[l];
                    sx2 += x2[l];
                }
                acc += d * (float)sc1 * qx1 - mn * (float)m1 * sx1;
                acc += d * (float)sc2 * qx2 - mn * (float)m2 * sx2;
            }
        }
    } else if (ty == KFO_TYPE_Q5_K) {  /* types/q5_k.rs:94-121 */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 176 * b;
            float d = f16_at(blk), mn = f16_at(blk + 2);
            const uint8_t* scales = blk + 4;
            const uint8_t* qh = blk + 16;
            const float* xs = x + 256 * b;
            for (int j = 0; j < 4; j++) {
                const uint8_t* ql = blk + 48 + 32 * j;
                uint8_t sc1, m1, sc2, m2;
                scale_min_k4(2 * j, scales, &sc1, &m1);
                scale_min_k4(2 * j + 1, scales, &sc2, &m2);
                const float* x1 = xs + 64 * j;
                const float* x2 = x1 + 32;
                float qx1 = 0.0f, sx1 = 0.0f, qx2 = 0.0f, sx2 = 0.0f;
                for (int l = 0; l < 32; l++) {
                    int h1 = ((qh[l] >> (2 * j)) & 1) << 4, h2 = ((qh[l] >> (2 * j + 1)) & 1) << 4;
                    qx1 += (float)((ql[l] & 0xF) | h1) * x1[l];
                    sx1 += x1[l];
                    qx2 += (float)((ql[l] >> 4) | h2) * x2[l];
                    sx2 += x2[l];
                }
                acc += d * (float)sc1 * qx1 - mn * (float)m1 * sx1;
                acc += d * (float)sc2 * qx2 - mn * (float)m2 * sx2;
            }
        }
    } else if (ty == KFO_TYPE_Q6_K) {  /* types/q6_k.rs:91-110 */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 210 * b;
            float d = f16_at(blk + 208);
            float sums[16] = {0};
            for (int h = 0; h < 2; h++) {
                const uint8_t* ql = blk + 64 * h;
                const uint8_t* qh = blk + 128 + 32 * h;
                const float* xn = x + 256 * b + 128 * h;
                for (int l = 0; l < 32; l++) {
                    int is = 8 * h + l / 16;
                    for (int k = 0; k < 4; k++) sums[is + 2 * k] += (float)q6_quad(ql, qh, l, k) * xn[l + 32 * k];
                }
            }
            for (int s = 0; s < 16; s++) acc += d * (float)(int8_t)blk[192 + s] * sums[s];
        }
    } else if (ty == KFO_TYPE_Q8_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 292 * b;
            uint32_t u = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) | ((uint32_t)blk[3] << 24);
            float d = bits_f32(u);
            float s = 0.0f;
            for (int j = 0; j < 256; j++) s += (float)(int8_t)blk[4 + j] * x[256 * b + j];
            acc += d * s;
        }
    }
    return acc;
}

/* ---------------------------------------------------------------- quantize_activations
 * crates/kf-quant/src/lib.rs:81-140 */
int kfo_quantize_activations(int kind, const float* x, int rows, int n, int8_t* q, float* d16, int32_t* sum16) {
    if (n % 16 != 0) return -1;
    int block;
    if (kind == KFO_ACT_Q8_0) block = 32;
    else if (kind == KFO_ACT_Q8K) block = 256;
    else return -1;
    if (n % block != 0) return -1;
    int n16 = n / 16;
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * n;
        int8_t* qr = q + (size_t)r * n;
        for (int bi = 0; bi < n / block; bi++) {
            const float* blk = xr + bi * block;
            int8_t* qb = qr + bi * block;
            float d;
            if (kind == KFO_ACT_Q8_0) {
                float amax = 0.0f;
                for (int j = 0; j < block; j++) amax = fmaxf(amax, fabsf(blk[j]));
                float dd = amax / 127.0f;
                float id = dd != 0.0f ? 1.0f / dd : 0.0f;
                for (int j = 0; j < block; j++) qb[j] = sat_i8(roundf(blk[j] * id));
                d = kfo_f16_to_f32(kfo_f32_to_f16(dd));
            } else {
                float amax = 0.0f, mx = 0.0f;
                for (int j = 0; j < block; j++) {
                    if (fabsf(blk[j]) > amax) {
                        amax = fabsf(blk[j]);
                        mx = blk[j];
                    }
                }
                if (amax == 0.0f) {
                    memset(qb, 0, (size_t)block);
                    d = 0.0f;
                } else {
                    float iscale = -127.0f / mx;
                    for (int j = 0; j < block; j++) {
                        int32_t v = nearest_int(iscale * blk[j]);
                        if (v > 127) v = 127;
                        qb[j] = (int8_t)v; /* `as i8` of an i32 keeps the low byte */
                    }
                    d = 1.0f / iscale;
                }
            }
            for (int g = 0; g < block / 16; g++) {
                int at = r * n16 + bi * (block / 16) + g;
                int32_t s = 0;
                for (int j = 0; j < 16; j++) s += qb[16 * g + j];
                d16[at] = d;
                sum16[at] = s;
            }
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- round_activations (int8 kinds)
 * crates/kf-quant/src/lib.rs:171-209, blocks taken with chunks() so a short last block is rounded on its own */
void kfo_round_activations(int kind, const float* x, int n, float* out) {
    if (kind == KFO_ACT_Q8_0) {
        for (int b0 = 0; b0 < n; b0 += 32) {
            int len = n - b0 < 32 ? n - b0 : 32;
            float amax = 0.0f;
            for (int j = 0; j < len; j++) amax = fmaxf(amax, fabsf(x[b0 + j]));
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            float dh = kfo_f16_to_f32(kfo_f32_to_f16(d));
            for (int j = 0; j < len; j++) out[b0 + j] = dh * roundf(x[b0 + j] * id);
        }
    } else if (kind == KFO_ACT_Q8K) {
        for (int b0 = 0; b0 < n; b0 += 256) {
            int len = n - b0 < 256 ? n - b0 : 256;
            float amax = 0.0f, mx = 0.0f;
            for (int j = 0; j < len; j++) {
                if (fabsf(x[b0 + j]) > amax) {
                    amax = fabsf(x[b0 + j]);
                    mx = x[b0 + j];
                }
            }
            if (amax == 0.0f) {
                for (int j = 0; j < len; j++) out[b0 + j] = 0.0f;
                continue;
            }
            float iscale = -127.0f / mx;
            float d = 1.0f / iscale;
            for (int j = 0; j < len; j++) {
                int32_t v = nearest_int(iscale * x[b0 + j]);
                if (v > 127) v = 127;
                out[b0 + j] = d * (float)v;
            }
        }
    } else {
        memcpy(out, x, sizeof(float) * (size_t)n);
    }
}

/* hsum_ps: crates/kf-quant/src/simd.rs:44-50, the 256-bit halves added, then movehl, then the last pair */
static float hsum8(const float* a) {
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

/* ---------------------------------------------------------------- dot_i8
 * q8_0 AVX2: crates/kf-quant/src/types/q8_0.rs:7-29; q4_K AVX2: types/q4_k.rs:7-58. Each int32 lane i of the AVX2
 * registers holds bytes 4i..4i+3 of a 32-byte run (maddubs then madd), and is scaled into its own f32 lane. */
static void dot_i8_q8_0_row(const uint8_t* src, int n, const int8_t* q, const float* d16, float* y) {
    float acc[8] = {0};
    for (int b = 0; b < n / 32; b++) {
        const uint8_t* blk = src + 34 * b;
        float dw = f16_at(blk);
        float s = dw * d16[b * 2];
        for (int i = 0; i < 8; i++) {
            int32_t dot = 0;
            for (int t = 0; t < 4; t++) dot += (int32_t)(int8_t)blk[2 + 4 * i + t] * (int32_t)q[32 * b + 4 * i + t];
            acc[i] = fmaf(s, (float)dot, acc[i]);
        }
    }
    *y = hsum8(acc);
}

static void dot_i8_q4_k_row(const uint8_t* src, int n, const int8_t* q, const float* d16, const int32_t* sum16, float* y) {
    float acc[8] = {0};
    for (int b = 0; b < n / 256; b++) {
        const uint8_t* blk = src + 144 * b;
        float d = f16_at(blk), dmin = f16_at(blk + 2);
        int32_t sc[8], mn[16];
        for (int s = 0; s < 8; s++) {
            uint8_t a, m;
            scale_min_k4(s, blk + 4, &a, &m);
            sc[s] = a;
            mn[2 * s] = m;
            mn[2 * s + 1] = m;
        }
        int32_t sumi[8] = {0};
        for (int j = 0; j < 4; j++) {
            const uint8_t* qs = blk + 16 + 32 * j;
            const int8_t* q0 = q + b * 256 + 64 * j;
            const int8_t* q1 = q0 + 32;
            for (int i = 0; i < 8; i++) {
                int32_t p0 = 0, p1 = 0;
                for (int t = 0; t < 4; t++) {
                    p0 += (int32_t)(qs[4 * i + t] & 0xF) * q0[4 * i + t];
                    p1 += (int32_t)(qs[4 * i + t] >> 4) * q1[4 * i + t];
                }
                sumi[i] += sc[2 * j] * p0 + sc[2 * j + 1] * p1;
            }
        }
        int at = b * 16;
        float dx = d16[at];
        float sd = d * dx, sm = dmin * dx;
        for (int i = 0; i < 8; i++) {
            int32_t mins = sum16[at + i] * mn[i] + sum16[at + 8 + i] * mn[8 + i];
            acc[i] = fmaf(sd, (float)sumi[i], acc[i]);
            acc[i] = fmaf(-sm, (float)mins, acc[i]);
        }
    }
    *y = hsum8(acc);
}

/* q5_K AVX2: crates/kf-quant/src/types/q5_k.rs:7-60. The fifth bit of a nibble comes from bit 2j (low nibbles) or
 * 2j + 1 (high nibbles) of qh[l]; otherwise q4_K's lanes. */
static void dot_i8_q5_k_row(const uint8_t* src, int n, const int8_t* q, const float* d16, const int32_t* sum16, float* y) {
    float acc[8] = {0};
    for (int b = 0; b < n / 256; b++) {
        const uint8_t* blk = src + 176 * b;
        float d = f16_at(blk), dmin = f16_at(blk + 2);
        int32_t sc[8], mn[16];
        for (int s = 0; s < 8; s++) {
            uint8_t a, m;
            scale_min_k4(s, blk + 4, &a, &m);
            sc[s] = a;
            mn[2 * s] = m;
            mn[2 * s + 1] = m;
        }
        const uint8_t* qh = blk + 16;
        int32_t sumi[8] = {0};
        for (int j = 0; j < 4; j++) {
            const uint8_t* qs = blk + 48 + 32 * j;
            const int8_t* q0 = q + b * 256 + 64 * j;
            const int8_t* q1 = q0 + 32;
            for (int i = 0; i < 8; i++) {
                int32_t p0 = 0, p1 = 0;
                for (int t = 0; t < 4; t++) {
                    const int e = 4 * i + t;
                    p0 += (int32_t)((qs[e] & 0xF) | (((qh[e] >> (2 * j)) & 1) << 4)) * q0[e];
                    p1 += (int32_t)((qs[e] >> 4) | (((qh[e] >> (2 * j + 1)) & 1) << 4)) * q1[e];
                }
                sumi[i] += sc[2 * j] * p0 + sc[2 * j + 1] * p1;
            }
        }
        int at = b * 16;
        float dx = d16[at];
        float sd = d * dx, sm = dmin * dx;
        for (int i = 0; i < 8; i++) {
            int32_t mins = sum16[at + i] * mn[i] + sum16[at + 8 + i] * mn[8 + i];
            acc[i] = fmaf(sd, (float)sumi[i], acc[i]);
            acc[i] = fmaf(-sm, (float)mins, acc[i]);
        }
    }
    *y = hsum8(acc);
}

/* q6_K AVX2: crates/kf-quant/src/types/q6_k.rs:17-59. The unsigned 6-bit values (0..63) against the int8
 * activations, lane i holding bytes 4i..4i+3 of each quad's 32-element run, lanes 0-3 scaled by sc[g] and 4-7 by
 * sc[g + 1] (g = 8h + 2k), minus the bias 32 sc * sum16 of groups i and 8 + i. */
static void dot_i8_q6_k_row(const uint8_t* src, int n, const int8_t* q, const float* d16, const int32_t* sum16, float* y) {
    float acc[8] = {0};
    for (int b = 0; b < n / 256; b++) {
        const uint8_t* blk = src + 210 * b;
        float d = f16_at(blk + 208);
        const int8_t* sc = (const int8_t*)(blk + 192);
        int32_t sumi[8] = {0};
        for (int h = 0; h < 2; h++) {
            const uint8_t* ql = blk + 64 * h;
            const uint8_t* qh = blk + 128 + 32 * h;
            for (int k = 0; k < 4; k++) {
                const int g = 8 * h + 2 * k;
                const int8_t* q8 = q + b * 256 + 16 * g;
                for (int i = 0; i < 8; i++) {
                    int32_t p = 0;
                    for (int t = 0; t < 4; t++) {
                        const int l = 4 * i + t;
                        p += (q6_quad(ql, qh, l, k) + 32) * q8[l];
                    }
                    sumi[i] += (i < 4 ? sc[g] : sc[g + 1]) * p;
                }
            }
        }
        int at = b * 16;
        float s = d * d16[at];
        for (int i = 0; i < 8; i++) {
            int32_t bias = sum16[at + i] * (sc[i] * 32) + sum16[at + 8 + i] * (sc[8 + i] * 32);
            acc[i] = fmaf(s, (float)(sumi[i] - bias), acc[i]);
        }
    }
    *y = hsum8(acc);
}

int kfo_dot_i8(uint32_t ty, const uint8_t* src, int n, const int8_t* q, const float* d16, const int32_t* sum16, int rows, float* y) {
    int n16 = n / 16;
    for (int r = 0; r < rows; r++) {
        const int8_t* qr = q + (size_t)r * n;
        const float* dr = d16 + (size_t)r * n16;
        const int32_t* sr = sum16 + (size_t)r * n16;
        if (ty == KFO_TYPE_Q8_0) dot_i8_q8_0_row(src, n, qr, dr, &y[r]);
        else if (ty == KFO_TYPE_Q4_K) dot_i8_q4_k_row(src, n, qr, dr, sr, &y[r]);
        else if (ty == KFO_TYPE_Q5_K) dot_i8_q5_k_row(src, n, qr, dr, sr, &y[r]);
        else if (ty == KFO_TYPE_Q6_K) dot_i8_q6_k_row(src, n, qr, dr, sr, &y[r]);
        else return -1;
    }
    return 0;
}

int kfo_block_ints(uint32_t ty, const uint8_t* src, int n, const int8_t* q, const int32_t* sum16, int32_t* ints) {
    if (ty == KFO_TYPE_Q8_0) {
        for (int b = 0; b < n / 32; b++) {
            int32_t s = 0;
            for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)src[34 * b + 2 + j] * q[32 * b + j];
            ints[b] = s;
        }
        return 0;
    }
    if (ty == KFO_TYPE_Q4_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 144 * b;
            int32_t sumi = 0, mins = 0;
            for (int s = 0; s < 8; s++) {
                uint8_t sc, m;
                scale_min_k4(s, blk + 4, &sc, &m);
                const uint8_t* qs = blk + 16 + 32 * (s / 2);
                int32_t dot = 0;
                for (int l = 0; l < 32; l++) {
                    int w = (s & 1) ? (qs[l] >> 4) : (qs[l] & 0xF);
                    dot += w * q[256 * b + 32 * s + l];
                }
                sumi += sc * dot;
                mins += m * (sum16[16 * b + 2 * s] + sum16[16 * b + 2 * s + 1]);
            }
            ints[2 * b] = sumi;
            ints[2 * b + 1] = mins;
        }
        return 0;
    }
    if (ty == KFO_TYPE_Q5_K) {  /* two per super-block, as q4_K: sum_s sc_s dot_s and sum_s m_s bsum_s */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 176 * b;
            const uint8_t* qh = blk + 16;
            int32_t sumi = 0, mins = 0;
            for (int s = 0; s < 8; s++) {
                uint8_t sc, m;
                scale_min_k4(s, blk + 4, &sc, &m);
                const uint8_t* qs = blk + 48 + 32 * (s / 2);
                int32_t dot = 0;
                for (int l = 0; l < 32; l++) {
                    int w = ((s & 1) ? (qs[l] >> 4) : (qs[l] & 0xF)) | (((qh[l] >> s) & 1) << 4);
                    dot += w * q[256 * b + 32 * s + l];
                }
                sumi += sc * dot;
                mins += m * (sum16[16 * b + 2 * s] + sum16[16 * b + 2 * s + 1]);
            }
            ints[2 * b] = sumi;
            ints[2 * b + 1] = mins;
        }
        return 0;
    }
    if (ty == KFO_TYPE_Q6_K) {  /* one per super-block: sum_g sc_g (dot_g of the unsigned values - 32 bsum_g) */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + 210 * b;
            const int8_t* sc = (const int8_t*)(blk + 192);
            int32_t tot = 0;
            for (int h = 0; h < 2; h++)
                for (int k = 0; k < 4; k++)
                    for (int half = 0; half < 2; half++) {
                        const int g = 8 * h + 2 * k + half;
                        int32_t dot = 0;
                        for (int l = 16 * half; l < 16 * half + 16; l++)
                            dot += (q6_quad(blk + 64 * h, blk + 128 + 32 * h, l, k) + 32) * q[256 * b + 128 * h + 32 * k + l];
                        tot += sc[g] * (dot - 32 * sum16[16 * b + g]);
                    }
            ints[b] = tot;
        }
        return 0;
    }
    return -1;
}

/* ---------------------------------------------------------------- matmul_slice (the CPU backend's product)
 * crates/kf-backend-cpu/src/ops.rs:304-346 */
int kfo_matmul_slice(uint32_t ty, const uint8_t* w, int n_in, int n_out, const float* x, int rows, const float* bias, float* y, int threads) {
    int block, size;
    if (kfo_type_info(ty, &block, &size) != 0 || n_in % block != 0 || rows < 0 || n_out < 0) return -1;
    int kind = kfo_act_kind(ty);
    size_t rb = (size_t)(n_in / block) * size;
    float* xr = (float*)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1) * n_in);
    if (!xr) return -2;
    for (int r = 0; r < rows; r++) kfo_round_activations(kind, x + (size_t)r * n_in, n_in, xr + (size_t)r * n_in);
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* tmp = (float*)malloc(sizeof(float) * (size_t)n_in);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int o = 0; o < n_out; o++) {
            const uint8_t* row = w + (size_t)o * rb;
            float b = bias ? bias[o] : 0.0f;
            if (rows <= 2) {
                for (int r = 0; r < rows; r++) y[(size_t)r * n_out + o] = kfo_dot_row(ty, row, xr + (size_t)r * n_in, n_in) + b;
            } else {
                kfo_dequant_row(ty, row, n_in, tmp);
                for (int r = 0; r < rows; r++) {
                    const float* xq = xr + (size_t)r * n_in;
                    float s = -0.0f; /* the neutral element of Rust's f32 Sum */
                    for (int k = 0; k < n_in; k++) s += xq[k] * tmp[k];
                    y[(size_t)r * n_out + o] = s + b;
                }
            }
        }
        free(tmp);
    }
    (void)threads;
    free(xr);
    return 0;
}

/* The integer products of the expert coprocessor (crates/kf-backend-cpu/src/experts.rs:93-124): one
 * quantize_activations of all rows, then Quant::dot_i8 of every weight row against them */
int kfo_matmul_i8(uint32_t ty, const uint8_t* w, int n_in, int n_out, const float* x, int rows, const float* bias, float* y, int threads) {
    int block, size;
    if (kfo_type_info(ty, &block, &size) != 0 || n_in % block != 0 || rows <= 0) return -1;
    int kind = kfo_act_kind(ty);
    size_t rb = (size_t)(n_in / block) * size;
    int8_t* q = (int8_t*)malloc((size_t)rows * n_in);
    float* d16 = (float*)malloc(sizeof(float) * (size_t)rows * (n_in / 16));
    int32_t* s16 = (int32_t*)malloc(sizeof(int32_t) * (size_t)rows * (n_in / 16));
    if (!q || !d16 || !s16) return -2;
    if (kfo_quantize_activations(kind, x, rows, n_in, q, d16, s16) != 0) {
        free(q); free(d16); free(s16);
        return -1;
    }
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* col = (float*)malloc(sizeof(float) * (size_t)rows);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int o = 0; o < n_out; o++) {
            kfo_dot_i8(ty, w + (size_t)o * rb, n_in, q, d16, s16, rows, col);
            float b = bias ? bias[o] : 0.0f;
            for (int r = 0; r < rows; r++) y[(size_t)r * n_out + o] = col[r] + b;
        }
        free(col);
    }
    (void)threads;
    free(q); free(d16); free(s16);
    return 0;
}

/* ops::silu: crates/kf-backend-cpu/src/ops.rs:6-8 */
float kfo_silu(float x) { return x / (1.0f + expf(-x)); }

/* ops::rms_norm: crates/kf-backend-cpu/src/ops.rs:222-239. The mean square sums f32 squares in f64 in column order,
 * divides by n in f64 and rounds to f32; inv = 1 / sqrt(ss + eps) in f32; each value is (v * inv) * w + b, w = 1 and
 * b = 0 where absent (both exact). w, b nullable. */
int kfo_rms_norm(const float* x, const float* w, const float* b, int rows, int n, float eps, float* out) {
    if (rows < 0 || n <= 0) return -1;
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * n;
        float* o = out + (size_t)r * n;
        double s = 0.0;
        for (int i = 0; i < n; i++) s += (double)(xr[i] * xr[i]);
        const float ss = (float)(s / (double)n);
        const float inv = 1.0f / sqrtf(ss + eps);
        for (int i = 0; i < n; i++) o[i] = xr[i] * inv * (w ? w[i] : 1.0f) + (b ? b[i] : 0.0f);
    }
    return 0;
}

/* ops::gated with no limit (crates/kf-backend-cpu/src/ops.rs:44-57) and ops::activate (:35-43) for the activations
 * whose reference formula is exact IEEE arithmetic plus exp: act 0 silu, 2 relu, 4 relu squared (the codes of the
 * reference GPU's kf_act, crates/kf-backend-cuda/src/kernels/common.cuh:93-99). gate and up rows are `stride` floats
 * apart (stride = 2 n: gate and up side by side in one row). Returns -1 for other activations. */
int kfo_gated(int act, const float* gate, const float* up, int rows, int n, int stride, float* out) {
    if (act != 0 && act != 2 && act != 4) return -1;
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) {
            const float g = gate[(size_t)r * stride + i], u = up[(size_t)r * stride + i];
            float a;
            if (act == 0) a = kfo_silu(g);
            else if (act == 2) a = fmaxf(g, 0.0f);
            else a = fmaxf(g, 0.0f) * fmaxf(g, 0.0f);
            out[(size_t)r * n + i] = a * u;
        }
    return 0;
}

/* expert_matvec: crates/kf-backend-cpu/src/moe.rs:7-24, rows of one expert against round_activations(x) */
static void expert_matvec(uint32_t ty, const uint8_t* w, int e, int n_in, int n_out, const float* x, float* y, float* xq, int nt) {
    int block, size;
    kfo_type_info(ty, &block, &size);
    size_t rb = (size_t)(n_in / block) * size;
    const uint8_t* base = w + (size_t)e * n_out * rb;
    kfo_round_activations(kfo_act_kind(ty), x, n_in, xq);
#ifdef _OPENMP
#pragma omp parallel for num_threads(nt) schedule(static)
#endif
    for (int o = 0; o < n_out; o++) y[o] = kfo_dot_row(ty, base + (size_t)o * rb, xq, n_in);
    (void)nt;
}

/* moe::exec with selected experts and expert_forward (crates/kf-backend-cpu/src/moe.rs:66-107,110-257) */
int kfo_moe_ffn(uint32_t ty, const uint8_t* gate, const uint8_t* up, const uint8_t* down, int n_exp, int n_embd, int n_ff,
                const float* x, int rows, const int32_t* sel, const float* wts, int n_used, float* out, int threads) {
    int block, size;
    if (kfo_type_info(ty, &block, &size) != 0 || n_embd % block != 0 || n_ff % block != 0) return -1;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#else
    int nt = 1;
#endif
    int big = n_embd > n_ff ? n_embd : n_ff;
    float* g = (float*)malloc(sizeof(float) * n_ff);
    float* u = (float*)malloc(sizeof(float) * n_ff);
    float* h = (float*)malloc(sizeof(float) * n_ff);
    float* ye = (float*)malloc(sizeof(float) * n_embd);
    float* xq = (float*)malloc(sizeof(float) * big);
    if (!g || !u || !h || !ye || !xq) return -2;
    int rc = 0;
    for (int r = 0; r < rows && rc == 0; r++) {
        float* acc = out + (size_t)r * n_embd;
        int first = 1;
        for (int k = 0; k < n_used; k++) {
            int e = sel[r * n_used + k];
            if (e < 0) continue;
            if (e >= n_exp) {
                rc = -1;
                break;
            }
            const float* xr = x + (size_t)r * n_embd;
            expert_matvec(ty, gate, e, n_embd, n_ff, xr, g, xq, nt);
            expert_matvec(ty, up, e, n_embd, n_ff, xr, u, xq, nt);
            for (int o = 0; o < n_ff; o++) h[o] = kfo_silu(g[o]) * u[o];
            expert_matvec(ty, down, e, n_ff, n_embd, h, ye, xq, nt);
            float wv = wts[r * n_used + k];
            for (int o = 0; o < n_embd; o++) acc[o] = first ? wv * ye[o] : acc[o] + wv * ye[o];
            first = 0;
        }
        if (first)
            for (int o = 0; o < n_embd; o++) acc[o] = 0.0f;
    }
    free(g); free(u); free(h); free(ye); free(xq);
    return rc;
}

/* The int8 expert path of the CPU backend, hidden_rows then down_cols (crates/kf-backend-cpu/src/experts.rs:93-124):
 * gate and up by dot_i8 on the quantized input row, hidden = silu(g) * u (ops::gated with Act::Silu, ops.rs:46-60),
 * the hidden row quantized again (Rows::new, experts.rs:48-53) and the down product by dot_i8; out[r] accumulates
 * wts * y in selection order. */
int kfo_moe_ffn_i8(uint32_t ty, const uint8_t* gate, const uint8_t* up, const uint8_t* down, int n_exp, int n_embd, int n_ff,
                   const float* x, int rows, const int32_t* sel, const float* wts, int n_used, float* out, int threads) {
    int block, size;
    if (kfo_type_info(ty, &block, &size) != 0 || n_embd % block != 0 || n_ff % block != 0) return -1;
    size_t rb_in = (size_t)(n_embd / block) * size, rb_ff = (size_t)(n_ff / block) * size;
    float* g = (float*)malloc(sizeof(float) * n_ff);
    float* u = (float*)malloc(sizeof(float) * n_ff);
    float* h = (float*)malloc(sizeof(float) * n_ff);
    float* ye = (float*)malloc(sizeof(float) * n_embd);
    if (!g || !u || !h || !ye) return -2;
    int rc = 0;
    for (int r = 0; r < rows && rc == 0; r++) {
        float* acc = out + (size_t)r * n_embd;
        for (int o = 0; o < n_embd; o++) acc[o] = 0.0f;
        const float* xr = x + (size_t)r * n_embd;
        for (int k = 0; k < n_used && rc == 0; k++) {
            int e = sel[r * n_used + k];
            if (e < 0) continue;
            if (e >= n_exp) {
                rc = -1;
                break;
            }
            rc |= kfo_matmul_i8(ty, gate + (size_t)e * n_ff * rb_in, n_embd, n_ff, xr, 1, NULL, g, threads);
            rc |= kfo_matmul_i8(ty, up + (size_t)e * n_ff * rb_in, n_embd, n_ff, xr, 1, NULL, u, threads);
            for (int o = 0; o < n_ff; o++) h[o] = kfo_silu(g[o]) * u[o];
            rc |= kfo_matmul_i8(ty, down + (size_t)e * n_embd * rb_ff, n_ff, n_embd, h, 1, NULL, ye, threads);
            float wv = wts[r * n_used + k];
            for (int o = 0; o < n_embd; o++) acc[o] += wv * ye[o];
        }
    }
    free(g); free(u); free(h); free(ye);
    return rc;
}
