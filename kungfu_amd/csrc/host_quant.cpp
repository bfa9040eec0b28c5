// Host-side weight encoders and synthetic data of kf-hip (CPU code, part of the library's C ABI).
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/kf_hip.h"
#include "kf_layout.h"

namespace {

// IEEE binary16 round-to-nearest-even, the conversion of half::f16::from_f32 (half 2.7.1). _Float16 conversions on
// x86-64 round to nearest even in software or with F16C.
uint16_t f32_to_f16_bits(float f) {
    const _Float16 h = (_Float16)f;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
}

// Rust's `f32::round_ties_even() as i32`, saturating
int32_t nearest_i32(float v) {
    if (v != v) return 0;
    const float r = std::nearbyint(v);
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return INT32_MIN;
    return (int32_t)r;
}

void q8_0_row(const float* x, int n, uint8_t* dst) {
    for (int b = 0; b < n / 32; b++) {
        const float* blk = x + 32 * b;
        uint8_t* out = dst + 34 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = std::fmax(amax, std::fabs(blk[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t h = f32_to_f16_bits(d);
        out[0] = (uint8_t)(h & 0xff);
        out[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) {
            int32_t v = nearest_i32(blk[j] * id);
            v = v < -127 ? -127 : (v > 127 ? 127 : v);
            out[2 + j] = (uint8_t)(int8_t)v;
        }
    }
}

// One q4_K super-block of 256 values: per sub-block of 32 an affine range [min(0, lo), hi] in 15 steps, then the
// 6-bit scales and mins against the largest of each over 63, stored as f16 d and dmin.
void q4_k_block(const float* x, uint8_t* out) {
    float scale[8], mins[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int s = 0; s < 8; s++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int l = 0; l < 32; l++) {
            lo = std::fmin(lo, x[32 * s + l]);
            hi = std::fmax(hi, x[32 * s + l]);
        }
        if (hi < lo) hi = lo;
        scale[s] = (hi - lo) / 15.0f;
        mins[s] = -lo;
        max_scale = std::fmax(max_scale, scale[s]);
        max_min = std::fmax(max_min, mins[s]);
    }
    const uint16_t dh = f32_to_f16_bits(max_scale / 63.0f);
    const uint16_t mh = f32_to_f16_bits(max_min / 63.0f);
    const float d = f16_bits_to_f32(dh), dmin = f16_bits_to_f32(mh);
    uint8_t sc[8], mn[8];
    for (int s = 0; s < 8; s++) {
        int32_t a = d > 0.0f ? nearest_i32(scale[s] / d) : 0;
        int32_t m = dmin > 0.0f ? nearest_i32(mins[s] / dmin) : 0;
        sc[s] = (uint8_t)(a < 0 ? 0 : (a > 63 ? 63 : a));
        mn[s] = (uint8_t)(m < 0 ? 0 : (m > 63 ? 63 : m));
    }
    out[0] = (uint8_t)(dh & 0xff);
    out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(mh & 0xff);
    out[3] = (uint8_t)(mh >> 8);
    // the packing scale_min_k4 (crates/kf-quant/src/types/mod.rs:86-94) reads back
    uint8_t* q = out + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    uint8_t nib[256];
    for (int s = 0; s < 8; s++) {
        const float ed = d * (float)sc[s], em = dmin * (float)mn[s];
        for (int l = 0; l < 32; l++) {
            int32_t v = ed > 0.0f ? nearest_i32((x[32 * s + l] + em) / ed) : 0;
            nib[32 * s + l] = (uint8_t)(v < 0 ? 0 : (v > 15 ? 15 : v));
        }
    }
    for (int j = 0; j < 4; j++)
        for (int l = 0; l < 32; l++) out[16 + 32 * j + l] = (uint8_t)(nib[64 * j + l] | (nib[64 * j + 32 + l] << 4));
}

// One q5_K super-block: q4_K's affine form with 31 steps per sub-block, the fifth bit of each value in qh
void q5_k_block(const float* x, uint8_t* out) {
    float scale[8], mins[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int s = 0; s < 8; s++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int l = 0; l < 32; l++) {
            lo = std::fmin(lo, x[32 * s + l]);
            hi = std::fmax(hi, x[32 * s + l]);
        }
        if (hi < lo) hi = lo;
        scale[s] = (hi - lo) / 31.0f;
        mins[s] = -lo;
        max_scale = std::fmax(max_scale, scale[s]);
        max_min = std::fmax(max_min, mins[s]);
    }
    const uint16_t dh = f32_to_f16_bits(max_scale / 63.0f);
    const uint16_t mh = f32_to_f16_bits(max_min / 63.0f);
    const float d = f16_bits_to_f32(dh), dmin = f16_bits_to_f32(mh);
    uint8_t sc[8], mn[8];
    for (int s = 0; s < 8; s++) {
        int32_t a = d > 0.0f ? nearest_i32(scale[s] / d) : 0;
        int32_t m = dmin > 0.0f ? nearest_i32(mins[s] / dmin) : 0;
        sc[s] = (uint8_t)(a < 0 ? 0 : (a > 63 ? 63 : a));
        mn[s] = (uint8_t)(m < 0 ? 0 : (m > 63 ? 63 : m));
    }
    out[0] = (uint8_t)(dh & 0xff);
    out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(mh & 0xff);
    out[3] = (uint8_t)(mh >> 8);
    uint8_t* q = out + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    uint8_t v5[256];
    for (int s = 0; s < 8; s++) {
        const float ed = d * (float)sc[s], em = dmin * (float)mn[s];
        for (int l = 0; l < 32; l++) {
            int32_t v = ed > 0.0f ? nearest_i32((x[32 * s + l] + em) / ed) : 0;
            v5[32 * s + l] = (uint8_t)(v < 0 ? 0 : (v > 31 ? 31 : v));
        }
    }
    uint8_t* qh = out + 16;
    for (int l = 0; l < 32; l++) {
        uint8_t h = 0;
        for (int s = 0; s < 8; s++) h |= (uint8_t)(((v5[32 * s + l] >> 4) & 1) << s);
        qh[l] = h;
    }
    for (int j = 0; j < 4; j++)
        for (int l = 0; l < 32; l++) out[48 + 32 * j + l] = (uint8_t)((v5[64 * j + l] & 15) | ((v5[64 * j + 32 + l] & 15) << 4));
}

// One q6_K super-block: per 16 values a scale amax / 31 (the values in -31..31 steps; -32 stays unused), the 16 scales
// as int8 against d = max scale / 127 (f16), then the values as 6-bit offsets from -32
void q6_k_block(const float* x, uint8_t* out) {
    float gs[16], max_abs = 0.0f;
    for (int g = 0; g < 16; g++) {
        float a = 0.0f;
        for (int l = 0; l < 16; l++) a = std::fmax(a, std::fabs(x[16 * g + l]));
        gs[g] = a / 31.0f;
        max_abs = std::fmax(max_abs, gs[g]);
    }
    const uint16_t dh = f32_to_f16_bits(max_abs / 127.0f);
    const float d = f16_bits_to_f32(dh);
    int8_t sc[16];
    uint8_t v6[256];
    for (int g = 0; g < 16; g++) {
        int32_t s = d > 0.0f ? nearest_i32(gs[g] / d) : 0;
        sc[g] = (int8_t)(s < -128 ? -128 : (s > 127 ? 127 : s));
        const float e = d * (float)sc[g];
        for (int l = 0; l < 16; l++) {
            int32_t v = e != 0.0f ? nearest_i32(x[16 * g + l] / e) : 0;
            v = v < -32 ? -32 : (v > 31 ? 31 : v);
            v6[16 * g + l] = (uint8_t)(v + 32);
        }
    }
    std::memset(out, 0, 208);
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++)
            for (int k = 0; k < 4; k++) {
                const uint8_t v = v6[128 * h + 32 * k + l];
                out[64 * h + l + 32 * (k & 1)] |= (uint8_t)((v & 15) << (4 * (k >> 1)));
                out[128 + 32 * h + l] |= (uint8_t)((v >> 4) << (2 * k));
            }
    for (int g = 0; g < 16; g++) out[192 + g] = (uint8_t)sc[g];
    out[208] = (uint8_t)(dh & 0xff);
    out[209] = (uint8_t)(dh >> 8);
}

uint64_t splitmix_next(uint64_t& state) {
    state += 0x9E3779B97F4A7C15ull;
    uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

extern "C" {

int kf_quantize_q8_0(const float* x, int64_t rows, int n, uint8_t* dst) {
    if (!x || !dst || rows < 0 || n <= 0 || n % 32 != 0) return KF_E_INVALID;
    const size_t rb = (size_t)(n / 32) * 34;
    for (int64_t r = 0; r < rows; r++) q8_0_row(x + (size_t)r * n, n, dst + (size_t)r * rb);
    return KF_OK;
}

int kf_quantize_q4_k(const float* x, int64_t rows, int n, uint8_t* dst) {
    if (!x || !dst || rows < 0 || n <= 0 || n % 256 != 0) return KF_E_INVALID;
    const size_t rb = (size_t)(n / 256) * 144;
    for (int64_t r = 0; r < rows; r++)
        for (int b = 0; b < n / 256; b++) q4_k_block(x + (size_t)r * n + 256 * b, dst + (size_t)r * rb + 144 * b);
    return KF_OK;
}

int kf_quantize_q5_k(const float* x, int64_t rows, int n, uint8_t* dst) {
    if (!x || !dst || rows < 0 || n <= 0 || n % 256 != 0) return KF_E_INVALID;
    const size_t rb = (size_t)(n / 256) * KF_Q5_K_BYTES;
    for (int64_t r = 0; r < rows; r++)
        for (int b = 0; b < n / 256; b++) q5_k_block(x + (size_t)r * n + 256 * b, dst + (size_t)r * rb + KF_Q5_K_BYTES * b);
    return KF_OK;
}

int kf_quantize_q6_k(const float* x, int64_t rows, int n, uint8_t* dst) {
    if (!x || !dst || rows < 0 || n <= 0 || n % 256 != 0) return KF_E_INVALID;
    const size_t rb = (size_t)(n / 256) * KF_Q6_K_BYTES;
    for (int64_t r = 0; r < rows; r++)
        for (int b = 0; b < n / 256; b++) q6_k_block(x + (size_t)r * n + 256 * b, dst + (size_t)r * rb + KF_Q6_K_BYTES * b);
    return KF_OK;
}

void kf_synth_normal(uint64_t seed, float sigma, float* out, size_t n) {
    uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = ((double)(splitmix_next(state) >> 11) + 0.5) * 0x1.0p-53;
        const double u2 = ((double)(splitmix_next(state) >> 11) + 0.5) * 0x1.0p-53;
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = (float)(sigma * r * std::cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(sigma * r * std::sin(two_pi * u2));
    }
}

}  // extern "C"
