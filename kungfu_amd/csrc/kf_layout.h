// Block layouts and the int8 activation scratch layout, shared by host and device code.
//
// GGUF block layouts consumed unchanged (crates/kf-quant/src/types/q8_0.rs:4, types/q4_k.rs:4):
//   q8_0: 32 elements in 34 bytes, f16 d then 32 x int8
//   q4_K: 256 elements in 144 bytes, f16 d, f16 dmin, 12 bytes of packed 6-bit scales and mins for 8 sub-blocks of
//         32, then 128 bytes of nibbles; pair j of sub-blocks (2j, 2j+1) lives in bytes 16+32j..48+32j, the low
//         nibble of byte 16+32j+l being element 64j+l and the high nibble element 64j+32+l.
//   q5_K (types/q5_k.rs:4): 256 elements in 176 bytes, q4_K's header (16 bytes), then qh[32] (bit s of qh[l] is the
//         fifth bit of element l of sub-block s), then q4_K's 128 bytes of low nibbles.
//   q6_K (types/q6_k.rs:4): 256 elements in 210 bytes, ql[128] (low 4 bits), qh[64] (high 2 bits), 16 int8 scales
//         (one per 16 elements), f16 d at byte 208; element 128h + 32k + l (h < 2, k < 4, l < 32) is
//         (ql[64h + l + 32 (k & 1)] >> 4 (k >> 1)) & 15 | ((qh[32h + l] >> 2k) & 3) << 4, minus 32.
#pragma once
#include <stddef.h>
#include <stdint.h>

#define KF_TYPE_Q8_0 8u
#define KF_TYPE_Q4_K 12u
#define KF_TYPE_Q5_K 13u
#define KF_TYPE_Q6_K 14u

#define KF_ACT_Q8_0 3
#define KF_ACT_Q8K 4

#define KF_Q8_0_BLOCK 32
#define KF_Q8_0_BYTES 34
#define KF_Q4_K_BLOCK 256
#define KF_Q4_K_BYTES 144
#define KF_Q5_K_BYTES 176
#define KF_Q6_K_BYTES 210

// Alignment of every section of the activation scratch
#define KF_ACT_ALIGN 256

static inline size_t kf_align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// The int8 activation scratch of `rows` rows of `n` columns: the reference's ActI8 (crates/kf-quant/src/lib.rs:48-78)
// plus per-32 copies of the scale and sum, each section KF_ACT_ALIGN aligned:
//   q    int8  [rows][n]
//   d16  f32   [rows][n/16]   scale of every 16 columns
//   s16  int32 [rows][n/16]   integer sum of every 16 columns
//   d32  f32   [rows][n/32]   scale of every 32 columns
//   s32  int32 [rows][n/32]   integer sum of every 32 columns
//   xa   f16   [rows][ceil(n/256)][16]  Q8K kind only: per 256 columns the matrix-core operand of the q4_K mins
//        term, hi_j = floor(s32_j / 64) for the eight 32-column groups j, then lo_j = s32_j - 64 hi_j (hi in
//        [-64, 63], lo in [0, 63], both exact in f16), the counterpart of the reference's fragment array xa
//        (crates/kf-backend-cuda/src/kf8.rs:338-357); left unwritten by the Q8_0 kind
struct kf_act_offsets {
    size_t q, d16, s16, d32, s32, xa, total;
};

static inline struct kf_act_offsets kf_act_layout(size_t rows, size_t n) {
    struct kf_act_offsets o;
    o.q = 0;
    o.d16 = kf_align_up(o.q + rows * n, KF_ACT_ALIGN);
    o.s16 = kf_align_up(o.d16 + rows * (n / 16) * 4, KF_ACT_ALIGN);
    o.d32 = kf_align_up(o.s16 + rows * (n / 16) * 4, KF_ACT_ALIGN);
    o.s32 = kf_align_up(o.d32 + rows * (n / 32) * 4, KF_ACT_ALIGN);
    o.xa = kf_align_up(o.s32 + rows * (n / 32) * 4, KF_ACT_ALIGN);
    o.total = kf_align_up(o.xa + rows * ((n + 255) / 256) * 32, KF_ACT_ALIGN);
    return o;
}

// Grouped products: up to KF_MAX_SEGS weight matrices with the same type and row width, stacked along the output
// rows and run against one quantized input. Stacked row o belongs to the last member k with start[k] <= o; its
// row (o - start[k]) of w[k] is multiplied and written to y[k] (+ bias[k], res[k], either may be null). n == 0 is the
// plain single product over the launch's own pointers.
#define KF_MAX_SEGS 4
struct KfSegs {
    int n;
    int start[KF_MAX_SEGS];
    const uint8_t* w[KF_MAX_SEGS];
    float* y[KF_MAX_SEGS];
    const float* bias[KF_MAX_SEGS];
    const float* res[KF_MAX_SEGS];
};
