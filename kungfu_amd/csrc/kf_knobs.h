// Tuning and comparison knobs of the launchers. Each knob is read from its KF_* environment variable once per process
// (at the first query of any knob, under std::call_once) and kept in an atomic, so launchers never scan the
// environment per call and never race a setenv. Tests and tuning scripts change them through kf_hip_set_knob, which
// stores into the same atomics. A flag knob is set by the variable's presence (any value), a value knob by its
// integer value; an unset knob reads -1 and the launchers then take their built-in choice.
#pragma once

enum KfKnob : int {
    KF_KNOB_GEMV_MAXIT,      // value: row iterations per GEMV block
    KF_KNOB_GEMV_NO_DMA,     // flag: register-staged GEMV
    KF_KNOB_GEMV_ONESHOT,    // flag: one-shot GEMV waves
    KF_KNOB_GEMV_NO_PIPE,    // flag: no persistent pipelined GEMV
    KF_KNOB_GEMV_DEPTH,      // value: rows in flight per GEMV wave (2..4)
    KF_KNOB_GEMV_BPC,        // value: GEMV blocks per CU
    KF_KNOB_MATMUL_NO_FUSE,  // flag: one-row matmul as quant_act + GEMV (two launches)
    KF_KNOB_ROWS_VALU,       // flag: per-lane few-row products instead of the matrix-core form
    KF_KNOB_RM_NB,           // value: stage buffers of the grouped matrix-core product
    KF_KNOB_RM_WHOLE,        // value: whole tiles a wave in the grouped matrix-core product
    KF_KNOB_RM1_TILES,       // value: tiles a block of the one-matrix few-row product
    KF_KNOB_Q4K_KQ,          // value: 0 / 1 forces the q4_K prefill GEMM kernel
    KF_KNOB_KQ_GEMM,         // value: 0 / 1 forces q5_K / q6_K few-row product or GEMM
    KF_KNOB_MOE_KQ,          // value: 0 selects the split-scale grouped MoE GEMM
    KF_KNOB_GEMM_NO_TAIL,    // flag: no K-split tail rounds in the tile GEMMs
    KF_KNOB_GEMM_TILE,       // flag: q8_0 always on the tile GEMM
    KF_KNOB_GEMM_SLICE,      // value: 0 / 1 forces 64-row slices for 65.. q8_0 rows
    KF_KNOB_GEMM_SK,         // value: 0 / 1 forces the q8_0 split-K small-batch product off / on
    KF_KNOB_GEMM_SK_S,       // value: splits of the split-K product
    KF_KNOB_GEMM_SK_V,       // value: split-K variant, 10 x groups a chunk + ring stages
    KF_KNOB_GEMM_NO_MR,      // flag: no 49..64-row one-pass product
    KF_KNOB_GEMM_MR,         // value: 11 / 14 forces a one-pass variant
    KF_KNOB_GEMM_SMALL_W,    // value: waves per block of the small-batch kernel
    KF_KNOB_GEMM_SMALL_TN,   // value: 16-column tiles a wave of the small-batch kernel
    KF_KNOB_CAPTURE_NO_SPLIT,  // flag: products under graph capture take the scratch-free forms
    KF_KNOB_GEMV_BURST,      // value: the burst GEMV takes grids of up to this many rows a wave (0: none; default 1)
    KF_KNOB_COUNT
};

// The knob's value, or -1 when unset
int kf_knob(KfKnob k);
inline bool kf_knob_on(KfKnob k) { return kf_knob(k) >= 0; }
inline int kf_knob_or(KfKnob k, int dflt) {
    const int v = kf_knob(k);
    return v >= 0 ? v : dflt;
}
