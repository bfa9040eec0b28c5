/*
 * kf_oracle — CPU restatement of kungfu's quantized linear-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product links, loads or calls this library. It is the checker the
 * parity tests, the smoke check and the CPU-baseline leg of the benchmark compare the HIP path against.
 *
 * Every function restates one piece of the Rust reference (nickheyer/kungfu) and cites the file:line it follows.
 * All paths are relative to the reference repository root.
 *
 * Activation kinds use the reference's rounding codes (crates/kf-backend-cuda/src/exec.rs:103-113):
 *   KFO_ACT_Q8_0 = 3  per-32 absmax scale, round half away from zero, scale stored f16-rounded
 *   KFO_ACT_Q8K  = 4  per-256 signed-max scale, round half to even, first index of the max wins ties
 */
#ifndef KF_ORACLE_H
#define KF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KFO_TYPE_Q8_0 8u
#define KFO_TYPE_Q4_K 12u
#define KFO_TYPE_Q5_K 13u
#define KFO_TYPE_Q6_K 14u
#define KFO_TYPE_Q8_K 15u

#define KFO_ACT_Q8_0 3
#define KFO_ACT_Q8K 4

/* half 2.7.1 f16::to_f32 / f16::from_f32 (IEEE binary16, round to nearest even) */
float kfo_f16_to_f32(uint16_t h);
uint16_t kfo_f32_to_f16(float f);

/* TypeInfo of q8_0 / q4_K / q5_K / q6_K / q8_K: returns 0 and fills block and byte size, -1 for another id */
int kfo_type_info(uint32_t ty, int* block, int* size);

/* Activation kind paired with a weight type (act_kind), -1 when the type is not restated here */
int kfo_act_kind(uint32_t ty);

/* q8_0::quantize_row */
void kfo_q8_0_quantize_row(const float* x, int n, uint8_t* dst);

/* Quant::dequant_row of q8_0, q4_K, q5_K, q6_K, q8_K; returns -1 for another type */
int kfo_dequant_row(uint32_t ty, const uint8_t* src, int n, float* dst);

/* Quant::dot_row (float path) */
float kfo_dot_row(uint32_t ty, const uint8_t* src, const float* x, int n);

/* quantize_activations: q [rows][n], d16 and sum16 [rows][n/16]; returns -1 where the reference returns None */
int kfo_quantize_activations(int kind, const float* x, int rows, int n, int8_t* q, float* d16, int32_t* sum16);

/* round_activations of one row of n values */
void kfo_round_activations(int kind, const float* x, int n, float* out);

/* Quant::dot_i8, restating the AVX2 kernels lane for lane: y[r] for every activation row r */
int kfo_dot_i8(uint32_t ty, const uint8_t* src, int n, const int8_t* q, const float* d16, const int32_t* sum16, int rows, float* y);

/*
 * The exact integer intermediates of dot_i8 for one weight row against one activation row:
 *   q8_0: one int32 per 32-block, sum of q_w * q_x                                  -> ints[n/32]
 *   q4_K: per 256 super-block, sumi = sum_j sc_j * dot_j and mins = sum_j m_j * bsum_j -> ints[2*(n/256)]
 */
int kfo_block_ints(uint32_t ty, const uint8_t* src, int n, const int8_t* q, const int32_t* sum16, int32_t* ints);

/*
 * ops::matmul_slice: y[rows][n_out] = x[rows][n_in] times the weight rows (+ bias), the float path of the CPU
 * backend (round_activations, then dot_row for rows <= 2 or dequant then f32 dot). threads <= 0 uses OpenMP's default.
 */
int kfo_matmul_slice(uint32_t ty, const uint8_t* w, int n_in, int n_out, const float* x, int rows, const float* bias, float* y, int threads);

/* The integer form: quantize_activations once, then dot_i8 of every weight row, parallel over weight rows */
int kfo_matmul_i8(uint32_t ty, const uint8_t* w, int n_in, int n_out, const float* x, int rows, const float* bias, float* y, int threads);

/*
 * moe::exec for selected experts (selected_in), silu gating, no biases, WeightNorm::None, scale 1:
 * out[r] = sum_k wts[r][k] * down_e(silu(gate_e(x_r)) * up_e(x_r)), e = sel[r][k]; experts with sel < 0 are skipped.
 * gate/up: [n_exp][n_ff][n_embd] blocks; down: [n_exp][n_embd][n_ff] blocks, all of one type.
 */
int kfo_moe_ffn(uint32_t ty, const uint8_t* gate, const uint8_t* up, const uint8_t* down, int n_exp, int n_embd, int n_ff,
                const float* x, int rows, const int32_t* sel, const float* wts, int n_used, float* out, int threads);

/* The CPU backend's int8 expert path, experts::hidden_rows then down_cols, silu gating, out = sum of wts * y in
 * selection order. */
int kfo_moe_ffn_i8(uint32_t ty, const uint8_t* gate, const uint8_t* up, const uint8_t* down, int n_exp, int n_embd, int n_ff,
                   const float* x, int rows, const int32_t* sel, const float* wts, int n_used, float* out, int threads);
/* ops::silu */
float kfo_silu(float x);

/* rms_norm of rows x [rows][n] with nullable weight w [n] and bias b [n] */
int kfo_rms_norm(const float* x, const float* w, const float* b, int rows, int n, float eps, float* out);

/* gated activation act(gate) * up, act 0 silu / 2 relu / 4 relu squared; gate/up rows `stride` floats apart */
int kfo_gated(int act, const float* gate, const float* up, int rows, int n, int stride, float* out);

#ifdef __cplusplus
}
#endif
#endif
