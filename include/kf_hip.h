/*
 * kf_hip.h — C ABI of the MI355X-native (gfx950) quantized linear-layer hot path of kungfu.
 *
 * This is the drop-in boundary a Rust `kf-backend-hip` crate binds (extern "C", plain pointers and sizes). It
 * replaces, entry point for entry point, what the reference's CUDA backend launches for `Op::MatMul` on int8-capable
 * weights (crates/kf-backend-cuda/src/exec.rs:2061-2109) and the backend trait methods around it
 * (crates/kf-core/src/backend.rs:206-269). Paths are relative to the reference repository root.
 *
 * Conventions
 *   - Weights are GGUF block bytes in their on-disk layout, unchanged: row-major [n_out][row_bytes], row_bytes =
 *     n_in / block * block_bytes (crates/kf-quant/src/lib.rs:17-20). Supported: q8_0 (id 8), q4_K (id 12).
 *   - Device pointers are HIP device addresses; `stream` is a hipStream_t (NULL = the null stream).
 *   - Every call returns 0 on success or a negative KF_E_* code; kf_hip_last_error() then describes the failure
 *     (per calling thread). No exception crosses the ABI. Shape checks mirror the reference's ensure!/bail! sites
 *     (crates/kf-backend-cpu/src/ops.rs:309-320, crates/kf-backend-cuda/src/exec.rs:2017,2066-2071).
 *   - Kernel-level entry points are stateless and asynchronous on `stream`; any number of threads may call them,
 *     one stream per thread.
 */
#ifndef KF_HIP_H
#define KF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KF_HIP_ABI_VERSION 2

/* ggml type ids (crates/kf-quant/src/types/q8_0.rs:4, q4_k.rs:4, q5_k.rs:4, q6_k.rs:4) */
#define KF_TYPE_Q8_0 8u
#define KF_TYPE_Q4_K 12u
#define KF_TYPE_Q5_K 13u
#define KF_TYPE_Q6_K 14u

/* activation rounding kinds, the reference's round codes (crates/kf-backend-cuda/src/exec.rs:103-113) */
#define KF_ACT_Q8_0 3
#define KF_ACT_Q8K 4

/* status codes */
#define KF_OK 0
#define KF_E_INVALID (-1)     /* bad shape, pointer or argument */
#define KF_E_UNSUPPORTED (-2) /* weight type or kind not on this path */
#define KF_E_HIP (-3)         /* a HIP runtime call or launch failed */
#define KF_E_NOMEM (-4)       /* device or host allocation failed */

/* ABI version of the loaded library (KF_HIP_ABI_VERSION it was built with). No reference counterpart. */
int kf_hip_abi_version(void);

/* Message of the last failed call on this thread ("" if none). Plays the role of the anyhow::Error text the reference
 * returns from Backend::run (crates/kf-core/src/backend.rs:212). */
const char* kf_hip_last_error(void);

/* ---------------------------------------------------------------------------------------------------------------
 * Activation quantization.
 * The int8 activation scratch of `rows` rows of `n` columns (the reference's ActI8, crates/kf-quant/src/lib.rs:48-78):
 *   q int8 [rows][n] | d16 f32 [rows][n/16] | s16 int32 [rows][n/16] | d32 f32 [rows][n/32] | s32 int32 [rows][n/32]
 *   | xa f16 [rows][ceil(n/256)][16]
 * each section 256-byte aligned from the base. xa (Q8K kind only) holds per 256 columns the eight per-32 sums split as
 * hi = floor(s / 64), lo = s - 64 hi (hi first), the operand of the q4_K GEMM's mins product.
 * This is NOT the reference's device layout act_scratch_all (crates/kf-backend-cuda/src/kf8.rs:338-357): that one
 * aligns sections to 16 bytes, keeps the sums as f32 and its fragment array xa in another form. A port sizes and
 * offsets this scratch with kf_hip_act_bytes / kf_hip_act_offsets, never with act_scratch_bytes. The integers and
 * scales themselves are the reference's, bit for bit. */

/* Bytes of that scratch. */
size_t kf_hip_act_bytes(int rows, int n);

/* Byte offsets of the six sections inside it (out[0..5] = q, d16, s16, d32, s32, xa). */
void kf_hip_act_offsets(int rows, int n, size_t out[6]);

/* Activation kind the reference pairs with a weight type (act_kind, crates/kf-quant/src/lib.rs:154-163), or
 * KF_E_UNSUPPORTED. */
int kf_hip_act_kind(uint32_t ty);

/* Quantizes x [rows][n] f32 (device, 16-byte aligned) into the scratch at `act` (device, 256-byte aligned).
 * Replaces quant_act (crates/kf-backend-cuda/src/kernels/fused.cu:12-21) and quant_launch (exec.rs:2053-2056);
 * bit-exact with quantize_activations (crates/kf-quant/src/lib.rs:81-140). n must be a multiple of 32 (Q8_0 kind) or
 * 256 (Q8K kind). */
int kf_hip_quant_act(const float* x, void* act, int rows, int n, int kind, void* stream);

/* Fused producers: the int8 activations straight from the preceding norm or gated activation, with no f32 round
 * trip through memory. Same scratch, kinds and width rules as kf_hip_quant_act; every f32 pointer 16-byte aligned.
 *
 * rms_norm of each row (x [rows][n], nullable weight w [n] and bias b [n], eps >= 0) then quantization. Replaces
 * rms_norm_q8 (crates/kf-backend-cuda/src/kernels/fused.cu:24-45, launched at exec.rs:2439); the values quantized are
 * the CPU backend's ops::rms_norm (crates/kf-backend-cpu/src/ops.rs:222-239) bit for bit: f64 sum of squares, IEEE
 * square root and division, unfused multiply-adds. */
int kf_hip_rms_norm_q8(const float* x, const float* w, const float* b, int rows, int n, float eps, int kind, void* act, void* stream);

/* Activation codes of kf_hip_gated_act_q8 (those of the reference GPU's kf_act, common.cuh:93-99). */
#define KF_GLU_SILU 0
#define KF_GLU_RELU 2
#define KF_GLU_RELU_SQR 4

/* act(gate) * up of each row, then quantization; gate and up rows are `stride` floats apart (stride = 2 n for the
 * two halves of one fused gate/up output row, n for separate tensors). Replaces gated_act_q8 (fused.cu:48-65,
 * exec.rs:2441-2444) for Op::GatedAct / Op::GatedActFused without a limit; the values are ops::gated
 * (crates/kf-backend-cpu/src/ops.rs:44-57) with silu's exp taken in f64 and rounded to f32. Other activations
 * return KF_E_UNSUPPORTED. */
int kf_hip_gated_act_q8(const float* gate, const float* up, int rows, int n, int stride, int act_fn, int kind, void* act, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Products on native block bytes against quantized activations.
 * y[r][o] = sum of the row's blocks (d_w * d_x * int32 dot, minus the q4_K min term) + bias[o] + res[r][o]
 * bias [n_out] and res [rows][n_out] are nullable device pointers. The weight base must be 16-byte aligned and
 * row_bytes must equal the type's row size for n (rows are packed). */

/* Decode and small-batch product of `rows` activation rows: one row is the streaming GEMV, several rows the
 * multi-row product that reads each weight row once per eight activation rows. Replaces matvec_i8_launch
 * (exec.rs:1996-2039) with the kernels matvec_i8 / matvec_i8_1 / matvec_i8_1s / mm_i8_{8,16,32} /
 * mm_frag_{8,16,24,32} (crates/kf-backend-cuda/src/kernels/quant.cuh:604-627, mm_frag.cuh:294-300).
 * q5_K and q6_K weights (Q8K-kind activations, any row count: one launch per eight activation rows) run their own
 * product, the reference's q5_K / q6_K loaders (kernels/quant_q5_K.cu, quant_q6_K.cu); q6_K rows need only 2-byte
 * alignment past the first. */
int kf_hip_gemv(uint32_t ty, const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y,
                int rows, int n, int n_out, void* stream);

/* Batched / prefill int8 GEMM on native rows: y [rows][n_out] from `rows` activation rows of the weight type's kind.
 * q8_0 (Q8_0-kind activations, n a multiple of 128): one int8 MFMA per 32-column group gives the exact int32 block
 * dots, rescaled by the group's activation and weight scales. q4_K (Q8K-kind activations, n a multiple of 256): the
 * 6-bit scales split into two 3-bit halves folded into two int8 operand planes, so two int8 MFMA chains form the
 * exact super-block integer; the mins term by an exact f16 MFMA per super-block, and the float rescale once per 256
 * columns. q5_K and q6_K (Q8K-kind activations, n a multiple of 256; q6_K: a multiple of 2048, so that its 210-byte
 * super-block rows start 16-byte aligned): one int8 MFMA per 32-column group (q6_K: per 16-column scale) gives the
 * exact int32 sub-block dots, the integer sub-scales are applied by multiply-adds into the exact super-block integer,
 * q5_K's mins by an exact f16 MFMA; other shapes return KF_E_UNSUPPORTED (kf_hip_gemv takes them).
 * Replaces kf8_gemm_dense / Store::gemm (crates/kf-backend-cuda/src/kernels/kf8.cu:375-395, HAS_M for q4_K / q5_K;
 * crates/kf-backend-cuda/src/kf8.rs:310-323) without the KF8 unpack pass (kf_unpack_i8, quant.cuh:585-601, instantiated
 * for q5_K / q6_K at quant_q5_K.cu:114 / quant_q6_K.cu:131): the native bytes are read directly. */
int kf_hip_gemm_i8(uint32_t ty, const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y,
                   int rows, int n, int n_out, void* stream);

/* The whole Op::MatMul of one weight: quantize x into `act` (device scratch of kf_hip_act_bytes(rows, n_in)) and run
 * the product the row count and shape select (q4_K: the few-row product or the tile GEMM, whichever a cost model
 * fitted on MI355X favours). Replaces matmul_launch (exec.rs:2061-2093). One row of q8_0 / q4_K (n_in <= 4096, x
 * and the weights 16-byte aligned) runs as one launch: the GEMV quantizes x itself, to the same integers, and `act`
 * is left unwritten (environment KF_MATMUL_NO_FUSE: two launches, as for other shapes). */
int kf_hip_matmul(uint32_t ty, const void* w, int n_in, int n_out, const float* x, int rows, void* act, const float* bias,
                  const float* res, float* y, void* stream);

/* kf_hip_rms_norm_q8 and kf_hip_matmul as one call: y = W . quant(rms_norm(x) * norm_w + norm_b) + bias + res, the
 * normalised rows quantized into `act` as kf_hip_rms_norm_q8 writes them, then the product kf_hip_matmul selects.
 * One row of q8_0 / q4_K (n_in <= 4096, x, norm_w, norm_b and the weights 16-byte aligned) runs as one launch: every
 * block of the GEMV normalises and quantizes the row itself (an f64 sum of squares, correctly rounded square root
 * and division and unfused multiply-adds, as kf_hip_rms_norm_q8; the f64 partial sums are added in another order, so
 * a row whose scaled value lies within an f64 rounding of a quantization boundary may get another integer there,
 * bit-identical on every tested shape) and `act` is left unwritten
 * (KF_MATMUL_NO_FUSE: two launches). Replaces the reference's rms_norm_q8 launch followed by matmul_launch
 * (exec.rs:2439, 2061-2093) for the decode products whose input is a normalised row (QKV, gate/up). */
int kf_hip_rms_norm_matmul(uint32_t ty, const void* w, int n_in, int n_out, const float* x, int rows, const float* norm_w, const float* norm_b,
                           float eps, void* act, const float* bias, const float* res, float* y, void* stream);

/* kf_hip_matmul without the `act` argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The activation
 * scratch is a static device array of KF_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until the process
 * ends; the call allocates nothing (no hipMalloc / hipFree / allocating library routine). Calls whose activations need
 * more (kf_hip_act_bytes(rows, n_in) > KF_NOALLOC_SCRATCH_BYTES, e.g. above 2048 x 16384) fail with KF_E_INVALID.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, two threads) race, so
 * callers serialise them (one stream per GPU, or events). The array keeps the last call's contents; nothing in it needs
 * to start at zero (each call overwrites what it reads). */
#define KF_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int kf_hip_matmul_noalloc(uint32_t ty, const void* w, int n_in, int n_out, const float* x, int rows, const float* bias,
                          const float* res, float* y, void* stream);

/* KF_NOALLOC_SCRATCH_BYTES of the loaded library. No reference counterpart. */
size_t kf_hip_noalloc_scratch_bytes(void);

/* The split-K products and the tile GEMMs' tail splits keep partial tiles and tickets in a static per-GPU array of
 * three slots. Two are stream slots: one goes to each (device, stream) on its first such product and stays with it;
 * launches on one stream are ordered, so a stream's products never share their slot with a running product. A stream
 * that finds both stream slots held by other streams runs the scratch-free forms (same results within the bar). The
 * third is the graph slot: every product recorded under HIP graph capture on that GPU uses it, and direct launches
 * never do, so a replay (on any stream) never shares tickets or partials with a direct product. Rule: two replays of
 * graphs that hold such products must not run at the same time on one GPU (serialise them on one stream, or with
 * events); knob KF_CAPTURE_NO_SPLIT records the scratch-free forms instead. This call waits for `stream`'s work and
 * returns its stream slot for other streams (a no-op if it holds none); call it before destroying a stream that ran
 * products. No reference counterpart. */
int kf_hip_release_stream(void* stream);

/* Grouped products sharing one input (Q/K/V, or gate and up stored as separate tensors): up to KF_HIP_MAX_SEGMENTS
 * weight matrices of one type and row width stacked along their output rows. The segment table is the reference's
 * (quant.cuh:301-305, built by matmul_group_launch, exec.rs:1305-1314), KF_SEG_WORDS int64 words per member in HOST
 * memory: [0] byte offset of the member's weights from w, [1] of its output from y, [2] of its bias from y or
 * KF_SEG_NONE, [3] of its residual from y or KF_SEG_NONE, [4] its first stacked row (members in order, no gaps), [5]
 * its row count. Member k writes y_k [rows][n_out_k]. One activation row of q8_0 / q4_K runs as one GEMV launch over
 * all stacked rows (the reference's segmented matvec_i8, quant.cuh:447-464); other row counts and types run each
 * member's product against the shared activations (the reference's per-member fallback, exec.rs:1334-1342). */
#define KF_HIP_MAX_SEGMENTS 4
#define KF_SEG_WORDS 6
#define KF_SEG_NONE (-0x7fffffffffffffffLL - 1)
int kf_hip_gemv_group(uint32_t ty, const void* w, int64_t row_bytes, const void* act, float* y, int rows, int n, const int64_t* segs,
                      int nseg, void* stream);

/* kf_hip_matmul for a group: quantize x once, then the grouped product (each member's product chosen by the row
 * count as kf_hip_matmul chooses it); one row of q8_0 / q4_K is one launch that quantizes x itself, as in
 * kf_hip_matmul. Replaces matmul_group_launch (exec.rs:1283-1346). */
int kf_hip_matmul_group(uint32_t ty, const void* w, int n_in, const float* x, int rows, void* act, float* y, const int64_t* segs, int nseg,
                        void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * MoE grouped experts (Op::MoeFfn with routed pairs: rows x n_used pairs rj = r * n_used + j, slot sel[rj] < 0 =
 * unused). Expert matrices are stacked: expert e's rows start at base + e * expert_bytes.
 * The CPU meaning is moe::exec / expert_forward (crates/kf-backend-cpu/src/moe.rs:66-107,110-257). */

/* Pairs grouped by slot: offsets[s] .. offsets[s + 1] index `order`, which lists the pair indices of slot s in
 * increasing order (deterministic; the reference's atomic placement leaves it unspecified). offsets has n_slots + 1
 * entries; slots outside [0, n_slots) are skipped; n_slots at most 4096. Replaces moe_group (crates/kf-backend-cuda/src/kernels/moe.cu:118-141). */
int kf_hip_moe_group(const int32_t* slots, int total, int n_slots, int32_t* order, int32_t* offsets, void* stream);

/* Grouped expert product: for each slot s and each pair p of its group, y[p][o] = W_s[o] . x, x the activation row p
 * (per_slot != 0) or p / n_used of `act` (act_rows rows of n columns, quantized with the weight type's kind). Each
 * expert row is read once per group (eight pairs at a time). With w_up non-null the gate (w) and up (w_up) experts
 * are multiplied together and y[p][o] = silu(gate . x) * (up . x). Replaces moe_matvec_i8 / moe_gate_up_i8
 * (crates/kf-backend-cuda/src/kernels/quant.cuh:519-581, launches exec.rs:2208-2237), which read each expert once
 * per pair. n at most 16384 (q4_K) or 8192 (q8_0). */
int kf_hip_moe_gemv(uint32_t ty, const void* w, const void* w_up, int64_t expert_bytes, int64_t row_bytes, const void* act, int act_rows, int n,
                    int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int n_used, int per_slot, float* y, void* stream);

/* Grouped tile GEMM of routed pairs (q4_K experts, n a multiple of 256): `act` holds `pairs` activation rows in group
 * order (the pairs of slot s are rows offsets[s]..offsets[s + 1], device offsets from kf_hip_moe_group); slot s
 * multiplies its expert w + s * expert_bytes ([n_out][row_bytes]) or, with w2 non-null, output columns below n_split
 * from w + s * expert_bytes and columns n_split.. from w2 + s * expert_bytes (gate and up as one product). Output row p
 * of the group order is written to y row out_rows[p] (device, nullable: row p); y is [*][n_out]. Rows of act past
 * offsets[n_slots] are not read. Replaces kf8_gemm_moe (crates/kf-backend-cuda/src/kernels/kf8.cu:400-416) without the
 * KF8 unpack; kf_hip_moe_ffn takes it past 64 routed pairs, as expert_gemm_chunks (exec.rs:2196-2237). A grid of at
 * most two rounds of the CUs runs each tile as two K halves through the split scratch (the stream's slot); the first
 * half's partial passes through the tile's rows of y before the sum lands there. */
int kf_hip_moe_gemm(uint32_t ty, const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, int n_split, const void* act,
                    int pairs, int n, int n_out, const int32_t* offsets, int n_slots, const int32_t* out_rows, float* y, void* stream);

/* out[r][o] = sum over j of wts[rj] * scale * part[rj][o] for the row's pairs with slots[rj] >= 0, in j order, plus
 * host[r][o] (nullable). Replaces moe_combine (moe.cu:153-164). */
int kf_hip_moe_combine(const float* part, const float* wts, const int32_t* slots, const float* host, float* out, int rows, int n_used, int n_embd,
                       float scale, void* stream);

/* Device scratch of one kf_hip_moe_ffn call. No reference counterpart (the reference sizes its per-node scratch in
 * the plan). */
size_t kf_hip_moe_scratch_bytes(int rows, int n_used, int n_embd, int n_ff, int n_slots);

/* The routed expert layer with silu gating: quantize x, group the pairs, fused gate/up product, quantize the hidden
 * rows, down product, weighted combine. Past 64 routed pairs of q4_K experts (n_embd and n_ff multiples of 256) the
 * products run as the grouped tile GEMM (kf_hip_moe_gemm) on the pairs' activation rows gathered in group order, with
 * the hidden rows quantized by kf_hip_gated_act_q8; otherwise as the grouped few-row products (kf_hip_moe_gemv). gate and up are [n_slots][n_ff][row of n_embd], down [n_slots][n_embd][row
 * of n_ff], all of type ty. out [rows][n_embd]. A pair whose slot is outside [0, n_slots) contributes nothing (the
 * grouping skips it and so does the combine). Replaces expert_launches (crates/kf-backend-cuda/src/exec.rs:2378-2386)
 * for int8-capable experts resident on the device. */
int kf_hip_moe_ffn(uint32_t ty, const void* gate, const void* up, const void* down, int n_slots, int n_embd, int n_ff, const float* x, int rows,
                   const int32_t* sel, const float* wts, int n_used, float scale, void* scratch, size_t scratch_bytes, float* out, void* stream);

/* Per-block int32 results of n_out weight rows against the `rows` activation rows of `act`: q8_0 one int32 per 32-block
 * (out [n_out][rows][n/32]); q4_K and q5_K (sumi, mins) per super-block (out [n_out][rows][n/256][2]); q6_K one
 * int32 per super-block, dot minus the 32-offset bias (out [n_out][rows][n/256]). The integers of dot_i8
 * (crates/kf-quant/src/types/q8_0.rs:10-29, q4_k.rs:10-58, q5_k.rs:7-60, q6_k.rs:17-59), computed by the same lane
 * code as the product kernels. No reference counterpart: it exists so the integer results can be checked bit-exact. */
int kf_hip_block_ints(uint32_t ty, const void* w, int64_t row_bytes, const void* act, int rows, int n, int n_out, int32_t* out,
                      void* stream);

/* Streaming read of `bytes` bytes at buf (16-byte aligned, bytes a multiple of 16, below 2^36) with plain 16-byte loads,
 * per_thread (4, 8 or 16) pieces a thread, all requested at launch; writes at most one word to sink (4 bytes). No
 * reference counterpart: the measurement's HBM read peak on the box, reported beside the spec peak. */
int kf_hip_stream_read(const void* buf, size_t bytes, int per_thread, uint32_t* sink, void* stream);

/* Launch knobs (KF_GEMV_MAXIT, KF_GEMM_NO_TAIL, ... : the kernel-variant and tuning switches the launchers consult).
 * The library reads each from its environment variable once per process, at the first knob query; afterwards only
 * kf_hip_set_knob changes them (value < 0 unsets the knob; a flag knob is on for any value >= 0). Returns KF_E_INVALID
 * for an unknown name. kf_hip_get_knob returns the value, -1 when unset, -2 for an unknown name. Knobs are
 * process-wide: a change applies to launches made after it on every thread. No reference counterpart (the reference
 * reads its KF_* variables with std::env at use, e.g. crates/kf-backend-cuda/src/exec.rs); these exist so tests and
 * tuning can compare kernel variants without racing the environment. */
int kf_hip_set_knob(const char* name, int value);
int kf_hip_get_knob(const char* name);

/* ---------------------------------------------------------------------------------------------------------------
 * Backend mirror (crates/kf-core/src/backend.rs:206-269 Backend; WeightSource :7-13). Host buffers in and out; the
 * backend owns device copies of its weights (ensure_weight, crates/kf-backend-cuda/src/exec.rs:1347-1359) and a
 * stream. Not thread-safe per handle (Backend is Send, not Sync). */
typedef struct kf_hip_backend kf_hip_backend;

/* A backend on HIP device `device`, or NULL (see kf_hip_last_error). */
kf_hip_backend* kf_hip_backend_new(int device);
void kf_hip_backend_free(kf_hip_backend* b);

/* Copies one weight tensor to the device. dims[0] = n_in (innermost), dims[1] = n_out, further dims stack matrices
 * (WeightSource::dims). Returns a weight id >= 0 or a negative status. */
int kf_hip_backend_add_weight(kf_hip_backend* b, uint32_t ty, const int64_t* dims, int ndims, const void* bytes, size_t nbytes);

/* Op::MatMul{weight, bias} on host rows: y [rows][n_out] = x [rows][cols] times the weight (+ bias [n_out], nullable).
 * The ops::matmul contract (crates/kf-backend-cpu/src/ops.rs:299-346): cols must equal n_in. Synchronous. */
int kf_hip_backend_matmul(kf_hip_backend* b, int wid, const float* x, int rows, int cols, const float* bias, float* y);

/* Op::MatMulSlice{weight, index} (ops.rs:304-346 with index): slice `index` of a weight whose third dim stacks matrices */
int kf_hip_backend_matmul_slice(kf_hip_backend* b, int wid, int index, const float* x, int rows, int cols, float* y);

/* ---------------------------------------------------------------------------------------------------------------
 * GGUF files (host). The reader of crates/kf-gguf/src/lib.rs: GGUF v2/v3, the typed key-value header (value kinds
 * 0..12 as in the file, arrays of any kind), tensor infos with ggml dims innermost first, the data section aligned to
 * general.alignment (32 when absent), and split files name-0000i-of-0000N.gguf opened as one. Shards are memory-mapped
 * read-only; kf_gguf_tensor_data returns a pointer into the map (valid until kf_gguf_close), which goes straight to
 * kf_hip_backend_add_weight as the reference's WeightSource::bytes borrows from its mmap (kf-engine/src/loader.rs).
 * Metadata is iterated in key order (the reference keeps a BTreeMap; a repeated key keeps its last value). */
typedef struct kf_gguf kf_gguf;

/* Gguf::open (lib.rs:181-203): NULL on failure, with the reason in kf_hip_last_error(). */
kf_gguf* kf_gguf_open(const char* path);
void kf_gguf_close(kf_gguf* g);
int kf_gguf_n_shards(const kf_gguf* g);

/* Tensors in file order, shard by shard; kf_gguf_find_tensor is Gguf::tensor (lib.rs:209-211), KF_E_INVALID if absent. */
int64_t kf_gguf_n_tensors(const kf_gguf* g);
int64_t kf_gguf_find_tensor(const kf_gguf* g, const char* name);

/* Tensor i: name (owned by g), up to max_dims dims, ggml type, shard, offset in its shard's data section and byte size
 * (TensorInfo::nbytes, lib.rs:157-160: -1 when the type has no known layout or the inner dim is not a multiple of its
 * block). Returns the number of dims. Nullable outputs. */
int kf_gguf_tensor_info(const kf_gguf* g, int64_t i, const char** name, int64_t* dims, int max_dims, uint32_t* ggml_type, int* shard,
                        uint64_t* offset, int64_t* nbytes);

/* Gguf::bytes (lib.rs:213-219): the tensor's bytes inside its shard's map, NULL when its size is unknown or the data
 * runs past the end of the file. */
const void* kf_gguf_tensor_data(const kf_gguf* g, int64_t i);

/* Metadata entry i (key order): key, value kind, element kind (arrays; the kind itself for scalars) and element count
 * (1 for scalars). Typed reads follow Value::as_u64 / as_i64 / as_f64 (lib.rs:28-62): unsigned reads take non-negative
 * signed values and bools, signed reads any integer, float reads floats and integers; idx selects an array element
 * (0 for a scalar). */
int64_t kf_gguf_n_kv(const kf_gguf* g);
int64_t kf_gguf_find_kv(const kf_gguf* g, const char* key);
int kf_gguf_kv(const kf_gguf* g, int64_t i, const char** key, uint32_t* kind, uint32_t* elem_kind, uint64_t* count);
int kf_gguf_kv_u64(const kf_gguf* g, int64_t i, uint64_t idx, uint64_t* out);
int kf_gguf_kv_i64(const kf_gguf* g, int64_t i, uint64_t idx, int64_t* out);
int kf_gguf_kv_f64(const kf_gguf* g, int64_t i, uint64_t idx, double* out);
int kf_gguf_kv_str(const kf_gguf* g, int64_t i, uint64_t idx, const char** out, uint64_t* len);

/* ---------------------------------------------------------------------------------------------------------------
 * Host utilities (CPU).
 * kf_quantize_q8_0: q8_0::quantize_row (crates/kf-quant/src/types/q8_0.rs:33-42, re-exported at lib.rs:2) over rows.
 * kf_quantize_q4_k: a q4_K encoder of this library's own. The reference has none (it only reads q4_K); this one fits
 *   per sub-block an affine min/max, then 6-bit scales and mins against f16 super-block d/dmin, rounding to nearest
 *   even. Any valid encoder suffices: parity is defined on the bytes.
 * kf_quantize_q5_k / kf_quantize_q6_k: encoders of this library's own for the same reason (q5_K: q4_K's form with 31
 *   steps and the fifth bit in qh; q6_K: per 16 values a signed scale amax / 32 as int8 against an f16 d).
 * kf_synth_normal: SplitMix64 (the generator of crates/kf-quant/tests/parity.rs:75-88) feeding Box-Muller pairs,
 *   sigma * N(0,1) as f32: the synthetic data of the benchmark configs. */
int kf_quantize_q8_0(const float* x, int64_t rows, int n, uint8_t* dst);
int kf_quantize_q4_k(const float* x, int64_t rows, int n, uint8_t* dst);
int kf_quantize_q5_k(const float* x, int64_t rows, int n, uint8_t* dst);
int kf_quantize_q6_k(const float* x, int64_t rows, int n, uint8_t* dst);
void kf_synth_normal(uint64_t seed, float sigma, float* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
