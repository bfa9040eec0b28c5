// C ABI of kf-hip: argument checks, kernel selection and the backend mirror. Declared in include/kf_hip.h.
//
// The selection logic plays the part of the reference's matmul_launch / matvec_i8_launch
// (crates/kf-backend-cuda/src/exec.rs:1850-2109): quantize the activations with the weight type's kind, then one
// product kernel chosen by the number of activation rows.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "kf_knobs.h"
#include "../../include/kf_hip.h"
#include "kf_host.h"
#include "kf_layout.h"

static_assert(KF_HIP_MAX_SEGMENTS == KF_MAX_SEGS, "one segment limit");

// Launchers in the .hip translation units
hipError_t kf_launch_quant_act(const float* x, void* act, int rows, int n, int kind, hipStream_t s);
hipError_t kf_launch_stream_read(const void* buf, size_t bytes, int per_thread, uint32_t* sink, hipStream_t s);
hipError_t kf_launch_gemv_k(uint32_t ty, const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y,
                            int rows, int n, int n_out, hipStream_t s);
hipError_t kf_launch_rms_norm_q8(const float* x, const float* w, const float* b, float eps, void* act, int rows, int n, int kind,
                                 hipStream_t s);
hipError_t kf_launch_gated_act_q8(const float* gate, const float* up, int stride, int act_fn, void* act, int rows, int n, int kind,
                                  hipStream_t s);
hipError_t kf_launch_gemv1(uint32_t ty, const void* w, int64_t row_bytes, const int8_t* xq, const int32_t* xs32, const float* xd32,
                           const float* bias, const float* res, float* y, int n, int n_out, int maxit, const KfSegs* segs, hipStream_t s);
hipError_t kf_launch_block_ints(uint32_t ty, const void* w, int64_t row_bytes, const void* act, int rows, int n, int n_out,
                                int32_t* out, hipStream_t s);
bool kf_rows_mma_1_ok(uint32_t ty, const void* w, int64_t row_bytes, int n, int n_out, int rows);
hipError_t kf_launch_rows_mma_1(uint32_t ty, const void* w, int64_t row_bytes, const int8_t* xq, const int32_t* xs32, const float* xd32, int n,
                                int n_out, int rows, const float* bias, const float* res, float* y, hipStream_t s);
hipError_t kf_launch_gemv1_fused(uint32_t ty, const void* w, int64_t row_bytes, const float* x, const float* bias, const float* res, float* y,
                                 int n, int n_out, const KfSegs* segs, hipStream_t s, const float* norm_w = nullptr, const float* norm_b = nullptr,
                                 float norm_eps = 0.0f, bool norm = false);
int kf_gemv_max_n();
hipError_t kf_launch_gemm_q8_0(const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y, int M,
                               int N, int K, hipStream_t s);
int kf_gemm_k_multiple();

bool kf_gemm_kq_ok(uint32_t ty, const void* w, int64_t row_bytes, int K, int N);
double kf_gemm_kq_sb_rounds(int M, int N, int K);
double kf_gemm_q4k_sb_rounds(int M, int N, int K);
hipError_t kf_launch_gemm_kq_moe(const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, int n_split, const void* act, int pairs,
                                 int n_slots, const int32_t* offsets, const int32_t* out_rows, float* y, int N, int K, hipStream_t s);
static bool q4k_gemm_kq_pays(int rows, int n_in, int n_out);
hipError_t kf_launch_gemm_kq(uint32_t ty, const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y,
                             int M, int N, int K, hipStream_t s);
hipError_t kf_launch_gemm_q4k(const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y, int M,
                              int N, int K, hipStream_t s);
int kf_rows_max_n(uint32_t ty);
hipError_t kf_launch_rows(uint32_t ty, const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, const void* act, int act_rows,
                          int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used, int per_slot,
                          const float* bias, const float* res, float* y, hipStream_t s);
hipError_t kf_launch_moe_group(const int32_t* slots, int total, int n_slots, int32_t* order, int32_t* offsets, hipStream_t s);
hipError_t kf_launch_moe_gather_act(const void* src, int src_rows, void* dst, int pairs, const int32_t* order, const int32_t* offsets,
                                    int n_slots, int n_used, int n, hipStream_t s);
hipError_t kf_launch_gemm_q4k_moe(const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, int n_split, const void* act,
                                  int pairs, int n_slots, const int32_t* offsets, const int32_t* out_rows, float* y, int N, int K,
                                  hipStream_t s);
hipError_t kf_launch_moe_combine(const float* part, const float* wts, const int32_t* slots, const float* host, float* out, int rows, int n_used,
                                 int n_embd, float scale, int n_slots, hipStream_t s);

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) { return fail(KF_E_HIP, "%s: %s", what, hipGetErrorString(e)); }

}  // namespace

// The thread's last error, for the other translation units of the library (gguf.cpp)
void kf_set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}

namespace {

bool type_info(uint32_t ty, int& block, int& bytes) {
    if (ty == KF_TYPE_Q8_0) {
        block = KF_Q8_0_BLOCK;
        bytes = KF_Q8_0_BYTES;
        return true;
    }
    if (ty == KF_TYPE_Q4_K || ty == KF_TYPE_Q5_K || ty == KF_TYPE_Q6_K) {
        block = KF_Q4_K_BLOCK;
        bytes = ty == KF_TYPE_Q4_K ? KF_Q4_K_BYTES : ty == KF_TYPE_Q5_K ? KF_Q5_K_BYTES : KF_Q6_K_BYTES;
        return true;
    }
    return false;
}

int kind_of(uint32_t ty) { return ty == KF_TYPE_Q8_0 ? KF_ACT_Q8_0 : KF_ACT_Q8K; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Row iterations per GEMV block (1, 2 or 4); KF_GEMV_MAXIT overrides the built-in choice (a tuning knob, like the
// reference's KF_* environment knobs)
int gemv_maxit() {
    return kf_knob_or(KF_KNOB_GEMV_MAXIT, 0);
}

// KF_MATMUL_NO_FUSE set: one-row matmuls quantize into `act` and run the GEMV as two launches (a comparison knob)
bool no_fusion() { return kf_knob_on(KF_KNOB_MATMUL_NO_FUSE); }

int product(uint32_t ty, const void* w, int64_t rb, const void* act, const float* bias, const float* res, float* y, int rows, int n_in,
            int n_out, void* stream);

int check_product(uint32_t ty, const void* w, int64_t row_bytes, const void* act, float* y, int rows, int n, int n_out) {
    int block, bytes;
    if (!type_info(ty, block, bytes)) return fail(KF_E_UNSUPPORTED, "ggml type %u is not on the int8 path (q8_0=8, q4_K=12, q5_K=13, q6_K=14)", ty);
    if (n <= 0 || n % block != 0) return fail(KF_E_INVALID, "%d columns against blocks of %d", n, block);
    if (rows < 1) return fail(KF_E_INVALID, "%d activation rows", rows);
    if (n_out < 0) return fail(KF_E_INVALID, "%d output rows", n_out);
    if (row_bytes != (int64_t)(n / block) * bytes)
        return fail(KF_E_INVALID, "row_bytes %lld for %d columns of type %u, want %lld", (long long)row_bytes, n, ty,
                    (long long)(n / block) * bytes);
    if (!w || !act || !y) return fail(KF_E_INVALID, "null weight, activation or output pointer");
    if (!aligned(w, 16)) return fail(KF_E_INVALID, "weight base must be 16-byte aligned");
    if (!aligned(act, KF_ACT_ALIGN)) return fail(KF_E_INVALID, "activation scratch must be %d-byte aligned", KF_ACT_ALIGN);
    return KF_OK;
}

}  // namespace

extern "C" {

int kf_hip_abi_version(void) { return KF_HIP_ABI_VERSION; }

const char* kf_hip_last_error(void) { return g_err.c_str(); }

size_t kf_hip_act_bytes(int rows, int n) {
    if (rows < 0 || n < 0) return 0;
    return kf_act_layout((size_t)rows, (size_t)n).total;
}

void kf_hip_act_offsets(int rows, int n, size_t out[6]) {
    const kf_act_offsets o = kf_act_layout((size_t)(rows < 0 ? 0 : rows), (size_t)(n < 0 ? 0 : n));
    out[0] = o.q;
    out[1] = o.d16;
    out[2] = o.s16;
    out[3] = o.d32;
    out[4] = o.s32;
    out[5] = o.xa;
}

int kf_hip_act_kind(uint32_t ty) {
    int block, bytes;
    if (!type_info(ty, block, bytes)) return fail(KF_E_UNSUPPORTED, "ggml type %u is not on the int8 path", ty);
    return kind_of(ty);
}

int kf_hip_quant_act(const float* x, void* act, int rows, int n, int kind, void* stream) {
    if (kind != KF_ACT_Q8_0 && kind != KF_ACT_Q8K) return fail(KF_E_UNSUPPORTED, "activation kind %d (3=Q8_0, 4=Q8K)", kind);
    const int block = kind == KF_ACT_Q8_0 ? 32 : 256;
    if (rows < 1 || n <= 0 || n % block != 0) return fail(KF_E_INVALID, "%d rows of %d columns for blocks of %d", rows, n, block);
    if (!x || !act) return fail(KF_E_INVALID, "null activation pointer");
    if (!aligned(x, 16) || !aligned(act, KF_ACT_ALIGN)) return fail(KF_E_INVALID, "x must be 16-byte and act 256-byte aligned");
    const hipError_t e = kf_launch_quant_act(x, act, rows, n, kind, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "quant_act launch");
}

// Shared checks of the fused producers: kind, widths, alignment of the f32 inputs (16 bytes) and of the scratch
static int check_producer(int kind, int rows, int n, const void* act) {
    if (kind != KF_ACT_Q8_0 && kind != KF_ACT_Q8K) return fail(KF_E_UNSUPPORTED, "activation kind %d (3=Q8_0, 4=Q8K)", kind);
    const int block = kind == KF_ACT_Q8_0 ? 32 : 256;
    if (rows < 1 || n <= 0 || n % block != 0) return fail(KF_E_INVALID, "%d rows of %d columns for blocks of %d", rows, n, block);
    if (!act || !aligned(act, KF_ACT_ALIGN)) return fail(KF_E_INVALID, "act must be a 256-byte aligned device pointer");
    return KF_OK;
}

int kf_hip_rms_norm_q8(const float* x, const float* w, const float* b, int rows, int n, float eps, int kind, void* act, void* stream) {
    const int rc = check_producer(kind, rows, n, act);
    if (rc != KF_OK) return rc;
    if (!x || !aligned(x, 16) || (w && !aligned(w, 16)) || (b && !aligned(b, 16)))
        return fail(KF_E_INVALID, "x (and w, b when given) must be 16-byte aligned device pointers");
    if (!(eps >= 0.0f)) return fail(KF_E_INVALID, "eps %g", (double)eps);
    const hipError_t e = kf_launch_rms_norm_q8(x, w, b, eps, act, rows, n, kind, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "rms_norm_q8 launch");
}

int kf_hip_gated_act_q8(const float* gate, const float* up, int rows, int n, int stride, int act_fn, int kind, void* act, void* stream) {
    const int rc = check_producer(kind, rows, n, act);
    if (rc != KF_OK) return rc;
    if (act_fn != KF_GLU_SILU && act_fn != KF_GLU_RELU && act_fn != KF_GLU_RELU_SQR)
        return fail(KF_E_UNSUPPORTED, "activation %d (0 silu, 2 relu, 4 relu squared)", act_fn);
    if (!gate || !up || !aligned(gate, 16) || !aligned(up, 16)) return fail(KF_E_INVALID, "gate and up must be 16-byte aligned device pointers");
    if (stride < n || stride % 4 != 0) return fail(KF_E_INVALID, "row stride %d for %d columns (a multiple of 4, at least n)", stride, n);
    const hipError_t e = kf_launch_gated_act_q8(gate, up, stride, act_fn, act, rows, n, kind, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "gated_act_q8 launch");
}

int kf_hip_gemv(uint32_t ty, const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y, int rows,
                int n, int n_out, void* stream) {
    const int rc = check_product(ty, w, row_bytes, act, y, rows, n, n_out);
    if (rc != KF_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // q5_K / q6_K: several rows on the matrix cores (16 activation rows a weight pass), one row (or a layout the
    // matrix-core form does not take: q6_K rows with an odd number of super-blocks) on their own per-lane product
    if ((ty == KF_TYPE_Q5_K || ty == KF_TYPE_Q6_K) && rows > 1 && !kf_knob_on(KF_KNOB_ROWS_VALU) && kf_rows_mma_1_ok(ty, w, row_bytes, n, n_out, rows)) {
        const kf_act_offsets o = kf_act_layout((size_t)rows, (size_t)n);
        const char* base = static_cast<const char*>(act);
        const hipError_t e = kf_launch_rows_mma_1(ty, w, row_bytes, reinterpret_cast<const int8_t*>(base + o.q), reinterpret_cast<const int32_t*>(base + o.s32),
                                                  reinterpret_cast<const float*>(base + o.d32), n, n_out, rows, bias, res, y, s);
        return e == hipSuccess ? KF_OK : hip_fail(e, "q5_K/q6_K multi-row product launch");
    }
    if (ty == KF_TYPE_Q5_K || ty == KF_TYPE_Q6_K) {
        const hipError_t e = kf_launch_gemv_k(ty, w, row_bytes, act, bias, res, y, rows, n, n_out, s);
        return e == hipSuccess ? KF_OK : hip_fail(e, "q5_K/q6_K product launch");
    }
    if (n > kf_gemv_max_n()) return fail(KF_E_UNSUPPORTED, "%d columns above the %d the GEMV stages in LDS", n, kf_gemv_max_n());
    const kf_act_offsets o = kf_act_layout((size_t)rows, (size_t)n);
    const char* base = static_cast<const char*>(act);
    // several rows: each weight row streamed once against up to eight staged activation rows
    if (rows > 1 && n <= kf_rows_max_n(ty)) {
        const hipError_t e = kf_launch_rows(ty, w, nullptr, 0, row_bytes, act, rows, n, n_out, nullptr, nullptr, 1, rows, 1, 1, bias, res, y, s);
        return e == hipSuccess ? KF_OK : hip_fail(e, "rows launch");
    }
    for (int r = 0; r < rows; r++) {
        const int8_t* xq = reinterpret_cast<const int8_t*>(base + o.q) + (size_t)r * n;
        const int32_t* xs32 = reinterpret_cast<const int32_t*>(base + o.s32) + (size_t)r * (n / 32);
        const float* xd32 = reinterpret_cast<const float*>(base + o.d32) + (size_t)r * (n / 32);
        const hipError_t e = kf_launch_gemv1(ty, w, row_bytes, xq, xs32, xd32, bias, res ? res + (size_t)r * n_out : nullptr,
                                             y + (size_t)r * n_out, n, n_out, gemv_maxit(), nullptr, s);
        if (e != hipSuccess) return hip_fail(e, "gemv launch");
    }
    return KF_OK;
}

int kf_hip_gemm_i8(uint32_t ty, const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y,
                   int rows, int n, int n_out, void* stream) {
    const int rc = check_product(ty, w, row_bytes, act, y, rows, n, n_out);
    if (rc != KF_OK) return rc;
    if (ty == KF_TYPE_Q4_K) {
        if (q4k_gemm_kq_pays(rows, n, n_out) && kf_gemm_kq_ok(ty, w, row_bytes, n, n_out)) {
            const hipError_t e = kf_launch_gemm_kq(ty, w, row_bytes, act, bias, res, y, rows, n_out, n, static_cast<hipStream_t>(stream));
            return e == hipSuccess ? KF_OK : hip_fail(e, "gemm launch");
        }
        const hipError_t e = kf_launch_gemm_q4k(w, row_bytes, act, bias, res, y, rows, n_out, n, static_cast<hipStream_t>(stream));
        return e == hipSuccess ? KF_OK : hip_fail(e, "gemm launch");
    }
    if (ty == KF_TYPE_Q5_K || ty == KF_TYPE_Q6_K) {
        if (!kf_gemm_kq_ok(ty, w, row_bytes, n, n_out))
            return fail(KF_E_UNSUPPORTED, "the q5_K/q6_K GEMM needs 16-byte aligned weights and rows (q6_K: %d columns, a multiple of 2048) and a matrix below 2 GB; kf_hip_gemv takes any", n);
        const hipError_t e = kf_launch_gemm_kq(ty, w, row_bytes, act, bias, res, y, rows, n_out, n, static_cast<hipStream_t>(stream));
        return e == hipSuccess ? KF_OK : hip_fail(e, "gemm launch");
    }
    if (ty != KF_TYPE_Q8_0) return fail(KF_E_UNSUPPORTED, "the int8 GEMM runs q8_0, q4_K, q5_K and q6_K weights (type %u given)", ty);
    if (n % kf_gemm_k_multiple() != 0) return fail(KF_E_INVALID, "%d columns, the GEMM needs a multiple of %d", n, kf_gemm_k_multiple());
    const hipError_t e = kf_launch_gemm_q8_0(w, row_bytes, act, bias, res, y, rows, n_out, n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "gemm launch");
}

int kf_hip_matmul(uint32_t ty, const void* w, int n_in, int n_out, const float* x, int rows, void* act, const float* bias,
                  const float* res, float* y, void* stream) {
    int block, bytes;
    if (!type_info(ty, block, bytes)) return fail(KF_E_UNSUPPORTED, "ggml type %u is not on the int8 path (q8_0=8, q4_K=12, q5_K=13, q6_K=14)", ty);
    if (n_in <= 0 || n_in % block != 0) return fail(KF_E_INVALID, "%d columns against blocks of %d", n_in, block);
    const int64_t rb = (int64_t)(n_in / block) * bytes;
    const int rc = check_product(ty, w, rb, act, y, rows, n_in, n_out);
    if (rc != KF_OK) return rc;
    if (rows == 1 && x && !no_fusion()) {
        // one launch: the GEMV quantizes its activation row itself
        const hipError_t e = kf_launch_gemv1_fused(ty, w, rb, x, bias, res, y, n_in, n_out, nullptr, static_cast<hipStream_t>(stream));
        if (e == hipSuccess) return KF_OK;
        if (e != hipErrorNotSupported) return hip_fail(e, "fused gemv launch");
    }
    const int q = kf_hip_quant_act(x, act, rows, n_in, kind_of(ty), stream);
    if (q != KF_OK) return q;
    return product(ty, w, rb, act, bias, res, y, rows, n_in, n_out, stream);
}

int kf_hip_rms_norm_matmul(uint32_t ty, const void* w, int n_in, int n_out, const float* x, int rows, const float* norm_w, const float* norm_b,
                           float eps, void* act, const float* bias, const float* res, float* y, void* stream) {
    int block, bytes;
    if (!type_info(ty, block, bytes)) return fail(KF_E_UNSUPPORTED, "ggml type %u is not on the int8 path (q8_0=8, q4_K=12, q5_K=13, q6_K=14)", ty);
    if (n_in <= 0 || n_in % block != 0) return fail(KF_E_INVALID, "%d columns against blocks of %d", n_in, block);
    const int64_t rb = (int64_t)(n_in / block) * bytes;
    const int rc = check_product(ty, w, rb, act, y, rows, n_in, n_out);
    if (rc != KF_OK) return rc;
    if (!x || !aligned(x, 16) || (norm_w && !aligned(norm_w, 16)) || (norm_b && !aligned(norm_b, 16)))
        return fail(KF_E_INVALID, "x (and norm_w, norm_b when given) must be 16-byte aligned device pointers");
    if (!(eps >= 0.0f)) return fail(KF_E_INVALID, "eps %g", (double)eps);
    if (rows == 1 && !no_fusion()) {
        // one launch: every block of the GEMV normalises and quantizes the row itself
        const hipError_t e = kf_launch_gemv1_fused(ty, w, rb, x, bias, res, y, n_in, n_out, nullptr, static_cast<hipStream_t>(stream), norm_w,
                                                   norm_b, eps, true);
        if (e == hipSuccess) return KF_OK;
        if (e != hipErrorNotSupported) return hip_fail(e, "fused rms_norm gemv launch");
    }
    const int q = kf_hip_rms_norm_q8(x, norm_w, norm_b, rows, n_in, eps, kind_of(ty), act, stream);
    if (q != KF_OK) return q;
    return product(ty, w, rb, act, bias, res, y, rows, n_in, n_out, stream);
}

}  // extern "C"

// q4_K GEMM costs (MI355X, Llama-3-8B QKV / O / gate / down shapes at 32-2048 rows, least squares over the rounds each
// launcher plans): the split-scale kernel (gemm_q4k.hip, 128 x 256 tiles, two K halves for a half-full last round)
// about 7.4 us plus 4.84 us per super-block of its rounds; the one-MFMA-per-group kernel (gemm_kq.hip, 64 x 256
// tiles, 2-4 K ranges for a half-full last round) 13.2 us plus 2.95 us. The first wins where its rounds are full
// (gate from about 384 rows, down from 768), the second on smaller grids.
static double q4k_gemm_us(int rows, int n_in, int n_out, bool kq) {
    return kq ? 13.2 + 2.95 * kf_gemm_kq_sb_rounds(rows, n_out, n_in) : 7.4 + 4.84 * kf_gemm_q4k_sb_rounds(rows, n_out, n_in);
}

// Which q4_K GEMM kf_hip_gemm_i8 runs: the one-MFMA-per-group kernel where it costs less (KF_Q4K_KQ=0 / 1 forces the
// choice, a comparison knob)
static bool q4k_gemm_kq_pays(int rows, int n_in, int n_out) {
    if (kf_knob_on(KF_KNOB_Q4K_KQ)) return kf_knob(KF_KNOB_Q4K_KQ) != 0;
    return q4k_gemm_us(rows, n_in, n_out, true) < q4k_gemm_us(rows, n_in, n_out, false);
}

// q4_K: whether the tile GEMM beats the few-row product. The few-row product streams the weights once per 16
// activation rows: about 0.28 us per MB and pass plus 1 us (fitted at the Llama shapes, 8-256 rows); the GEMM costs
// the cheaper of the two kernels above. Rows wider than the few-row product stages go one GEMV launch per row, so the
// GEMM takes them from 96 rows.
static bool q4k_gemm_pays(int rows, int n_in, int n_out, int64_t row_bytes) {
    if (rows < 2) return false;
    if (n_in > kf_rows_max_n(KF_TYPE_Q4_K)) return rows >= 96;
    const double mb = (double)n_out * row_bytes / 1e6;
    const double t_rows = ((rows + 15) / 16) * (0.28 * mb + 1.0);
    const double t_gemm = std::min(q4k_gemm_us(rows, n_in, n_out, true), q4k_gemm_us(rows, n_in, n_out, false));
    return t_gemm < t_rows;
}

// q5_K / q6_K: whether the tile GEMM beats the few-row product. The few-row product streams the weights once per 64
// activation rows, about 1.05 (q5_K) / 1.55 (q6_K) us per MB and pass; the GEMM costs about 14.5 us plus 3.23 / 5.72
// us per super-block of its rounds (kf_gemm_kq_sb_rounds: one 64 x 256 tile a CU a round, a last round at most half
// full split over 2 or 4 K ranges). Fitted on MI355X at the Llama-3-8B gate and down shapes, 32-512 rows: the model
// picks the faster product at every measured point. KF_KQ_GEMM=0 / 1 forces the choice (a comparison knob).
static bool kq_gemm_pays(uint32_t ty, int rows, int n_in, int n_out, int64_t row_bytes) {
    if (kf_knob_on(KF_KNOB_KQ_GEMM)) return kf_knob(KF_KNOB_KQ_GEMM) != 0;
    if (rows < 2) return false;
    const bool q6 = ty == KF_TYPE_Q6_K;
    const double mb = (double)n_out * row_bytes / 1e6;
    const double t_rows = rows / 64.0 * mb * (q6 ? 1.55 : 1.05);
    const double t_gemm = 14.5 + kf_gemm_kq_sb_rounds(rows, n_out, n_in) * (q6 ? 5.72 : 3.23);
    return t_gemm < t_rows;
}

namespace {

// The product of kf_hip_matmul once the activations are quantized
int product(uint32_t ty, const void* w, int64_t rb, const void* act, const float* bias, const float* res, float* y, int rows, int n_in,
            int n_out, void* stream) {
    // the row count picks the product, as matvec_rows / multi_kind do (exec.rs:1877-1945): one row is the GEMV;
    // several q8_0 rows are the int8 GEMM, which reads each weight byte once per 128 rows
    if (rows > 1 && ty == KF_TYPE_Q8_0 && n_in % kf_gemm_k_multiple() == 0 && n_out > 0)
        return kf_hip_gemm_i8(ty, w, rb, act, bias, res, y, rows, n_in, n_out, stream);
    if (ty == KF_TYPE_Q4_K && n_out > 0 && q4k_gemm_pays(rows, n_in, n_out, rb))
        return kf_hip_gemm_i8(ty, w, rb, act, bias, res, y, rows, n_in, n_out, stream);
    if ((ty == KF_TYPE_Q5_K || ty == KF_TYPE_Q6_K) && n_out > 0 && kq_gemm_pays(ty, rows, n_in, n_out, rb) && kf_gemm_kq_ok(ty, w, rb, n_in, n_out))
        return kf_hip_gemm_i8(ty, w, rb, act, bias, res, y, rows, n_in, n_out, stream);
    return kf_hip_gemv(ty, w, rb, act, bias, res, y, rows, n_in, n_out, stream);
}

// A grouped product's members from the reference's segment words (quant.cuh:301-305): per member the byte offsets of
// its weights from w and of its output, bias and residual from y (KF_SEG_NONE: none), its first stacked row and its
// row count. Members must be stacked in order without gaps.
struct Member {
    const uint8_t* w;
    float* y;
    const float* bias;
    const float* res;
    int start, n_out;
};

int unpack_segs(const void* w, float* y, const int64_t* segs, int nseg, std::vector<Member>& out, int& total) {
    if (!segs || nseg < 1 || nseg > KF_MAX_SEGS) return fail(KF_E_INVALID, "%d segments (1 to %d, non-null table)", nseg, KF_MAX_SEGS);
    if (!w || !y) return fail(KF_E_INVALID, "null leader weight or output pointer");
    out.clear();
    total = 0;
    char* yb = reinterpret_cast<char*>(y);
    for (int i = 0; i < nseg; i++) {
        const int64_t* e = segs + (size_t)i * KF_SEG_WORDS;
        if (e[0] == KF_SEG_NONE || e[1] == KF_SEG_NONE) return fail(KF_E_INVALID, "segment %d has no weights or output", i);
        if (e[4] != total) return fail(KF_E_INVALID, "segment %d starts at row %lld, want %d (members stacked in order)", i, (long long)e[4], total);
        if (e[5] < 1 || e[5] > (int64_t)0x7fffffff - total) return fail(KF_E_INVALID, "segment %d has %lld rows", i, (long long)e[5]);
        Member m;
        m.w = static_cast<const uint8_t*>(w) + e[0];
        m.y = reinterpret_cast<float*>(yb + e[1]);
        m.bias = e[2] == KF_SEG_NONE ? nullptr : reinterpret_cast<const float*>(yb + e[2]);
        m.res = e[3] == KF_SEG_NONE ? nullptr : reinterpret_cast<const float*>(yb + e[3]);
        m.start = total;
        m.n_out = (int)e[5];
        if (!aligned(m.w, 16)) return fail(KF_E_INVALID, "segment %d weights must be 16-byte aligned", i);
        if (!aligned(m.y, 4) || (m.bias && !aligned(m.bias, 4)) || (m.res && !aligned(m.res, 4)))
            return fail(KF_E_INVALID, "segment %d output, bias or residual not 4-byte aligned", i);
        total += m.n_out;
        out.push_back(m);
    }
    return KF_OK;
}

// The kernels' member table of a group
KfSegs seg_table(const std::vector<Member>& ms) {
    KfSegs sg{};
    sg.n = (int)ms.size();
    for (size_t i = 0; i < ms.size(); i++) {
        sg.start[i] = ms[i].start;
        sg.w[i] = ms[i].w;
        sg.y[i] = ms[i].y;
        sg.bias[i] = ms[i].bias;
        sg.res[i] = ms[i].res;
    }
    return sg;
}

// The grouped product over quantized activations: one GEMV launch over the stacked rows for one activation row of
// q8_0 / q4_K, otherwise each member's product against the shared activations
int group_product(uint32_t ty, const std::vector<Member>& ms, int64_t rb, const void* act, int rows, int n, int total, bool select,
                  void* stream) {
    if (rows == 1 && (ty == KF_TYPE_Q8_0 || ty == KF_TYPE_Q4_K) && n <= kf_gemv_max_n()) {
        const KfSegs sg = seg_table(ms);
        const kf_act_offsets o = kf_act_layout(1, (size_t)n);
        const char* base = static_cast<const char*>(act);
        const hipError_t e = kf_launch_gemv1(ty, ms[0].w, rb, reinterpret_cast<const int8_t*>(base + o.q), reinterpret_cast<const int32_t*>(base + o.s32),
                                             reinterpret_cast<const float*>(base + o.d32), nullptr, nullptr, ms[0].y, n, total, gemv_maxit(), &sg,
                                             static_cast<hipStream_t>(stream));
        return e == hipSuccess ? KF_OK : hip_fail(e, "grouped gemv launch");
    }
    for (const Member& m : ms) {
        const int rc = select ? product(ty, m.w, rb, act, m.bias, m.res, m.y, rows, n, m.n_out, stream)
                              : kf_hip_gemv(ty, m.w, rb, act, m.bias, m.res, m.y, rows, n, m.n_out, stream);
        if (rc != KF_OK) return rc;
    }
    return KF_OK;
}

}  // namespace

extern "C" {

int kf_hip_gemv_group(uint32_t ty, const void* w, int64_t row_bytes, const void* act, float* y, int rows, int n, const int64_t* segs, int nseg,
                      void* stream) {
    std::vector<Member> ms;
    int total = 0;
    int rc = unpack_segs(w, y, segs, nseg, ms, total);
    if (rc != KF_OK) return rc;
    rc = check_product(ty, w, row_bytes, act, y, rows, n, total);
    if (rc != KF_OK) return rc;
    return group_product(ty, ms, row_bytes, act, rows, n, total, false, stream);
}

int kf_hip_matmul_group(uint32_t ty, const void* w, int n_in, const float* x, int rows, void* act, float* y, const int64_t* segs, int nseg,
                        void* stream) {
    int block, bytes;
    if (!type_info(ty, block, bytes)) return fail(KF_E_UNSUPPORTED, "ggml type %u is not on the int8 path (q8_0=8, q4_K=12, q5_K=13, q6_K=14)", ty);
    if (n_in <= 0 || n_in % block != 0) return fail(KF_E_INVALID, "%d columns against blocks of %d", n_in, block);
    const int64_t rb = (int64_t)(n_in / block) * bytes;
    std::vector<Member> ms;
    int total = 0;
    int rc = unpack_segs(w, y, segs, nseg, ms, total);
    if (rc != KF_OK) return rc;
    rc = check_product(ty, w, rb, act, y, rows, n_in, total);
    if (rc != KF_OK) return rc;
    if (rows == 1 && x && !no_fusion()) {
        // one launch over the stacked rows, quantizing the activation row itself
        const KfSegs sg = seg_table(ms);
        const hipError_t e = kf_launch_gemv1_fused(ty, ms[0].w, rb, x, nullptr, nullptr, ms[0].y, n_in, total, &sg, static_cast<hipStream_t>(stream));
        if (e == hipSuccess) return KF_OK;
        if (e != hipErrorNotSupported) return hip_fail(e, "fused grouped gemv launch");
    }
    rc = kf_hip_quant_act(x, act, rows, n_in, kind_of(ty), stream);
    if (rc != KF_OK) return rc;
    return group_product(ty, ms, rb, act, rows, n_in, total, true, stream);
}

int kf_hip_moe_group(const int32_t* slots, int total, int n_slots, int32_t* order, int32_t* offsets, void* stream) {
    if (total < 0 || n_slots < 1) return fail(KF_E_INVALID, "%d pairs over %d slots", total, n_slots);
    if (n_slots > 4096) return fail(KF_E_UNSUPPORTED, "%d slots (at most 4096)", n_slots);
    if ((total > 0 && (!slots || !order)) || !offsets) return fail(KF_E_INVALID, "null slot, order or offset pointer");
    const hipError_t e = kf_launch_moe_group(slots, total, n_slots, order, offsets, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "moe_group launch");
}

int kf_hip_moe_gemv(uint32_t ty, const void* w, const void* w_up, int64_t expert_bytes, int64_t row_bytes, const void* act, int act_rows, int n,
                    int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int n_used, int per_slot, float* y, void* stream) {
    const int rc = check_product(ty, w, row_bytes, act, y, act_rows, n, n_out);
    if (rc != KF_OK) return rc;
    if (ty != KF_TYPE_Q8_0 && ty != KF_TYPE_Q4_K) return fail(KF_E_UNSUPPORTED, "grouped expert products run q8_0 and q4_K weights (type %u)", ty);
    if (w_up && !aligned(w_up, 16)) return fail(KF_E_INVALID, "up weight base must be 16-byte aligned");
    if (!order || !offsets || n_slots < 1 || n_used < 1) return fail(KF_E_INVALID, "null order/offsets or %d slots, %d used", n_slots, n_used);
    if (expert_bytes < (int64_t)n_out * row_bytes || expert_bytes % 16 != 0)
        return fail(KF_E_INVALID, "expert stride %lld for %d rows of %lld bytes (16-byte multiple)", (long long)expert_bytes, n_out, (long long)row_bytes);
    if (n > kf_rows_max_n(ty)) return fail(KF_E_UNSUPPORTED, "%d columns above the %d of the grouped product", n, kf_rows_max_n(ty));
    const hipError_t e = kf_launch_rows(ty, w, w_up, expert_bytes, row_bytes, act, act_rows, n, n_out, order, offsets, n_slots, 0, n_used,
                                        per_slot ? 1 : 0, nullptr, nullptr, y, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "moe product launch");
}

int kf_hip_moe_gemm(uint32_t ty, const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, int n_split, const void* act,
                    int pairs, int n, int n_out, const int32_t* offsets, int n_slots, const int32_t* out_rows, float* y, void* stream) {
    const int rc = check_product(ty, w, row_bytes, act, y, pairs, n, n_out);
    if (rc != KF_OK) return rc;
    if (ty != KF_TYPE_Q4_K) return fail(KF_E_UNSUPPORTED, "the grouped GEMM runs q4_K experts (type %u)", ty);
    if (n % 256 != 0) return fail(KF_E_INVALID, "%d columns, the grouped GEMM needs a multiple of 256", n);
    if (!offsets || n_slots < 1) return fail(KF_E_INVALID, "null offsets or %d slots", n_slots);
    const int mat_rows = w2 ? n_split : n_out;
    if (w2 && (n_split < 1 || n_split >= n_out || n_split % 256 != 0 || !aligned(w2, 16)))
        return fail(KF_E_INVALID, "split at column %d of %d (a multiple of 256 inside the output) or unaligned second matrix", n_split, n_out);
    if (expert_bytes < (int64_t)mat_rows * row_bytes || expert_bytes % 16 != 0)
        return fail(KF_E_INVALID, "expert stride %lld for %d rows of %lld bytes (16-byte multiple)", (long long)expert_bytes, mat_rows, (long long)row_bytes);
    // the one-MFMA-per-group kernel (64-row tiles: less of each slot's partial tile idle; 839 against 894 us for the
    // split-scale kernel at 512 tokens top-2 over 8 experts) unless KF_MOE_KQ=0 (a comparison knob)
    const bool kq = kf_knob(KF_KNOB_MOE_KQ) != 0 && row_bytes % 16 == 0 && aligned(w, 16);
    const hipError_t e = kq ? kf_launch_gemm_kq_moe(w, w2, expert_bytes, row_bytes, w2 ? n_split : 0, act, pairs, n_slots, offsets, out_rows, y,
                                                    n_out, n, static_cast<hipStream_t>(stream))
                            : kf_launch_gemm_q4k_moe(w, w2, expert_bytes, row_bytes, w2 ? n_split : 0, act, pairs, n_slots, offsets, out_rows, y,
                                                     n_out, n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "grouped GEMM launch");
}

int kf_hip_moe_combine(const float* part, const float* wts, const int32_t* slots, const float* host, float* out, int rows, int n_used, int n_embd,
                       float scale, void* stream) {
    if (rows < 0 || n_used < 1 || n_embd < 0) return fail(KF_E_INVALID, "%d rows, %d used, %d columns", rows, n_used, n_embd);
    if (rows > 0 && n_embd > 0 && (!part || !wts || !slots || !out)) return fail(KF_E_INVALID, "null combine pointer");
    // every pair with a slot >= 0 has a part row: the caller wrote them
    const hipError_t e = kf_launch_moe_combine(part, wts, slots, host, out, rows, n_used, n_embd, scale, INT_MAX, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "moe_combine launch");
}

namespace {
// Scratch of one MoE layer: x activations | order | offsets | hidden f32 | hidden activations | pair outputs, and for
// the grouped GEMM the pairs' activation rows in group order; hidden holds [pairs][2 n_ff] (gate | up for the GEMM)
struct MoeScratch {
    size_t xact, order, offsets, hidden, hact, part, xg, total;
};
MoeScratch moe_scratch(int rows, int n_used, int n_embd, int n_ff, int n_slots) {
    MoeScratch m{};
    const size_t pairs = (size_t)rows * n_used;
    size_t at = 0;
    m.xact = at;
    at += kf_align_up(kf_act_layout((size_t)rows, (size_t)n_embd).total, 256);
    m.order = at;
    at += kf_align_up(pairs * 4, 256);
    m.offsets = at;
    at += kf_align_up(((size_t)n_slots + 1) * 4, 256);
    m.hidden = at;
    at += kf_align_up(pairs * n_ff * 2 * 4, 256);
    m.hact = at;
    at += kf_align_up(kf_act_layout(pairs, (size_t)n_ff).total, 256);
    m.part = at;
    at += kf_align_up(pairs * n_embd * 4, 256);
    m.xg = at;
    at += kf_align_up(kf_act_layout(pairs, (size_t)n_embd).total, 256);
    m.total = at;
    return m;
}

// Routed pairs past which the q4_K expert products run as the grouped tile GEMM (each expert's weights read once per
// 128 pairs) instead of the few-row product (once per 16); the reference switches to its tensor-core GEMM past
// MOE_MATVEC_ROWS = 64 pairs (crates/kf-backend-cuda/src/exec.rs:2196)
constexpr int KF_MOE_GEMM_PAIRS = 64;
}  // namespace

size_t kf_hip_moe_scratch_bytes(int rows, int n_used, int n_embd, int n_ff, int n_slots) {
    if (rows < 0 || n_used < 1 || n_embd < 0 || n_ff < 0 || n_slots < 1) return 0;
    return moe_scratch(rows, n_used, n_embd, n_ff, n_slots).total;
}

int kf_hip_moe_ffn(uint32_t ty, const void* gate, const void* up, const void* down, int n_slots, int n_embd, int n_ff, const float* x, int rows,
                   const int32_t* sel, const float* wts, int n_used, float scale, void* scratch, size_t scratch_bytes, float* out, void* stream) {
    int block, bytes;
    if (!type_info(ty, block, bytes)) return fail(KF_E_UNSUPPORTED, "ggml type %u is not on the int8 path (q8_0=8, q4_K=12, q5_K=13, q6_K=14)", ty);
    if (ty != KF_TYPE_Q8_0 && ty != KF_TYPE_Q4_K) return fail(KF_E_UNSUPPORTED, "the MoE layer runs q8_0 and q4_K experts (type %u)", ty);
    if (rows < 1 || n_used < 1 || n_slots < 1) return fail(KF_E_INVALID, "%d rows, %d used of %d slots", rows, n_used, n_slots);
    if (n_embd <= 0 || n_ff <= 0 || n_embd % block != 0 || n_ff % block != 0) return fail(KF_E_INVALID, "%d / %d columns against blocks of %d", n_embd, n_ff, block);
    if (!gate || !up || !down || !x || !sel || !wts || !scratch || !out) return fail(KF_E_INVALID, "null MoE pointer");
    const MoeScratch m = moe_scratch(rows, n_used, n_embd, n_ff, n_slots);
    if (scratch_bytes < m.total) return fail(KF_E_INVALID, "scratch of %zu bytes, the layer needs %zu", scratch_bytes, m.total);
    if (!aligned(scratch, 256)) return fail(KF_E_INVALID, "scratch must be 256-byte aligned");
    const int64_t rb_in = (int64_t)(n_embd / block) * bytes, rb_ff = (int64_t)(n_ff / block) * bytes;
    const int64_t eb_gu = kf_align_up((size_t)(n_ff * rb_in), 16), eb_dn = kf_align_up((size_t)(n_embd * rb_ff), 16);
    if (eb_gu != (int64_t)n_ff * rb_in || eb_dn != (int64_t)n_embd * rb_ff)
        return fail(KF_E_UNSUPPORTED, "expert matrices must be whole multiples of 16 bytes");
    char* base = static_cast<char*>(scratch);
    void* xact = base + m.xact;
    auto* order = reinterpret_cast<int32_t*>(base + m.order);
    auto* offsets = reinterpret_cast<int32_t*>(base + m.offsets);
    auto* hidden = reinterpret_cast<float*>(base + m.hidden);
    void* hact = base + m.hact;
    auto* part = reinterpret_cast<float*>(base + m.part);
    const int pairs = rows * n_used;
    int rc = kf_hip_quant_act(x, xact, rows, n_embd, kind_of(ty), stream);
    if (rc == KF_OK) rc = kf_hip_moe_group(sel, pairs, n_slots, order, offsets, stream);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (rc == KF_OK && ty == KF_TYPE_Q4_K && pairs > KF_MOE_GEMM_PAIRS && n_embd % 256 == 0 && n_ff % 256 == 0) {
        // many pairs: the grouped GEMM (the reference's expert_gemm_chunks, exec.rs:2196-2237). The pairs' activation
        // rows in group order; gate and up as one product of 2 n_ff columns; the gated activation quantized; down
        // written to each pair's row; the weighted combine
        void* xg = base + m.xg;
        hipError_t e = kf_launch_moe_gather_act(xact, rows, xg, pairs, order, offsets, n_slots, n_used, n_embd, st);
        if (e != hipSuccess) return hip_fail(e, "moe gather launch");
        rc = kf_hip_moe_gemm(ty, gate, up, eb_gu, rb_in, n_ff, xg, pairs, n_embd, 2 * n_ff, offsets, n_slots, nullptr, hidden, stream);
        if (rc == KF_OK) rc = kf_hip_gated_act_q8(hidden, hidden + n_ff, pairs, n_ff, 2 * n_ff, KF_GLU_SILU, kind_of(ty), hact, stream);
        if (rc == KF_OK) rc = kf_hip_moe_gemm(ty, down, nullptr, eb_dn, rb_ff, 0, hact, pairs, n_ff, n_embd, offsets, n_slots, order, part, stream);
        if (rc != KF_OK) return rc;
        e = kf_launch_moe_combine(part, wts, sel, nullptr, out, rows, n_used, n_embd, scale, n_slots, st);
        return e == hipSuccess ? KF_OK : hip_fail(e, "moe_combine launch");
    }
    if (rc == KF_OK)
        rc = kf_hip_moe_gemv(ty, gate, up, eb_gu, rb_in, xact, rows, n_embd, n_ff, order, offsets, n_slots, n_used, 0, hidden, stream);
    if (rc == KF_OK) rc = kf_hip_quant_act(hidden, hact, pairs, n_ff, kind_of(ty), stream);
    if (rc == KF_OK) rc = kf_hip_moe_gemv(ty, down, nullptr, eb_dn, rb_ff, hact, pairs, n_ff, n_embd, order, offsets, n_slots, n_used, 1, part, stream);
    // moe_group skips pairs whose slot is n_slots or more, so their part rows are never written: the combine skips them
    // too rather than reading stale scratch
    if (rc == KF_OK) {
        const hipError_t e = kf_launch_moe_combine(part, wts, sel, nullptr, out, rows, n_used, n_embd, scale, n_slots, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) rc = hip_fail(e, "moe_combine launch");
    }
    return rc;
}

int kf_hip_block_ints(uint32_t ty, const void* w, int64_t row_bytes, const void* act, int rows, int n, int n_out, int32_t* out,
                      void* stream) {
    const int rc = check_product(ty, w, row_bytes, act, reinterpret_cast<float*>(out), rows, n, n_out);
    if (rc != KF_OK) return rc;
    const hipError_t e = kf_launch_block_ints(ty, w, row_bytes, act, rows, n, n_out, out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "block_ints launch");
}

int kf_hip_stream_read(const void* buf, size_t bytes, int per_thread, uint32_t* sink, void* stream) {
    if (!buf || !sink) return fail(KF_E_INVALID, "null buffer or sink");
    if (reinterpret_cast<uintptr_t>(buf) % 16 != 0 || bytes % 16 != 0 || bytes == 0 || bytes >= (1ull << 36))
        return fail(KF_E_INVALID, "%zu bytes at a %s address: the probe reads 16-byte aligned pieces, below 64 GB", bytes,
                    reinterpret_cast<uintptr_t>(buf) % 16 ? "misaligned" : "16-byte aligned");
    if (per_thread != 4 && per_thread != 8 && per_thread != 16) return fail(KF_E_INVALID, "%d pieces a thread (4, 8 or 16)", per_thread);
    const hipError_t e = kf_launch_stream_read(buf, bytes, per_thread, sink, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KF_OK : hip_fail(e, "stream_read launch");
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------ backend mirror

struct kf_hip_weight {
    uint32_t ty;
    std::vector<int64_t> dims;
    void* dev;
    size_t nbytes;
};

struct kf_hip_backend {
    int device;
    hipStream_t stream;
    std::vector<kf_hip_weight> weights;
    void* scratch = nullptr;  // x | act | y, grown on demand (the per-graph pool of exec.rs:603-711, reduced to one op)
    size_t scratch_bytes = 0;
};

namespace {

int ensure_scratch(kf_hip_backend* b, size_t need) {
    if (need <= b->scratch_bytes) return KF_OK;
    if (b->scratch) hipFree(b->scratch);
    b->scratch = nullptr;
    b->scratch_bytes = 0;
    const hipError_t e = hipMalloc(&b->scratch, need);
    if (e != hipSuccess) return fail(KF_E_NOMEM, "scratch of %zu bytes: %s", need, hipGetErrorString(e));
    b->scratch_bytes = need;
    return KF_OK;
}

int backend_matmul(kf_hip_backend* b, int wid, int index, const float* x, int rows, int cols, const float* bias, float* y) {
    if (!b) return fail(KF_E_INVALID, "null backend");
    if (wid < 0 || wid >= (int)b->weights.size()) return fail(KF_E_INVALID, "weight id %d of %zu", wid, b->weights.size());
    const kf_hip_weight& w = b->weights[wid];
    const int64_t n_in = w.dims[0];
    const int64_t n_out = w.dims.size() > 1 ? w.dims[1] : 1;
    int64_t n_slices = 1;
    for (size_t i = 2; i < w.dims.size(); i++) n_slices *= w.dims[i];
    if (cols != n_in) return fail(KF_E_INVALID, "%d columns against %lld inputs", cols, (long long)n_in);
    if (index < 0 || index >= n_slices) return fail(KF_E_INVALID, "slice %d of %lld", index, (long long)n_slices);
    if (rows < 0 || (rows > 0 && (!x || !y))) return fail(KF_E_INVALID, "null rows");
    if (rows == 0 || n_out == 0) return KF_OK;
    int block, bytes;
    type_info(w.ty, block, bytes);
    const int64_t rb = n_in / block * bytes;
    const size_t xb = kf_align_up(sizeof(float) * (size_t)rows * n_in, 256);
    const size_t ab = kf_act_layout((size_t)rows, (size_t)n_in).total;
    const size_t yb = kf_align_up(sizeof(float) * (size_t)rows * n_out, 256);
    const size_t bb = bias ? kf_align_up(sizeof(float) * (size_t)n_out, 256) : 0;
    int rc = ensure_scratch(b, xb + ab + yb + bb);
    if (rc != KF_OK) return rc;
    char* base = static_cast<char*>(b->scratch);
    float* dx = reinterpret_cast<float*>(base);
    void* act = base + xb;
    float* dy = reinterpret_cast<float*>(base + xb + ab);
    float* dbias = bias ? reinterpret_cast<float*>(base + xb + ab + yb) : nullptr;
    hipError_t e = hipMemcpyAsync(dx, x, sizeof(float) * (size_t)rows * n_in, hipMemcpyHostToDevice, b->stream);
    if (e == hipSuccess && bias) e = hipMemcpyAsync(dbias, bias, sizeof(float) * (size_t)n_out, hipMemcpyHostToDevice, b->stream);
    if (e != hipSuccess) return hip_fail(e, "copy of the input rows");
    const char* wslice = static_cast<const char*>(w.dev) + (size_t)index * n_out * rb;
    rc = kf_hip_matmul(w.ty, wslice, (int)n_in, (int)n_out, dx, rows, act, dbias, nullptr, dy, b->stream);
    if (rc != KF_OK) return rc;
    e = hipMemcpyAsync(y, dy, sizeof(float) * (size_t)rows * n_out, hipMemcpyDeviceToHost, b->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(b->stream);
    return e == hipSuccess ? KF_OK : hip_fail(e, "matmul");
}

}  // namespace

extern "C" {

kf_hip_backend* kf_hip_backend_new(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || device < 0 || device >= count) {
        fail(KF_E_INVALID, "device %d of %d", device, count);
        return nullptr;
    }
    e = hipSetDevice(device);
    if (e != hipSuccess) {
        hip_fail(e, "hipSetDevice");
        return nullptr;
    }
    hipStream_t s;
    e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
        hip_fail(e, "hipStreamCreate");
        return nullptr;
    }
    kf_hip_backend* b = new kf_hip_backend;
    b->device = device;
    b->stream = s;
    return b;
}

void kf_hip_backend_free(kf_hip_backend* b) {
    if (!b) return;
    hipSetDevice(b->device);
    hipStreamSynchronize(b->stream);
    for (auto& w : b->weights) hipFree(w.dev);
    if (b->scratch) hipFree(b->scratch);
    hipStreamDestroy(b->stream);
    delete b;
}

int kf_hip_backend_add_weight(kf_hip_backend* b, uint32_t ty, const int64_t* dims, int ndims, const void* bytes, size_t nbytes) {
    if (!b) return fail(KF_E_INVALID, "null backend");
    int block, bsz;
    if (!type_info(ty, block, bsz)) return fail(KF_E_UNSUPPORTED, "ggml type %u is not on the int8 path", ty);
    if (!dims || ndims < 1 || !bytes) return fail(KF_E_INVALID, "null dims or bytes");
    int64_t rows = 1;
    for (int i = 1; i < ndims; i++) {
        if (dims[i] < 0) return fail(KF_E_INVALID, "negative dim");
        rows *= dims[i];
    }
    if (dims[0] <= 0 || dims[0] % block != 0) return fail(KF_E_INVALID, "%lld columns against blocks of %d", (long long)dims[0], block);
    const size_t want = (size_t)(dims[0] / block) * bsz * (size_t)rows;
    if (nbytes != want) return fail(KF_E_INVALID, "%zu bytes for a tensor of %zu", nbytes, want);
    hipSetDevice(b->device);
    void* dev = nullptr;
    // 16 spare bytes past the tensor, as the reference's ensure_weight keeps (exec.rs:1347-1359)
    hipError_t e = hipMalloc(&dev, nbytes + 16);
    if (e != hipSuccess) return fail(KF_E_NOMEM, "weight of %zu bytes: %s", nbytes, hipGetErrorString(e));
    e = hipMemcpy(dev, bytes, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(static_cast<char*>(dev) + nbytes, 0, 16);
    if (e != hipSuccess) {
        hipFree(dev);
        return hip_fail(e, "weight upload");
    }
    b->weights.push_back(kf_hip_weight{ty, std::vector<int64_t>(dims, dims + ndims), dev, nbytes});
    return (int)b->weights.size() - 1;
}

int kf_hip_backend_matmul(kf_hip_backend* b, int wid, const float* x, int rows, int cols, const float* bias, float* y) {
    if (b) hipSetDevice(b->device);
    return backend_matmul(b, wid, 0, x, rows, cols, bias, y);
}

int kf_hip_backend_matmul_slice(kf_hip_backend* b, int wid, int index, const float* x, int rows, int cols, float* y) {
    if (b) hipSetDevice(b->device);
    return backend_matmul(b, wid, index, x, rows, cols, nullptr, y);
}

}  // extern "C"
