// Activation quantizer: rows of f32 activations into the int8 scratch the products consume, in place of the
// reference's quant_act (crates/kf-backend-cuda/src/kernels/fused.cu:12-21, kf_quant_span common.cuh:231-309). The
// per-lane arithmetic (crates/kf-quant/src/lib.rs:81-140) is kf_qa_quant; the integer results are bit-exact with the
// CPU reference.
#include "kf_qa.h"

// The producers' own f32 arithmetic (rms_norm, the gated activation) is written unfused, as the CPU rounds it.
#pragma clang fp contract(off)

namespace {

constexpr int QA_THREADS = 256;
constexpr int QA_SPAN = QA_THREADS * 4;  // columns one block covers

// Quantizes the four columns c0.. of one row held by this thread (v, zeros past n) and writes q, the per-16 and
// per-32 scales and integer sums, and (Q8K) the mins operand of the q4_K GEMM. Every thread of the wave calls it.
__device__ __forceinline__ void qa_emit(const float (&v)[4], int c0, bool in, int n, int kind, int row, int8_t* __restrict__ q,
                                        float* __restrict__ d16, int32_t* __restrict__ s16, float* __restrict__ d32,
                                        int32_t* __restrict__ s32, _Float16* __restrict__ xa) {
    const int lane = threadIdx.x & 63;
    const KfQa r = kf_qa_quant(v, c0, in, kind);
    if (!in) return;
    *reinterpret_cast<uint32_t*>(q + (size_t)row * n + c0) = r.packed;
    if ((lane & 3) == 0) {
        const size_t g = (size_t)row * (n >> 4) + (c0 >> 4);
        d16[g] = r.d;
        s16[g] = r.sum16;
    }
    if ((lane & 7) == 0) {
        const size_t g = (size_t)row * (n >> 5) + (c0 >> 5);
        d32[g] = r.d;
        s32[g] = r.sum32;
        if (kind == KF_ACT_Q8K) {
            // the mins operand of the q4_K GEMM: sum32 = 64 hi + lo
            _Float16* xr = xa + ((size_t)row * ((n + 255) >> 8) + (c0 >> 8)) * 16 + ((c0 >> 5) & 7);
            xr[0] = (_Float16)(float)(r.sum32 >> 6);
            xr[8] = (_Float16)(float)(r.sum32 & 63);
        }
    }
}

__device__ __forceinline__ void qa_load4(const float* p, bool in, float (&v)[4]) {
    v[0] = v[1] = v[2] = v[3] = 0.0f;
    if (in) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    }
}

#define QA_OUT int8_t *__restrict__ q, float *__restrict__ d16, int32_t *__restrict__ s16, float *__restrict__ d32, int32_t *__restrict__ s32, _Float16 *__restrict__ xa

__global__ void __launch_bounds__(QA_THREADS) quant_act_kernel(const float* __restrict__ x, QA_OUT, int n, int kind) {
    const int row = blockIdx.y;
    const int c0 = blockIdx.x * QA_SPAN + threadIdx.x * 4;
    const bool in = c0 < n;
    float v[4];
    qa_load4(x + (size_t)row * n + c0, in, v);
    qa_emit(v, c0, in, n, kind, row, q, d16, s16, d32, s32, xa);
}

// rms_norm (crates/kf-backend-cpu/src/ops.rs:222-239) fused with the quantization, in place of the reference's
// rms_norm_q8 (crates/kf-backend-cuda/src/kernels/fused.cu:24-45). One block per row sums the row's f32 squares in f64
// (the CPU's accumulator type; a fixed reduction tree), rounds ss / n to f32, takes inv = 1 / sqrt(ss + eps) with
// correctly rounded f32 square root and division, then walks the row's 1024-column spans computing (v * inv) * w + b
// unfused: the values the CPU rounds, so the quantized integers agree bit for bit (an f64 sum in another order rounds
// to the same f32 except within ~1e-16 of a rounding boundary). The second pass over the row hits L2.
// T threads a row: 256 when the rows fill the GPU, 1024 for a few rows (decode), where one block's passes over the
// row are the whole latency
template <int T>
__global__ void __launch_bounds__(T) rms_norm_q8_kernel(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
                                                        float eps, QA_OUT, int n, int kind) {
    constexpr int SPAN = 4 * T;
    __shared__ double part[T / 64];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * n;
    double s = 0.0;
    for (int i = threadIdx.x * 4; i < n; i += SPAN) {
        const float4 t = *reinterpret_cast<const float4*>(xr + i);
        const float a0 = t.x * t.x, a1 = t.y * t.y, a2 = t.z * t.z, a3 = t.w * t.w;
        s += (double)a0;
        s += (double)a1;
        s += (double)a2;
        s += (double)a3;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int k = 0; k < T / 64; k++) t += part[k];
    const float ss = (float)(t / (double)n);
    // f32 square root and division, each correctly rounded: evaluated in f64 and rounded once (exact for both
    // operations, since 53 >= 2 * 24 + 2); the f32 intrinsics measured one ulp off on some rows
    const float r = (float)sqrt((double)(ss + eps));
    const float inv = (float)(1.0 / (double)r);
    for (int base = 0; base < n; base += SPAN) {
        const int c0 = base + threadIdx.x * 4;
        const bool in = c0 < n;
        float v[4];
        qa_load4(xr + c0, in, v);
        if (in) {
            float wv[4] = {1.0f, 1.0f, 1.0f, 1.0f}, bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (w) qa_load4(w + c0, true, wv);
            if (b) qa_load4(b + c0, true, bv);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float u = v[j] * inv;
                u = u * wv[j];
                v[j] = u + bv[j];
            }
        }
        qa_emit(v, c0, in, n, kind, row, q, d16, s16, d32, s32, xa);
    }
}

// The gated activation act(gate) * up (crates/kf-backend-cpu/src/ops.rs:44-57, no limit) fused with the
// quantization, in place of the reference's gated_act_q8 (crates/kf-backend-cuda/src/kernels/fused.cu:48-65).
// act 0 silu: g / (1 + exp(-g)) with exp evaluated in f64 and rounded to f32 (the correctly rounded value the CPU's
// libm expf returns but for rare last-ulp cases), IEEE division; act 2 relu; act 4 relu squared. Rows of gate and up
// are `stride` floats apart.
__global__ void __launch_bounds__(QA_THREADS) gated_act_q8_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                                  int stride, int act, QA_OUT, int n, int kind) {
    const int row = blockIdx.y;
    const int c0 = blockIdx.x * QA_SPAN + threadIdx.x * 4;
    const bool in = c0 < n;
    float g[4], u[4], v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    qa_load4(gate + (size_t)row * stride + c0, in, g);
    qa_load4(up + (size_t)row * stride + c0, in, u);
    if (in) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float a;
            if (act == 0) {
                const float e = (float)exp(-(double)g[j]);
                a = (float)((double)g[j] / (double)(1.0f + e));  // correctly rounded f32 division
            } else {
                const float r = fmaxf(g[j], 0.0f);
                a = act == 4 ? r * r : r;
            }
            v[j] = a * u[j];
        }
    }
    qa_emit(v, c0, in, n, kind, row, q, d16, s16, d32, s32, xa);
}

}  // namespace

#define QA_ARGS(act)                                                                                          \
    const kf_act_offsets o = kf_act_layout((size_t)rows, (size_t)n);                                          \
    char* base = static_cast<char*>(act);                                                                     \
    int8_t* q = reinterpret_cast<int8_t*>(base + o.q);                                                        \
    float* d16 = reinterpret_cast<float*>(base + o.d16);                                                      \
    int32_t* s16 = reinterpret_cast<int32_t*>(base + o.s16);                                                  \
    float* d32 = reinterpret_cast<float*>(base + o.d32);                                                      \
    int32_t* s32 = reinterpret_cast<int32_t*>(base + o.s32);                                                  \
    _Float16* xa = reinterpret_cast<_Float16*>(base + o.xa);                                                  \
    dim3 grid((n + QA_SPAN - 1) / QA_SPAN, rows)

// Host launchers, validated by the caller (api.cpp): n a multiple of the kind's block, rows >= 1
hipError_t kf_launch_quant_act(const float* x, void* act, int rows, int n, int kind, hipStream_t s) {
    QA_ARGS(act);
    quant_act_kernel<<<grid, QA_THREADS, 0, s>>>(x, q, d16, s16, d32, s32, xa, n, kind);
    return hipGetLastError();
}

hipError_t kf_launch_rms_norm_q8(const float* x, const float* w, const float* b, float eps, void* act, int rows, int n, int kind,
                                 hipStream_t s) {
    QA_ARGS(act);
    (void)grid;
    if (rows < 64)
        rms_norm_q8_kernel<1024><<<rows, 1024, 0, s>>>(x, w, b, eps, q, d16, s16, d32, s32, xa, n, kind);
    else
        rms_norm_q8_kernel<QA_THREADS><<<rows, QA_THREADS, 0, s>>>(x, w, b, eps, q, d16, s16, d32, s32, xa, n, kind);
    return hipGetLastError();
}

hipError_t kf_launch_gated_act_q8(const float* gate, const float* up, int stride, int act_fn, void* act, int rows, int n, int kind,
                                  hipStream_t s) {
    QA_ARGS(act);
    gated_act_q8_kernel<<<grid, QA_THREADS, 0, s>>>(gate, up, stride, act_fn, q, d16, s16, d32, s32, xa, n, kind);
    return hipGetLastError();
}
