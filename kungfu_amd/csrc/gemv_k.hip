// Decode and few-row product for q5_K and q6_K weights (SURVEY's second "next" row: the other K-quant weight types on
// the same product; Q4_K_M files carry q6_K head and down projections). y[r][o] = sum over super-blocks of the
// reference's dot_i8 integers scaled back to floats (crates/kf-quant/src/types/q5_k.rs:7-60, q6_k.rs:17-59) + bias +
// res; it replaces the reference's q5_K / q6_K loaders of kf_matvec_i8 (crates/kf-backend-cuda/src/kernels/quant_q6_K.cu,
// quant_q5_K.cu, launched by matvec_i8_launch, exec.rs:1996-2039).
//
// Design: one wave per output row at a time, four lanes per super-block (the lane units KfQ5Lane / KfQ6Lane), so a
// wave pass covers 16 super-blocks (4096 columns) of the row; up to eight activation rows against every weight pass
// (the weights are read once per eight rows). Activations are read from the scratch in global memory (a few KB per
// row, L2-resident). The q6_K super-block is 210 bytes, so its loads are 2-byte aligned 16-byte loads.
#include "kf_blocks.h"

#include <algorithm>

namespace {

constexpr int GK_THREADS = 256;
constexpr int GK_WAVES = GK_THREADS / 64;

template <uint32_t TY, int R>
__global__ void __launch_bounds__(GK_THREADS) gemv_k_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                            const int32_t* __restrict__ xs16, const int32_t* __restrict__ xs32,
                                                            const float* __restrict__ xd16, const float* __restrict__ bias,
                                                            const float* __restrict__ res, float* __restrict__ y, int rows, int n, int n_out,
                                                            int ld_y) {
    constexpr int BYTES = TY == KF_TYPE_Q6_K ? KF_Q6_K_BYTES : KF_Q5_K_BYTES;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsb = n / 256, n16 = n / 16, n32 = n / 32;
    const int j = lane & 3;
    for (int row = blockIdx.x * GK_WAVES + wave; row < n_out; row += gridDim.x * GK_WAVES) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        const uint8_t* wr = w + (int64_t)row * row_bytes;
        for (int sb0 = 0; sb0 < nsb; sb0 += 16) {
            const int sb = sb0 + (lane >> 2);
            if (sb < nsb) {
                const uint8_t* blk = wr + (int64_t)sb * BYTES;
                if constexpr (TY == KF_TYPE_Q6_K) {
                    KfQ6Lane u;
                    u.load(blk, j);
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        if (r < rows) {
                            const int isum = u.dot(xq + (int64_t)r * n + 256 * sb, xs16 + (int64_t)r * n16 + 16 * sb, j);
                            acc[r] = fmaf(u.d * xd16[(int64_t)r * n16 + 16 * sb], (float)isum, acc[r]);
                        }
                    }
                } else {
                    KfQ5Lane u;
                    u.load(blk, j);
                    const float d = kf_h2f(u.hdr.x & 0xffffu), dmin = kf_h2f(u.hdr.x >> 16);
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        if (r < rows) {
                            int isum, imin;
                            u.dot(xq + (int64_t)r * n + 256 * sb, xs32 + (int64_t)r * n32 + 8 * sb, j, isum, imin);
                            const float dx = xd16[(int64_t)r * n16 + 16 * sb];
                            acc[r] = fmaf(-(dmin * dx), (float)imin, fmaf(d * dx, (float)isum, acc[r]));
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r < rows) {
                const float v = kf_wave_sum(acc[r]);
                if (lane == 0) {
                    const int64_t o = (int64_t)r * ld_y + row;
                    y[o] = v + (bias ? bias[row] : 0.0f) + (res ? res[o] : 0.0f);
                }
            }
        }
    }
}

template <uint32_t TY>
hipError_t launch_k(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const int32_t* xs16, const int32_t* xs32, const float* xd16,
                    const float* bias, const float* res, float* y, int rows, int n, int n_out, hipStream_t s) {
    const int grid = (n_out + GK_WAVES - 1) / GK_WAVES;
    // rows of one launch: 1, 2, 4 or 8 (the kernel skips rows past `rows`)
    if (rows == 1)
        gemv_k_kernel<TY, 1><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
    else if (rows == 2)
        gemv_k_kernel<TY, 2><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
    else if (rows <= 4)
        gemv_k_kernel<TY, 4><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
    else
        gemv_k_kernel<TY, 8><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
    return hipGetLastError();
}

}  // namespace

// Host launcher, validated by the caller (api.cpp): ty q5_K or q6_K, n a multiple of 256, Q8K-kind activations in
// `act`. Activation rows go in chunks of eight, each chunk one launch that reads the weights once.
hipError_t kf_launch_gemv_k(uint32_t ty, const void* wv, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y,
                            int rows, int n, int n_out, hipStream_t s) {
    if (n_out == 0) return hipSuccess;
    const kf_act_offsets o = kf_act_layout((size_t)rows, (size_t)n);
    const char* base = static_cast<const char*>(act);
    const auto* w = static_cast<const uint8_t*>(wv);
    for (int r0 = 0; r0 < rows; r0 += 8) {
        const int rc = std::min(8, rows - r0);
        const int8_t* xq = reinterpret_cast<const int8_t*>(base + o.q) + (size_t)r0 * n;
        const int32_t* xs16 = reinterpret_cast<const int32_t*>(base + o.s16) + (size_t)r0 * (n / 16);
        const int32_t* xs32 = reinterpret_cast<const int32_t*>(base + o.s32) + (size_t)r0 * (n / 32);
        const float* xd16 = reinterpret_cast<const float*>(base + o.d16) + (size_t)r0 * (n / 16);
        float* yc = y + (size_t)r0 * n_out;
        const float* rcp = res ? res + (size_t)r0 * n_out : nullptr;
        const hipError_t e = ty == KF_TYPE_Q6_K ? launch_k<KF_TYPE_Q6_K>(w, row_bytes, xq, xs16, xs32, xd16, bias, rcp, yc, rc, n, n_out, s)
                                                : launch_k<KF_TYPE_Q5_K>(w, row_bytes, xq, xs16, xs32, xd16, bias, rcp, yc, rc, n, n_out, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
