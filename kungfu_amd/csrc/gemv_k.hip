// Decode and few-row product for q5_K and q6_K weights (SURVEY's second "next" row: the other K-quant weight types on
// the same product; Q4_K_M files carry q6_K head and down projections). y[r][o] = sum over super-blocks of the
// reference's dot_i8 integers scaled back to floats (crates/kf-quant/src/types/q5_k.rs:7-60, q6_k.rs:17-59) + bias +
// res; it replaces the reference's q5_K / q6_K loaders of kf_matvec_i8 (crates/kf-backend-cuda/src/kernels/quant_q6_K.cu,
// quant_q5_K.cu, launched by matvec_i8_launch, exec.rs:1996-2039).
//
// Design: one wave per output row at a time, four lanes per super-block (the lane units KfQ5Lane / KfQ6Lane), so a
// wave pass covers 16 super-blocks (4096 columns) of the row; up to eight activation rows against every weight pass
// (the weights are read once per eight rows). Activations are read from the scratch in global memory (a few KB per
// row, L2-resident). With 16-byte aligned rows (q5_K always, q6_K when the row has a multiple of eight super-blocks)
// a pass's bytes travel as contiguous 16-byte pieces (lane l takes pieces l, l + 64, ...: every wave load
// instruction reads 1 KB of consecutive bytes, the pattern that streams at the chip's read rate), are parked in the
// wave's own LDS buffer and read back by the lanes; otherwise each lane loads its unit's bytes straight from memory
// (2-byte aligned 16-byte loads for q6_K's 210-byte super-blocks).
#include "kf_blocks.h"

#include <algorithm>

namespace {

constexpr int GK_THREADS = 256;
constexpr int GK_WAVES = GK_THREADS / 64;
constexpr int GK_PIECES = 4;  // 16-byte pieces a lane moves per pass: 210 (q6_K) or 176 (q5_K) over 64 lanes
constexpr int GK_WBUF = 16 * KF_Q6_K_BYTES;  // one pass of 16 super-blocks

template <uint32_t TY, int R, bool PARK>
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
    __shared__ __align__(16) uint8_t park[PARK ? GK_WAVES * GK_WBUF : 16];
    uint8_t* wbuf = park + (PARK ? wave * GK_WBUF : 0);
    const int stride = gridDim.x * GK_WAVES;
    const int npass = (nsb + 15) / 16;
    int row = blockIdx.x * GK_WAVES + wave;  // wave-uniform
    uint4 v[GK_PIECES];                      // the next (row, pass) item's pieces in flight (PARK)
    auto fetch = [&](int rw, int sb0) {
        // 16-byte pieces clamped onto the pass's last 16 bytes (no byte past the pass is read)
        const int len = min(16, nsb - sb0) * BYTES;
        const uint8_t* src = w + (int64_t)rw * row_bytes + (int64_t)sb0 * BYTES;
#pragma unroll
        for (int i = 0; i < GK_PIECES; i++) v[i] = kf_load_stream_u4(src + min(16 * (lane + 64 * i), len - 16));
    };
    if constexpr (PARK) {
        if (row < n_out) fetch(row, 0);
    }
    for (; row < n_out; row += stride) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        const uint8_t* wr = w + (int64_t)row * row_bytes;
        for (int p = 0; p < npass; p++) {
            const int sb0 = 16 * p;
            const int sb = sb0 + (lane >> 2);
            const uint8_t* blk;
            if constexpr (PARK) {
                const int len = min(16, nsb - sb0) * BYTES;
#pragma unroll
                for (int i = 0; i < GK_PIECES; i++) *reinterpret_cast<uint4*>(wbuf + min(16 * (lane + 64 * i), len - 16)) = v[i];
                // the wave's next item (this row's next pass, or its next row's first) is requested before this
                // pass is multiplied; one wave's LDS operations complete in order, so no barrier guards the buffer
                if (p + 1 < npass) fetch(row, sb0 + 16);
                else if (row + stride < n_out) fetch(row + stride, 0);
                blk = wbuf + (lane >> 2) * BYTES;
            } else {
                blk = wr + (int64_t)sb * BYTES;
            }
            if (sb < nsb) {
                if constexpr (TY == KF_TYPE_Q6_K) {
                    KfQ6Lane u;
                    u.template load<PARK>(blk, j);
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        if (r < rows) {
                            const int isum = u.dot(xq + (int64_t)r * n + 256 * sb, xs16 + (int64_t)r * n16 + 16 * sb, j);
                            acc[r] = fmaf(u.d * xd16[(int64_t)r * n16 + 16 * sb], (float)isum, acc[r]);
                        }
                    }
                } else {
                    KfQ5Lane u;
                    u.template load<PARK>(blk, j);
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
                const float vs = kf_wave_sum(acc[r]);
                if (lane == 0) {
                    const int64_t o = (int64_t)r * ld_y + row;
                    y[o] = vs + (bias ? bias[row] : 0.0f) + (res ? res[o] : 0.0f);
                }
            }
        }
    }
}

int gk_cus() {
    static const int cus = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1)
            v = 256;
        return v;
    }();
    return cus;
}

template <uint32_t TY, bool PARK>
hipError_t launch_k(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const int32_t* xs16, const int32_t* xs32, const float* xd16,
                    const float* bias, const float* res, float* y, int rows, int n, int n_out, hipStream_t s) {
    // a resident grid of four blocks per CU; each wave walks its rows with the next (row, pass) in flight
    const int grid = std::min((n_out + GK_WAVES - 1) / GK_WAVES, 4 * gk_cus());
    // rows of one launch: 1, 2, 4 or 8 (the kernel skips rows past `rows`)
    if (rows == 1)
        gemv_k_kernel<TY, 1, PARK><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
    else if (rows == 2)
        gemv_k_kernel<TY, 2, PARK><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
    else if (rows <= 4)
        gemv_k_kernel<TY, 4, PARK><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
    else
        gemv_k_kernel<TY, 8, PARK><<<grid, GK_THREADS, 0, s>>>(w, row_bytes, xq, xs16, xs32, xd16, bias, res, y, rows, n, n_out, n_out);
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
        // parking needs 16-byte aligned passes: the weight base and every row start
        const bool park = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
        hipError_t e;
        if (ty == KF_TYPE_Q6_K)
            e = park ? launch_k<KF_TYPE_Q6_K, true>(w, row_bytes, xq, xs16, xs32, xd16, bias, rcp, yc, rc, n, n_out, s)
                     : launch_k<KF_TYPE_Q6_K, false>(w, row_bytes, xq, xs16, xs32, xd16, bias, rcp, yc, rc, n, n_out, s);
        else
            e = park ? launch_k<KF_TYPE_Q5_K, true>(w, row_bytes, xq, xs16, xs32, xd16, bias, rcp, yc, rc, n, n_out, s)
                     : launch_k<KF_TYPE_Q5_K, false>(w, row_bytes, xq, xs16, xs32, xd16, bias, rcp, yc, rc, n, n_out, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
