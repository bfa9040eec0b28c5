// Batch-1 decode GEMV on native GGUF bytes: y[o] = sum over the row's blocks of (d_w * d_x) * int32 dot (+ min term
// for q4_K) + bias[o] + res[o].
//
// Replaces the reference's matvec_i8_1 / kf_matvec_i8<T,1> (crates/kf-backend-cuda/src/kernels/quant.cuh:435-512)
// and its launch (crates/kf-backend-cuda/src/exec.rs:1996-2039). The arithmetic per block is the reference's dot_i8
// (crates/kf-quant/src/types/q8_0.rs:10-29, types/q4_k.rs:10-58); the per-block int32 results are bit-exact.
//
// Design for gfx950 (wave64, 256 CUs, HBM3E):
//   * A block of 8 waves stages the quantized activation row (int8 + per-32 integer sums + scales) in LDS once and
//     every wave then streams whole weight rows, one row per wave at a time, reading only HBM weight bytes.
//   * q4_K: four lanes own one 144-byte super-block, each lane a 32-byte pair of sub-blocks (two 16-byte loads) plus
//     the 16-byte header (one request per four lanes), so a wave step covers 16 super-blocks = 4096 columns and every
//     load is a 128-bit load. All of a row's loads are issued before any arithmetic (template STEPS).
//   * q8_0: one lane owns one 34-byte block read as a 2-byte-skewed dword window and realigned with v_perm_b32; a wave
//     step covers 64 consecutive blocks = 2176 contiguous bytes.
//   * Integer dots use v_dot4_i32_i8; the per-block float combine happens per lane; one wave reduction per row.
#include "kf_blocks.h"

namespace {

constexpr int GV_THREADS = 512;
constexpr int GV_WAVES = GV_THREADS / 64;

// LDS bytes of the staged activation row of n columns for either kind
__host__ __device__ constexpr size_t gv_smem(int n) { return (size_t)n + (size_t)(n / 32) * 4 + (size_t)(n / 32) * 4; }

// Stages q (n bytes), the per-32 integer sums and the per-32 scales of one activation row into LDS
__device__ __forceinline__ void gv_stage(uint8_t* smem, const int8_t* __restrict__ xq, const int32_t* __restrict__ xs32,
                                         const float* __restrict__ xd32, int n) {
    uint4* sq = reinterpret_cast<uint4*>(smem);
    const uint4* gq = reinterpret_cast<const uint4*>(xq);
    for (int i = threadIdx.x; i < (n >> 4); i += GV_THREADS) sq[i] = gq[i];
    int32_t* ss = reinterpret_cast<int32_t*>(smem + n);
    float* sd = reinterpret_cast<float*>(smem + n + (n / 32) * 4);
    for (int i = threadIdx.x; i < (n >> 5); i += GV_THREADS) {
        ss[i] = xs32[i];
        sd[i] = xd32[i];
    }
    __syncthreads();
}

template <int STEPS>
__global__ void __launch_bounds__(GV_THREADS) gemv_q4k_kernel(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                              const int8_t* __restrict__ xq, const int32_t* __restrict__ xs32,
                                                              const float* __restrict__ xd32, const float* __restrict__ bias,
                                                              const float* __restrict__ res, float* __restrict__ y, int n,
                                                              int n_out) {
    extern __shared__ __align__(16) uint8_t smem[];
    gv_stage(smem, xq, xs32, xd32, n);
    const int8_t* sx = reinterpret_cast<const int8_t*>(smem);
    const int32_t* ss = reinterpret_cast<const int32_t*>(smem + n);
    const float* sd = reinterpret_cast<const float*>(smem + n + (n / 32) * 4);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sbl = lane >> 2;  // super-block of the lane within a step
    const int j = lane & 3;     // sub-block pair of the lane
    const int nsb = n >> 8;
    for (int o = blockIdx.x * GV_WAVES + wave; o < n_out; o += gridDim.x * GV_WAVES) {
        const uint8_t* row = w + (int64_t)o * row_bytes;
        uint4 hdr[STEPS], qa[STEPS], qb[STEPS];
#pragma unroll
        for (int s = 0; s < STEPS; s++) {
            const int sb = s * 16 + sbl;
            if (sb < nsb) {
                const uint8_t* blk = row + (int64_t)sb * KF_Q4_K_BYTES;
                hdr[s] = kf_load_stream_u4(blk);
                qa[s] = kf_load_stream_u4(blk + 16 + 32 * j);
                qb[s] = kf_load_stream_u4(blk + 32 + 32 * j);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < STEPS; s++) {
            const int sb = s * 16 + sbl;
            if (sb < nsb) {
                const uint4* xs = reinterpret_cast<const uint4*>(sx + sb * 256 + 64 * j);
                const int2 bs = *reinterpret_cast<const int2*>(ss + sb * 8 + 2 * j);
                int isum, imin;
                kf_q4k_lane(hdr[s], qa[s], qb[s], j, xs[0], xs[1], xs[2], xs[3], bs.x, bs.y, isum, imin);
                const float dx = sd[sb * 8];
                const float d = kf_h2f(hdr[s].x & 0xffffu) * dx;
                const float dm = kf_h2f(hdr[s].x >> 16) * dx;
                acc = fmaf(d, (float)isum, acc);
                acc = fmaf(-dm, (float)imin, acc);
            }
        }
        acc = kf_wave_sum(acc);
        if (lane == 0) y[o] = acc + (bias ? bias[o] : 0.0f) + (res ? res[o] : 0.0f);
    }
}

template <int STEPS>
__global__ void __launch_bounds__(GV_THREADS) gemv_q8_0_kernel(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                               const int8_t* __restrict__ xq, const int32_t* __restrict__ xs32,
                                                               const float* __restrict__ xd32, const float* __restrict__ bias,
                                                               const float* __restrict__ res, float* __restrict__ y, int n,
                                                               int n_out) {
    extern __shared__ __align__(16) uint8_t smem[];
    gv_stage(smem, xq, xs32, xd32, n);
    const int8_t* sx = reinterpret_cast<const int8_t*>(smem);
    const float* sd = reinterpret_cast<const float*>(smem + n + (n / 32) * 4);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nb = n >> 5;
    for (int o = blockIdx.x * GV_WAVES + wave; o < n_out; o += gridDim.x * GV_WAVES) {
        const uint8_t* row = w + (int64_t)o * row_bytes;
        float acc = 0.0f;
        // groups of four steps: the loads of a group go out before its arithmetic
        for (int s0 = 0; s0 < STEPS; s0 += 4) {
            uint32_t win[4][9];
            bool sk[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int b = (s0 + u) * 64 + lane;
                if (s0 + u < STEPS && b < nb) kf_q8_0_window(row + (int64_t)b * KF_Q8_0_BYTES, win[u], sk[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int b = (s0 + u) * 64 + lane;
                if (s0 + u < STEPS && b < nb) {
                    uint32_t dbits, wq[8];
                    kf_q8_0_unpack(win[u], sk[u], dbits, wq);
                    const uint4* xs = reinterpret_cast<const uint4*>(sx + b * 32);
                    const int dot = kf_q8_0_dot(wq, xs[0], xs[1]);
                    acc = fmaf(kf_h2f(dbits) * sd[b], (float)dot, acc);
                }
            }
        }
        acc = kf_wave_sum(acc);
        if (lane == 0) y[o] = acc + (bias ? bias[o] : 0.0f) + (res ? res[o] : 0.0f);
    }
}

// Per-block integers of weight rows against activation rows, one thread per (weight row, activation row, block):
// q8_0 one int32 per 32-block, q4_K (sumi, mins) per super-block. The check that pins the GEMV's lane arithmetic.
__global__ void block_ints_kernel(uint32_t ty, const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                  const int32_t* __restrict__ xs32, int n, int n_out, int rows, int32_t* __restrict__ out) {
    const int per = ty == KF_TYPE_Q8_0 ? n / 32 : n / 256;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)n_out * rows * per) return;
    const int b = (int)(t % per);
    const int r = (int)((t / per) % rows);
    const int o = (int)(t / ((int64_t)per * rows));
    const uint8_t* row = w + (int64_t)o * row_bytes;
    const int8_t* x = xq + (int64_t)r * n;
    if (ty == KF_TYPE_Q8_0) {
        uint32_t win[9], dbits, wq[8];
        bool sk;
        kf_q8_0_window(row + (int64_t)b * KF_Q8_0_BYTES, win, sk);
        kf_q8_0_unpack(win, sk, dbits, wq);
        const uint4* xs = reinterpret_cast<const uint4*>(x + b * 32);
        out[t] = kf_q8_0_dot(wq, xs[0], xs[1]);
    } else {
        const uint8_t* blk = row + (int64_t)b * KF_Q4_K_BYTES;
        const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
        const int32_t* bs = xs32 + (int64_t)r * (n / 32) + b * 8;
        int sumi = 0, mins = 0;
        for (int j = 0; j < 4; j++) {
            const uint4 qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * j);
            const uint4 qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * j);
            const uint4* xs = reinterpret_cast<const uint4*>(x + b * 256 + 64 * j);
            int isum, imin;
            kf_q4k_lane(hdr, qa, qb, j, xs[0], xs[1], xs[2], xs[3], bs[2 * j], bs[2 * j + 1], isum, imin);
            sumi += isum;
            mins += imin;
        }
        out[2 * t] = sumi;
        out[2 * t + 1] = mins;
    }
}

int g_cu_count = 0;

int cu_count() {
    if (g_cu_count == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            g_cu_count = v;
        else
            g_cu_count = 256;
    }
    return g_cu_count;
}

}  // namespace

// Largest row width the single-row GEMV stages in LDS
int kf_gemv_max_n() { return 32768; }

int kf_gemv_blocks(int n_out, int blocks_per_cu) {
    const int want = (n_out + GV_WAVES - 1) / GV_WAVES;
    const int cap = cu_count() * (blocks_per_cu > 0 ? blocks_per_cu : 2);
    return want < cap ? want : cap;
}

#define KF_GEMV_CASE(KERN, S)                                                                                               \
    case S:                                                                                                                 \
        KERN<S><<<grid, GV_THREADS, smem, s>>>(w, row_bytes, xq, xs32, xd32, bias, res, y, n, n_out);                       \
        break;

// Host launcher for one activation row, validated by the caller (api.cpp): n a multiple of the type's block,
// n <= kf_gemv_max_n(). xq / xs32 / xd32 point at the row's int8 values, per-32 sums and per-32 scales.
hipError_t kf_launch_gemv1(uint32_t ty, const void* wv, int64_t row_bytes, const int8_t* xq, const int32_t* xs32, const float* xd32,
                           const float* bias, const float* res, float* y, int n, int n_out, int blocks_per_cu, hipStream_t s) {
    const uint8_t* w = static_cast<const uint8_t*>(wv);
    const size_t smem = gv_smem(n);
    const int grid = kf_gemv_blocks(n_out, blocks_per_cu);
    if (n_out == 0) return hipSuccess;
    if (ty == KF_TYPE_Q4_K) {
        const int steps = (n / 256 + 15) / 16;
        switch (steps) {
            KF_GEMV_CASE(gemv_q4k_kernel, 1)
            KF_GEMV_CASE(gemv_q4k_kernel, 2)
            KF_GEMV_CASE(gemv_q4k_kernel, 3)
            KF_GEMV_CASE(gemv_q4k_kernel, 4)
            KF_GEMV_CASE(gemv_q4k_kernel, 5)
            KF_GEMV_CASE(gemv_q4k_kernel, 6)
            KF_GEMV_CASE(gemv_q4k_kernel, 7)
            KF_GEMV_CASE(gemv_q4k_kernel, 8)
            default: return hipErrorInvalidValue;
        }
    } else {
        const int steps = (n / 32 + 63) / 64;
        switch ((steps + 3) / 4 * 4) {
            KF_GEMV_CASE(gemv_q8_0_kernel, 4)
            KF_GEMV_CASE(gemv_q8_0_kernel, 8)
            KF_GEMV_CASE(gemv_q8_0_kernel, 12)
            KF_GEMV_CASE(gemv_q8_0_kernel, 16)
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

hipError_t kf_launch_block_ints(uint32_t ty, const void* w, int64_t row_bytes, const void* act, int rows, int n, int n_out,
                                int32_t* out, hipStream_t s) {
    const kf_act_offsets off = kf_act_layout((size_t)rows, (size_t)n);
    const char* base = static_cast<const char*>(act);
    const int per = ty == KF_TYPE_Q8_0 ? n / 32 : n / 256;
    const int64_t total = (int64_t)n_out * rows * per;
    if (total == 0) return hipSuccess;
    const int threads = 256;
    block_ints_kernel<<<(unsigned)((total + threads - 1) / threads), threads, 0, s>>>(
        ty, static_cast<const uint8_t*>(w), row_bytes, reinterpret_cast<const int8_t*>(base + off.q),
        reinterpret_cast<const int32_t*>(base + off.s32), n, n_out, rows, out);
    return hipGetLastError();
}
