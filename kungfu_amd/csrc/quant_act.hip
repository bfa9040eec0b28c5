// Activation quantizer: rows of f32 activations into the int8 scratch the products consume.
//
// Restates crates/kf-quant/src/lib.rs:81-140 (quantize_activations) on the GPU, in place of the reference's
// quant_act (crates/kf-backend-cuda/src/kernels/fused.cu:12-21, kf_quant_span common.cuh:231-309):
//   kind 3 (Q8_0): per 32 columns d = amax/127, q = round-half-away(v / d) with 1/d taken from the unrounded d,
//                  d stored f16-rounded
//   kind 4 (Q8K):  per 256 columns, the first value of largest magnitude `mx`, iscale = -127/mx,
//                  q = min(round-half-even(iscale * v), 127), d = 1/iscale
// A wave of 64 lanes covers 256 columns, four consecutive columns a lane, so a Q8K block is one wave and a Q8_0 block
// eight lanes. The integer results are bit-exact with the CPU reference.
#include "kf_device.h"

// The reference rounds the f32 product v * id: with contraction, roundf's expansion (trunc, then p - trunc(p)) becomes
// fma(v, id, -trunc(p)), which sees the unrounded product and turns ties such as 58.4999999 -> 58.5 into 58.
#pragma clang fp contract(off)

namespace {

constexpr int QA_THREADS = 256;
constexpr int QA_SPAN = QA_THREADS * 4;  // columns one block covers

__global__ void __launch_bounds__(QA_THREADS) quant_act_kernel(const float* __restrict__ x, int8_t* __restrict__ q,
                                                               float* __restrict__ d16, int32_t* __restrict__ s16,
                                                               float* __restrict__ d32, int32_t* __restrict__ s32,
                                                               int n, int kind) {
    const int row = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int c0 = blockIdx.x * QA_SPAN + threadIdx.x * 4;
    const bool in = c0 < n;
    const float* xr = x + (size_t)row * n;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (in) {
        const float4 t = *reinterpret_cast<const float4*>(xr + c0);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    }
    int qi[4];
    float d;
    if (kind == KF_ACT_Q8_0) {
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        // eight lanes make a block of 32
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) qi[j] = (int)roundf(v[j] * id);
        d = kf_round_f16(dd);
    } else {
        // first index of the largest magnitude: lexicographic max of (|v|, -index) over the wave
        float a = -1.0f, mx = 0.0f;
        int idx = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float aj = in ? fabsf(v[j]) : -1.0f;
            if (aj > a) {
                a = aj;
                idx = c0 + j;
                mx = v[j];
            }
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float oa = __shfl_xor(a, o, 64);
            const int oi = __shfl_xor(idx, o, 64);
            const float om = __shfl_xor(mx, o, 64);
            if (oa > a || (oa == a && oi < idx)) {
                a = oa;
                idx = oi;
                mx = om;
            }
        }
        if (a > 0.0f) {
            const float iscale = -127.0f / mx;
            d = 1.0f / iscale;
#pragma unroll
            for (int j = 0; j < 4; j++) qi[j] = min((int)rintf(iscale * v[j]), 127);
        } else {
            d = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) qi[j] = 0;
        }
    }
    // four lanes make a group of 16, eight a group of 32
    int sum16 = qi[0] + qi[1] + qi[2] + qi[3];
    sum16 += __shfl_xor(sum16, 1, 64);
    sum16 += __shfl_xor(sum16, 2, 64);
    const int sum32 = sum16 + __shfl_xor(sum16, 4, 64);
    if (!in) return;
    const uint32_t packed = (uint32_t)(qi[0] & 0xff) | ((uint32_t)(qi[1] & 0xff) << 8) | ((uint32_t)(qi[2] & 0xff) << 16) |
                            ((uint32_t)(qi[3] & 0xff) << 24);
    *reinterpret_cast<uint32_t*>(q + (size_t)row * n + c0) = packed;
    if ((lane & 3) == 0) {
        const size_t g = (size_t)row * (n >> 4) + (c0 >> 4);
        d16[g] = d;
        s16[g] = sum16;
    }
    if ((lane & 7) == 0) {
        const size_t g = (size_t)row * (n >> 5) + (c0 >> 5);
        d32[g] = d;
        s32[g] = sum32;
    }
}

}  // namespace

// Host launcher, validated by the caller (api.cpp): n a multiple of the kind's block, rows >= 1
hipError_t kf_launch_quant_act(const float* x, void* act, int rows, int n, int kind, hipStream_t s) {
    const kf_act_offsets o = kf_act_layout((size_t)rows, (size_t)n);
    char* base = static_cast<char*>(act);
    dim3 grid((n + QA_SPAN - 1) / QA_SPAN, rows);
    quant_act_kernel<<<grid, QA_THREADS, 0, s>>>(x, reinterpret_cast<int8_t*>(base + o.q), reinterpret_cast<float*>(base + o.d16),
                                                 reinterpret_cast<int32_t*>(base + o.s16), reinterpret_cast<float*>(base + o.d32),
                                                 reinterpret_cast<int32_t*>(base + o.s32), n, kind);
    return hipGetLastError();
}
