// Prefill / batched int8 GEMM on native q8_0 weight bytes: y[m][n] = sum over 32-column groups g of
// d_x[m][g] * d_w[n][g] * I_g[m][n] (+ bias[n] + res[m][n]), with I_g the exact int32 dot of the group.
//
// Replaces the reference's KF8 GEMM (crates/kf-backend-cuda/src/kernels/kf8.cu:116-395, host kf8.rs:258-323), which
// first unpacks native bytes into an int8 + f32-scale form; here the q8_0 rows are read unchanged (a q8_0 block is
// already int8 with one f16 scale per 32) and only their 32 weight bytes are moved into LDS tiles.
//
// gfx950 design:
//   * A block computes a 128 x 128 output tile with four waves of 64 x 64 (2 x 2 tiles of 32 x 32).
//   * K advances 128 columns (four groups) per stage. Global loads of the next stage are in flight in registers
//     while the current stage is multiplied from LDS; LDS is double-buffered, one barrier per stage.
//   * LDS holds each 32 x 32 operand tile in MFMA operand order (lane l's 16 bytes at 16 * l), so every operand read
//     is a contiguous 1 KB and bank-conflict free.
//   * Per group and 32 x 32 tile: one v_mfma_i32_32x32x32_i8 gives the exact int32 dots I_g; one
//     v_mfma_f32_32x32x16_f16 with a single non-zero k slot gives the exact outer product d_x (x) d_w of the group's
//     f16 scales (q8_0 weight scales are f16, Q8_0-kind activation scales are f16-rounded); the VALU then converts
//     I_g and accumulates with one FMA. The per-element rescale (a convert and an FMA per group) is the VALU work
//     that bounds this GEMM, not the MFMA.
#include "kf_device.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 128;  // tile sizes; BK spans four 32-column groups
constexpr int GM_THREADS = 256;
constexpr int GM_G = GM_BK / 32;  // groups per stage
// LDS of one stage: A and B operand tiles (16 KB each) and f16 scales of A rows and B columns (1 KB each)
constexpr int GM_A_BYTES = GM_BM * GM_BK, GM_B_BYTES = GM_BN * GM_BK;
constexpr int GM_SA = GM_A_BYTES + GM_B_BYTES, GM_SB = GM_SA + GM_G * GM_BM * 2;
constexpr int GM_STAGE = GM_SB + GM_G * GM_BN * 2;

// Byte offset in an operand tile of the 16-byte piece (group g, row r of the 128, half h of the 32 columns):
// tiles of 32 rows are stored as [half][row % 32] so a wave reads one tile as 64 consecutive 16-byte pieces
__device__ __forceinline__ int gm_piece(int g, int r, int h) { return (((g * 4 + (r >> 5)) * 2 + h) * 32 + (r & 31)) * 16; }

struct GmPrefetch {
    uint4 a[4], b[4];
    uint32_t dw[2];
    float dx[2];
};

__global__ void __launch_bounds__(GM_THREADS, 2) gemm_q8_0_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xd32, const float* __restrict__ bias,
                                                                  const float* __restrict__ res, float* __restrict__ y, int M, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * GM_BM, n0 = blockIdx.x * GM_BN;
    const int kg = K >> 5;  // groups per row
    const int stages = K / GM_BK;

    auto load = [&](GmPrefetch& p, int st) {
        const int gb = st * GM_G;  // first group of the stage
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + GM_THREADS * i;  // 1024 pieces: row c / 8, group (c % 8) / 2, half c % 2
            const int r = c >> 3, g = (c >> 1) & 3, h = c & 1;
            const int m = min(m0 + r, M - 1), n = min(n0 + r, N - 1);
            p.a[i] = *reinterpret_cast<const uint4*>(xq + (int64_t)m * K + (gb + g) * 32 + 16 * h);
            p.b[i] = kf_load_stream_u4_unaligned(w + (int64_t)n * row_bytes + (int64_t)(gb + g) * KF_Q8_0_BYTES + 2 + 16 * h);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = tid + GM_THREADS * i;  // 512 scales: row c / 4, group c % 4
            const int r = c >> 2, g = c & 3;
            const int m = min(m0 + r, M - 1), n = min(n0 + r, N - 1);
            p.dx[i] = xd32[(int64_t)m * kg + gb + g];
            p.dw[i] = *reinterpret_cast<const uint16_t*>(w + (int64_t)n * row_bytes + (int64_t)(gb + g) * KF_Q8_0_BYTES);
        }
    };
    auto store = [&](const GmPrefetch& p, uint8_t* buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + GM_THREADS * i;
            const int r = c >> 3, g = (c >> 1) & 3, h = c & 1;
            *reinterpret_cast<uint4*>(buf + gm_piece(g, r, h)) = p.a[i];
            *reinterpret_cast<uint4*>(buf + GM_A_BYTES + gm_piece(g, r, h)) = p.b[i];
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = tid + GM_THREADS * i;
            const int r = c >> 2, g = c & 3;
            // Q8_0-kind activation scales are f16-rounded values, so this conversion is exact
            reinterpret_cast<_Float16*>(buf + GM_SA)[g * GM_BM + r] = (_Float16)p.dx[i];
            reinterpret_cast<uint16_t*>(buf + GM_SB)[g * GM_BN + r] = (uint16_t)p.dw[i];
        }
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v16f{};

    GmPrefetch pf;
    load(pf, 0);
    store(pf, smem);
    __syncthreads();
    for (int st = 0; st < stages; st++) {
        const uint8_t* buf = smem + (st & 1) * GM_STAGE;
        if (st + 1 < stages) load(pf, st + 1);
#pragma unroll 1
        for (int g = 0; g < GM_G; g++) {
            v4i a[2], b[2];
            v8h sa[2], sb[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                a[t] = *reinterpret_cast<const v4i*>(buf + gm_piece(g, (wm * 2 + t) * 32, 0) + 16 * lane);
                b[t] = *reinterpret_cast<const v4i*>(buf + GM_A_BYTES + gm_piece(g, (wn * 2 + t) * 32, 0) + 16 * lane);
                sa[t] = v8h{};
                sb[t] = v8h{};
                if (lane < 32) {
                    sa[t][0] = reinterpret_cast<const _Float16*>(buf + GM_SA)[g * GM_BM + (wm * 2 + t) * 32 + lane];
                    sb[t][0] = reinterpret_cast<const _Float16*>(buf + GM_SB)[g * GM_BN + (wn * 2 + t) * 32 + lane];
                }
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                v16i c[2];
                v16f s[2];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], v16i{}, 0, 0, 0);
                    s[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa[i], sb[j], v16f{}, 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf((float)c[j][r], s[j][r], acc[i][j][r]);
            }
        }
        if (st + 1 < stages) store(pf, smem + ((st + 1) & 1) * GM_STAGE);
        __syncthreads();
    }

    // 32 x 32 accumulator layout: lane l holds column l % 32; register r holds row (r % 4) + 8 * (r / 4) + 4 * (l / 32)
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + (wn * 2 + j) * 32 + (lane & 31);
            if (n >= N) continue;
            const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + (wm * 2 + i) * 32 + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
                if (m < M) y[(int64_t)m * N + n] = acc[i][j][r] + bn + (res ? res[(int64_t)m * N + n] : 0.0f);
            }
        }
}

}  // namespace

// Host launcher, validated by the caller (api.cpp): K a multiple of 128, Q8_0-kind activations in `act`
hipError_t kf_launch_gemm_q8_0(const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y, int M,
                               int N, int K, hipStream_t s) {
    const kf_act_offsets o = kf_act_layout((size_t)M, (size_t)K);
    const char* base = static_cast<const char*>(act);
    dim3 grid((N + GM_BN - 1) / GM_BN, (M + GM_BM - 1) / GM_BM);
    static bool lds_set = false;  // the double-buffered stage needs 68 KB of LDS per block
    if (!lds_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_q8_0_kernel), hipFuncAttributeMaxDynamicSharedMemorySize, 2 * GM_STAGE);
        if (e != hipSuccess) return e;
        lds_set = true;
    }
    gemm_q8_0_kernel<<<grid, GM_THREADS, 2 * GM_STAGE, s>>>(static_cast<const uint8_t*>(w), row_bytes, reinterpret_cast<const int8_t*>(base + o.q),
                                                           reinterpret_cast<const float*>(base + o.d32), bias, res, y, M, N, K);
    return hipGetLastError();
}

int kf_gemm_k_multiple() { return GM_BK; }
