// Batched / prefill int8 GEMM on native q8_0 weight bytes: y[m][n] = sum over 32-column groups g of
// d_x[m][g] * d_w[n][g] * I_g[m][n] (+ bias[n] + res[m][n]), with I_g the exact int32 dot of the group.
//
// Replaces the reference's KF8 GEMM (crates/kf-backend-cuda/src/kernels/kf8.cu:116-395, host kf8.rs:258-323), which
// first unpacks native bytes into an int8 + f32-scale form; here the q8_0 rows are read unchanged (a q8_0 block is
// already int8 with one f16 scale per 32) and only their 32 weight bytes are moved into LDS tiles.
//
// gfx950 design:
//   * Four waves per block in a WM x WN grid, each computing TM x TN tiles of 32 x 32, so a block tile is
//     (32 WM TM) x (32 WN TN): 128 x 128 for prefill, 32 x 128 / 64 x 128 for small batches.
//   * K advances 128 columns (four groups) per stage. The next stage's global loads are in flight in registers while
//     the current one is multiplied from LDS; LDS is double-buffered with one barrier per stage.
//   * An operand tile of 32 rows x 32 bytes sits in LDS as two halves of 32 slots of 16 bytes, in the order the MFMA
//     consumes (lane l reads slot l % 32 of half l / 32), with the slot XOR-swizzled by the piece's (group, half) so
//     that both the row-contiguous stores and the operand reads hit 16 distinct bank quads per 16 lanes.
//   * Per group and 32 x 32 tile: one v_mfma_i32_32x32x32_i8 gives the exact int32 dots I_g; one
//     v_mfma_f32_32x32x16_f16 with a single non-zero k slot gives the exact outer product d_x (x) d_w of the group's
//     f16 scales (q8_0 weight scales are f16, Q8_0-kind activation scales are f16-rounded); the VALU converts I_g and
//     accumulates with one FMA. Those two VALU ops per output per group bound the kernel, not the MFMA: the VALU does
//     64 lane-ops a clock per CU against the int8 MFMA's ~4096 multiply-adds, i.e. at most 32 outputs x 32 columns
//     per clock, a quarter of the int8 peak.
//   * Up to 64 rows (decode batches) the tile GEMM has too few tiles and too little in flight to stream the weights, so
//     gemm_q8_0_small_kernel takes over: a block owns 32 output columns, its W waves split K among themselves, every
//     lane loads its MFMA operand pieces straight from memory (no LDS staging) several groups ahead, and the waves'
//     partial tiles are summed in LDS in a fixed tree order.
#include "kf_knobs.h"
#include "kf_blocks.h"
#include "kf_host.h"
#include "kf_device.h"

#include <algorithm>
#include <type_traits>
#include <cstdlib>

// The split-K fixups rely on gfx9 cache behaviour (system-scope relaxed atomics write through to memory, stores are
// counted in vmcnt), not on a release/acquire pair: build for gfx950 only.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the split-K fixups assume gfx950's cache and counter behaviour"
#endif

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int GM_BK = 128;  // columns per stage: four 32-column groups
constexpr int GM_G = GM_BK / 32;
constexpr int GM_THREADS = 256;

template <int WM, int WN, int TM, int TN>
struct GmCfg {
    static_assert(WM * WN == 4, "four waves");
    static constexpr int BM = 32 * WM * TM, BN = 32 * WN * TN;
    static constexpr int A_BYTES = BM * GM_BK, B_BYTES = BN * GM_BK;
    static constexpr int SA = A_BYTES + B_BYTES;          // f16 activation scales [g][BM]
    static constexpr int SB = SA + GM_G * BM * 2;         // f16 weight scales [g][BN]
    static constexpr int STAGE = SB + GM_G * BN * 2;
    static constexpr int PA = BM * 8 / GM_THREADS;        // 16-byte pieces a thread moves per stage
    static constexpr int PB = BN * 8 / GM_THREADS;
    static constexpr int QA = (BM * GM_G + GM_THREADS - 1) / GM_THREADS;  // scales a thread moves per stage
    static constexpr int QB = (BN * GM_G + GM_THREADS - 1) / GM_THREADS;
    static_assert(PA >= 1 && PB >= 1, "a block tile spans at least 32 rows");
};

// Byte offset of the 16-byte piece (group g, tile row r, half h) in an operand tile of `tiles` 32-row tiles
__device__ __forceinline__ int gm_slot(int tiles, int g, int r, int h) {
    return (((g * tiles + (r >> 5)) * 2 + h) * 32 + ((r & 31) ^ ((g * 2 + h) << 1))) * 16;
}

// The piece a lane reads for the MFMA operand of tile t, group g: row lane % 32, half lane / 32
__device__ __forceinline__ int gm_operand(int tiles, int g, int t, int lane) {
    const int h = lane >> 5;
    return (((g * tiles + t) * 2 + h) * 32 + ((lane & 31) ^ ((g * 2 + h) << 1))) * 16;
}

template <class C>
struct GmStage {
    uint4 a[C::PA], b[C::PB];
    float dx[C::QA];
    uint32_t dw[C::QB];

    __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                         const float* __restrict__ xd32, int m0, int n0, int M, int N, int K, int st, int tid) {
        const int gb = st * GM_G;
        const int kg = K >> 5;
#pragma unroll
        for (int i = 0; i < C::PA; i++) {
            const int c = tid + GM_THREADS * i;  // eight consecutive threads read one row's 128 bytes
            const int m = min(m0 + (c >> 3), M - 1);
            a[i] = *reinterpret_cast<const uint4*>(xq + (int64_t)m * K + gb * 32 + (c & 7) * 16);
        }
#pragma unroll
        for (int i = 0; i < C::PB; i++) {
            const int c = tid + GM_THREADS * i;
            const int n = min(n0 + (c >> 3), N - 1);
            const int p = c & 7;
            const u32x4_a2 v = *reinterpret_cast<const u32x4_a2*>(w + (int64_t)n * row_bytes + (int64_t)(gb + (p >> 1)) * KF_Q8_0_BYTES + 2 +
                                                                  16 * (p & 1));
            b[i] = make_uint4(v.x, v.y, v.z, v.w);
        }
#pragma unroll
        for (int i = 0; i < C::QA; i++) {
            const int c = min(tid + GM_THREADS * i, C::BM * GM_G - 1);  // row c / 4, group c % 4
            const int m = min(m0 + (c >> 2), M - 1);
            dx[i] = xd32[(int64_t)m * kg + gb + (c & 3)];
        }
#pragma unroll
        for (int i = 0; i < C::QB; i++) {
            const int c = min(tid + GM_THREADS * i, C::BN * GM_G - 1);
            const int n = min(n0 + (c >> 2), N - 1);
            dw[i] = *reinterpret_cast<const uint16_t*>(w + (int64_t)n * row_bytes + (int64_t)(gb + (c & 3)) * KF_Q8_0_BYTES);
        }
    }

    __device__ __forceinline__ void store(uint8_t* buf, int tid) const {
#pragma unroll
        for (int i = 0; i < C::PA; i++) {
            const int c = tid + GM_THREADS * i;
            const int p = c & 7;
            *reinterpret_cast<uint4*>(buf + gm_slot(C::BM / 32, p >> 1, c >> 3, p & 1)) = a[i];
        }
#pragma unroll
        for (int i = 0; i < C::PB; i++) {
            const int c = tid + GM_THREADS * i;
            const int p = c & 7;
            *reinterpret_cast<uint4*>(buf + C::A_BYTES + gm_slot(C::BN / 32, p >> 1, c >> 3, p & 1)) = b[i];
        }
#pragma unroll
        for (int i = 0; i < C::QA; i++) {
            const int c = tid + GM_THREADS * i;
            // Q8_0-kind activation scales are f16-rounded values, so this conversion is exact
            if (C::QA * GM_THREADS == C::BM * GM_G || c < C::BM * GM_G)
                reinterpret_cast<_Float16*>(buf + C::SA)[(c & 3) * C::BM + (c >> 2)] = (_Float16)dx[i];
        }
#pragma unroll
        for (int i = 0; i < C::QB; i++) {
            const int c = tid + GM_THREADS * i;
            if (C::QB * GM_THREADS == C::BN * GM_G || c < C::BN * GM_G)
                reinterpret_cast<uint16_t*>(buf + C::SB)[(c & 3) * C::BN + (c >> 2)] = (uint16_t)dw[i];
        }
    }
};

// One block: output tile (blockIdx.y, blockIdx.x) over all of K
template <int WM, int WN, int TM, int TN>
__global__ void __launch_bounds__(GM_THREADS, 2) gemm_q8_0_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xd32, const float* __restrict__ bias,
                                                                  const float* __restrict__ res, float* __restrict__ y, int M, int N, int K) {
    using C = GmCfg<WM, WN, TM, TN>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * C::BM, n0 = blockIdx.x * C::BN;
    const int st0 = 0, st1 = K / GM_BK;

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = v16f{};

    GmStage<C> pf;
    pf.load(w, row_bytes, xq, xd32, m0, n0, M, N, K, st0, tid);
    pf.store(smem, tid);
    __syncthreads();
    for (int st = st0; st < st1; st++) {
        const uint8_t* buf = smem + ((st - st0) & 1) * C::STAGE;
        // the last stage reloads itself: an unconditional load keeps the prefetch registers out of any phi
        pf.load(w, row_bytes, xq, xd32, m0, n0, M, N, K, min(st + 1, st1 - 1), tid);
        // the operands of group g + 1 are read from LDS while group g is multiplied and rescaled; the scale operands
        // of the outer-product MFMA carry one f16 in k slot 0 (lanes < 32; lanes >= 32 hold k slots 8..15) and
        // zeros elsewhere, and only their first dword changes from group to group
        struct Ops {
            v4i a[TM], b[TN];
            uint32_t sa[TM], sb[TN];
        };
        auto read_ops = [&](Ops& o, int g) {
#pragma unroll
            for (int t = 0; t < TM; t++) {
                o.a[t] = *reinterpret_cast<const v4i*>(buf + gm_operand(C::BM / 32, g, wm * TM + t, lane));
                const uint16_t v = reinterpret_cast<const uint16_t*>(buf + C::SA)[g * C::BM + (wm * TM + t) * 32 + (lane & 31)];
                o.sa[t] = lane < 32 ? v : 0u;
            }
#pragma unroll
            for (int t = 0; t < TN; t++) {
                o.b[t] = *reinterpret_cast<const v4i*>(buf + C::A_BYTES + gm_operand(C::BN / 32, g, wn * TN + t, lane));
                o.sb[t] = reinterpret_cast<const uint16_t*>(buf + C::SB)[g * C::BN + (wn * TN + t) * 32 + (lane & 31)];
            }
        };
        Ops cur;
        read_ops(cur, 0);
#pragma unroll 1
        for (int g = 0; g < GM_G; g++) {
            Ops nxt;
            read_ops(nxt, min(g + 1, GM_G - 1));
#pragma unroll
            for (int i = 0; i < TM; i++) {
                v16i c[TN];
                v16f s[TN];
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[i], cur.b[j], v16i{}, 0, 0, 0);
                    const v4u sa = {cur.sa[i], 0u, 0u, 0u}, sb = {cur.sb[j], 0u, 0u, 0u};
                    s[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, sa), __builtin_bit_cast(v8h, sb), v16f{}, 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf((float)c[j][r], s[j][r], acc[i][j][r]);
            }
            cur = nxt;
        }
        if (st + 1 < st1) pf.store(smem + ((st + 1 - st0) & 1) * C::STAGE, tid);
        __syncthreads();
    }

    // 32 x 32 accumulator layout: lane l holds column l % 32; register r holds row (r % 4) + 8 * (r / 4) + 4 * (l / 32)
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + (wn * TN + j) * 32 + (lane & 31);
            if (n >= N) continue;
            const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + (wm * TM + i) * 32 + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
                if (m >= M) continue;
                const int64_t o = (int64_t)m * N + n;
                y[o] = acc[i][j][r] + bn + (res ? res[o] : 0.0f);
            }
        }
}

// Decode-batch product (up to MR activation rows). Block x owns 32 output columns [32 x, +32); its W waves take the
// 8-group chunks of K round-robin. A chunk is 272 bytes of each of the 32 weight rows (17 aligned 16-byte pieces, so a
// wave's loads cover about four rows each); the next chunk is in flight in registers while the current one is
// multiplied out of the wave's own LDS region (row stride 304 bytes, 76 dwords: consecutive rows start on distinct
// bank quads). Per group, 16 x 16 tile pair and activation tile, one v_mfma_i32_16x16x32_i8 gives the int32 dots (the
// weight operand read from LDS at its 2-byte aligned address, the activation operand loaded from memory in MFMA order:
// lane l holds row l % 16, bytes [8 (l / 16), +8) of the group, reused for both weight tiles) and one
// v_mfma_f32_16x16x16_f16 the outer product of the f16 scales. The waves' partial tiles are summed by a fixed-order
// tree in LDS.
typedef long v1l;
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t v2u_sk __attribute__((ext_vector_type(2)));
typedef int v4i_ __attribute__((ext_vector_type(4)));

// The 8 bytes at a 2-byte aligned LDS address as a long: aligned dwords realigned by v_alignbyte_b32 (an LDS read
// that is not dword aligned stalls). Reads only the dwords that hold the 8 bytes: a third one when they straddle it.
__device__ __forceinline__ long sk_lds_u64_a2(const uint8_t* p) {
    const uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(p) & 2u;
    const uint32_t* ap = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t d0 = ap[0], d1 = ap[1], d2 = ap[1 + (sh >> 1)];
    return (long)kf_alignbyte(d1, d0, sh) | ((long)kf_alignbyte(d2, d1, sh) << 32);
}

// Ablation switch for measurement builds only (0 in the product): bit 1 drops the MFMA/VALU arithmetic, bit 2 the
// LDS staging and operand reads, bit 4 the activation loads
#ifndef KF_SK_ABLATE
#define KF_SK_ABLATE 0
#endif
constexpr int SK_G = 8;                        // groups per chunk
constexpr int SK_WB = SK_G * KF_Q8_0_BYTES;    // 272 weight bytes per row per chunk
constexpr int SK_WP = SK_WB / 16;              // 17 pieces
constexpr int SK_STRIDE = 304;                 // LDS row stride
// A wave's weight tile: TN 16-column tiles (two for wide outputs, one when the output has at most one block of 16
// columns per CU, so that every CU gets a block)
template <int TN>
struct SkGeo {
    static constexpr int ROWS = 16 * TN;                     // weight rows of a wave
    static constexpr int WI = (ROWS * SK_WP + 63) / 64;      // load instructions for the weights (9 for TN = 2)
    static constexpr int WAVE_LDS = ROWS * SK_STRIDE;        // 9728 bytes for TN = 2: also holds one partial tile
};

// The activation operands and scales of one chunk, loaded together when the chunk starts (they are small and stay
// in L2, shared by every block)
template <int MR>
struct SkAct {
    static constexpr int TM = MR / 16;  // 16-row activation tiles
    uint32_t aq[TM][SK_G][2];           // this lane's 8 activation bytes of each tile and group
    v4f dx[TM][2];                      // the scales of this lane's activation row (lanes < 16 use them)

    __device__ __forceinline__ void load(const int8_t* __restrict__ xq, const float* __restrict__ xd32, const uint32_t (&aoff)[TM],
                                         const uint32_t (&doff)[TM], int ch) {
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const uint32_t ab = (uint32_t)ch * SK_G * 32;
#pragma unroll
        for (int t = 0; t < TM; t++) {
#pragma unroll
            for (int g = 0; g < SK_G; g++) {
                const v2u v = *reinterpret_cast<const v2u*>(xq + (aoff[t] + ab + 32 * g));
                aq[t][g][0] = v.x;
                aq[t][g][1] = v.y;
            }
            dx[t][0] = *reinterpret_cast<const v4f*>(xd32 + doff[t] + ch * SK_G);
            dx[t][1] = *reinterpret_cast<const v4f*>(xd32 + doff[t] + ch * SK_G + 4);
        }
    }
};

template <int MR, int SK_TN>
__global__ void __launch_bounds__(512) gemm_q8_0_small_kernel(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                                               const int8_t* __restrict__ xq, const float* __restrict__ xd32,
                                                                               const float* __restrict__ bias, const float* __restrict__ res,
                                                                               float* __restrict__ y, int M, int N, int K) {
    constexpr int TM = SkAct<MR>::TM;
    constexpr int SK_ROWS = SkGeo<SK_TN>::ROWS, SK_WI = SkGeo<SK_TN>::WI, SK_WAVE_LDS = SkGeo<SK_TN>::WAVE_LDS;
    extern __shared__ __align__(16) uint8_t smem[];
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t* lw = smem + wave * SK_WAVE_LDS;
    // XCD-aware order (a 1-D grid of gx weight tiles x gy row blocks): the hardware deals blocks to the 8 XCDs in
    // turn (block b to XCD b % 8), so XCD x takes a contiguous range of (tile, row block) pairs with a tile's row
    // blocks next to each other: they run together on one XCD and its L2 serves the tile's weights to all of them
    int tn, tm;
    {
        const int gy = (M + MR - 1) / MR, T = (int)gridDim.x, b = (int)blockIdx.x;
        const int t = (T & 7) ? b : (b & 7) * (T >> 3) + (b >> 3);
        tn = t / gy;
        tm = t - tn * gy;
    }
    const int n0 = tn * SK_ROWS, m0 = tm * MR;
    const int q = lane >> 4, c = lane & 15;  // operand k-quarter and row/column
    const int kg = K >> 5;
    const int chunks = kg / SK_G;  // K % 256 == 0: whole chunks

    // weight piece p = 64 i + lane is row p / 17, piece p % 17 (clamped: duplicates of the last piece). Byte offsets
    // fit in 32 bits (the launcher checks the weight and activation sizes).
    uint32_t woff[SK_WI];
#pragma unroll
    for (int i = 0; i < SK_WI; i++) {
        const int p = min(64 * i + lane, SK_ROWS * SK_WP - 1);
        woff[i] = (uint32_t)min(n0 + p / SK_WP, N - 1) * (uint32_t)row_bytes + 16 * (p % SK_WP);
    }
    uint32_t aoff[TM], doff[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) {
        const int m = min(m0 + 16 * t + c, M - 1);
        aoff[t] = (uint32_t)m * (uint32_t)K + 8 * q;
        doff[t] = (uint32_t)m * (uint32_t)kg;
    }

    v4f acc[TM][SK_TN];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int j = 0; j < SK_TN; j++) acc[t][j] = v4f{};
    // software pipeline over this wave's chunks. Loads complete in issue order (one vmcnt counter), so each
    // iteration issues chunk j+1's activations before its weights: multiplying chunk j then needs nothing in flight,
    // and the next iteration's single wait (for chunk j+1's weights) covers both. LDS operations of one wave complete
    // in order, so no barrier separates the staging from the reads, nor the reads of chunk j from the staging of j+1.
    v4u wq[SK_WI];
    auto load_w = [&](int chk) {
        const uint32_t wb = (uint32_t)chk * SK_WB;
#pragma unroll
        for (int i = 0; i < SK_WI; i++) wq[i] = *reinterpret_cast<const v4u*>(w + (woff[i] + wb));
    };
    int ch = wave;
    SkAct<MR> nact;
    nact.load(xq, xd32, aoff, doff, min(ch, chunks - 1));
    load_w(min(ch, chunks - 1));
    for (; ch < chunks; ch += W) {
        if (!(KF_SK_ABLATE & 2)) {
#pragma unroll
            for (int i = 0; i < SK_WI; i++) {
                const int p = min(64 * i + lane, SK_ROWS * SK_WP - 1);
                *reinterpret_cast<v4u*>(lw + (p / SK_WP) * SK_STRIDE + 16 * (p % SK_WP)) = wq[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < SK_WI; i++) acc[0][0][0] += __builtin_bit_cast(float, wq[i].x ^ wq[i].w);
        }
        const SkAct<MR> act = nact;
        if (ch + W < chunks) {  // uniform
            if (!(KF_SK_ABLATE & 4)) nact.load(xq, xd32, aoff, doff, ch + W);
            load_w(ch + W);
        }

#pragma unroll
        for (int g = 0; g < SK_G; g++) {
            if (KF_SK_ABLATE & 3) {
                if (!(KF_SK_ABLATE & 2)) acc[0][0][0] += __builtin_bit_cast(float, *reinterpret_cast<const uint32_t*>(lw + c * SK_STRIDE + 34 * g));
                acc[0][0][1] += __builtin_bit_cast(float, act.aq[0][g][0]);
                continue;
            }
            long b[SK_TN];
            v4h sb[SK_TN];
#pragma unroll
            for (int j = 0; j < SK_TN; j++) {
                const uint8_t* wp = lw + (16 * j + c) * SK_STRIDE + g * KF_Q8_0_BYTES;
                b[j] = sk_lds_u64_a2(wp + 2 + 8 * q);
                sb[j] = v4h{};
                sb[j][0] = q == 0 ? *reinterpret_cast<const _Float16*>(wp) : (_Float16)0.0f;
            }
#pragma unroll
            for (int t = 0; t < TM; t++) {
                const long a = (long)act.aq[t][g][0] | ((long)act.aq[t][g][1] << 32);
                const float d = act.dx[t][g >> 2][g & 3];
                v4h sa = v4h{};
                sa[0] = q == 0 ? (_Float16)d : (_Float16)0.0f;  // f16-rounded scales: exact
#pragma unroll
                for (int j = 0; j < SK_TN; j++) {
                    const v4i_ ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b[j], v4i_{}, 0, 0, 0);
                    const v4f sc = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, sb[j], v4f{}, 0, 0, 0);
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[t][j][k] = fmaf((float)ci[k], sc[k], acc[t][j][k]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the groups apart: bounded registers
        }
    }

    // fixed-order tree over the waves (W a power of two): the upper half stores its tile, the lower half adds
    __syncthreads();
    for (int half = W / 2; half >= 1; half >>= 1) {
        if (wave >= half && wave < 2 * half) {
            float* p = reinterpret_cast<float*>(smem + (wave - half) * SK_WAVE_LDS) + lane;
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int j = 0; j < SK_TN; j++)
#pragma unroll
                    for (int k = 0; k < 4; k++) p[((t * SK_TN + j) * 4 + k) * 64] = acc[t][j][k];
        }
        __syncthreads();
        if (wave < half) {
            const float* p = reinterpret_cast<const float*>(smem + wave * SK_WAVE_LDS) + lane;
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int j = 0; j < SK_TN; j++)
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[t][j][k] += p[((t * SK_TN + j) * 4 + k) * 64];
        }
        __syncthreads();
    }
    if (wave != 0) return;
    // 16 x 16 accumulator layout: lane l holds column l % 16, register k holds row 4 (l / 16) + k
#pragma unroll
    for (int j = 0; j < SK_TN; j++) {
        const int n = n0 + 16 * j + c;
        if (n >= N) continue;
        const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int t = 0; t < TM; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int m = m0 + 16 * t + 4 * q + k;
                if (m >= M) continue;
                const int64_t o = (int64_t)m * N + n;
                y[o] = acc[t][j][k] + bn + (res ? res[o] : 0.0f);
            }
    }
}

// XCD-aware tile order. Workgroups go to the eight XCDs round-robin by linear block id, and each XCD has its own L2.
// Block b runs tile t = (b % 8) * (T / 8) + b / 8, so XCD x works through the contiguous tile range
// [x T / 8, (x + 1) T / 8). Tiles are numbered M-fastest, so an XCD's range is a few weight tiles against every
// activation panel: the blocks in flight on an XCD share their weight tiles, every weight byte crosses HBM once, and
// only the (smaller, MALL-resident) activations are streamed per XCD. Numbered N-fastest, each XCD would stream the
// whole weight matrix once per activation panel pair (measured: about 1 GB per 62 MB GEMM and no faster kernel).
// Identity when T is not a multiple of eight.
__device__ __forceinline__ void gm_tile(int nt, int mt, int& tm, int& tn) {
    const int T = nt * mt, b = blockIdx.x;
    const int t = (T & 7) ? b : (b & 7) * (T >> 3) + (b >> 3);
    tn = t / mt;
    tm = t - tn * mt;
}

// The grid's tail (the DMA GEMM, two blocks a CU): when the tiles leave a last round of blocks at most half full, the
// tiles from `full` on run as two blocks each over the two halves of K; each half writes its partial tile to `part`
// ([tail tile][half][register][thread]) and the second to arrive (a ticket per tail tile) adds the other's in half
// order and stores the tile. part == nullptr: no split.
struct GmTail {
    float* part;
    int* tickets;
    int full;
};

// ----------------------------------------------------------------------------------- q8_0 prefill GEMM, DMA staging
// The product of gemm_q8_0_kernel (per group and 32 x 32 tile: the exact int32 dots I_g from v_mfma_i32_32x32x32_i8,
// the outer product d_x (x) d_w of the f16 scales from one v_mfma_f32_32x32x16_f16 with a single non-zero k slot,
// then a convert and an FMA per output) with all staging done by buffer_load ... lds DMA over buffer resources (per-lane
// offsets fixed for the K loop, a stage adding a scalar offset), as in the q4_K GEMM:
//   * activations: [group][32-row tile] 1 KB blocks in MFMA order, one DMA instruction each;
//   * weights: a stage's four q8_0 blocks of a row are 136 bytes at row offset 136 st, 8-byte aligned; each row's
//     16-byte aligned 144-byte window around them is copied whole ([row][144] in LDS: nine 16-byte pieces, the
//     stage's data at offset (136 st) % 16), so the DMA needs only aligned pieces. Rows are 16-byte aligned when
//     K % 256 == 0, and the last stage (st odd) ends exactly at the row's end;
//   * activation scales: [row][4] f32 per stage.
// The DMA is inline assembly (kf_adma16): issued through the builtin, it carries no alias information, so the
// compiler waited for every DMA in flight (the next stage's included) before the first LDS read of each stage and the
// double buffer never overlapped. The waits are explicit instead: each stage ends with vmcnt(0) and a barrier, after
// which the other buffer's DMA (issued at the stage's start) has landed. Eight waves, each a 64 x 32 tile;
// blocks in XCD order. Wave tiles of 2 x 2 measured slower (their 128 x 256 block halves the blocks per CU).
// gemm_q8_0_kernel (register staging) remains for K % 256 != 0.
template <int WM, int WN, int TM, int TN>
struct GqCfg {
    static constexpr int W = WM * WN, THREADS = 64 * W;
    static constexpr int BM = 32 * WM * TM, BN = 32 * WN * TN;
    static constexpr int MT = BM / 32, NT = BN / 32;
    static constexpr int ROW = 144;                       // LDS bytes of a weight row's window
    static constexpr int A_BYTES = MT * GM_G * 1024;
    static constexpr int B_OFF = A_BYTES, B_BYTES = BN * ROW;
    static constexpr int D_OFF = B_OFF + B_BYTES, D_BYTES = ((BM + 63) / 64) * 1024;
    static constexpr int STAGE = D_OFF + D_BYTES;
    static constexpr int NA = MT * GM_G, NB = (BN * 9 + 63) / 64, ND = (BM + 63) / 64;
    static_assert(BN * 9 % 64 == 0, "whole DMA instructions for the weight windows");
};

template <int WM, int WN, int TM, int TN>
__global__ void __launch_bounds__(64 * WM * WN, 8 / (WM * WN)) gemm_q8_0_dma_kernel(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                                     const int8_t* __restrict__ xq, const float* __restrict__ xd32,
                                                                     const float* __restrict__ bias, const float* __restrict__ res,
                                                                     float* __restrict__ y, int M, int N, int K, GmTail tail) {
    using C = GqCfg<WM, WN, TM, TN>;
    __shared__ __align__(16) uint8_t buf0[C::STAGE];
    __shared__ __align__(16) uint8_t buf1[C::STAGE];
    __shared__ int last;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int mt = (M + C::BM - 1) / C::BM;
    const int kg = K >> 5;
    const int nst = K / GM_BK;
    int tm, tn;
    int s0 = 0, s1 = nst, half_k = -1, tt = 0;  // stages [s0, s1) (even counts); a tail block's half and tail tile
    if (tail.part && (int)blockIdx.x >= tail.full) {
        const int b = blockIdx.x - tail.full;
        tt = b >> 1;
        half_k = b & 1;
        const int t = tail.full + tt;
        tn = t / mt;
        tm = t - tn * mt;
        s0 = half_k ? nst / 2 : 0;
        s1 = half_k ? nst : nst / 2;
    } else {
        const int T = tail.part ? tail.full : ((N + C::BN - 1) / C::BN) * mt, b = blockIdx.x;
        const int t = (T & 7) ? b : (b & 7) * (T >> 3) + (b >> 3);
        tn = t / mt;
        tm = t - tn * mt;
    }
    const int m0 = tm * C::BM, n0 = tn * C::BN;
    const int half = lane >> 5, r32 = lane & 31;

    // DMA sources: buffer resources over the tile's first rows; per-lane offsets fixed for the K loop, a stage adds
    // only a scalar offset (rows past M or N are clamped to the last one)
    const auto rw = kf_arsrc(w + (int64_t)n0 * row_bytes, (uint64_t)(N - n0) * row_bytes);
    const auto rx = kf_arsrc(xq + (int64_t)m0 * K, (uint64_t)(M - m0) * K);
    const auto rd = kf_arsrc(xd32 + (int64_t)m0 * kg, (uint64_t)(M - m0) * kg * 4);
    constexpr int IA = (C::NA + C::W - 1) / C::W, IB = (C::NB + C::W - 1) / C::W, ID = (C::ND + C::W - 1) / C::W;
    int va[IA], vb[IB], vd[ID];
#pragma unroll
    for (int it = 0; it < IA; it++) {
        const int q = wave + it * C::W, g = q / C::MT, t = q % C::MT;
        va[it] = (min(m0 + t * 32 + r32, M - 1) - m0) * K + g * 32 + half * 16;
    }
#pragma unroll
    for (int it = 0; it < IB; it++) {
        const int p = (wave + it * C::W) * 64 + lane, r = p / 9, pc = p - 9 * r;
        vb[it] = (min(n0 + r, N - 1) - n0) * (int)row_bytes + 16 * pc;
    }
#pragma unroll
    for (int it = 0; it < ID; it++) vd[it] = (min(m0 + (wave + it * C::W) * 64 + lane, M - 1) - m0) * kg * 4;
    auto dma = [&](int st, uint8_t* buf) {
#pragma unroll
        for (int it = 0; it < IA; it++) {
            const int q = wave + it * C::W;
            if (C::NA % C::W == 0 || q < C::NA) kf_adma16(rx, va[it], st * GM_BK, buf + q * 1024);
        }
        const int wbase = (136 * st) & ~15;
#pragma unroll
        for (int it = 0; it < IB; it++) {
            const int q = wave + it * C::W;
            if (C::NB % C::W == 0 || q < C::NB) kf_adma16(rw, vb[it], wbase, buf + C::B_OFF + q * 1024);
        }
#pragma unroll
        for (int it = 0; it < ID; it++) {
            const int q = wave + it * C::W;
            if (q < C::ND) kf_adma16(rd, vd[it], st * GM_G * 4, buf + C::D_OFF + q * 1024);
        }
    };

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = v16f{};

    // one group per trip: fully unrolled, the scheduler hoists every group's MFMAs above the rescales and spills
    // the scales' operand tuples (the f16 scale at k = 0, zeros elsewhere) live across the stages: only their first
    // register changes per group, so the zeros are not rebuilt every time
    v4u ua[TM], ub[TN];
#pragma unroll
    for (int i = 0; i < TM; i++) ua[i] = v4u{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < TN; j++) ub[j] = v4u{0u, 0u, 0u, 0u};
    auto stage = [&](const uint8_t* buf, int st) {
        const int wo = (136 * st) & 15;  // the stage's offset in its weight windows
#pragma unroll 1
        for (int g = 0; g < GM_G; g++) {
            v4i a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                a[i] = *reinterpret_cast<const v4i*>(buf + ((g * C::MT + wm * TM + i) * 64 + lane) * 16);
                // Q8_0-kind activation scales are f16-rounded values, so this conversion is exact
                const float dx = reinterpret_cast<const float*>(buf + C::D_OFF)[((wm * TM + i) * 32 + r32) * 4 + g];
                ua[i].x = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)dx) & (uint32_t)(half - 1);  // lanes >= 32: zero
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint8_t* rp = buf + C::B_OFF + ((wn * TN + j) * 32 + r32) * C::ROW + wo + g * KF_Q8_0_BYTES;
                // the 16 weight bytes start 2 bytes past a dword boundary in even groups and on one in odd groups
                // (windows and rows are 16-byte aligned, blocks 34 bytes): five aligned dwords and a byte realignment
                // instead of a 2-byte aligned 16-byte read, which stalls the LDS
                const int sh = (g & 1) ? 0 : 2;
                const uint32_t* ap = reinterpret_cast<const uint32_t*>(rp + 2 + 16 * half - sh);
                const uint32_t d0 = ap[0], d1 = ap[1], d2 = ap[2], d3 = ap[3], d4 = ap[4];
                b[j] = v4i{(int)kf_alignbyte(d1, d0, sh), (int)kf_alignbyte(d2, d1, sh), (int)kf_alignbyte(d3, d2, sh),
                           (int)kf_alignbyte(d4, d3, sh)};
                ub[j].x = *reinterpret_cast<const uint16_t*>(rp);
            }
            v16i c[TM][TN];
            v16f s[TM][TN];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], v16i{}, 0, 0, 0);
                    s[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, ua[i]), __builtin_bit_cast(v8h, ub[j]), v16f{}, 0, 0, 0);
                }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf((float)c[i][j][r], s[i][j][r], acc[i][j][r]);
        }
    };

    dma(s0, buf0);
    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
    __syncthreads();
#pragma unroll 1
    for (int st = s0; st < s1; st += 2) {
        // the stage count is even (K % 256 == 0; halves: K % 512 == 0)
        dma(st + 1, buf1);
        stage(buf0, st);
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
        if (st + 2 < s1) dma(st + 2, buf0);
        stage(buf1, st + 1);
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
    }

    if (half_k >= 0) {
        // a tail half: its partial tile through system-scope stores (they write through to memory, so the other
        // half's block sees them from any XCD without an L2 write-back), a ticket, and the second to arrive adds
        constexpr int R = TM * TN * 16;
        float* pp = tail.part + (size_t)(2 * tt + half_k) * R * C::THREADS + tid;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    __hip_atomic_store(pp + ((i * TN + j) * 16 + r) * C::THREADS, acc[i][j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
        if (tid == 0) last = __hip_atomic_fetch_add(&tail.tickets[tt], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 1;
        __syncthreads();
        if (!last) return;
        const float* po = tail.part + (size_t)(2 * tt + (half_k ^ 1)) * R * C::THREADS + tid;
        float other[R];
#pragma unroll
        for (int k = 0; k < R; k++) other[k] = __hip_atomic_load(po + k * C::THREADS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float o = other[(i * TN + j) * 16 + r];
                    acc[i][j][r] = half_k ? o + acc[i][j][r] : acc[i][j][r] + o;
                }
        if (tid == 0) __hip_atomic_store(&tail.tickets[tt], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }

    // 32 x 32 accumulator layout: lane l holds column l % 32; register r holds row (r % 4) + 8 (r / 4) + 4 (l / 32)
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + (wn * TN + j) * 32 + r32;
            if (n >= N) continue;
            const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + (wm * TM + i) * 32 + (r & 3) + 8 * (r >> 2) + 4 * half;
                if (m >= M) continue;
                const int64_t o = (int64_t)m * N + n;
                y[o] = acc[i][j][r] + bn + (res ? res[o] : 0.0f);
            }
        }
}

// ------------------------------------------------------------------------------------------------ 49..64 rows
// gemm_q8_0_small_kernel holds a wave's activation operands in registers, so it carries 16 rows (32 spill); past 16
// rows each further 16-row block streams the weights again. Here a wave holds all 64 (MR_ROWS) rows of its K chunk
// in LDS instead: per chunk of 4 groups (128 columns) it DMAs the rows' 128 int8 bytes, their 4 scales (group-major)
// and its weight rows' 136 bytes into one of three buffers, two chunks ahead of the one it multiplies, so a weight
// byte is read once for all the rows. Rows of a buffer are 128 bytes with 16-byte slot s of row r holding piece
// s ^ (r % 8), so the MFMA operand reads (16 rows, 8 bytes each) spread over the banks; rows past M and N read as
// zeros (buffer range check) and are not stored. The block's W waves split K (chunk c to wave c % W) and meet in a
// fixed-order tree. Per output and group: one int8 MFMA lane result, d_x d_w (exact: both are f16 values) and one
// FMA, as the small kernel. What bounds it: every block re-reads all M x K activation bytes, M / 16 times its weight
// bytes, so it beats four 16-row passes only where it measured so (see the launcher).
constexpr int MR_ROWS = 64, MR_TM = MR_ROWS / 16;
constexpr int MR_G = 4;                                   // groups per chunk
constexpr int MR_ACT = MR_ROWS * MR_G * 32;               // 8192 bytes of activations a chunk
constexpr int MR_ABUF = MR_ACT + MR_ROWS * MR_G * 4;      // + the scales: 9216
constexpr int MR_WCH = MR_G * KF_Q8_0_BYTES;              // 136 weight bytes a row and chunk


// The kernel below issues its LDS DMA through inline assembly (kf_adma16 / kf_adma4): the compiler's own waits for
// DMA-written LDS were conservative here (a read of one buffer waited for the DMA into another, serializing the
// chunks); every wait is explicit instead.
template <int TN, int W>
__global__ void __launch_bounds__(64 * W) gemm_q8_0_mr_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                              const float* __restrict__ xd32, const float* __restrict__ bias,
                                                              const float* __restrict__ res, float* __restrict__ y, int M, int N, int K) {
    constexpr int ROWS = 16 * TN;                  // weight rows of the block (every wave: all of them, its own K chunks)
    constexpr int WB = ROWS * MR_WCH;              // weight bytes a chunk, rows MR_WCH apart in the buffer
    constexpr int WI = (WB / 4 + 63) / 64;         // dword DMA instructions for them
    constexpr int BUF = MR_ABUF + WI * 256;        // one chunk: activations, scales, weights
    constexpr int NI = MR_ROWS / 8 + MR_G + WI;    // memory instructions a chunk
    static_assert(2 * NI <= 63, "two chunks in flight fit the vmcnt counter");
    static_assert(BUF >= MR_TM * TN * 4 * 64 * 4, "a wave's buffer holds its partial tile for the tree");
    __shared__ __align__(16) uint8_t abuf0[W * BUF];
    __shared__ __align__(16) uint8_t abuf1[W * BUF];
    __shared__ __align__(16) uint8_t abuf2[W * BUF];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * ROWS;
    const int kg = K >> 5;
    const int chunks = K / (32 * MR_G);
    uint8_t* const ab[3] = {abuf0 + wave * BUF, abuf1 + wave * BUF, abuf2 + wave * BUF};

    // activation DMA sources: instruction i (rows 8 i..) lane l: row 8 i + l / 8, piece (l % 8) ^ (row % 8); scales:
    // lane l row l, 16 bytes
    const kf_arsrc_t rx = kf_arsrc(xq, (uint64_t)M * K);
    const kf_arsrc_t rd = kf_arsrc(xd32, (uint64_t)M * kg * 4);
    const int xr = lane >> 3, xs = lane & 7;
    const int va = xr * K + 16 * (xs ^ (xr & 7));  // + 8 i K for instruction i (row 8 i + xr: same row % 8)
    const int vd = lane * kg * 4;  // scales: instruction g moves group g of the 64 rows (lane l: row l), [group][row]
    // weight DMA: instruction i lane l moves the dword at byte e = 256 i + 4 l of the chunk's [ROWS][136] block: row
    // e / 136, offset e % 136 (rows past N read as zeros: the resource ends at the matrix's last row)
    const kf_arsrc_t rw = kf_arsrc(w + (int64_t)n0 * row_bytes, (uint64_t)max(N - n0, 0) * row_bytes);
    int vw[WI];
#pragma unroll
    for (int i = 0; i < WI; i++) {
        const int e = min(256 * i + 4 * lane, WB - 4);
        const int r = e / MR_WCH;
        vw[i] = r * (int)row_bytes + (e - r * MR_WCH);
    }

    // every wave issues the same number of memory instructions per chunk slot (a slot past its last chunk reloads the
    // last one), so the vmcnt counts below are exact
    const int last = chunks - 1;
    auto issue = [&](auto kb, int ch) __attribute__((always_inline)) {
        constexpr int B = decltype(kb)::value;
        const int cc = min(ch, last);
#pragma unroll
        for (int i = 0; i < MR_ROWS / 8; i++) kf_adma16(rx, va + 8 * i * K, cc * (32 * MR_G), ab[B] + 1024 * i);
#pragma unroll
        for (int g = 0; g < MR_G; g++) kf_adma4(rd, vd, (cc * MR_G + g) * 4, ab[B] + MR_ACT + 256 * g);
#pragma unroll
        for (int i = 0; i < WI; i++) kf_adma4(rw, vw[i], cc * MR_WCH, ab[B] + MR_ABUF + 256 * i);
    };

    v4f acc[MR_TM][TN];
#pragma unroll
    for (int t = 0; t < MR_TM; t++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[t][j] = v4f{};

    // one chunk out of activation buffer B and the parked weights
    auto compute = [&](auto kb) __attribute__((always_inline)) {
        constexpr int B = decltype(kb)::value;
        const uint8_t* a_b = ab[B];
#pragma unroll
        for (int g = 0; g < MR_G; g++) {
            long b[TN];
            float dw[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint8_t* wp = a_b + MR_ABUF + (16 * j + c) * MR_WCH + g * KF_Q8_0_BYTES;
                b[j] = sk_lds_u64_a2(wp + 2 + 8 * q);
                dw[j] = (float)*reinterpret_cast<const _Float16*>(wp);
            }
#pragma unroll
            for (int t = 0; t < MR_TM; t++) {
                const int r = 16 * t + c;
                const int sl = (2 * g + (q >> 1)) ^ (r & 7);
                const long a = *reinterpret_cast<const long*>(a_b + r * (32 * MR_G) + 16 * sl + 8 * (q & 1));
                // the output lane holds activation rows 16 t + 4 q + k: their four scales of group g, one read
                const v4f dx = *reinterpret_cast<const v4f*>(a_b + MR_ACT + 256 * g + 4 * (16 * t + 4 * q));
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i_ ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b[j], v4i_{}, 0, 0, 0);
                    // d_x d_w I: the f32 products the reference forms (d_x and d_w are f16 values, so d_x d_w is exact)
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[t][j][k] = fmaf((float)ci[k], dx[k] * dw[j], acc[t][j][k]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the groups apart: bounded registers
        }
    };

    // the wave's chunks wave, wave + W, ...: slot i uses buffer i % 3, and chunk i + 2 is requested before chunk i is
    // multiplied. Loads complete in issue order, so waiting until the two later chunks' 2 NI instructions are the only
    // ones outstanding lands chunk i (DMA into LDS, which the compiler's register waits do not track). Nothing in the
    // loop writes LDS, so the compiler adds no waits of its own for the DMA in flight.
    const int mine = chunks > wave ? (chunks - wave + W - 1) / W : 0;
    auto step = [&](auto kb, int i) __attribute__((always_inline)) {
        constexpr int B = decltype(kb)::value;
        constexpr int B2 = (B + 2) % 3;
        issue(std::integral_constant<int, B2>{}, wave + (i + 2) * W);
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(2 * NI));
        compute(kb);
    };
    if (mine > 0) {
        issue(std::integral_constant<int, 0>{}, wave);
        issue(std::integral_constant<int, 1>{}, wave + W);
        step(std::integral_constant<int, 0>{}, 0);
        for (int i = 1; i < mine; i += 3) {
            step(std::integral_constant<int, 1>{}, i);
            if (i + 1 >= mine) break;
            step(std::integral_constant<int, 2>{}, i + 1);
            if (i + 2 >= mine) break;
            step(std::integral_constant<int, 0>{}, i + 2);
        }
    }
    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));  // the reloads past the last chunk land before the buffers are reused

    // fixed-order tree over the waves (W a power of two): the upper half stores its tile, the lower half adds
    if (W > 1) {
        __syncthreads();
        for (int half = W / 2; half >= 1; half >>= 1) {
            if (wave >= half && wave < 2 * half) {
                float* p = reinterpret_cast<float*>(abuf0 + (wave - half) * BUF) + lane;
#pragma unroll
                for (int t = 0; t < MR_TM; t++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int k = 0; k < 4; k++) p[((t * TN + j) * 4 + k) * 64] = acc[t][j][k];
            }
            __syncthreads();
            if (wave < half) {
                const float* p = reinterpret_cast<const float*>(abuf0 + wave * BUF) + lane;
#pragma unroll
                for (int t = 0; t < MR_TM; t++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int k = 0; k < 4; k++) acc[t][j][k] += p[((t * TN + j) * 4 + k) * 64];
            }
            __syncthreads();
        }
    }
    if (wave != 0) return;
    // 16 x 16 accumulator layout: lane l holds weight row l % 16 of tile j, register k activation row 4 (l / 16) + k
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + 16 * j + c;
        if (n >= N) continue;
        const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int t = 0; t < MR_TM; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int m = 16 * t + 4 * q + k;
                if (m >= M) continue;
                const int64_t o = (int64_t)m * N + n;
                y[o] = acc[t][j][k] + bn + (res ? res[o] : 0.0f);
            }
    }
}

// ------------------------------------------------------------------------------------------------ split K
// 1..64 rows with K split across blocks. A block of four waves owns 64 TN weight rows (16 TN a wave) and all TM x 16
// activation rows, over its share of K in chunks of G groups: the activation chunk (TM x 16 rows x 32 G columns and
// their group scales, 16-byte piece s of row r staged in slot s ^ (r % 2G) for bank-spread operand reads) is DMA'd
// once per block and read by all four waves, so the activation bytes moved are about M / (64 TN) times the weight
// bytes; the K split gives the grid about two blocks a CU even where the N / (64 TN) tiles are few. A row's 34 G
// weight bytes of a chunk touch 2, 3 or 5 cache lines for G = 4, 8, 16: the L1's outstanding requests bound the
// rate, so longer chunks move more bytes a request. NS stages ring (NS - 1 chunks in flight while one is
// multiplied), one barrier a chunk.
// Each block writes its partial tile to the scratch, and the last block of a tile to arrive (an atomic ticket per
// tile) adds the partials in split order (deterministic whatever the arrival order), adds bias and residual, stores y
// and resets the ticket; nothing waits on another block. All of the DMA goes through kf_adma16 / kf_adma4 with
// explicit waits (the compiler would otherwise drain the ring before every LDS read).
template <int TM, int TN, int G>
struct SplitGeo {
    static constexpr int R = 16 * TM;                      // activation rows staged
    static constexpr int BR = 64 * TN;                     // weight rows of a block
    static constexpr int RB = 32 * G;                      // bytes of an activation row of a chunk
    static constexpr int P = 2 * G;                        // its 16-byte pieces
    static constexpr int RI = 1024 / RB;                   // rows a 16-byte DMA instruction covers
    static constexpr int ACT = R * RB;                     // activation bytes of a chunk
    static constexpr int AB = ACT + G * R * 4;             // + the scales, group-major [group][row]
    static constexpr int WCH = G * KF_Q8_0_BYTES;          // weight bytes a row and chunk
    static constexpr int WB = 16 * TN * WCH;               // a wave's weight bytes of a chunk
    static constexpr int WI = (WB / 4 + 63) / 64;          // dword DMA instructions for them
    static constexpr int STAGE = AB + 4 * WB;
    static constexpr int AI = R / (4 * RI);                // 16-byte activation DMA instructions a wave
    static constexpr int DI = G / 4;                       // scale DMA instructions a wave (one group each)
    static constexpr int NI = AI + DI + WI;                // DMA instructions a wave issues per chunk
    static constexpr int TILE = 64 * BR;                   // floats of a partial tile (64 rows at most)
    static_assert(R % (4 * RI) == 0 && G % 4 == 0, "whole instructions a wave");
};

// wait until at most `rem` chunks after the current one (NI instructions each) are still in flight (rem <= RMAX)
template <int NI, int RMAX>
__device__ __forceinline__ void sk_wait(int rem) {
    if constexpr (RMAX == 0) {
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
    } else {
        if (rem >= RMAX)
            __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(NI * RMAX));
        else
            sk_wait<NI, RMAX - 1>(rem);
    }
}

// Ablation switch for measurement builds only (0 in the product): bit 1 drops the MFMA / VALU work of a chunk, bit 2
// the split epilogue (partials, ticket and fixup: each block stores its own tile), bit 4 the chunks' DMA (the compute
// reads whatever the LDS holds)
#ifndef SK_ABL
#define SK_ABL 0
#endif


template <int TM, int TN, int G, int NS>
__global__ void __launch_bounds__(256) gemm_q8_0_sk_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                           const float* __restrict__ xd32, const float* __restrict__ bias,
                                                           const float* __restrict__ res, float* __restrict__ y, int M, int N, int K, int S,
                                                           int* __restrict__ tickets, float* __restrict__ part) {
    using Geo = SplitGeo<TM, TN, G>;
    extern __shared__ __align__(16) uint8_t sk_ring[];     // NS stages of Geo::STAGE bytes
    __shared__ int last;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    // the splits of a tile are consecutive blocks: they run together, and the last of them finishes the tile
    const int tile = blockIdx.x / S, sp = blockIdx.x - tile * S;
    const int n0 = tile * Geo::BR;
    const int kg = K >> 5;
    const int chunks = K / (32 * G);
    const int ch0 = (int)((int64_t)chunks * sp / S), ch1 = (int)((int64_t)chunks * (sp + 1) / S);
    const int nch = ch1 - ch0;

    // activation DMA: RI-row instructions w + 4 i (lane l: row RI (w + 4 i) + l / P, piece (l % P) ^ (row % P)),
    // and the scales of groups w + 4 i (lane l: row l, lanes past the staged rows idle)
    const kf_arsrc_t rx = kf_arsrc(xq, (uint64_t)M * K);
    const kf_arsrc_t rd = kf_arsrc(xd32, (uint64_t)M * kg * 4);
    const int xr = lane / Geo::P, xs = lane % Geo::P;
    int va[Geo::AI];
#pragma unroll
    for (int i = 0; i < Geo::AI; i++) {
        const int row = Geo::RI * (wave + 4 * i) + xr;
        va[i] = row * K + 16 * (xs ^ (row % Geo::P));
    }
    const int vd = lane * kg * 4;
    // weight DMA: the wave's 16 TN rows, dword e = 64 i + lane of the chunk's [16 TN][136] block (rows past N read
    // zeros)
    const int wr0 = n0 + 16 * TN * wave;
    const kf_arsrc_t rw = kf_arsrc(w + (int64_t)min(wr0, N) * row_bytes, (uint64_t)max(N - wr0, 0) * row_bytes);
    int vw[Geo::WI];
#pragma unroll
    for (int i = 0; i < Geo::WI; i++) {
        const int e = min(256 * i + 4 * lane, Geo::WB - 4);
        const int r = e / Geo::WCH;
        vw[i] = r * (int)row_bytes + (e - r * Geo::WCH);
    }
    auto issue = [&](auto kb, int ch) __attribute__((always_inline)) {
        if (SK_ABL & 4) return;
        uint8_t* b = sk_ring + decltype(kb)::value * Geo::STAGE;
        const int cc = ch0 + ch;
#pragma unroll
        for (int i = 0; i < Geo::AI; i++) kf_adma16(rx, va[i], cc * Geo::RB, b + 1024 * (wave + 4 * i));
#pragma unroll
        for (int i = 0; i < Geo::DI; i++)
            if (Geo::R == 64 || lane < Geo::R) kf_adma4(rd, vd, (cc * G + wave + 4 * i) * 4, b + Geo::ACT + Geo::R * 4 * (wave + 4 * i));
        uint8_t* wb = b + Geo::AB + wave * Geo::WB;
        // the last instruction on the lanes that still hold bytes of the rows (an instruction writes 256 bytes)
#pragma unroll
        for (int i = 0; i < Geo::WI; i++)
            if ((Geo::WB / 4) % 64 == 0 || i + 1 < Geo::WI || lane < (Geo::WB / 4) % 64) kf_adma4(rw, vw[i], cc * Geo::WCH, wb + 256 * i);
    };

    v4f acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[t][j] = v4f{};
    auto compute = [&](auto kb) __attribute__((always_inline)) {
        const uint8_t* b = sk_ring + decltype(kb)::value * Geo::STAGE;
        const uint8_t* wr = b + Geo::AB + wave * Geo::WB + c * Geo::WCH;
#pragma unroll
        for (int g = 0; g < G; g++) {
            // the scales' outer product d_x d_w on the matrix cores (A and B hold them at k = 0, zeros elsewhere):
            // both are f16 values, so the f32 products are exact, and the VALU keeps one conversion and one FMA
            long bq[TN];
            v4h sb[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint8_t* wp = wr + 16 * j * Geo::WCH + g * KF_Q8_0_BYTES;
                bq[j] = sk_lds_u64_a2(wp + 2 + 8 * q);
                const _Float16 dw = *reinterpret_cast<const _Float16*>(wp);
                sb[j] = v4h{};
                sb[j][0] = q == 0 ? dw : (_Float16)0.0f;
            }
#pragma unroll
            for (int t = 0; t < TM; t++) {
                const int r = 16 * t + c;
                const int sl = (2 * g + (q >> 1)) ^ (r % Geo::P);
                const long a = *reinterpret_cast<const long*>(b + r * Geo::RB + 16 * sl + 8 * (q & 1));
                // the row's scale at k = 0 of every k-block: sb is zero past k = 0, so the copies on lanes q > 0 meet
                // zeros; Q8_0-kind activation scales are f16-rounded values, so the truncating conversion is exact
                const float dx = *reinterpret_cast<const float*>(b + Geo::ACT + Geo::R * 4 * g + 4 * r);
                const v4h sa = __builtin_bit_cast(v4h, v2u_sk{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(dx, 0.0f)), 0u});
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i_ ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq[j], v4i_{}, 0, 0, 0);
                    const v4f sc = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, sb[j], v4f{}, 0, 0, 0);
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[t][j][k] = fmaf((float)ci[k], sc[k], acc[t][j][k]);
                }
            }
        }
    };
    // chunk i: wait for this wave's share of it (loads complete in issue order; the chunks after it, up to NS - 2,
    // may stay in flight), the barrier makes every wave's share visible and frees the stage chunk i + NS - 1 lands in
    // (chunk i - 1's)
    auto step = [&](auto kb, int i) __attribute__((always_inline)) {
        constexpr int B = decltype(kb)::value;
        sk_wait<Geo::NI, NS - 2>(min(nch - 1 - i, NS - 2));
        __syncthreads();
        if (i + NS - 1 < nch) issue(std::integral_constant<int, (B + NS - 1) % NS>{}, i + NS - 1);
        if (!(SK_ABL & 1)) compute(kb);
    };
    static_assert(NS >= 2 && NS <= 4, "two to four stages");
    issue(std::integral_constant<int, 0>{}, 0);  // nch >= 1: the launcher gives every split a chunk
    if constexpr (NS > 2)
        if (1 < nch) issue(std::integral_constant<int, 1>{}, 1);
    if constexpr (NS > 3)
        if (2 < nch) issue(std::integral_constant<int, 2>{}, 2);
    for (int i = 0; i < nch; i += NS) {
        step(std::integral_constant<int, 0>{}, i);
        if (i + 1 >= nch) break;
        step(std::integral_constant<int, 1>{}, i + 1);
        if constexpr (NS > 2) {
            if (i + 2 >= nch) break;
            step(std::integral_constant<int, 2>{}, i + 2);
        }
        if constexpr (NS > 3) {
            if (i + 3 >= nch) break;
            step(std::integral_constant<int, 3>{}, i + 3);
        }
    }

    // the partial tile [row][BR columns]: lane (c, q) of wave w holds rows 16 t + 4 q + k, column 16 (TN w + j) + c.
    // Partials and tickets are read and written with system-scope relaxed atomics, which go through the caches to
    // memory, so the blocks of a tile on different XCDs (each with its own L2) see each other's partials without an L2
    // write-back (a __threadfence here, one per block, cost more than the product). Every lane waits for its partial
    // stores to complete before the barrier, and the ticket is taken after it.
    if (SK_ABL & 2) {
#pragma unroll
        for (int t = 0; t < TM; t++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int m = 16 * t + 4 * q + k, n = n0 + 16 * (TN * wave + j) + c;
                    if (m < M && n < N) y[(int64_t)m * N + n] = acc[t][j][k];
                }
        return;
    }
    float* pt = part + (size_t)blockIdx.x * Geo::TILE;
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int k = 0; k < 4; k++)
                __hip_atomic_store(pt + (16 * t + 4 * q + k) * Geo::BR + 16 * (TN * wave + j) + c, acc[t][j][k], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
    __syncthreads();
    if (threadIdx.x == 0) last = __hip_atomic_fetch_add(&tickets[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == S - 1;
    __syncthreads();
    if (!last) return;
    // the thread's V outputs (idx = threadIdx.x + 256 u: row idx / BR, column idx % BR), the partials of all of them
    // in flight per split: each load is a trip to memory, so the split loop (four splits a round) waits about S / 4
    // times, not S V times
    constexpr int V = TM * 16 * Geo::BR / 256;
    constexpr int RPU = 256 / Geo::BR;                     // rows a step of u advances
    const int col = threadIdx.x % Geo::BR, row0 = threadIdx.x / Geo::BR;
    const float* p0 = part + (size_t)tile * S * Geo::TILE;
    float v[V];
#pragma unroll
    for (int u = 0; u < V; u++) v[u] = 0.0f;
#pragma unroll 4
    for (int k = 0; k < S; k++) {
        float x[V];
#pragma unroll
        for (int u = 0; u < V; u++)
            x[u] = __hip_atomic_load(p0 + (size_t)k * Geo::TILE + threadIdx.x + 256 * u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
        for (int u = 0; u < V; u++) v[u] += x[u];
    }
    // bias and residual with clamped (always valid) indices, so all of their loads are in flight together too
    const int n = min(n0 + col, N - 1);
    const float bn = bias ? bias[n] : 0.0f;
    float r[V];
#pragma unroll
    for (int u = 0; u < V; u++) r[u] = res ? res[(int64_t)min(row0 + RPU * u, M - 1) * N + n] : 0.0f;
#pragma unroll
    for (int u = 0; u < V; u++) {
        const int m = row0 + RPU * u;
        if (m < M && n0 + col < N) y[(int64_t)m * N + n] = v[u] + bn + r[u];
    }
    if (threadIdx.x == 0) __hip_atomic_store(&tickets[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The split-K launch: S splits of K per weight tile, about BPC blocks a CU (as many as the stages' LDS lets a CU
// hold, at most two), as many as the scratch holds; hipErrorNotSupported when the scratch cannot be had (a stream
// under graph capture, or every slot held by other streams)
template <int TM, int TN, int G, int NS>
hipError_t gemm_sk_launch(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const float* xd32, const float* bias, const float* res,
                          float* y, int M, int N, int K, hipStream_t s) {
    using Geo = SplitGeo<TM, TN, G>;
    constexpr int LDS = NS * Geo::STAGE;
    constexpr int BPC = std::min(2, 160 * 1024 / (LDS + 256));
    static_assert(BPC >= 1, "the stages fit one CU");
    auto* fn = gemm_q8_0_sk_kernel<TM, TN, G, NS>;
    const int tiles = (N + Geo::BR - 1) / Geo::BR, chunks = K / (32 * G);
    int S = std::max(1, BPC * kf_cu_count() / tiles);
    S = std::min(S, std::max(1, chunks / 3));  // at least three chunks a split
    if (kf_knob_on(KF_KNOB_GEMM_SK_S)) S = std::max(1, std::min(kf_knob(KF_KNOB_GEMM_SK_S), chunks));  // a comparison knob
    const size_t room = (KF_SPLIT_SCRATCH - (size_t)KF_SPLIT_TICKETS * 4) / ((size_t)tiles * Geo::TILE * 4);
    S = std::min<int>(S, (int)std::min<size_t>(room, 1 << 20));
    if (tiles > KF_SPLIT_TICKETS || S < 1) return hipErrorNotSupported;
    char* scr = static_cast<char*>(kf_split_scratch(s));
    if (!scr) return hipErrorNotSupported;
    const hipError_t le = kf_raise_lds(reinterpret_cast<const void*>(fn), LDS);
    if (le != hipSuccess) return le;
    int* tickets = reinterpret_cast<int*>(scr);
    float* part = reinterpret_cast<float*>(scr + (size_t)KF_SPLIT_TICKETS * 4);
    fn<<<tiles * S, 256, LDS, s>>>(w, row_bytes, xq, xd32, bias, res, y, M, N, K, S, tickets, part);
    return hipGetLastError();
}

template <int TN, int W>
hipError_t gemm_mr_launch(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const float* xd32, const float* bias, const float* res,
                          float* y, int M, int N, int K, hipStream_t s) {
    gemm_q8_0_mr_kernel<TN, W><<<(N + 16 * TN - 1) / (16 * TN), 64 * W, 0, s>>>(w, row_bytes, xq, xd32, bias, res, y, M, N, K);
    return hipGetLastError();
}

template <int WM, int WN, int TM, int TN>
hipError_t gemm_q8_0_dma_launch(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const float* xd32, const float* bias, const float* res,
                                float* y, int M, int N, int K, hipStream_t s) {
    using C = GqCfg<WM, WN, TM, TN>;
    const int T = ((N + C::BN - 1) / C::BN) * ((M + C::BM - 1) / C::BM);
    // the tail split: a last round (8 / (WM WN) blocks a CU) at most half full runs its tiles as K halves in one round
    // of half the length; it needs the split scratch and K % 512 == 0 (even stage counts; KF_GEMM_NO_TAIL turns it
    // off, a comparison knob)
    GmTail tail{nullptr, nullptr, T};
    int blocks = T;
    const int slots = kf_cu_count() * (8 / (WM * WN)), rem = T % slots;
    const size_t part_bytes = (size_t)rem * 2 * TM * TN * 16 * C::THREADS * 4;
    if (rem > 0 && rem <= slots / 2 && K % 512 == 0 && K / GM_BK >= 4 && rem <= KF_SPLIT_TICKETS &&
        part_bytes <= KF_SPLIT_SCRATCH - (size_t)KF_SPLIT_TICKETS * 4 && !kf_knob_on(KF_KNOB_GEMM_NO_TAIL)) {
        if (char* scr = static_cast<char*>(kf_split_scratch(s))) {
            tail = GmTail{reinterpret_cast<float*>(scr + (size_t)KF_SPLIT_TICKETS * 4), reinterpret_cast<int*>(scr), T - rem};
            blocks = T + rem;
        }
    }
    gemm_q8_0_dma_kernel<WM, WN, TM, TN><<<blocks, C::THREADS, 0, s>>>(w, row_bytes, xq, xd32, bias, res, y, M, N, K, tail);
    return hipGetLastError();
}

template <int WM, int WN, int TM, int TN>
hipError_t gemm_launch(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const float* xd32, const float* bias, const float* res, float* y,
                       int M, int N, int K, hipStream_t s) {
    using C = GmCfg<WM, WN, TM, TN>;
    auto* fn = gemm_q8_0_kernel<WM, WN, TM, TN>;
    // the double-buffered stage needs more than the default 64 KB of LDS
    const hipError_t e = kf_raise_lds(reinterpret_cast<const void*>(fn), 2 * C::STAGE);
    if (e != hipSuccess) return e;
    dim3 grid((N + C::BN - 1) / C::BN, (M + C::BM - 1) / C::BM);
    fn<<<grid, GM_THREADS, 2 * C::STAGE, s>>>(w, row_bytes, xq, xd32, bias, res, y, M, N, K);
    return hipGetLastError();
}

template <int MR, int TN>
hipError_t gemm_small_launch(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const float* xd32, const float* bias, const float* res,
                             float* y, int M, int N, int K, int W, hipStream_t s) {
    static_assert(SkGeo<TN>::WAVE_LDS >= SkAct<MR>::TM * TN * 4 * 64 * 4, "a wave region holds a partial tile");
    auto* fn = gemm_q8_0_small_kernel<MR, TN>;
    const hipError_t e = kf_raise_lds(reinterpret_cast<const void*>(fn), 8 * SkGeo<TN>::WAVE_LDS);
    if (e != hipSuccess) return e;
    fn<<<dim3(((N + SkGeo<TN>::ROWS - 1) / SkGeo<TN>::ROWS) * ((M + MR - 1) / MR)), 64 * W, W * SkGeo<TN>::WAVE_LDS, s>>>(w, row_bytes, xq, xd32, bias, res,
                                                                                                                 y, M, N, K);
    return hipGetLastError();
}

// Waves per block of the small-batch kernel: enough blocks x waves to fill the GPU (about 4096 waves), at least two
// chunks a wave, a power of two, at most four; KF_GEMM_SMALL_W overrides it (a tuning knob)
int small_waves(int M, int N, int K, int rows_per_block) {
    const int forced = kf_knob_or(KF_KNOB_GEMM_SMALL_W, 0);
    const int cap = 4;  // measured: four waves (more chunks each) beat eight on every Llama shape at M = 8..64
    const int rblocks = (M + 15) / 16;
    if (forced == 1 || forced == 2 || forced == 4 || forced == 8) return forced;
    const int tiles = (N + rows_per_block - 1) / rows_per_block, chunks = K / 256;
    int w = 1;
    while (w < cap && tiles * rblocks * w < 4096 && chunks / (2 * w) >= 2) w *= 2;
    return w;
}

}  // namespace

int kf_gemm_k_multiple() { return GM_BK; }



// Host launcher, validated by the caller (api.cpp): K a multiple of 128, Q8_0-kind activations in `act`
// Whether 65.. q8_0 rows run faster as 64-row slices through the small-batch products than on the tile GEMM
// (MI355X, Llama-3-8B shapes at 96-512 rows; the model picks the faster form at all 24 measured points): a 64-row
// slice costs about 9 us + 0.45 us per weight MB, the tile GEMM about 3 us per 128-column stage per round of one
// block a CU (a last round at most half full as K halves: half a round; the kernel is VALU-bound, so a second block
// on a CU does not shorten a round). KF_GEMM_SLICE=0 / 1 forces the choice (a comparison knob).
static bool q8_0_slices_pay(int M, int N, int K, int64_t row_bytes) {
    if (kf_knob_on(KF_KNOB_GEMM_SLICE)) return kf_knob(KF_KNOB_GEMM_SLICE) != 0;
    const double mb = (double)N * row_bytes / 1e6;
    const double t_slices = ((M + 63) / 64) * (9.0 + 0.45 * mb);
    const int cus = kf_cu_count();
    const int64_t T = (int64_t)((N + 127) / 128) * ((M + 127) / 128), rem = T % cus;
    const double rounds = (double)(T / cus) + (rem == 0 ? 0.0 : rem <= cus / 2 && K % 512 == 0 ? 0.5 : 1.0);
    const double t_tile = 3.0 * (K / 128) * rounds;
    return t_slices < t_tile;
}

// The small-batch products of 1..64 activation rows (K % 256 == 0, 16-byte aligned rows): hipErrorNotSupported when
// none takes the shape
static hipError_t small_q8_0(const uint8_t* wb, int64_t row_bytes, const int8_t* xq, const float* xd, const float* bias, const float* res,
                             float* y, int M, int N, int K, hipStream_t s) {
    // 1..64 rows with K split across blocks, for matrices above 4096 x 4096 (MI355X, Llama-3-8B shapes, 32 / 64
    // rows: QKV 17.0 / 23.4 against 21.1 / 28.4 us, gate 26.4 / 38.2 against 35.6 / 50.0, down 27.8 / 38.9
    // against 31.4 / 48.0; O at 4096 x 4096 15.2 / 20.5 against 12.1 / 18.4, so not there). KF_GEMM_SK=0 turns
    // it off, KF_GEMM_SK=1 on for every size (comparison knobs)
    const bool sk = kf_knob_on(KF_KNOB_GEMM_SK) ? kf_knob(KF_KNOB_GEMM_SK) != 0 : (int64_t)N * K > (1ll << 24);
    if (M <= 64 && K % 128 == 0 && (K / 32) % 2 == 0 && sk) {
        const int var = kf_knob_or(KF_KNOB_GEMM_SK_V, 0);  // 10 G + NS (groups a chunk, ring stages): a tuning knob
        // 8-group chunks in two stages where K allows (MI355X, Llama-3-8B shapes at 32 / 64 rows: gate 25.1 / 37.2
        // against 26.0 / 38.3 us with 4-group chunks in three, down 24.5 / 37.4 against 25.3 / 39.3)
        const int v = var ? var : K % 256 == 0 ? 82 : 43;
        hipError_t e = hipErrorNotSupported;
        if (K % (32 * (v / 10)) == 0) {
            // 1..16 rows: one staged 16-row tile (MI355X, Llama-3-8B shapes at 8 / 16 rows: QKV 11.0 / 11.4 against
            // 12.1 / 12.9 us for the small-batch kernel, gate 17.9 / 19.0 against 21.3 / 21.9, down 18.0 / 18.2
            // against 19.4 / 23.1: that kernel fills fewer than one wave a SIMD on these grids); 8-group chunks only
            // (a 16-row tile of 4-group chunks is not whole DMA instructions)
            if (M <= 16) {
                if (K % 256 == 0) e = gemm_sk_launch<1, 1, 8, 2>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
            } else if (M <= 32)
                e = v == 83    ? gemm_sk_launch<2, 1, 8, 3>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s)
                    : v == 82  ? gemm_sk_launch<2, 1, 8, 2>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s)
                    : v == 162 ? gemm_sk_launch<2, 1, 16, 2>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s)
                               : gemm_sk_launch<2, 1, 4, 3>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
            else
                e = v == 83    ? gemm_sk_launch<4, 1, 8, 3>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s)
                    : v == 82  ? gemm_sk_launch<4, 1, 8, 2>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s)
                    : v == 162 ? gemm_sk_launch<4, 1, 16, 2>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s)
                               : gemm_sk_launch<4, 1, 4, 3>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
        }
        if (e != hipErrorNotSupported) return e;
    }
    if (M > 48 && M <= MR_ROWS && K % (32 * MR_G) == 0 && !kf_knob_on(KF_KNOB_GEMM_NO_MR)) {
        // 49..64 rows in one weight pass where it measured faster than four 16-row blocks (MI355X, Llama-3-8B
        // shapes at 64 rows: O 18.4 against 21.6 us, down 48.3 against 57.0, gate 49.8 against 55.2; QKV and
        // 17..48 rows: no gain). One 16-row weight tile a block, 4 waves splitting K for N <= 4096 (too few tiles
        // otherwise), one wave for wide outputs. KF_GEMM_MR=11 / 14 forces a variant (a comparison knob)
        const int v = kf_knob_or(KF_KNOB_GEMM_MR, N >= 8192 ? 11 : N <= 4096 ? 14 : 0);
        if (v == 11) return gemm_mr_launch<1, 1>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
        if (v == 14) return gemm_mr_launch<1, 4>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
    }
    if (M <= 64) {  // M / 16 row blocks
        // one 16-column tile a wave when that still gives at most one block per CU (a block holds a CU), else two
        const int tn = kf_knob_or(KF_KNOB_GEMM_SMALL_TN, 0);  // a tuning knob
        if (tn == 1 || (tn != 2 && (int64_t)((N + 15) / 16) * ((M + 15) / 16) <= kf_cu_count()))
            return gemm_small_launch<16, 1>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, small_waves(M, N, K, 16), s);
        return gemm_small_launch<16, 2>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, small_waves(M, N, K, 32), s);
    }
    return hipErrorNotSupported;
}

hipError_t kf_launch_gemm_q8_0(const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y, int M,
                               int N, int K, hipStream_t s) {
    const kf_act_offsets o = kf_act_layout((size_t)M, (size_t)K);
    const char* base = static_cast<const char*>(act);
    const auto* xq = reinterpret_cast<const int8_t*>(base + o.q);
    const auto* xd = reinterpret_cast<const float*>(base + o.d32);
    const auto* wb = static_cast<const uint8_t*>(w);
    // the small-batch kernels read whole 16-byte pieces of rows, which needs 16-byte aligned rows (K % 256 == 0)
    if (K % 256 == 0 && row_bytes % 16 == 0 && (int64_t)N * row_bytes < (1ll << 31) && (int64_t)M * K < (1ll << 31) && !kf_knob_on(KF_KNOB_GEMM_TILE)) {
        if (M <= 64) {
            const hipError_t e = small_q8_0(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
            if (e != hipErrorNotSupported) return e;
        } else if (q8_0_slices_pay(M, N, K, row_bytes)) {
            // 65.. rows as 64-row slices through the small-batch products (each slice its own weight pass)
            for (int m0 = 0; m0 < M; m0 += 64) {
                const hipError_t e = small_q8_0(wb, row_bytes, xq + (int64_t)m0 * K, xd + (int64_t)m0 * (K / 32), bias,
                                                res ? res + (int64_t)m0 * N : nullptr, y + (int64_t)m0 * N, std::min(64, M - m0), N, K, s);
                if (e != hipSuccess) return e;
            }
            return hipSuccess;
        }
    }
    if (K % 256 == 0 && row_bytes % 16 == 0) return gemm_q8_0_dma_launch<2, 4, 2, 1>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
    return gemm_launch<2, 2, 2, 2>(wb, row_bytes, xq, xd, bias, res, y, M, N, K, s);
}
