// Prefill GEMM on native q5_K and q6_K bytes: y[m][n] = sum over super-blocks b of dx[m][b] * (d[n][b] * S_b[m][n]
// - dmin[n][b] * mins_b[m][n]) (+ bias[n] + res[m][n]), with S_b the reference's exact super-block integer:
//   * q5_K (crates/kf-quant/src/types/q5_k.rs): S_b = sum_g sc_g I_g over the eight 32-column groups, I_g the int32
//     dot of the group's 5-bit values (the fifth bit from qh) with the int8 activations; mins_b = sum_g m_g bsum_g;
//   * q6_K (crates/kf-quant/src/types/q6_k.rs): S_b = sum_s sc_s (dot_s - 32 bsum_s) over the sixteen 16-column
//     sub-blocks with int8 scales, formed as sum_s sc_s dot'_s with the operand q - 32 (an int8); no mins term.
// It replaces the reference's unpack + KF8 GEMM for these types (crates/kf-backend-cuda/src/kernels/quant.cuh:585-601,
// KF_QUANT_KERNELS_I8 in quant_q5_K.cu:114 / quant_q6_K.cu:131, kf8.cu:116-369), reading the native bytes directly.
//
// Arithmetic: per group and 32 x 32 tile one v_mfma_i32_32x32x32_i8 gives I_g exactly (q6_K: two, each with the
// other 16 columns' operand bytes zeroed, for the two scales of the group); S_b accumulates by 24-bit multiply-adds
// with the integer sub-scales (every product below 2^23), mins_b by one exact v_mfma_f32_32x32x16_f16 against
// quant_act's split sums (as the q4_K GEMM), and the float rescale runs once per super-block and output.
//
// Schedule: eight waves (two a SIMD), one block a CU, block tile 64 x 256: each wave a 64 x 32 tile (two 32 x 32
// MFMA tiles down M, one weight column tile), so a wave's weight operands serve two MFMAs. One super-block (K = 256)
// per stage, two stage buffers: activations [row 64][256] with the 16-byte chunk swizzle c ^ (row % 16), weights
// [row 256][WROW] (q5_K: the 176-byte super-block; q6_K: the 224-byte 16-byte aligned window around the 210-byte
// block, which needs rows that start 16-byte aligned: K a multiple of 2048), the stage's activation scales and (q5_K)
// mins operands. Every DMA instruction reads whole 16-byte pieces of consecutive rows, issued through inline assembly
// with explicit waits; rows past M or N read as zeros through the hardware range check. Blocks run in XCD order (each
// XCD a contiguous range of tiles, M fastest), so the blocks in flight on an XCD share their weight tiles in its L2.
#include "kf_knobs.h"
#include "kf_blocks.h"
#include "kf_device.h"
#include "kf_host.h"

#include <type_traits>

// The split-K fixups rely on gfx9 cache behaviour (system-scope relaxed atomics write through to memory, stores are
// counted in vmcnt), not on a release/acquire pair: build for gfx950 only.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the split-K fixups assume gfx950's cache and counter behaviour"
#endif

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));

constexpr int KQ_WAVES = 8, KQ_THREADS = 64 * KQ_WAVES;
constexpr int KQ_TM = 2;                       // 32-row tiles per wave (all of the block's rows)
constexpr int KQ_BM = 32 * KQ_TM;              // 64
constexpr int KQ_BN = 32 * KQ_WAVES;           // 256: one 32-column tile per wave

template <uint32_t TY>
struct KqGeo {
    static constexpr bool Q6 = TY == KF_TYPE_Q6_K, Q4 = TY == KF_TYPE_Q4_K;
    static constexpr int SBB = Q6 ? KF_Q6_K_BYTES : Q4 ? KF_Q4_K_BYTES : KF_Q5_K_BYTES;  // bytes of a super-block
    static constexpr int WROW = Q6 ? 224 : SBB;                      // LDS bytes of a weight row's super-block
    static constexpr int QS = Q4 ? 16 : 48;                          // q4_K / q5_K: the nibbles' offset
    static constexpr int PR = WROW / 16;                             // its 16-byte pieces
    static constexpr int A = 0;                                      // activations [row 64][256]
    static constexpr int W = A + KQ_BM * 256;                        // weights [row 256][WROW]
    static constexpr int DX = W + KQ_BN * WROW;                      // activation scales [row 64] f32
    static constexpr int XS = DX + KQ_BM * 4;                        // q5_K: mins operands [row 64][16] f16
    static constexpr int STAGE = XS + (Q6 ? 0 : KQ_BM * 32);
    static constexpr int NA = KQ_BM * 256 / 1024;                    // activation DMA instructions (4 rows each)
    static constexpr int NW = (KQ_BN * PR + 63) / 64;                // weight DMA instructions (64 pieces each)
    static_assert(NA % KQ_WAVES == 0, "whole activation instructions a wave");
    static_assert(2 * STAGE <= 160 * 1024, "two stages fit the LDS");
};

// XCD-aware tile order over the first T tiles: block b < T runs tile (b % 8) (T / 8) + b / 8 (tiles numbered
// M-fastest), so XCD x (blocks go to the eight XCDs round-robin) works through a contiguous range of weight tiles
// against every activation panel. Identity when T is not a multiple of eight.
__device__ __forceinline__ void kq_tile(int T, int mt, int b, int& tm, int& tn) {
    const int t = (T & 7) ? b : (b & 7) * (T >> 3) + (b >> 3);
    tn = t / mt;
    tm = t - tn * mt;
}

// The grid's tail: the tiles from `full` on (a last round of blocks at most half full, or a whole grid below half
// the CUs) run as S blocks each over S consecutive ranges of K; each writes its 64 x 256 partial tile to `part`
// ([tail tile][split][register][thread]), and the last of them to arrive (a ticket per tail tile) adds all S in split
// order and stores the tile. part == nullptr: no split.
struct KqTail {
    float* part;
    int* tickets;
    int full, S;
};

// The grouped (MoE) form: the activation rows are routed pairs in group order (slot s: rows offsets[s]..offsets[s + 1]),
// slot s multiplies its own expert matrix (w + s expert_bytes; with w2, output columns from n_split on come from
// w2 + s expert_bytes, row n - n_split), and output row p goes to y row out_rows[p] (or p). n_slots == 0: one matrix.
struct KqMoe {
    const int32_t* offsets;
    const int32_t* out_rows;
    const uint8_t* w2;
    int64_t expert_bytes;
    int n_slots, n_split;
};

template <uint32_t TY, bool MOE>
__global__ void __launch_bounds__(KQ_THREADS, 1) gemm_kq_kernel(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                                 const int8_t* __restrict__ xq, const _Float16* __restrict__ xa,
                                                                 const float* __restrict__ xd32, const float* __restrict__ bias,
                                                                 const float* __restrict__ res, float* __restrict__ y, int M, int N, int K,
                                                                 KqTail tail_arg, KqMoe moe) {
    const KqTail tail = MOE ? KqTail{nullptr, nullptr, 0, 1} : tail_arg;  // the dense form's tail split
    // the grouped form splits K in two over every tile when its launcher passes the scratch (msplit)
    const bool msplit = MOE && tail_arg.part != nullptr;
    using G = KqGeo<TY>;
    __shared__ __align__(16) uint8_t buf0[G::STAGE];
    __shared__ __align__(16) uint8_t buf1[G::STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5, r32 = lane & 31;
    __shared__ int last;
    const int mt = (M + KQ_BM - 1) / KQ_BM;
    const int kg = K >> 5;
    const int nsb = K >> 8;
    int tm, tn;
    int s0 = 0, s1 = nsb, sp = -1, tt = 0;  // super-blocks [s0, s1); a tail block's split and tail tile
    if (!MOE && tail.part && (int)blockIdx.x >= tail.full) {
        const int b = blockIdx.x - tail.full;
        tt = b / tail.S;
        sp = b - tt * tail.S;
        const int t = tail.full + tt;
        tn = t / mt;
        tm = t - tn * mt;
        s0 = nsb * sp / tail.S;
        s1 = nsb * (sp + 1) / tail.S;
    } else if (msplit) {
        // the two K halves of tile tt, in XCD order: XCD x (blocks go to the eight XCDs round-robin) takes a contiguous
        // range of tiles, both halves of each, so the blocks of an expert's weight tiles share them in its L2
        const int T = ((N + KQ_BN - 1) / KQ_BN) * mt, b = blockIdx.x;
        if ((T & 7) == 0) {
            tt = (b & 7) * (T >> 3) + (b >> 4);
            sp = (b >> 3) & 1;
        } else {
            tt = b >> 1;
            sp = b & 1;
        }
        tn = tt / mt;
        tm = tt - tn * mt;
        s0 = nsb * sp / 2;
        s1 = nsb * (sp + 1) / 2;
    } else {
        kq_tile(tail.part ? tail.full : ((N + KQ_BN - 1) / KQ_BN) * mt, mt, blockIdx.x, tm, tn);
    }
    int m0 = tm * KQ_BM;
    const int n0 = tn * KQ_BN;
    int m_end = M;  // rows of the block's slot end here
    const uint8_t* wt = w + (int64_t)n0 * row_bytes;
    int n_end = N;  // columns of the block's matrix end here (as output columns)
    if (MOE) {
        // M counts the grid's row tiles over all slots (an upper bound): tile tm is the slot's tile tm - (the tiles of
        // the slots before it); past the last slot's tiles the block has nothing to do
        int sl = 0, t0 = 0;
        for (; sl < moe.n_slots; sl++) {
            const int rows = moe.offsets[sl + 1] - moe.offsets[sl], t = (rows + KQ_BM - 1) / KQ_BM;
            if (tm < t0 + t) break;
            t0 += t;
        }
        if (sl == moe.n_slots) return;  // whole block, before any barrier
        m0 = moe.offsets[sl] + (tm - t0) * KQ_BM;
        m_end = moe.offsets[sl + 1];
        if (moe.w2 && n0 >= moe.n_split) {
            wt = moe.w2 + sl * moe.expert_bytes + (int64_t)(n0 - moe.n_split) * row_bytes;
        } else {
            wt = w + sl * moe.expert_bytes + (int64_t)n0 * row_bytes;
            if (moe.w2) n_end = moe.n_split;
        }
    }

    const kf_arsrc_t rw = kf_arsrc(wt, (uint64_t)(n_end - n0) * row_bytes);
    const kf_arsrc_t rx = kf_arsrc(xq + (int64_t)m0 * K, (uint64_t)(m_end - m0) * K);
    const kf_arsrc_t rs = kf_arsrc(xa + (int64_t)m0 * nsb * 16, (uint64_t)(m_end - m0) * nsb * 32);
    const kf_arsrc_t rd = kf_arsrc(xd32 + (int64_t)m0 * kg, (uint64_t)(m_end - m0) * kg * 4);
    // activation instruction i (rows 4 i..) is wave i % 8's: lane l takes chunk (l % 16) ^ (row % 16) of row
    // 4 i + l / 16 and writes it at position l % 16, so the MFMA operand reads below hit distinct banks
    int va[G::NA / KQ_WAVES];
#pragma unroll
    for (int k = 0; k < G::NA / KQ_WAVES; k++) {
        const int row = 4 * (wave + KQ_WAVES * k) + (lane >> 4);
        va[k] = row * K + 16 * ((lane & 15) ^ (row & 15));
    }
    // weight piece q = 64 i + l of a stage: row q / PR, piece q % PR
    auto wpiece = [&](int i) __attribute__((always_inline)) {
        const int q = min(64 * i + lane, KQ_BN * G::PR - 1), row = q / G::PR;
        return row * (int)row_bytes + 16 * (q - G::PR * row);
    };
    auto dma = [&](uint8_t* buf, int sb) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < G::NA / KQ_WAVES; k++) kf_adma16(rx, va[k], sb * 256, buf + G::A + (wave + KQ_WAVES * k) * 1024);
        const int wo = G::Q6 ? (sb * G::SBB) & ~15 : sb * G::SBB;
#pragma unroll
        for (int k = 0; k < (G::NW + KQ_WAVES - 1) / KQ_WAVES; k++) {
            const int i = wave + KQ_WAVES * k;
            if (i < G::NW) kf_adma16(rw, wpiece(i), wo, buf + G::W + i * 1024);
        }
        if (wave == 0) kf_adma4(rd, lane * kg * 4, sb * 32, buf + G::DX);
        if (!G::Q6 && (wave == 1 || wave == 2))
            kf_adma16(rs, ((wave - 1) * 32 + (lane >> 1)) * nsb * 32 + (lane & 1) * 16, sb * 32, buf + G::XS + (wave - 1) * 1024);
    };

    v16f acc[KQ_TM];
#pragma unroll
    for (int i = 0; i < KQ_TM; i++) acc[i] = v16f{};
    const int wcol = (wave * 32 + r32) * G::WROW;  // the wave's weight row (tile column) for this lane
    const int sw = r32 & 15;

    // group g's activation operand of tile i: chunk 2 g + half of the lane's row, stored at (2 g + half) ^ (row % 16)
    auto aop = [&](const uint8_t* cur, int g, int i) __attribute__((always_inline)) {
        return *reinterpret_cast<const v4i*>(cur + G::A + (i * 32 + r32) * 256 + 16 * ((2 * g + half) ^ sw));
    };

    // TLC: the 32-row tiles of the block that hold rows (a grouped tile with at most 32 rows skips its second)
    auto stage = [&](auto tlc, const uint8_t* cur, int sb) __attribute__((always_inline)) {
        constexpr int TL = decltype(tlc)::value;
        v16i S[KQ_TM];
#pragma unroll
        for (int i = 0; i < TL; i++) S[i] = v16i{};
        float d, dm = 0.0f;
        v8h mo;
        if constexpr (!G::Q6) {
            // q5_K: d, dmin, 12 bytes of 6-bit scales / mins, qh[32], qs[128]; the lane's 16 columns of group g are
            // bytes 16 half.. of qs[32 (g / 2)..] (low nibbles: g even) with bit g of qh[16 half..]
            const uint8_t* wr = cur + G::W + wcol;
            const uint4 hd = *reinterpret_cast<const uint4*>(wr);
            const uint4 qh = G::Q4 ? make_uint4(0u, 0u, 0u, 0u) : *reinterpret_cast<const uint4*>(wr + 16 + 16 * half);
            const uint32_t qhv[4] = {qh.x, qh.y, qh.z, qh.w};
            const uint32_t m4 = 0x0f0f0f0fu, m1 = 0x01010101u;
            uint4 raw[4];
            uint32_t sc2[4], scv[2], mnv[2];
            kf_q4k_scales8(hd.y, hd.z, hd.w, scv, mnv);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                raw[p] = *reinterpret_cast<const uint4*>(wr + G::QS + 32 * p + 16 * half);
                sc2[p] = kf_pair(scv, p);
                const uint32_t m2 = kf_pair(mnv, p);
                mo[2 * p] = (_Float16)(float)((half ? 1u : 64u) * (m2 & 0xffu));
                mo[2 * p + 1] = (_Float16)(float)((half ? 1u : 64u) * (m2 >> 8));
            }
            // group g's MFMAs (operand: 0..31 per byte, the fifth bit from qh)
            auto issue = [&](auto gc, v16i (&I)[KQ_TM]) __attribute__((always_inline)) {
                constexpr int g = decltype(gc)::value;
                const uint32_t v[4] = {raw[g / 2].x, raw[g / 2].y, raw[g / 2].z, raw[g / 2].w};
                v4i b;
#pragma unroll
                for (int e = 0; e < 4; e++) b[e] = (int)((((g & 1) ? v[e] >> 4 : v[e]) & m4) | (((qhv[e] >> g) & m1) << 4));
#pragma unroll
                for (int i = 0; i < TL; i++) I[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop(cur, g, i), b, v16i{}, 0, 0, 0);
            };
            // Software-pipelined by one group: group g + 1's MFMAs are issued before group g's multiply-adds, which
            // depend on none of them, so the adds run while the matrix core works. The running sums are
            // materialized after each group (left free, the compiler reassociates the integer adds across groups
            // and holds every product), and the sched barriers keep the groups in this order.
            v16i Ia[KQ_TM], Ib[KQ_TM];
            auto mads = [&](int g, const v16i (&I)[KQ_TM]) __attribute__((always_inline)) {
                const int sc = (int)((g & 1) ? sc2[g / 2] >> 8 : sc2[g / 2] & 0xffu);
#pragma unroll
                for (int i = 0; i < TL; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) S[i][r] += __mul24(sc, I[i][r]);  // |sc I| < 2^22
#pragma unroll
                for (int i = 0; i < TL; i++) __asm__ volatile("" : "+v"(S[i]));
            };
            issue(std::integral_constant<int, 0>{}, Ia);
            __builtin_amdgcn_sched_barrier(0);
            issue(std::integral_constant<int, 1>{}, Ib);
            mads(0, Ia);
            __builtin_amdgcn_sched_barrier(0);
            issue(std::integral_constant<int, 2>{}, Ia);
            mads(1, Ib);
            __builtin_amdgcn_sched_barrier(0);
            issue(std::integral_constant<int, 3>{}, Ib);
            mads(2, Ia);
            __builtin_amdgcn_sched_barrier(0);
            issue(std::integral_constant<int, 4>{}, Ia);
            mads(3, Ib);
            __builtin_amdgcn_sched_barrier(0);
            issue(std::integral_constant<int, 5>{}, Ib);
            mads(4, Ia);
            __builtin_amdgcn_sched_barrier(0);
            issue(std::integral_constant<int, 6>{}, Ia);
            mads(5, Ib);
            __builtin_amdgcn_sched_barrier(0);
            issue(std::integral_constant<int, 7>{}, Ib);
            mads(6, Ia);
            __builtin_amdgcn_sched_barrier(0);
            mads(7, Ib);
            __builtin_amdgcn_sched_barrier(0);
            d = kf_h2f(hd.x & 0xffffu);
            dm = kf_h2f(hd.x >> 16);
        } else {
            // q6_K: ql[128], qh[64], int8 scales[16], d; the super-block starts at the window's shift (sb * 210) % 16,
            // 2-byte aligned. Group g = 4 h + gg (columns 128 h + 32 gg..): the lane's 16 columns l = 16 half.. take
            // the low (gg < 2) or high nibbles of ql[64 h + 32 (gg % 2) + l] and bits 2 gg.. of qh[32 h + l]; scales
            // 8 h + 2 gg (columns 0-15 of the group) and 8 h + 2 gg + 1 (16-31)
            const uint8_t* wr = cur + G::W + wcol + ((sb * G::SBB) & 15);
            const u32x4_a2 scv = *reinterpret_cast<const u32x4_a2*>(wr + 192);
            const uint32_t scw[4] = {scv.x, scv.y, scv.z, scv.w};
            const uint32_t m4 = 0x0f0f0f0fu, m3 = 0x03030303u, hb = 0x80808080u, k32 = 0x20202020u;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const u32x4_a2 la = *reinterpret_cast<const u32x4_a2*>(wr + 64 * h + 16 * half);
                const u32x4_a2 lb = *reinterpret_cast<const u32x4_a2*>(wr + 64 * h + 32 + 16 * half);
                const u32x4_a2 qq = *reinterpret_cast<const u32x4_a2*>(wr + 128 + 32 * h + 16 * half);
#pragma unroll
                for (int gg = 0; gg < 4; gg++) {
                    const u32x4_a2 src = (gg & 1) ? lb : la;
                    v4i bw;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t lo = (gg >> 1) ? (src[e] >> 4) & m4 : src[e] & m4;
                        const uint32_t v = lo | (((qq[e] >> (2 * gg)) & m3) << 4);  // q in [0, 63] per byte
                        bw[e] = (int)(((v | hb) - k32) ^ hb);                         // q - 32 per byte, no borrows
                    }
                    const v4i b0 = half ? v4i{} : bw, b1 = half ? bw : v4i{};  // columns 0-15, then 16-31
                    const int si = 8 * h + 2 * gg;
                    const int s0 = (int)(int8_t)(uint8_t)(scw[si >> 2] >> (8 * (si & 3)));
                    const int s1 = (int)(int8_t)(uint8_t)(scw[(si + 1) >> 2] >> (8 * ((si + 1) & 3)));
#pragma unroll
                    for (int i = 0; i < TL; i++) {
                        const v4i a = aop(cur, 4 * h + gg, i);
                        const v16i I0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b0, v16i{}, 0, 0, 0);
                        const v16i I1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b1, v16i{}, 0, 0, 0);
                        // |dot| <= 16 * 128 * 32 and |sc| <= 128: the 24-bit products are exact
#pragma unroll
                        for (int r = 0; r < 16; r++) S[i][r] += __mul24(s0, I0[r]) + __mul24(s1, I1[r]);
                    }
#pragma unroll
                    for (int i = 0; i < TL; i++) __asm__ volatile("" : "+v"(S[i]));
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            d = kf_h2f(*reinterpret_cast<const uint16_t*>(wr + 208));
        }
        // acc += dx (d S - dmin mins); accumulator register r holds row (r % 4) + 8 (r / 4) + 4 (lane / 32)
#pragma unroll
        for (int i = 0; i < TL; i++) {
            v16f mins = v16f{};
            if constexpr (!G::Q6) {
                const v8h xo = *reinterpret_cast<const v8h*>(cur + G::XS + (i * 32 + r32) * 32 + half * 16);
                mins = __builtin_amdgcn_mfma_f32_32x32x16_f16(xo, mo, v16f{}, 0, 0, 0);
            }
            const float* dxp = reinterpret_cast<const float*>(cur + G::DX) + i * 32 + half * 4;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const v4f dx = *reinterpret_cast<const v4f*>(dxp + 8 * q);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = 4 * q + e;
                    const float t = G::Q6 ? d * (float)S[i][r] : fmaf(-dm, mins[r], d * (float)S[i][r]);
                    acc[i][r] = fmaf(t, dx[e], acc[i][r]);
                }
            }
        }
    };

    // stage sb multiplies one buffer while sb + 1 lands in the other; every DMA wait is explicit
    auto kloop = [&](auto tlc) __attribute__((always_inline)) {
        dma(buf0, s0);
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
#pragma unroll 1
        for (int sb = s0; sb < s1; sb += 2) {
            if (sb + 1 < s1) dma(buf1, sb + 1);
            stage(tlc, buf0, sb);
            __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
            __syncthreads();
            if (sb + 1 < s1) {
                if (sb + 2 < s1) dma(buf0, sb + 2);
                stage(tlc, buf1, sb + 1);
                __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
                __syncthreads();
            }
        }
    };
    // a grouped slot's last tile often holds a few rows: with at most 32 the second 32-row tile's MFMAs, adds and
    // rescale are skipped (its accumulators stay zero and its rows are not stored)
    if (MOE && m_end - m0 <= 32)
        kloop(std::integral_constant<int, 1>{});
    else
        kloop(std::integral_constant<int, KQ_TM>{});

    if (!MOE && sp >= 0) {
        // a split: its partial tile through system-scope stores (they write through to memory, so the other splits'
        // blocks see them from any XCD without an L2 write-back), a ticket, and the last to arrive adds all S
        constexpr int R = KQ_TM * 16;
        float* pp = tail.part + (size_t)(tail.S * tt + sp) * R * KQ_THREADS + tid;
#pragma unroll
        for (int i = 0; i < KQ_TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) __hip_atomic_store(pp + (i * 16 + r) * KQ_THREADS, acc[i][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
        if (tid == 0) last = __hip_atomic_fetch_add(&tail.tickets[tt], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == tail.S - 1;
        __syncthreads();
        if (!last) return;
        const float* p0 = tail.part + (size_t)tail.S * tt * R * KQ_THREADS + tid;
#pragma unroll
        for (int i = 0; i < KQ_TM; i++) acc[i] = v16f{};
        for (int k = 0; k < tail.S; k++) {
            float part[R];
#pragma unroll
            for (int e = 0; e < R; e++) part[e] = __hip_atomic_load(p0 + ((size_t)k * R + e) * KQ_THREADS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
            for (int i = 0; i < KQ_TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][r] += part[i * 16 + r];
        }
        if (tid == 0) __hip_atomic_store(&tail.tickets[tt], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }

    const int n = n0 + wave * 32 + r32;
    if (MOE && msplit) {
        // The two K halves of a grouped tile. The first half leaves its partial in y (the tile's output rows) and the
        // second in the scratch, each with system-scope stores, which write through to memory, then each takes the
        // tile's ticket; the second to arrive reads the other's partial from its place and stores the sum. A sum of
        // two is the same in either order, so the result does not depend on which half arrives last.
        constexpr int R = KQ_TM * 16;
        float* pp = tail_arg.part + (size_t)tt * R * KQ_THREADS + tid;
        auto yo = [&](int i, int r) __attribute__((always_inline)) {
            const int m = m0 + i * 32 + (r & 3) + 8 * (r >> 2) + 4 * half;
            return m >= m_end ? (int64_t)-1 : (int64_t)(moe.out_rows ? moe.out_rows[m] : m) * N + n;
        };
        if (sp == 1) {
#pragma unroll
            for (int i = 0; i < KQ_TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) __hip_atomic_store(pp + (i * 16 + r) * KQ_THREADS, acc[i][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        } else if (n < N) {
#pragma unroll
            for (int i = 0; i < KQ_TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int64_t o = yo(i, r);
                    if (o >= 0) __hip_atomic_store(y + o, acc[i][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
        }
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
        if (tid == 0) last = __hip_atomic_fetch_add(&tail_arg.tickets[tt], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 1;
        __syncthreads();
        if (!last) return;
        if (sp == 0) {
            float other[R];
#pragma unroll
            for (int e = 0; e < R; e++) other[e] = __hip_atomic_load(pp + e * KQ_THREADS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
            for (int i = 0; i < KQ_TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][r] = acc[i][r] + other[i * 16 + r];
        } else if (n < N) {
            float other[R];
#pragma unroll
            for (int i = 0; i < KQ_TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int64_t o = yo(i, r);
                    other[i * 16 + r] = o >= 0 ? __hip_atomic_load(y + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : 0.0f;
                }
#pragma unroll
            for (int i = 0; i < KQ_TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][r] = other[i * 16 + r] + acc[i][r];
        }
        if (tid == 0) __hip_atomic_store(&tail_arg.tickets[tt], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    if (n < N) {
        const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < KQ_TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + i * 32 + (r & 3) + 8 * (r >> 2) + 4 * half;
                if (m >= m_end) continue;
                const int64_t o = (int64_t)(MOE && moe.out_rows ? moe.out_rows[m] : m) * N + n;
                y[o] = acc[i][r] + bn + (res ? res[o] : 0.0f);
            }
    }
}

}  // namespace

// Whether the q5_K / q6_K GEMM takes these weights: K a multiple of 256 with 16-byte aligned rows (q5_K: always, 176-byte
// super-blocks), q6_K rows that start 16-byte aligned (210-byte super-blocks: K a multiple of 2048), matrices below
// 2 GB (row offsets travel as 32-bit values)
bool kf_gemm_kq_ok(uint32_t ty, const void* w, int64_t row_bytes, int K, int N) {
    if (K % 256 != 0 || (int64_t)N * row_bytes >= (1ll << 31) || (reinterpret_cast<uintptr_t>(w) & 15) != 0) return false;
    if (ty == KF_TYPE_Q4_K || ty == KF_TYPE_Q5_K) return row_bytes % 16 == 0;
    if (ty == KF_TYPE_Q6_K) return row_bytes % 16 == 0;
    return false;
}

// The tail split of an M x N x K launch: the number of K ranges the last round's tiles run as (1: none) and the rounds'
// length in super-blocks (full rounds of nsb, plus nsb / S for a split tail), as the launcher plans them
static int kq_splits(int T, int nsb, int cus) {
    const int rem = T % cus;
    int S = 1;
    while (S < 4 && rem * S * 2 <= cus && nsb / (S * 2) >= 2) S *= 2;
    return S;
}

double kf_gemm_kq_sb_rounds(int M, int N, int K) {
    const int T = ((N + KQ_BN - 1) / KQ_BN) * ((M + KQ_BM - 1) / KQ_BM), nsb = K / 256, cus = kf_cu_count();
    const int rem = T % cus, S = kq_splits(T, nsb, cus);
    return (double)(T / cus) * nsb + (rem == 0 ? 0.0 : (double)nsb / S);
}

// Host launcher, validated by the caller (kf_gemm_kq_ok; Q8K-kind activations in `act`)
hipError_t kf_launch_gemm_kq(uint32_t ty, const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y,
                             int M, int N, int K, hipStream_t s) {
    const kf_act_offsets o = kf_act_layout((size_t)M, (size_t)K);
    const char* base = static_cast<const char*>(act);
    const int T = ((N + KQ_BN - 1) / KQ_BN) * ((M + KQ_BM - 1) / KQ_BM);
    // the tail split (one block a CU): the tiles of a last round at most half full run as S = 2 or 4 blocks over K
    // ranges of at least two super-blocks, S as large as the round holds (KF_GEMM_NO_TAIL turns it off, a comparison
    // knob); it needs the split scratch
    KqTail tail{nullptr, nullptr, T, 1};
    int blocks = T;
    const int cus = kf_cu_count(), rem = T % cus;
    const int S = kq_splits(T, K / 256, cus);
    const size_t part_bytes = (size_t)rem * S * KQ_TM * 16 * KQ_THREADS * 4;
    if (S > 1 && rem <= KF_SPLIT_TICKETS && part_bytes <= KF_SPLIT_SCRATCH - (size_t)KF_SPLIT_TICKETS * 4 && !kf_knob_on(KF_KNOB_GEMM_NO_TAIL)) {
        if (char* scr = static_cast<char*>(kf_split_scratch(s))) {
            tail = KqTail{reinterpret_cast<float*>(scr + (size_t)KF_SPLIT_TICKETS * 4), reinterpret_cast<int*>(scr), T - rem, S};
            blocks = T - rem + rem * S;
        }
    }
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* xq = reinterpret_cast<const int8_t*>(base + o.q);
    const auto* xa = reinterpret_cast<const _Float16*>(base + o.xa);
    const auto* xd = reinterpret_cast<const float*>(base + o.d32);
    if (ty == KF_TYPE_Q4_K)
        gemm_kq_kernel<KF_TYPE_Q4_K, false><<<blocks, KQ_THREADS, 0, s>>>(wb, row_bytes, xq, xa, xd, bias, res, y, M, N, K, tail, KqMoe{});
    else if (ty == KF_TYPE_Q5_K)
        gemm_kq_kernel<KF_TYPE_Q5_K, false><<<blocks, KQ_THREADS, 0, s>>>(wb, row_bytes, xq, xa, xd, bias, res, y, M, N, K, tail, KqMoe{});
    else
        gemm_kq_kernel<KF_TYPE_Q6_K, false><<<blocks, KQ_THREADS, 0, s>>>(wb, row_bytes, xq, xa, xd, bias, res, y, M, N, K, tail, KqMoe{});
    return hipGetLastError();
}

// Grouped (MoE) form on q4_K experts: `act` holds `pairs` activation rows in group order (slot s: rows
// offsets[s]..offsets[s + 1], device offsets), slot s multiplies w + s expert_bytes (N output columns; with w2,
// columns n_split.. from w2), output row p goes to y row out_rows[p] (nullable: p). Validated by the caller: K a
// multiple of 256, n_split a multiple of 256, 16-byte aligned matrices and rows.
hipError_t kf_launch_gemm_kq_moe(const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, int n_split, const void* act, int pairs,
                                 int n_slots, const int32_t* offsets, const int32_t* out_rows, float* y, int N, int K, hipStream_t s) {
    const kf_act_offsets o = kf_act_layout((size_t)pairs, (size_t)K);
    const char* base = static_cast<const char*>(act);
    // row tiles over all slots: each slot adds at most one partial tile
    const int mt = (pairs + KQ_BM - 1) / KQ_BM + n_slots;
    const KqMoe moe{offsets, out_rows, static_cast<const uint8_t*>(w2), expert_bytes, n_slots, n_split};
    // Grids of at most two rounds of the CUs (by the tile bound; down at 512 tokens top-2: 384 tiles, about 320 live)
    // run every tile as two K halves: a second round a quarter full would otherwise take as long as a full one. It
    // needs the split scratch, one partial tile per tile (KF_GEMM_NO_TAIL turns it off, a comparison knob)
    const int T = ((N + KQ_BN - 1) / KQ_BN) * mt;
    KqTail split{nullptr, nullptr, 0, 1};
    int blocks = T;
    if (T <= 2 * kf_cu_count() && K / 256 >= 4 && T <= KF_SPLIT_TICKETS &&
        (size_t)T * KQ_TM * 16 * KQ_THREADS * 4 <= KF_SPLIT_SCRATCH - (size_t)KF_SPLIT_TICKETS * 4 && !kf_knob_on(KF_KNOB_GEMM_NO_TAIL)) {
        if (char* scr = static_cast<char*>(kf_split_scratch(s))) {
            split = KqTail{reinterpret_cast<float*>(scr + (size_t)KF_SPLIT_TICKETS * 4), reinterpret_cast<int*>(scr), 0, 2};
            blocks = 2 * T;
        }
    }
    gemm_kq_kernel<KF_TYPE_Q4_K, true><<<blocks, KQ_THREADS, 0, s>>>(
        static_cast<const uint8_t*>(w), row_bytes, reinterpret_cast<const int8_t*>(base + o.q), reinterpret_cast<const _Float16*>(base + o.xa),
        reinterpret_cast<const float*>(base + o.d32), nullptr, nullptr, y, mt * KQ_BM, N, K, split, moe);
    return hipGetLastError();
}
