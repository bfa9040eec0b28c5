// Prefill GEMM on native q4_K bytes: y[m][n] = sum over super-blocks b of
// dx[m][b] * (d[n][b] * S_b[m][n] - dmin[n][b] * mins_b[m][n]) (+ bias[n] + res[m][n]), with S_b = sum_j sc_j[n] I_j[m][n]
// and mins_b = sum_j m_j[n] bsum_j[m] the reference's exact per-super-block integers (crates/kf-quant/src/types/q4_k.rs:10-58).
// It replaces the reference's unpack + KF8 GEMM with offsets (crates/kf-backend-cuda/src/kernels/quant.cuh:585-601,
// kf8.cu:253-310, HAS_M), reading the native bytes directly.
//
// Arithmetic: the 6-bit scale splits as sc = 8 sh + sl (both in [0, 7]), so the nibble products q sl and q sh (at most
// 105) are int8 operands; per 32-column group and 32 x 32 tile two v_mfma_i32_32x32x32_i8 chains form S_lo and S_hi,
// S_b = S_lo + 8 S_hi exactly; mins_b comes from one exact v_mfma_f32_32x32x16_f16 per super-block and tile (the
// activation group sums split 64 hi + lo by quant_act's xa section); the float rescale runs once per super-block and
// output: five VALU operations.
//
// Schedule (gfx950), each choice measured with ablation builds (G4_ABL below) and a rate probe:
//   * eight waves (two a SIMD), one block a CU, block tile 128 x 256, each wave a 128 x 32 tile (four 32 x 32 MFMA
//     tiles down M), so a wave expands a weight sub-block pair into its two operand planes once for four MFMA tiles.
//     The 64 int32 and 64 f32 accumulator registers a tile needs per lane cap the wave tile: four tiles use all 256
//     registers two waves a SIMD allow;
//   * one super-block (K = 256) per stage, two stage buffers: the activations as [row][256] and the weights as
//     [row][144], the rows' whole super-blocks. Every DMA instruction reads whole rows (four activation rows, or 64
//     consecutive 16-byte pieces of the weight rows), so each 128-byte line crosses from L2 once per instruction: the
//     first form, which read 32-byte pieces of 32 rows per instruction in MFMA order, moved four times the bytes per
//     instruction from L2 and its staging alone took 253 us at the gate/up shape against 91 us now. The MFMA operand
//     order is restored by the 16-byte chunk swizzle c ^ (row % 16) of the activation rows;
//   * the rescale runs out of phase on the two waves of a SIMD: waves 0-3 (early) rescale a super-block at the end of
//     its stage, waves 4-7 (late) convert their S chains to f32 there and finish the rescale at the start of the next
//     stage, while the early wave of their SIMD issues MFMAs. The activation side of a rescale (scales, mins operands)
//     sits in a ring of three records so the late waves still find it one stage later; only the early waves move
//     records, so a late wave's record reads never wait for a DMA in flight;
//   * the MFMA phase runs at raised wave priority (s_setprio 1), so a SIMD's MFMA-issuing wave goes first and its
//     rescaling neighbour fills the issue slots left (8% faster);
//   * staging is buffer_load ... lds DMA over buffer resources based at the tile's first rows; rows past M or N read
//     as zeros through the hardware range check. The DMA is inline assembly (kf_adma16 / kf_adma4) with explicit
//     waits (vmcnt(0) and a barrier at each stage's end): through the builtin it carries no alias information and
//     the compiler waited for the next stage's DMA before each MFMA phase (3% slower). Blocks run in XCD order
//     (each XCD a contiguous range of tiles, M fastest), so the blocks in flight on an XCD share their weight tiles
//     in its L2.
// Measured at M = 2048 (ablation builds with the builtin DMA, gate / down, us): 305-314 / 271-278 in all (300 / 268
// with the DMA in assembly); the MFMA phase alone (no DMA, rescale or plane expansion) 218-225 / 186-189, with the
// plane expansion 225 / 186, with the rescale 265 / 229, with the DMA 245 / 216. The MFMA phase itself keeps the
// matrix cores about half busy, and the rescale and the DMA add to it.
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

// Ablation switch for measurement builds only (0 in the product): bit 1 drops the K loop's DMA, bit 2 the rescale,
// bit 4 the plane expansion, bit 8 the MFMAs
#ifndef G4_ABL
#define G4_ABL 0
#endif

// Packed 16-bit multiply of the bytes of x by a small s: exact per byte while every byte product stays below 256
__device__ __forceinline__ uint32_t g4_pmul(uint32_t x, uint32_t s) {
    typedef unsigned short v2us __attribute__((ext_vector_type(2)));
    const v2us r = __builtin_bit_cast(v2us, x) * v2us{(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, r);
}

// XCD-aware tile order over the first T tiles: block b < T runs tile (b % 8) (T / 8) + b / 8 (tiles numbered
// M-fastest), so XCD x (blocks go to the eight XCDs round-robin) works through a contiguous range of weight tiles
// against every activation panel. Identity when T is not a multiple of eight.
__device__ __forceinline__ void g4_tile(int T, int mt, int b, int& tm, int& tn) {
    const int t = (T & 7) ? b : (b & 7) * (T >> 3) + (b >> 3);
    tn = t / mt;
    tm = t - tn * mt;
}

// The grid's tail: when the tiles leave a last round of blocks at most half full (tiles % CUs <= CUs / 2), the tiles
// from `full` on run as two blocks each, over the two halves of K. Each half writes its 128 x 256 partial tile to
// `part` ([tail tile][half][register][thread]); the second to arrive (a ticket per tail tile) adds the other's, in
// half order, and stores the tile. part == nullptr: no split.
struct G4Tail {
    float* part;
    int* tickets;
    int full;
};

#ifndef G4_PRIO
#define G4_PRIO 1
#endif
#ifndef G4_SWZ
#define G4_SWZ 15
#endif

constexpr int G4_WAVES = 8, G4_THREADS = 64 * G4_WAVES;
#ifndef G4_TILES
#define G4_TILES 4
#endif
constexpr int G4_TM = G4_TILES;              // 32-row tiles per wave (all of the block's rows)
constexpr int G4_BM = 32 * G4_TM;
constexpr int G4_BN = 32 * G4_WAVES;         // 256: one 32-column tile per wave

// Stage buffer layout (bytes): one super-block (K = 256) of the block tile
constexpr int G4_A = 0;                         // activations [row 128][256], 16-byte chunk c of row r at c ^ (r % 8)
constexpr int G4_W = G4_A + G4_BM * 256;        // weight super-blocks [row 256][144] (header, then the nibble pairs)
constexpr int G4_STAGE = G4_W + G4_BN * 144;
// Record layout (bytes): the activation side of a super-block's rescale, in a ring of three
constexpr int G4_DX = 0;                        // activation scales [row 128] f32
constexpr int G4_XS = G4_DX + 128 * 4;          // activation mins operands [row BM][16] f16 (scales: room for 128)
constexpr int G4_REC = G4_XS + G4_BM * 32;
constexpr int G4_NA = G4_BM * 256 / 1024;       // DMA instructions of a stage: activations (4 rows each)
constexpr int G4_NW = G4_BN * 144 / 1024;       // weights (64 16-byte pieces each)
static_assert(G4_BN * 144 % 1024 == 0 && G4_NA % G4_WAVES == 0 && G4_BN * 9 <= 2304, "whole DMA instructions");
static_assert(2 * G4_STAGE + 3 * G4_REC <= 160 * 1024, "two stages and three records fit the LDS");

// The grouped (MoE) form: the activation rows are routed pairs in group order (pairs of slot s are rows
// offsets[s]..offsets[s + 1]), slot s multiplies its own expert matrix (w + s expert_bytes; with w2, output columns from
// n_split on come from w2 + s expert_bytes, row n - n_split), and output row p goes to y row out_rows[p] (or p)
struct G4Moe {
    const int32_t* offsets;
    const int32_t* out_rows;
    const uint8_t* w2;
    int64_t expert_bytes;
    int n_slots, n_split;
};

template <bool MOE>
__global__ void __launch_bounds__(G4_THREADS, 1) gemm_q4k_kernel(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                                  const int8_t* __restrict__ xq, const _Float16* __restrict__ xa,
                                                                  const float* __restrict__ xd32, const float* __restrict__ bias,
                                                                  const float* __restrict__ res, float* __restrict__ y, int M, int N,
                                                                  int K, G4Moe moe, G4Tail tail_arg) {
    // the grouped form never splits: its tail is a compile-time nothing there
    const G4Tail tail = MOE ? G4Tail{nullptr, nullptr, 0} : tail_arg;
    __shared__ __align__(16) uint8_t buf0[G4_STAGE];
    __shared__ __align__(16) uint8_t buf1[G4_STAGE];
    __shared__ __align__(16) uint8_t recs[3 * G4_REC];  // records of super-blocks sb % 3
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5, r32 = lane & 31;
    const int kg = K >> 5;
    const int nsb = K >> 8;
    // the block's tile, and for a tail half its half (else -1) and tail tile; the super-blocks it runs are [s0, s1),
    // literal bounds in the grouped instantiation (bounds derived from the tail fields left it 17 more spilled
    // registers: the stage code's lambdas capture them by reference)
    struct Place {
        int tm, tn, half, tt;
    };
    const Place pl = [&]() {
        Place r{0, 0, -1, 0};
        const int mt = (M + G4_BM - 1) / G4_BM;
        if (!MOE && tail.part && (int)blockIdx.x >= tail.full) {
            const int b = blockIdx.x - tail.full;
            r.tt = b >> 1;
            r.half = b & 1;
            const int t = tail.full + r.tt;
            r.tn = t / mt;
            r.tm = t - r.tn * mt;
        } else {
            g4_tile(tail.part ? tail.full : ((N + G4_BN - 1) / G4_BN) * mt, mt, blockIdx.x, r.tm, r.tn);
        }
        return r;
    }();
    const int tm = pl.tm, tn = pl.tn, half_k = pl.half, tt = pl.tt;
    const int s0 = MOE ? 0 : half_k > 0 ? nsb / 2 : 0, s1 = MOE ? nsb : half_k == 0 ? nsb / 2 : nsb;
    int m0 = tm * G4_BM, n0 = tn * G4_BN;
    int m_end = M;  // rows of the block's slot end here
    const uint8_t* wt = w + (int64_t)n0 * row_bytes;
    int n_end = N;  // columns of the block's matrix end here (as output columns)
    if (MOE) {
        // M counts the grid's row tiles over all slots (an upper bound): tile tm is the slot's tile tm - (the tiles of
        // the slots before it); past the last slot's tiles the block has nothing to do
        int s = 0, t0 = 0;
        for (; s < moe.n_slots; s++) {
            const int rows = moe.offsets[s + 1] - moe.offsets[s], t = (rows + G4_BM - 1) / G4_BM;
            if (tm < t0 + t) break;
            t0 += t;
        }
        if (s == moe.n_slots) return;  // whole block, before any barrier
        m0 = moe.offsets[s] + (tm - t0) * G4_BM;
        m_end = moe.offsets[s + 1];
        if (moe.w2 && n0 >= moe.n_split) {
            wt = moe.w2 + s * moe.expert_bytes + (int64_t)(n0 - moe.n_split) * row_bytes;
        } else {
            wt = w + s * moe.expert_bytes + (int64_t)n0 * row_bytes;
            if (moe.w2) n_end = moe.n_split;
        }
    }

    // DMA sources: buffer resources over the tile's first rows to the end of the matrix; rows past M or N read as
    // zeros (the hardware range check), and their outputs are not stored
    const auto rw = kf_arsrc(wt, (uint64_t)(n_end - n0) * row_bytes);
    const auto rx = kf_arsrc(xq + (int64_t)m0 * K, (uint64_t)(m_end - m0) * K);
    const auto rs = kf_arsrc(xa + (int64_t)m0 * nsb * 16, (uint64_t)(m_end - m0) * nsb * 32);
    const auto rd = kf_arsrc(xd32 + (int64_t)m0 * kg, (uint64_t)(m_end - m0) * kg * 4);
    // Every DMA instruction reads whole rows: 4 activation rows of 256 bytes, or 64 consecutive 16-byte pieces of the
    // weight rows' 144-byte super-blocks (about seven rows), so each 128-byte line a stage needs crosses from L2 once
    // per instruction. Activation instruction i (rows 4 i..) is wave i % 8's; lane l takes chunk (l % 16) ^ (row % 8)
    // of row 4 i + l / 16 and writes it at position l % 16, so the MFMA operand reads below hit distinct banks.
    const int arow = 4 * wave + (lane >> 4);
    const int va = arow * K + 16 * ((lane & 15) ^ (arow & G4_SWZ));  // + 32 K k for instruction wave + 8 k
    // weight piece q = 64 i + l of a stage: row q / 9, piece q % 9 (computed per stage: cheaper than 5 registers)
    auto wpiece = [&](int i) __attribute__((always_inline)) {
        const int q = 64 * i + lane, row = (q * 7282) >> 16;  // q / 9 for q < 2304
        return row * (int)row_bytes + 16 * (q - 9 * row);
    };
    const int vd = ((wave & 1) * 64 + lane) * kg * 4;              // waves 0-1: activation scales
    const int vs = (((wave & 3) * 32 + (lane >> 1)) * nsb * 32) + (lane & 1) * 16;  // waves 0-3: mins operands
    const bool late = wave >= 4;  // waves 4-7 finish a super-block's rescale at the start of the next one

    auto record = [&](int sb) __attribute__((always_inline)) { return recs + (sb % 3) * G4_REC; };
    // A stage's operands; its record comes from the early waves (so a late wave's code holds no record DMA that its
    // reads of the previous records would wait for)
    auto dma = [&](uint8_t* buf, int sb) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < G4_NA / G4_WAVES; k++) kf_adma16(rx, va, sb * 256 + 32 * K * k, buf + G4_A + (wave + G4_WAVES * k) * 1024);
#pragma unroll
        for (int k = 0; k < (G4_NW + G4_WAVES - 1) / G4_WAVES; k++)
            if (wave + G4_WAVES * k < G4_NW)
                kf_adma16(rw, wpiece(wave + G4_WAVES * k), sb * KF_Q4_K_BYTES, buf + G4_W + (wave + G4_WAVES * k) * 1024);
        if (!late) {
            uint8_t* rec = record(sb);
            if (wave < 2) kf_adma4(rd, vd, sb * 32, rec + G4_DX + wave * 256);
            if (wave * 32 < G4_BM) kf_adma16(rs, vs, sb * 32, rec + G4_XS + wave * 1024);
        }
    };

    v16f acc[G4_TM];
    v16i slo[G4_TM], shi[G4_TM];
#pragma unroll
    for (int i = 0; i < G4_TM; i++) acc[i] = v16f{};

    // the wave's weight row (tile column) and the activation chunk swizzle of its lane's rows
    const int wrow = (wave * 32 + r32) * 144;
    const int sw = r32 & G4_SWZ;

    // The super-block's four sub-block pairs into the S chains
    auto mfma_sb = [&](const uint8_t* buf) __attribute__((always_inline)) {
        const uint4 hd = *reinterpret_cast<const uint4*>(buf + G4_W + wrow);
        uint32_t scv[2], mnv[2];
        kf_q4k_scales8(hd.y, hd.z, hd.w, scv, mnv);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint4 raw = *reinterpret_cast<const uint4*>(buf + G4_W + wrow + 16 + 32 * p + 16 * half);
            const uint32_t sc2 = kf_pair(scv, p);
            const uint32_t s0 = sc2 & 0xffu, s1 = sc2 >> 8;
            const uint32_t l0 = s0 & 7u, u0 = s0 >> 3, l1 = s1 & 7u, u1 = s1 >> 3;
            const uint32_t m4 = 0x0f0f0f0fu;
            const uint32_t v[4] = {raw.x, raw.y, raw.z, raw.w};
            v4i bl[2], bh[2];
            if (G4_ABL & 4) {
                // the high plane a permutation of the low one: identical operands let the compiler merge the two
                // MFMAs of a tile and group, halving the matrix-core work the ablation measures
                bl[0] = bl[1] = v4i{(int)raw.x, (int)raw.y, (int)raw.z, (int)raw.w};
                bh[0] = bh[1] = v4i{(int)raw.y, (int)raw.z, (int)raw.w, (int)raw.x};
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t lo = v[e] & m4, hi = (v[e] >> 4) & m4;
                    bl[0][e] = (int)g4_pmul(lo, l0);
                    bh[0][e] = (int)g4_pmul(lo, u0);
                    bl[1][e] = (int)g4_pmul(hi, l1);
                    bh[1][e] = (int)g4_pmul(hi, u1);
                }
            }
#pragma unroll
            for (int gg = 0; gg < 2; gg++) {
                const int g = 2 * p + gg;
                const bool z = g == 0;
                // chunk 2 g + half of the lane's row, stored at (2 g + half) ^ (row % 8)
                const int ao = G4_A + r32 * 256 + 16 * ((2 * g + half) ^ sw);
#pragma unroll
                for (int i = 0; i < G4_TM; i++) {
                    const v4i a = *reinterpret_cast<const v4i*>(buf + ao + i * 32 * 256);
                    if (G4_ABL & 8) {
                        slo[i][0] = (z ? 0 : slo[i][0]) ^ a[0] ^ bl[gg][0];
                        shi[i][0] = (z ? 0 : shi[i][0]) ^ a[1] ^ bh[gg][1];
                        continue;
                    }
                    slo[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bl[gg], z ? v16i{} : slo[i], 0, 0, 0);
                    shi[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bh[gg], z ? v16i{} : shi[i], 0, 0, 0);
                }
            }
        }
    };

    // The super-block's rescale, acc += dx (d S - dmin mins), in two parts. Part one turns the S chains into f32
    // (S = S_lo + 8 S_hi, exact); part two takes the mins by MFMA and the scales from the header hd and the record rec.
    v16f sf[G4_TM];
    auto rescale1 = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < G4_TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) sf[i][r] = (float)(slo[i][r] + (shi[i][r] << 3));  // |S| < 2^25: exact
    };
    auto rescale2 = [&](const uint4 hd, const uint8_t* rec) __attribute__((always_inline)) {
        if (G4_ABL & 2) {
#pragma unroll
            for (int i = 0; i < G4_TM; i++) acc[i][0] += sf[i][0];
            return;
        }
        v8h mo;
        uint32_t scv[2], mnv[2];
        kf_q4k_scales8(hd.y, hd.z, hd.w, scv, mnv);
#pragma unroll
        for (int pj = 0; pj < 4; pj++) {
            const uint32_t m2 = kf_pair(mnv, pj);
            const uint32_t f = half ? 1u : 64u;
            mo[2 * pj] = (_Float16)(float)(f * (m2 & 0xffu));
            mo[2 * pj + 1] = (_Float16)(float)(f * (m2 >> 8));
        }
        const float dd = kf_h2f(hd.x & 0xffffu), dm = kf_h2f(hd.x >> 16);
#pragma unroll
        for (int i = 0; i < G4_TM; i++) {
            // the row's mins operand: sums split as 64 hi + lo (lanes < 32: hi, lanes >= 32: lo), from quant_act
            const v8h xo = *reinterpret_cast<const v8h*>(rec + G4_XS + (i * 32 + r32) * 32 + half * 16);
            const v16f mins = __builtin_amdgcn_mfma_f32_32x32x16_f16(xo, mo, v16f{}, 0, 0, 0);
            // accumulator register r holds row (r % 4) + 8 (r / 4) + 4 (lane / 32) of the tile
            const float* dxp = reinterpret_cast<const float*>(rec + G4_DX) + i * 32 + half * 4;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const v4f dx = *reinterpret_cast<const v4f*>(dxp + 8 * q);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = 4 * q + e;
                    const float t = fmaf(-dm, mins[r], dd * sf[i][r]);
                    acc[i][r] = fmaf(t, dx[e], acc[i][r]);
                }
            }
            // one tile at a time: every tile's mins and scales at once would need 128 more registers
            __asm__ volatile("" ::: "memory");
        }
    };

    // Stage sb (operands in cur) of one half of the block. Early waves (LATE false) rescale sb at its end; late waves
    // turn their S chains into f32 at its end and finish the rescale at the start of stage sb + 1, while the early
    // waves of their SIMDs issue MFMAs.
    uint4 hprev = make_uint4(0u, 0u, 0u, 0u);  // late waves: the header of the previous super-block
    auto stage = [&](auto latec, const uint8_t* cur, uint8_t* nxt, int sb) __attribute__((always_inline)) {
        constexpr bool LATE = decltype(latec)::value;
        if (sb + 1 < s1 && !(G4_ABL & 1)) dma(nxt, sb + 1);
        if (LATE && sb > s0) rescale2(hprev, record(sb - 1));
        __builtin_amdgcn_sched_barrier(0);
        // the MFMA phase at raised issue priority: a SIMD's other wave, in its rescale, fills the issue slots the MFMAs
        // leave
        if (G4_PRIO) __builtin_amdgcn_s_setprio(1);
        mfma_sb(cur);
        if (G4_PRIO) __builtin_amdgcn_s_setprio(0);
        const uint4 hd = *reinterpret_cast<const uint4*>(cur + G4_W + wrow);
        rescale1();
        if (LATE)
            hprev = hd;
        else
            rescale2(hd, record(sb));
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
    };
    auto kloop = [&](auto latec) __attribute__((always_inline)) {
#pragma unroll 1
        for (int sb = s0; sb < s1; sb += 2) {
            stage(latec, buf0, buf1, sb);
            if (sb + 1 < s1) stage(latec, buf1, buf0, sb + 1);
        }
        if (decltype(latec)::value) rescale2(hprev, record(s1 - 1));
    };

    dma(buf0, s0);
    if (G4_ABL & 1) dma(buf1, 0);
    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
    __syncthreads();
    if (late)
        kloop(std::true_type{});
    else
        kloop(std::false_type{});


    if (!MOE && half_k >= 0) {
        __shared__ int last;
        // a tail half: its partial tile through system-scope stores (they write through to memory, so the other
        // half's block sees them from any XCD without an L2 write-back), a ticket, and the second to arrive adds
        float* pp = tail.part + (size_t)(2 * tt + half_k) * G4_TM * 16 * G4_THREADS + tid;
#pragma unroll
        for (int i = 0; i < G4_TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) __hip_atomic_store(pp + (i * 16 + r) * G4_THREADS, acc[i][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
        __syncthreads();
        if (tid == 0) last = __hip_atomic_fetch_add(&tail.tickets[tt], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 1;
        __syncthreads();
        if (!last) return;
        const float* po = tail.part + (size_t)(2 * tt + (half_k ^ 1)) * G4_TM * 16 * G4_THREADS + tid;
        float other[G4_TM * 16];
#pragma unroll
        for (int k = 0; k < G4_TM * 16; k++) other[k] = __hip_atomic_load(po + k * G4_THREADS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
        for (int i = 0; i < G4_TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][r] = half_k ? other[i * 16 + r] + acc[i][r] : acc[i][r] + other[i * 16 + r];
        if (tid == 0) __hip_atomic_store(&tail.tickets[tt], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }

    const int n = n0 + wave * 32 + r32;
    if (n < N) {
        const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < G4_TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // row m0 + 32 i + (r % 4) + 8 (r / 4) + 4 half: a wave-uniform row base and the lane's offset
                const int mb = m0 + i * 32 + (r & 3) + 8 * (r >> 2);
                if (mb + 4 * half >= m_end) continue;
                if (MOE && moe.out_rows) {
                    const int64_t o = (int64_t)moe.out_rows[mb + 4 * half] * N + n;
                    y[o] = acc[i][r] + bn + (res ? res[o] : 0.0f);
                    continue;
                }
                const int64_t ob = (int64_t)mb * N;
                const int lo = 4 * half * N + n;
                y[ob + lo] = acc[i][r] + bn + (res ? res[ob + lo] : 0.0f);
            }
    }
}

}  // namespace

// The rounds of an M x N x K launch in super-blocks, as the launcher plans them: one 128 x 256 tile a CU a round, a
// last round at most half full as two K halves (half a round)
double kf_gemm_q4k_sb_rounds(int M, int N, int K) {
    const int T = ((N + G4_BN - 1) / G4_BN) * ((M + G4_BM - 1) / G4_BM), cus = kf_cu_count(), rem = T % cus, nsb = K / 256;
    const double last = rem == 0 ? 0.0 : rem <= cus / 2 && nsb >= 4 ? 0.5 : 1.0;
    return ((double)(T / cus) + last) * nsb;
}

// Host launcher of the q4_K prefill GEMM, validated by the caller (api.cpp): K a multiple of 256, Q8K-kind activations
// in `act`
hipError_t kf_launch_gemm_q4k(const void* w, int64_t row_bytes, const void* act, const float* bias, const float* res, float* y, int M,
                              int N, int K, hipStream_t s) {
    const kf_act_offsets o = kf_act_layout((size_t)M, (size_t)K);
    const char* base = static_cast<const char*>(act);
    const int T = ((N + G4_BN - 1) / G4_BN) * ((M + G4_BM - 1) / G4_BM);
    // the tail split (one block a CU): a last round at most half full runs its tiles as K halves in one round of
    // half the length; it needs the split scratch (KF_GEMM_NO_TAIL turns it off, a comparison knob)
    G4Tail tail{nullptr, nullptr, T};
    int blocks = T;
    const int cus = kf_cu_count(), rem = T % cus;
    const size_t part_bytes = (size_t)rem * 2 * G4_TM * 16 * G4_THREADS * 4;
    if (rem > 0 && rem <= cus / 2 && K / 256 >= 4 && rem <= KF_SPLIT_TICKETS &&
        part_bytes <= KF_SPLIT_SCRATCH - (size_t)KF_SPLIT_TICKETS * 4 && !kf_knob_on(KF_KNOB_GEMM_NO_TAIL)) {
        if (char* scr = static_cast<char*>(kf_split_scratch(s))) {
            tail = G4Tail{reinterpret_cast<float*>(scr + (size_t)KF_SPLIT_TICKETS * 4), reinterpret_cast<int*>(scr), T - rem};
            blocks = T + rem;
        }
    }
    gemm_q4k_kernel<false><<<blocks, G4_THREADS, 0, s>>>(static_cast<const uint8_t*>(w), row_bytes, reinterpret_cast<const int8_t*>(base + o.q),
                                                          reinterpret_cast<const _Float16*>(base + o.xa),
                                                          reinterpret_cast<const float*>(base + o.d32), bias, res, y, M, N, K, G4Moe{}, tail);
    return hipGetLastError();
}

// Grouped (MoE) form: `act` holds `pairs` activation rows in group order (slot s: rows offsets[s]..offsets[s + 1],
// device offsets), slot s multiplies w + s expert_bytes (N output columns; with w2, columns n_split.. from w2), output
// row p goes to y row out_rows[p] (nullable: p). Validated by the caller: K a multiple of 256, n_split a multiple of 256.
hipError_t kf_launch_gemm_q4k_moe(const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, int n_split, const void* act,
                                  int pairs, int n_slots, const int32_t* offsets, const int32_t* out_rows, float* y, int N, int K,
                                  hipStream_t s) {
    const kf_act_offsets o = kf_act_layout((size_t)pairs, (size_t)K);
    const char* base = static_cast<const char*>(act);
    // row tiles over all slots: each slot adds at most one partial tile
    const int mt = (pairs + G4_BM - 1) / G4_BM + n_slots;
    dim3 grid(((N + G4_BN - 1) / G4_BN) * mt);
    const G4Moe moe{offsets, out_rows, static_cast<const uint8_t*>(w2), expert_bytes, n_slots, n_split};
    gemm_q4k_kernel<true><<<grid, G4_THREADS, 0, s>>>(static_cast<const uint8_t*>(w), row_bytes, reinterpret_cast<const int8_t*>(base + o.q),
                                                       reinterpret_cast<const _Float16*>(base + o.xa),
                                                       reinterpret_cast<const float*>(base + o.d32), nullptr, nullptr, y, mt * G4_BM, N, K,
                                                       moe, G4Tail{nullptr, nullptr, 0});
    return hipGetLastError();
}
