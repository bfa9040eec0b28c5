// Multi-row q4_K product on the matrix cores: up to 16 activation rows against each weight row, for the MoE grouped
// expert products (grid row = expert slot, activation rows = the pairs routed to it) and the few-row product of one
// matrix. Same interface and results as rows_kernel (rows.hip), which it replaces for q4_K weights: the super-block
// integers are the reference's dot_i8 integers (crates/kf-quant/src/types/q4_k.rs:10-58, sumi and mins), exact; the
// float combine is the GEMV's. The reference runs these products as per-pair matvecs (kf_moe_matvec_i8 /
// kf_moe_gate_up_i8, crates/kf-backend-cuda/src/kernels/quant.cuh:519-581) and its small-batch q4_K form as fragment
// MMAs (kf_mm_frag, crates/kf-backend-cuda/src/kernels/mm_frag.cuh:60-292).
//
// Why: the per-lane dot4 form costs about 35 vector instructions per activation row and weight step, so with four to
// eight rows a weight byte it is bound by the VALU rather than by HBM. Here a wave owns 16 weight rows and the
// matrix core forms all rows' integer dots at once; the vector work per weight byte no longer grows with the rows.
//
// Per wave, per super-block of its 16 weight rows (2304 bytes):
//   * operands, MFMA layouts (16 x 16 x 32 int8): A = activations (lane l: row l % 16, bytes 8 (l / 16).. of the
//     group), B = weights (lane l: weight row l % 16, the same bytes of the group). For sub-block pair p a lane loads
//     the 8 nibble bytes 16 + 32 p + 8 (l / 16).. of its row: the low nibbles are its B operand of group 2 p, the high
//     nibbles of group 2 p + 1, unscaled (0..15);
//   * I_g = v_mfma_i32_16x16x32_i8 per group, exact int32; S = sum_g sc_g I_g by 24-bit multiply-adds (every
//     product below 2^22): the output lane holds weight row l % 16 for four activation rows, so its scales are one
//     row's;
//   * mins = sum_g m_g bsum_g by one v_mfma_f32_16x16x16_f16 (bsum_g = 64 hi + lo split at staging, m_g and 64 m_g
//     against them: every product and partial sum is an integer below 2^24, exact);
//   * acc += dx (d S - dmin mins).
// Weights: each wave's super-block of 16 rows x 144 bytes is fetched whole by DMA (buffer_load ... lds: contiguous
// 16-byte pieces, every cache line used by one instruction) into one of two LDS buffers of its own, the next one
// landing while the current one is multiplied, continuing across the wave's tiles; operand loads from global memory
// per lane (16 rows x 32 bytes an instruction) measured 25% slower. Activations are staged in LDS once per chunk of RT
// rows by DMA, in K phases when all n columns do not fit beside the weight buffers.
// Measured (Mixtral-style layer, 8 Q4_K experts, 16 tokens top-2): fused gate/up 129 us against 203 us for the
// per-lane form.
#include "kf_knobs.h"
#include "kf_blocks.h"
#include "kf_host.h"

#include <algorithm>

namespace {

typedef float rm_v4f __attribute__((ext_vector_type(4)));
typedef int rm_v4i __attribute__((ext_vector_type(4)));
typedef _Float16 rm_v4h __attribute__((ext_vector_type(4)));
typedef uint32_t rm_v2u __attribute__((ext_vector_type(2)));
typedef uint32_t rm_v4u __attribute__((ext_vector_type(4)));

constexpr int RM_WAVES = 8;
constexpr int RM_THREADS = 64 * RM_WAVES;

// LDS of one chunk of RT staged rows: A operands [group][RT][32 bytes], the split group sums [super-block][RT][16 f16],
// the activation scales [super-block][RT] f32
struct RmLds {
    int a, x, d, total;
};

__host__ __device__ inline RmLds rm_lds(int n, int rt) {
    RmLds l;
    const int nsb = n / KF_Q4_K_BLOCK;
    l.a = 0;
    l.x = rt * n;
    l.d = l.x + nsb * rt * 32;
    l.total = l.d + nsb * rt * 4;
    return l;
}

constexpr int RM_TILE_BYTES = 16 * KF_Q4_K_BYTES;  // one super-block of a wave's 16 weight rows

// One super-block of one weight operand row set: the lane's header and its four 8-byte nibble pieces (q5_K: and the
// high bits of its eight columns, qh bytes 8 q..)
struct RmW {
    rm_v4u hd;
    rm_v2u q[4];
    rm_v2u qh;
};

// S and mins of one super-block for the lane's weight row against the staged rows; a_at / x_at: the lane's A operand
// and split-sum addresses of this super-block (group 0)
template <bool Q5 = false>
__device__ __forceinline__ void rm_block(const RmW& v, const uint8_t* a_at, int a_gstride, rm_v4h xo, int q, rm_v4i& S, rm_v4f& mins) {
    const uint32_t m4 = 0x0f0f0f0fu, m1 = 0x01010101u;
    S = rm_v4i{0, 0, 0, 0};
    // the eight 6-bit scales and mins at once (crates/kf-quant/src/types/mod.rs:86-94); mq: the lane's quarter q,
    // groups 2q and 2q+1
    uint32_t sc[2], mn[2];
    kf_q4k_scales8(v.hd.y, v.hd.z, v.hd.w, sc, mn);
    const uint32_t mq = kf_pair(mn, q);
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t sc2 = kf_pair(sc, p);
        uint32_t l0 = v.q[p].x & m4, l1 = v.q[p].y & m4, h0 = (v.q[p].x >> 4) & m4, h1 = (v.q[p].y >> 4) & m4;
        if constexpr (Q5) {  // the fifth bit of group g is bit g of the column's qh byte (q5_k.rs:7-60)
            l0 |= ((v.qh.x >> (2 * p)) & m1) << 4;
            l1 |= ((v.qh.y >> (2 * p)) & m1) << 4;
            h0 |= ((v.qh.x >> (2 * p + 1)) & m1) << 4;
            h1 |= ((v.qh.y >> (2 * p + 1)) & m1) << 4;
        }
        const long blo = (long)l0 | ((long)l1 << 32);
        const long bhi = (long)h0 | ((long)h1 << 32);
        const long a0 = *reinterpret_cast<const long*>(a_at + (2 * p) * a_gstride);
        const long a1 = *reinterpret_cast<const long*>(a_at + (2 * p + 1) * a_gstride);
        const rm_v4i i0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, blo, rm_v4i{0, 0, 0, 0}, 0, 0, 0);
        const rm_v4i i1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bhi, rm_v4i{0, 0, 0, 0}, 0, 0, 0);
        const int s0 = (int)(sc2 & 0xffu), s1 = (int)(sc2 >> 8);
#pragma unroll
        for (int e = 0; e < 4; e++) S[e] += __mul24(s0, i0[e]) + __mul24(s1, i1[e]);
    }
    // k slots of the lane's quarter q: groups 2q and 2q+1, each as (64 m, m) against the split sum (hi, lo)
    rm_v4h mo;
    mo[0] = (_Float16)(float)(64u * (mq & 0xffu));
    mo[1] = (_Float16)(float)(mq & 0xffu);
    mo[2] = (_Float16)(float)(64u * (mq >> 8));
    mo[3] = (_Float16)(float)(mq >> 8);
    mins = __builtin_amdgcn_mfma_f32_16x16x16f16(xo, mo, rm_v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
}

// ops::silu (crates/kf-backend-cpu/src/ops.rs): x / (1 + e^-x)
__device__ __forceinline__ float rm_silu(float x) { return x / (1.0f + expf(-x)); }

// Block (x, slot): weight rows [x * rpb, +rpb) of the slot's matrix (w + slot * expert_bytes; with GLU also w2's)
// against the slot's pairs offsets[slot] .. offsets[slot + 1] of `order` (identity without order; one slot [0,
// pairs) without offsets), RT at a time. The activation row of pair p is p (per_slot) or p / n_used. Outputs
// y[p][o]: GLU ? silu(gate . x) * (up . x) : w . x + bias[o] + res[p][o].
// K runs in phases of kc columns when a chunk's staged rows of all n columns do not fit beside the weight buffers;
// then every wave owns one 16-row tile (rpb = 16 x waves) and its accumulators carry across the phases.
template <bool GLU, int RT, int NB>
__global__ void __launch_bounds__(RM_THREADS) rows_mma_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int64_t expert_bytes,
                                                              int64_t row_bytes, const int8_t* __restrict__ xq, const int32_t* __restrict__ xs32,
                                                              const float* __restrict__ xd32, int n, int n_out, const int32_t* __restrict__ order,
                                                              const int32_t* __restrict__ offsets, int pairs, int n_used, int per_slot,
                                                              const float* __restrict__ bias, const float* __restrict__ res, float* __restrict__ y,
                                                              int rpb, int kc) {
    extern __shared__ __align__(16) uint8_t smem[];
    // a wave's super-blocks of weights land whole in its LDS buffers (NB of them, in rotation), rows contiguous
    constexpr int NW = GLU ? 2 : 1;
    static_assert(NB >= 2 && NB <= 5, "two to five weight buffers");
    __shared__ __align__(16) uint8_t pk[NB][RM_WAVES * NW * RM_TILE_BYTES];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = blockIdx.y;
    const int p0 = offsets ? offsets[slot] : 0;
    const int p1 = offsets ? offsets[slot + 1] : pairs;
    if (p0 >= p1) return;
    const int nsb = n / KF_Q4_K_BLOCK, nsum = n / 32;
    const int kcs = kc / KF_Q4_K_BLOCK, nph = (nsb + kcs - 1) / kcs;
    const int o0 = blockIdx.x * rpb;
    const int o1 = min(o0 + rpb, n_out);
    const int tiles = (o1 - o0 + 15) / 16;
    const RmLds L = rm_lds(kc, RT);
    const int c = lane & 15, q = lane >> 4;

    // weights: a buffer resource from the tile's first row to the slot matrix's last (rows past it read as zeros);
    // DMA instruction i of a super-block moves the 16-byte pieces s = 64 i + lane of the tile's 16 rows x 144 bytes
    // (row s / 9, piece s % 9; the third instruction only on lanes below 16): 3 instructions per matrix, the
    // super-block adding sb * 144 as a scalar offset
    const uint8_t* wbase = w + (int64_t)slot * expert_bytes;
    const uint8_t* ubase = GLU ? w2 + (int64_t)slot * expert_bytes : wbase;
    int vpk[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int s2 = min(64 * i + lane, 143);
        vpk[i] = (s2 / 9) * (int)row_bytes + 16 * (s2 % 9);
    }
    // the wave's items in a phase: (tile t, super-block) for tiles t = wave, wave + WAVES, ..., super-block fastest
    const int my_tiles = tiles > wave ? (tiles - wave + RM_WAVES - 1) / RM_WAVES : 0;
    auto park = [&](int sb0, int nsbp, int it, uint8_t* buf) {
        const int t = wave + (it / nsbp) * RM_WAVES, sb = sb0 + it % nsbp;
        // the resource starts at the tile's first row and ends at the matrix's last, so the hardware range check on
        // the per-lane offset returns zeros for the tile's rows past n_out instead of reading past the matrix
        const int trow = o0 + 16 * t;
        const int64_t tb = (int64_t)trow * row_bytes;
        const uint64_t left = (uint64_t)(n_out - trow) * row_bytes;
        const int so = sb * KF_Q4_K_BYTES;
#pragma unroll
        for (int k = 0; k < NW; k++) {
            uint8_t* b = buf + (wave * NW + k) * RM_TILE_BYTES;
            const auto r = kf_rsrc((k == 0 ? wbase : ubase) + tb, left);
            kf_bdma16(r, vpk[0], so, b);
            kf_bdma16(r, vpk[1], so, b + 1024);
            if (lane < 16) kf_bdma16(r, vpk[2], so, b + 2048);
        }
    };
    auto unpark = [&](RmW& v, const uint8_t* buf, int k) {
        const uint8_t* b = buf + (wave * NW + k) * RM_TILE_BYTES + c * KF_Q4_K_BYTES;
        v.hd = *reinterpret_cast<const rm_v4u*>(b);
#pragma unroll
        for (int p = 0; p < 4; p++) v.q[p] = *reinterpret_cast<const rm_v2u*>(b + 16 + 32 * p + 8 * q);
    };
    auto xrow_of = [&](int c0, int R, int r) {
        const int pr = c0 + min(r, R - 1);
        const int p = order ? order[pr] : pr;
        return per_slot ? p : p / n_used;
    };

    for (int c0 = p0; c0 < p1; c0 += RT) {
        const int R = min(RT, p1 - c0);
        // the pairs of the lane's output rows 4q .. 4q + 3 (loaded once: a load at a tile's end would make the wave
        // wait for every weight request in flight)
        int pidx[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = min(4 * q + e, R - 1);
            pidx[e] = order ? order[c0 + m] : c0 + m;
        }
        rm_v4f acc = rm_v4f{0.0f, 0.0f, 0.0f, 0.0f}, accu = rm_v4f{0.0f, 0.0f, 0.0f, 0.0f};
        for (int ph = 0; ph < nph; ph++) {
            const int sb0 = ph * kcs, nsbp = min(kcs, nsb - sb0);
            const int items = my_tiles * nsbp;
            const bool last_phase = ph == nph - 1;
            // the first NB super-blocks of weights go out before the phase's activations are staged
#pragma unroll
            for (int b = 0; b < NB; b++)
                if (items > b) park(sb0, nsbp, b, pk[b]);
            // stage: A operands by DMA (instruction i fills LDS bytes [1024 i, +1024): slot s = 64 i + lane of 16
            // bytes is group s / (2 RT) of the phase, row (s / 2) % RT, half s % 2), rows past R repeat row R - 1
            {
                const int ninst = RT * nsbp / 4;
                for (int i = wave; i < ninst; i += RM_WAVES) {
                    const int s = 64 * i + lane, g = s / (2 * RT), r = (s >> 1) % RT, h = s & 1;
                    kf_dma16(xq + (int64_t)xrow_of(c0, R, r) * n + (int64_t)sb0 * KF_Q4_K_BLOCK + 32 * g + 16 * h, smem + L.a + 1024 * i);
                }
                // split group sums (f16 hi, lo of bsum = 64 hi + lo, exact) and scales, per (super-block, row)
                for (int idx = threadIdx.x; idx < nsbp * RT; idx += RM_THREADS) {
                    const int sb = idx / RT, r = idx % RT;
                    const int xrow = xrow_of(c0, R, r);
                    const int32_t* bs = xs32 + (int64_t)xrow * nsum + (sb0 + sb) * 8;
                    _Float16* xo = reinterpret_cast<_Float16*>(smem + L.x) + (size_t)idx * 16;
#pragma unroll
                    for (int g = 0; g < 8; g++) {
                        const int b = bs[g];
                        xo[2 * g] = (_Float16)(float)(b >> 6);
                        xo[2 * g + 1] = (_Float16)(float)(b & 63);
                    }
                    reinterpret_cast<float*>(smem + L.d)[idx] = xd32[(int64_t)xrow * nsum + (sb0 + sb) * 8];
                }
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();

            // lane constants: A operand of row c (rows past RT alias the staged ones; their outputs are not stored),
            // split sums of row c, scales of rows 4q .. 4q + 3
            const uint8_t* a_lane = smem + L.a + (c % RT) * 32 + 8 * q;
            const int a_g = RT * 32;  // bytes between groups
            auto process = [&](const RmW& v, const RmW& vu, int it) {
                const int sb = it % nsbp;
                const rm_v4h xo = *reinterpret_cast<const rm_v4h*>(smem + L.x + (sb * RT + c % RT) * 32 + 8 * q);
                const rm_v4f dx = *reinterpret_cast<const rm_v4f*>(smem + L.d + (sb * RT + (4 * q) % RT) * 4);
                const uint8_t* a_at = a_lane + sb * 8 * a_g;
                rm_v4i S;
                rm_v4f mins;
                rm_block(v, a_at, a_g, xo, q, S, mins);
                const float d = kf_h2f(v.hd.x & 0xffffu), dm = kf_h2f(v.hd.x >> 16);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = fmaf(dx[e], fmaf(-dm, mins[e], d * (float)S[e]), acc[e]);
                if constexpr (GLU) {
                    rm_block(vu, a_at, a_g, xo, q, S, mins);
                    const float du = kf_h2f(vu.hd.x & 0xffffu), dmu = kf_h2f(vu.hd.x >> 16);
#pragma unroll
                    for (int e = 0; e < 4; e++) accu[e] = fmaf(dx[e], fmaf(-dmu, mins[e], du * (float)S[e]), accu[e]);
                }
                if (last_phase && sb == nsbp - 1) {  // the tile is done: lane (c, q) holds weight row c for rows 4q ..
                    const int t = wave + (it / nsbp) * RM_WAVES;
                    const int o = o0 + 16 * t + c;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int m = 4 * q + e;
                        if (m < R && o < o1) {
                            const int p = pidx[e];
                            float* yo = y + (int64_t)p * n_out + o;
                            if constexpr (GLU)
                                *yo = rm_silu(acc[e]) * accu[e];
                            else
                                *yo = acc[e] + (bias ? bias[o] : 0.0f) + (res ? res[(int64_t)p * n_out + o] : 0.0f);
                        }
                    }
                    acc = rm_v4f{0.0f, 0.0f, 0.0f, 0.0f};
                    accu = rm_v4f{0.0f, 0.0f, 0.0f, 0.0f};
                }
            };
            // NB buffers in rotation: item j is multiplied from one while j + 1 .. j + NB - 1 land in the others; each
            // wait leaves only those items' DMA instructions (3 NW each) outstanding
            constexpr int NI = 3 * NW;
            auto step = [&](uint8_t* buf, int j) {
                const int ahead = min(NB - 1, items - 1 - j);
                if (NB > 4 && ahead >= 4)
                    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(4 * NI));
                else if (NB > 3 && ahead == 3)
                    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(3 * NI));
                else if (ahead == 2)
                    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(2 * NI));
                else if (ahead == 1)
                    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(NI));
                else
                    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
                RmW v, vu;
                unpark(v, buf, 0);
                if constexpr (GLU) unpark(vu, buf, 1);
                process(v, vu, j);
                if (j + NB < items) {
                    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(63) & ~(15 << 8));  // this buffer's reads are done
                    park(sb0, nsbp, j + NB, buf);
                }
            };
            for (int it = 0; it < items; it += NB) {
#pragma unroll
                for (int b = 0; b < NB; b++)
                    if (it + b < items) step(pk[b], it + b);
            }
            __syncthreads();  // before the next phase or chunk restages
        }
    }
}

// LDS budget of a block: the chunk's staged rows (dynamic) and the two weight buffers (static)
constexpr int RM_LDS_MAX = 160 * 1024;

struct RmPlan {
    int rt, nb, kc, rpb;
};

// Staged rows per chunk (16 or 8), weight buffers per wave (3 or 2) and K phases. Preferred: 16 rows with three
// buffers; with few pairs a slot (at most 8 on average) 8 rows with three buffers before 16 with two; K phases (each
// wave then owns one tile) when even 8 rows of all n columns do not fit.
RmPlan rm_plan(int n, int n_out, int slots, bool glu, int avg_rows) {
    const int buf = RM_WAVES * (glu ? 2 : 1) * RM_TILE_BYTES;
    auto fits = [&](int rt, int nb) { return rm_lds(n, rt).total + nb * buf <= RM_LDS_MAX; };
    RmPlan pl{8, 2, n, 0};
    if (fits(16, 3))
        pl = RmPlan{16, 3, n, 0};
    else if (avg_rows <= 8 && fits(8, 3))
        pl = RmPlan{8, 3, n, 0};
    else if (fits(16, 2))
        pl = RmPlan{16, 2, n, 0};
    else if (fits(8, 3))
        pl = RmPlan{8, 3, n, 0};
    else if (fits(8, 2))
        pl = RmPlan{8, 2, n, 0};
    else {
        // the fewest phases three buffers allow; then, without GLU, as many buffers (up to five) as fit beside a
        // phase of that width, so more weight bytes stay in flight (C5 down: 8 rows of 7168 columns and five buffers)
        const int nsb = n / KF_Q4_K_BLOCK;
        auto phases = [&](int nb) {
            int max_sb = nsb;
            while (max_sb > 1 && rm_lds(max_sb * KF_Q4_K_BLOCK, 8).total + nb * buf > RM_LDS_MAX) max_sb--;
            return (nsb + max_sb - 1) / max_sb;
        };
        const int nph = phases(3);
        pl = RmPlan{8, 3, ((nsb + nph - 1) / nph) * KF_Q4_K_BLOCK, 0};  // balanced phases
        if (!glu)
            for (int nb = 5; nb > 3; nb--)
                if (rm_lds(pl.kc, 8).total + nb * buf <= RM_LDS_MAX) {
                    pl.nb = nb;
                    break;
                }
    }
    const int forced_nb = kf_knob_or(KF_KNOB_RM_NB, 0);  // a measurement knob: fewer buffers (2 to 4)
    if (forced_nb >= 2 && forced_nb < pl.nb) pl.nb = forced_nb;
    if (pl.kc < n) {
        pl.rpb = 16 * RM_WAVES;
    } else {
        // whole 16-row tiles, at most 16 tiles a wave (a block stages its activation rows once for all of them), and
        // as many blocks over all slots as the CUs hold at once: a grid of one round (C5, 8 experts: 224 blocks,
        // 199 us, against 448 blocks in two rounds, 206 us, and 384 blocks, 235 us)
        const int tiles = (n_out + 15) / 16;
        const int per_cu = std::max(1, RM_LDS_MAX / (int)(rm_lds(pl.kc, pl.rt).total + pl.nb * buf));
        const int want = std::max(1, kf_cu_count() * per_cu / slots);
        // tiles a block: enough that the slots' blocks fill one round, at least one a wave, at most 16 a wave; not
        // necessarily a multiple of the waves (C5: 28 tiles a block, 256 blocks, where whole tiles a wave gave 32 and
        // 224 blocks, leaving 32 CUs idle)
        const int whole = kf_knob_or(KF_KNOB_RM_WHOLE, 0);  // 1: whole tiles a wave (a comparison knob)
        int tpb = std::max(RM_WAVES, std::min(16 * RM_WAVES, (tiles + want - 1) / want));
        if (whole) tpb = RM_WAVES * std::max(1, std::min(16, (tiles + want * RM_WAVES - 1) / (want * RM_WAVES)));
        pl.rpb = 16 * tpb;
    }
    return pl;
}

template <bool GLU, int RT, int NB>
hipError_t rows_mma_launch(const uint8_t* w, const uint8_t* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                           const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                           int per_slot, const float* bias, const float* res, float* y, const RmPlan& pl, hipStream_t s) {
    auto* fn = rows_mma_kernel<GLU, RT, NB>;
    const int lds = rm_lds(pl.kc, RT).total;
    const hipError_t e = kf_raise_lds(reinterpret_cast<const void*>(fn), lds);
    if (e != hipSuccess) return e;
    const int slots = offsets ? n_slots : 1;
    dim3 grid((n_out + pl.rpb - 1) / pl.rpb, slots);
    fn<<<grid, RM_THREADS, lds, s>>>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, pairs, n_used, per_slot, bias, res, y,
                                     pl.rpb, pl.kc);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------ one-slot form
// The few-row product of one matrix (no slots) has too few 16-row tiles to give every wave its own, and staging the
// activation rows per block would cost as much as the block's weights. Here a block's eight waves split K over
// TILES tiles (KP = 8 / TILES waves a tile, each taking super-blocks kpart, kpart + KP, ...), and each wave fetches,
// per super-block, its tile's weights and exactly the activation data it multiplies them with (16 rows x 256 int8
// columns in MFMA order, their 32-column sums and scales) by DMA into one of its two LDS buffers. (Operand loads into
// registers instead made the compiler copy the loaded registers at every loop pass, waiting for all loads in flight.)
// The KP partials of a tile are summed in LDS in kpart order (deterministic). Rows run in chunks of 16, up to four
// chunks (64 rows) per pass over the weights: a super-block's weights stay while its chunks of staged rows pass.
// The same kernel runs q5_K and q6_K (replacing the per-lane dot form of gemv_k.hip for several rows):
//   * q5_K: q4_K's arithmetic with 5-bit operands (the fifth bit from qh, q5_k.rs:7-60); 176-byte rows;
//   * q6_K: the operand is q - 32 (in [-32, 31], an int8), so the super-block integer sum_s sc_s (dot_s - 32 bsum_s)
//     of the reference (q6_k.rs) is sum_s sc_s dot'_s with no sums term; the int8 scales cover 16 columns, so each
//     32-column group takes two MFMAs with the other 16 columns' operand bytes zeroed (lane quarters 0-1 hold columns
//     0-15, quarters 2-3 columns 16-31). Its 210-byte blocks are 2-byte aligned: each row's super-block comes as the
//     212-byte dword window [start & ~3, +212) (rows are 4-byte aligned when the row has an even number of
//     super-blocks, which the launcher requires), read back at the window's 0- or 2-byte shift.
template <uint32_t TY>
struct RdGeo {
    static constexpr int WROW = TY == KF_TYPE_Q4_K ? KF_Q4_K_BYTES : TY == KF_TYPE_Q5_K ? KF_Q5_K_BYTES : 212;  // LDS row
    static constexpr int WB = (16 * WROW + 15) / 16 * 16;  // one weight buffer: the tile's super-block
    static constexpr int A = 0, S = A + 8 * 16 * 32, D = S + 16 * 8 * 4, AB = D + 16 * 4 + 64;  // one activation buffer
    static constexpr bool DW = TY == KF_TYPE_Q6_K;         // dword DMA (2-byte aligned blocks) instead of 16-byte
    static constexpr int UNITS = DW ? 16 * WROW / 4 : 16 * WROW / 16;  // DMA units of the tile's weights
    static constexpr int WI = (UNITS + 63) / 64;           // weight DMA instructions a super-block
    static constexpr int NA = 4 + (TY == KF_TYPE_Q6_K ? 0 : 1) + 1;  // activation DMA instructions a chunk
};

// CM: row chunks of 16 a block carries through one pass over its weights (1 up to 16 rows; 4 above: 64 rows a pass)
template <uint32_t TY, int TILES, int CM>
__global__ void __launch_bounds__(RM_THREADS) rows_mma_1_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                                const int32_t* __restrict__ xs32, const float* __restrict__ xd32, int n, int n_out,
                                                                int rows, const float* __restrict__ bias, const float* __restrict__ res,
                                                                float* __restrict__ y) {
    using G = RdGeo<TY>;
    constexpr int KP = RM_WAVES / TILES;
    constexpr int SBB = TY == KF_TYPE_Q4_K ? KF_Q4_K_BYTES : TY == KF_TYPE_Q5_K ? KF_Q5_K_BYTES : KF_Q6_K_BYTES;
    // a wave's two weight buffers (super-blocks alternate) and two activation buffers (items alternate)
    __shared__ __align__(16) uint8_t pw0[RM_WAVES * G::WB];
    __shared__ __align__(16) uint8_t pw1[RM_WAVES * G::WB];
    __shared__ __align__(16) uint8_t pa0[RM_WAVES * G::AB];
    __shared__ __align__(16) uint8_t pa1[RM_WAVES * G::AB];
    __shared__ __align__(16) rm_v4f part[RM_WAVES * 64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tl = wave / KP, kpart = wave % KP;
    const int c = lane & 15, q = lane >> 4;
    const int nsb = n / KF_Q4_K_BLOCK, nsum = n / 32;
    const int orow = (blockIdx.x * TILES + tl) * 16;  // the wave's tile
    const int msb = nsb > kpart ? (nsb - kpart + KP - 1) / KP : 0;  // the wave's super-blocks

    // the resource starts at the wave's tile (the last tile's start for a wave past n_out) and ends at the matrix's
    // last row: the hardware range check on the per-lane offset returns zeros for rows past n_out
    const int trow = min(orow, (n_out - 1) & ~15);
    const kf_arsrc_t rw = kf_arsrc(w + (int64_t)trow * row_bytes, (uint64_t)(n_out - trow) * row_bytes);
    // weight DMA unit u = 64 i + lane: row u / per, unit u % per of the row's super-block (clamped duplicates)
    int vpk[G::WI];
#pragma unroll
    for (int i = 0; i < G::WI; i++) {
        constexpr int per = G::DW ? G::WROW / 4 : G::WROW / 16;
        const int u = min(64 * i + lane, G::UNITS - 1);
        vpk[i] = (u / per) * (int)row_bytes + (G::DW ? 4 : 16) * (u % per);
    }

    // one super-block of the tile against one chunk of 16 staged rows: weights at wb, activations at ab
    auto compute = [&](const uint8_t* wb, const uint8_t* ab, int sb, rm_v4f& acc) __attribute__((always_inline)) {
        const rm_v4f dx = *reinterpret_cast<const rm_v4f*>(ab + G::D + 16 * q);
        const uint8_t* a_at = ab + G::A + c * 32 + 8 * q;
        if constexpr (TY == KF_TYPE_Q6_K) {
            const uint8_t* wr = wb + c * G::WROW + ((sb * SBB) & 3);  // the lane's row of the super-block
            typedef uint32_t v2a2 __attribute__((ext_vector_type(2), aligned(2)));
            typedef uint32_t v4a2 __attribute__((ext_vector_type(4), aligned(2)));
            const v4a2 scv = *reinterpret_cast<const v4a2*>(wr + 192);  // the row's sixteen int8 scales
            const uint32_t scw[4] = {scv.x, scv.y, scv.z, scv.w};
            rm_v4i S = rm_v4i{0, 0, 0, 0};
            const uint32_t m4 = 0x0f0f0f0fu, m3 = 0x03030303u, hb = 0x80808080u, k32 = 0x20202020u;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const v2a2 la = *reinterpret_cast<const v2a2*>(wr + 64 * h + 8 * q);
                const v2a2 lb = *reinterpret_cast<const v2a2*>(wr + 64 * h + 32 + 8 * q);
                const v2a2 qh = *reinterpret_cast<const v2a2*>(wr + 128 + 32 * h + 8 * q);
#pragma unroll
                for (int gg = 0; gg < 4; gg++) {
                    const v2a2 src = (gg & 1) ? lb : la;
                    uint32_t wv[2];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t lo = (gg >> 1) ? (src[e] >> 4) & m4 : src[e] & m4;
                        const uint32_t v = lo | (((qh[e] >> (2 * gg)) & m3) << 4);  // q in [0, 63] per byte
                        wv[e] = ((v | hb) - k32) ^ hb;                            // q - 32 per byte, no borrows
                    }
                    const long bw = (long)wv[0] | ((long)wv[1] << 32);
                    const long b0 = q < 2 ? bw : 0, b1 = q < 2 ? 0 : bw;  // columns 0-15, then 16-31
                    const long a = *reinterpret_cast<const long*>(a_at + (4 * h + gg) * (16 * 32));
                    const rm_v4i i0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b0, rm_v4i{0, 0, 0, 0}, 0, 0, 0);
                    const rm_v4i i1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, rm_v4i{0, 0, 0, 0}, 0, 0, 0);
                    // scales 8 h + 2 gg and 8 h + 2 gg + 1 (ggml's q6_K order: 16 columns a scale)
                    const int si = 8 * h + 2 * gg;
                    const int s0 = (int)(int8_t)(uint8_t)(scw[si >> 2] >> (8 * (si & 3)));
                    const int s1 = (int)(int8_t)(uint8_t)(scw[(si + 1) >> 2] >> (8 * ((si + 1) & 3)));
                    // |dot| <= 32 * 128 * 16 and |sc| <= 128: 24-bit multiplies are exact
#pragma unroll
                    for (int e = 0; e < 4; e++) S[e] += __mul24(s0, i0[e]) + __mul24(s1, i1[e]);
                }
            }
            const float d = kf_h2f(*reinterpret_cast<const uint16_t*>(wr + 208));
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = fmaf(dx[e], d * (float)S[e], acc[e]);
        } else {
            constexpr int QS = TY == KF_TYPE_Q5_K ? 48 : 16;  // the nibbles' offset in the block
            RmW v;
            v.hd = *reinterpret_cast<const rm_v4u*>(wb + c * G::WROW);
#pragma unroll
            for (int p = 0; p < 4; p++) v.q[p] = *reinterpret_cast<const rm_v2u*>(wb + c * G::WROW + QS + 32 * p + 8 * q);
            if constexpr (TY == KF_TYPE_Q5_K) v.qh = *reinterpret_cast<const rm_v2u*>(wb + c * G::WROW + 16 + 8 * q);
            const int2 bs = *reinterpret_cast<const int2*>(ab + G::S + (c * 8 + 2 * q) * 4);
            rm_v4h xo;
            xo[0] = (_Float16)(float)(bs.x >> 6);
            xo[1] = (_Float16)(float)(bs.x & 63);
            xo[2] = (_Float16)(float)(bs.y >> 6);
            xo[3] = (_Float16)(float)(bs.y & 63);
            rm_v4i S;
            rm_v4f mins;
            rm_block<TY == KF_TYPE_Q5_K>(v, a_at, 16 * 32, xo, q, S, mins);
            const float d = kf_h2f(v.hd.x & 0xffffu), dm = kf_h2f(v.hd.x >> 16);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = fmaf(dx[e], fmaf(-dm, mins[e], d * (float)S[e]), acc[e]);
        }
    };

    // Rows in groups of up to 64; within a group the wave walks items j = (super-block i, chunk cc), j = i C + cc:
    // a super-block's weights are fetched with its first chunk and stay while all C chunks of staged rows pass, so a
    // weight byte is read once per 64 rows. Item j + 2 is requested once item j is multiplied. The DMA goes through
    // kf_adma16 / kf_adma4 (the buffers are picked at run time, and the compiler's own waits would drain the ring):
    // every wait below is explicit.
    for (int g0 = 0; g0 < rows; g0 += 16 * CM) {
        const int Rg = min(16 * CM, rows - g0);
        const int C = (Rg + 15) / 16;
        const int items = msb * C;
        // activation sources of the group (rows past Rg repeat row Rg - 1): A pieces (instruction i: groups 2 i, 2 i + 1;
        // lane l: group 2 i + l / 32, row 16 cc + (l / 2) % 16, half l % 2), sums (lane l < 32: row l / 2, four sums from
        // 4 (l % 2)), scales (lane l < 16: row l)
        const kf_arsrc_t rx = kf_arsrc(xq + (int64_t)g0 * n, (uint64_t)Rg * n);
        const kf_arsrc_t rs = kf_arsrc(xs32 + (int64_t)g0 * nsum, (uint64_t)Rg * nsum * 4);
        const kf_arsrc_t rd = kf_arsrc(xd32 + (int64_t)g0 * nsum, (uint64_t)Rg * nsum * 4);
        auto park = [&](int j) {
            const int i = j / C, cc = j - i * C;
            const int sb = kpart + KP * i;
            if (cc == 0) {
                uint8_t* b = ((i & 1) ? pw1 : pw0) + wave * G::WB;
                if constexpr (G::DW) {
                    const int so = (sb * SBB) & ~3;  // the window's start (rows 4-byte aligned)
#pragma unroll
                    for (int k = 0; k < G::WI; k++)
                        if (G::UNITS % 64 == 0 || k + 1 < G::WI || lane < G::UNITS % 64) kf_adma4(rw, vpk[k], so, b + 256 * k);
                } else {
                    const int so = sb * SBB;
#pragma unroll
                    for (int k = 0; k < G::WI; k++)
                        if (G::UNITS % 64 == 0 || k + 1 < G::WI || lane < G::UNITS % 64) kf_adma16(rw, vpk[k], so, b + 1024 * k);
                }
            }
            uint8_t* b = ((j & 1) ? pa1 : pa0) + wave * G::AB;
            const int r16 = 16 * cc;
            const int ra = min(r16 + ((lane >> 1) & 15), Rg - 1);
#pragma unroll
            for (int k = 0; k < 4; k++)
                kf_adma16(rx, ra * n + 32 * (2 * k + (lane >> 5)) + 16 * (lane & 1), sb * KF_Q4_K_BLOCK, b + G::A + 1024 * k);
            if constexpr (TY != KF_TYPE_Q6_K)
                if (lane < 32) kf_adma16(rs, ra * nsum * 4 + 16 * (lane & 1), sb * 32, b + G::S);
            if (lane < 16) kf_adma4(rd, min(r16 + lane, Rg - 1) * nsum * 4, sb * 32, b + G::D);
        };
        rm_v4f acc[CM];
#pragma unroll
        for (int k = 0; k < CM; k++) acc[k] = rm_v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (items > 0) park(0);
        if (items > 1) park(1);
        for (int i = 0; i < msb; i++) {
            const int sb = kpart + KP * i;
            const uint8_t* wb = ((i & 1) ? pw1 : pw0) + wave * G::WB;
#pragma unroll
            for (int cc = 0; cc < CM; cc++) {
                if (cc < C) {
                    const int j = i * C + cc;
                    // loads complete in issue order: wait until only item j + 1's DMA is outstanding
                    if (j + 1 >= items)
                        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(0));
                    else if ((j + 1) % C == 0)
                        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(G::NA + G::WI));
                    else
                        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(G::NA));
                    compute(wb, ((j & 1) ? pa1 : pa0) + wave * G::AB, sb, acc[cc]);
                    if (j + 2 < items) {
                        __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(63) & ~(15 << 8));  // this item's reads are done
                        park(j + 2);
                    }
                }
            }
        }
        // per chunk, the KP partials of each tile in kpart order
#pragma unroll
        for (int cc = 0; cc < CM; cc++) {
            if (cc < C) {
                part[wave * 64 + lane] = acc[cc];
                __syncthreads();
                if (kpart == 0) {
                    rm_v4f t = part[(tl * KP) * 64 + lane];
#pragma unroll
                    for (int k = 1; k < KP; k++) t += part[(tl * KP + k) * 64 + lane];
                    const int o = orow + c;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int m = 16 * cc + 4 * q + e;
                        if (m < Rg && o < n_out) {
                            const int64_t at = (int64_t)(g0 + m) * n_out + o;
                            y[at] = t[e] + (bias ? bias[o] : 0.0f) + (res ? res[at] : 0.0f);
                        }
                    }
                }
                __syncthreads();  // before the next chunk's partials
            }
        }
    }
}

}  // namespace

// Whether the matrix-core product takes this launch: it needs 16-byte aligned weight rows (q4_K always), matrices
// below 2 GB and a grid that fills the GPU; a K-phased launch (one tile a wave) over few slots has too few blocks, and
// the per-lane dot form takes it
bool kf_rows_mma_ok(int n, int n_out, int slots, bool glu, int avg_rows) {
    // row offsets within a matrix travel as 32-bit scalar offsets
    if ((int64_t)n_out * (n / KF_Q4_K_BLOCK) * KF_Q4_K_BYTES >= (1ll << 31)) return false;
    const RmPlan pl = rm_plan(n, n_out, slots, glu, avg_rows);
    return pl.kc == n || (int64_t)((n_out + pl.rpb - 1) / pl.rpb) * slots >= 128;
}

// Host launcher of the q4_K multi-row / grouped product on the matrix cores, validated by the caller (api.cpp): n a
// multiple of 256 and at most 16384, rows 16-byte aligned, every matrix (expert_bytes apart) below 2 GB.
hipError_t kf_launch_rows_mma(const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                              const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                              int per_slot, int avg_rows, const float* bias, const float* res, float* y, hipStream_t s) {
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* ub = static_cast<const uint8_t*>(w2);
    const RmPlan pl = rm_plan(n, n_out, offsets ? n_slots : 1, w2 != nullptr, avg_rows);
#define KF_RM(G, RT_, NB_) \
    return rows_mma_launch<G, RT_, NB_>(wb, ub, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, pl, s)
#define KF_RM_NB(G, RT_) \
    if (pl.nb == 3) KF_RM(G, RT_, 3); \
    KF_RM(G, RT_, 2)
    if (w2) {
        if (pl.rt == 16) { KF_RM_NB(true, 16); }
        KF_RM_NB(true, 8);
    }
    if (pl.rt == 16) { KF_RM_NB(false, 16); }
    if (pl.nb == 5) KF_RM(false, 8, 5);
    if (pl.nb == 4) KF_RM(false, 8, 4);
    KF_RM_NB(false, 8);
#undef KF_RM_NB
#undef KF_RM
}

// Whether the one-slot matrix-core product takes a q4_K / q5_K / q6_K weight: row offsets travel as 32-bit values (the
// matrix and the activation rows below 2 GB), 16-byte aligned weights, and for q6_K 4-byte aligned rows (an even
// number of super-blocks a row)
bool kf_rows_mma_1_ok(uint32_t ty, const void* w, int64_t row_bytes, int n, int n_out, int rows) {
    if (n % KF_Q4_K_BLOCK != 0 || (int64_t)n_out * row_bytes >= (1ll << 31) || (int64_t)rows * n >= (1ll << 31)) return false;
    if ((reinterpret_cast<uintptr_t>(w) & 15) != 0) return false;
    if (ty == KF_TYPE_Q6_K) return row_bytes % 4 == 0;
    return (ty == KF_TYPE_Q4_K || ty == KF_TYPE_Q5_K) && row_bytes % 16 == 0;
}

// Host launcher of the one-slot few-row product (rows_mma_1_kernel) for q4_K, q5_K and q6_K weights, validated by the
// caller (kf_rows_mma_1_ok). Tiles per block chosen so the grid has about one block per CU or more.
hipError_t kf_launch_rows_mma_1(uint32_t ty, const void* w, int64_t row_bytes, const int8_t* xq, const int32_t* xs32, const float* xd32, int n,
                                int n_out, int rows, const float* bias, const float* res, float* y, hipStream_t s) {
    if (!kf_rows_mma_1_ok(ty, w, row_bytes, n, n_out, rows)) return hipErrorInvalidValue;
    const int tiles = (n_out + 15) / 16;
    const int forced = kf_knob_or(KF_KNOB_RM1_TILES, 0);  // a tuning knob (1, 2, 4 or 8 tiles a block)
    // a block's two stage buffers per wave hold most of a CU's LDS, so one block runs per CU: the fewest tiles a block
    // whose grid still fits in one round of the CUs (QKV at 4096 x 6144: 192 blocks of two tiles, 8.5 us at 8 rows,
    // against 384 blocks of one tile in two rounds, 10.7 us)
    int tpb = forced == 1 || forced == 2 || forced == 4 || forced == 8 ? forced : 0;
    if (tpb == 0) {
        const int cus = kf_cu_count();
        tpb = 8;
        for (int t = 1; t < 8; t *= 2)
            if ((tiles + t - 1) / t <= cus) {
                tpb = t;
                break;
            }
    }
    const auto* wb = static_cast<const uint8_t*>(w);
#define KF_R1(TY, T)                                                                                               \
    {                                                                                                              \
        if (rows <= 16)                                                                                            \
            rows_mma_1_kernel<TY, T, 1><<<(tiles + T - 1) / T, RM_THREADS, 0, s>>>(wb, row_bytes, xq, xs32, xd32, n, n_out, rows, bias, res, y); \
        else                                                                                                       \
            rows_mma_1_kernel<TY, T, 4><<<(tiles + T - 1) / T, RM_THREADS, 0, s>>>(wb, row_bytes, xq, xs32, xd32, n, n_out, rows, bias, res, y); \
        return hipGetLastError();                                                                                  \
    }
#define KF_R1_T(TY)          \
    if (tpb == 8) KF_R1(TY, 8) \
    if (tpb == 4) KF_R1(TY, 4) \
    if (tpb == 2) KF_R1(TY, 2) \
    KF_R1(TY, 1)
    if (ty == KF_TYPE_Q6_K) { KF_R1_T(KF_TYPE_Q6_K) }
    if (ty == KF_TYPE_Q5_K) { KF_R1_T(KF_TYPE_Q5_K) }
    KF_R1_T(KF_TYPE_Q4_K)
#undef KF_R1_T
#undef KF_R1
}

