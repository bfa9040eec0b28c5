// Multi-row products on native GGUF bytes and the MoE pieces around them.
//
//  * rows_kernel: each weight row is streamed once and multiplied against up to RMAX activation rows staged in LDS.
//    It is the grouped expert product of the MoE layer (grid row = expert slot, activation rows = the pairs routed to
//    that slot, from the moe_group order and offsets), optionally fused gate + up with the gated activation, and the
//    plain few-row product of one matrix. The per-block integer arithmetic is the GEMV's (kf_blocks.h), so the int32
//    block results are the reference's dot_i8 (crates/kf-quant/src/types/q8_0.rs:10-29, types/q4_k.rs:10-58).
//    Replaces kf_moe_matvec_i8 / kf_moe_gate_up_i8 (crates/kf-backend-cuda/src/kernels/quant.cuh:519-581), which read
//    an expert's rows once per routed pair; here they are read once per slot (chunks of RMAX pairs).
//  * moe_group_kernel: pairs grouped by slot (counts, offsets, order), replacing moe_group
//    (crates/kf-backend-cuda/src/kernels/moe.cu:118-141); the order within a slot is the pair order (stable), where
//    the reference's atomic placement leaves it unspecified.
//  * moe_combine_kernel: the routing-weighted sum of each row's pairs, replacing moe_combine (moe.cu:153-164).
//
// gfx950 layout: a wave owns one weight row at a time and walks its steps (q4_K: 16 super-blocks = 2304 bytes, four
// lanes a super-block, each lane a 32-byte pair of sub-blocks plus the 16-byte header; q8_0: 64 blocks = 2176 bytes,
// one lane a block). Activation rows sit in LDS wave-transposed (a lane's 16-byte pieces are contiguous across the
// wave, conflict free), with their per-32 integer sums and scales. The next row's weights are requested before the
// current row is multiplied.
#include "kf_knobs.h"
#include "kf_blocks.h"
#include "kf_host.h"

#include <algorithm>

hipError_t kf_launch_rows_mma(const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                              const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                              int per_slot, int avg_rows, const float* bias, const float* res, float* y, hipStream_t s);
bool kf_rows_mma_ok(int n, int n_out, int slots, bool glu, int avg_rows);
bool kf_rows_mma_1_ok(uint32_t ty, const void* w, int64_t row_bytes, int n, int n_out, int rows);
hipError_t kf_launch_rows_mma_1(uint32_t ty, const void* w, int64_t row_bytes, const int8_t* xq, const int32_t* xs32, const float* xd32, int n, int n_out,
                                int rows, const float* bias, const float* res, float* y, hipStream_t s);

namespace {

template <uint32_t TY>
struct RwType {
    static constexpr int STEP_BYTES = TY == KF_TYPE_Q4_K ? 16 * KF_Q4_K_BYTES : 64 * KF_Q8_0_BYTES;
    static constexpr int STEP_PIECES = TY == KF_TYPE_Q4_K ? 256 : 128;  // 16-byte activation pieces per step
    static constexpr int PER_STEP = TY == KF_TYPE_Q4_K ? 16 : 64;       // blocks per step
    static constexpr int BLOCK = TY == KF_TYPE_Q4_K ? 256 : 32;
};

// LDS bytes of one staged activation row of n columns: transposed int8 values (whole steps), per-32 sums (q4_K), per-32
// scales
template <uint32_t TY>
__host__ __device__ inline int rw_row_lds(int n) {
    using T = RwType<TY>;
    const int steps = (n / T::BLOCK + T::PER_STEP - 1) / T::PER_STEP;
    return steps * T::STEP_PIECES * 16 + (TY == KF_TYPE_Q4_K ? (n / 32) * 4 : 0) + (n / 32) * 4;
}

// One lane's weight registers for one step of one row
struct RwLaneW {
    uint4 a, b, c;  // q4_K: header, nibble halves; q8_0: quant halves (a, b) and the scale in c.x
};

template <uint32_t TY>
__device__ __forceinline__ void rw_load(RwLaneW& v, const uint8_t* row, int s, int nblk, int lane) {
    if constexpr (TY == KF_TYPE_Q4_K) {
        const int sb = min(s * 16 + (lane >> 2), nblk - 1), j = lane & 3;
        const uint8_t* blk = row + (int64_t)sb * KF_Q4_K_BYTES;
        v.a = *reinterpret_cast<const uint4*>(blk);
        v.b = *reinterpret_cast<const uint4*>(blk + 16 + 32 * j);
        v.c = *reinterpret_cast<const uint4*>(blk + 32 + 32 * j);
    } else {
        const int b = min(s * 64 + lane, nblk - 1);
        const uint8_t* blk = row + (int64_t)b * KF_Q8_0_BYTES;
        const kf_u32x4_a2 q0 = *reinterpret_cast<const kf_u32x4_a2*>(blk + 2);
        const kf_u32x4_a2 q1 = *reinterpret_cast<const kf_u32x4_a2*>(blk + 18);
        v.a = make_uint4(q0.x, q0.y, q0.z, q0.w);
        v.b = make_uint4(q1.x, q1.y, q1.z, q1.w);
        v.c = make_uint4(*reinterpret_cast<const uint16_t*>(blk), 0, 0, 0);
    }
}

// The weight side of one lane's step, decoded once and reused against every staged activation row: q4_K nibbles
// split into low and high halves, the sub-block pair's 6-bit scales and mins, the super-block's f16 scales; q8_0 the
// int8 quants and the f16 scale.
// Scheduling barrier between staged pairs (bounds the registers a row's dots hold; 0 lets the compiler interleave)
#ifndef KF_RW_PAIR_BARRIER
#define KF_RW_PAIR_BARRIER 1
#endif

struct RwPrep {
    uint32_t q[16];
    int sc0, sc1, m0, m1;
    float d, dm;
};

template <uint32_t TY>
__device__ __forceinline__ void rw_prep(RwPrep& u, const RwLaneW& v, int lane) {
    if constexpr (TY == KF_TYPE_Q4_K) {
        const uint32_t m4 = 0x0f0f0f0fu;
        const uint32_t qa[4] = {v.b.x, v.b.y, v.b.z, v.b.w}, qb[4] = {v.c.x, v.c.y, v.c.z, v.c.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            u.q[i] = qa[i] & m4;
            u.q[4 + i] = qb[i] & m4;
            u.q[8 + i] = (qa[i] >> 4) & m4;
            u.q[12 + i] = (qb[i] >> 4) & m4;
        }
        uint32_t sc2, m2;
        kf_q4k_scales(v.a.y, v.a.z, v.a.w, lane & 3, sc2, m2);
        u.sc0 = (int)(sc2 & 0xffu);
        u.sc1 = (int)(sc2 >> 8);
        u.m0 = (int)(m2 & 0xffu);
        u.m1 = (int)(m2 >> 8);
        u.d = kf_h2f(v.a.x & 0xffffu);
        u.dm = kf_h2f(v.a.x >> 16);
    } else {
        const uint32_t w[8] = {v.a.x, v.a.y, v.a.z, v.a.w, v.b.x, v.b.y, v.b.z, v.b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) u.q[i] = w[i];
        u.d = kf_h2f(v.c.x);
    }
}

// The lane's float contribution of one step against one staged activation row at xr (LDS). The integers are those of
// kf_q4k_lane / kf_q8_0_dot (the reference's dot_i8 integers), the float combine that of the GEMV.
template <uint32_t TY>
__device__ __forceinline__ float rw_dot(const RwPrep& u, const uint8_t* xr, int n, int s, int lane) {
    using T = RwType<TY>;
    const uint4* xs = reinterpret_cast<const uint4*>(xr) + (s * T::STEP_PIECES) + lane;
    const int32_t* ss = reinterpret_cast<const int32_t*>(xr + (n / T::BLOCK + T::PER_STEP - 1) / T::PER_STEP * T::STEP_PIECES * 16);
    if constexpr (TY == KF_TYPE_Q4_K) {
        const float* sd = reinterpret_cast<const float*>(ss + n / 32);
        const int sb = s * 16 + (lane >> 2), j = lane & 3;
        const int2 bs = *reinterpret_cast<const int2*>(ss + sb * 8 + 2 * j);
        const uint4 x0 = xs[0], x1 = xs[64], x2 = xs[128], x3 = xs[192];
        const uint32_t xv[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w, x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) lo = kf_dot4(u.q[i], xv[i], lo);
#pragma unroll
        for (int i = 8; i < 16; i++) hi = kf_dot4(u.q[i], xv[i], hi);
        // 24-bit multiplies are exact: scales and mins are 6-bit, |dot| <= 15*127*32 and |bsum| <= 128*32
        const int isum = __mul24(u.sc0, lo) + __mul24(u.sc1, hi);
        const int imin = __mul24(u.m0, bs.x) + __mul24(u.m1, bs.y);
        const float dx = sd[sb * 8];
        return fmaf(-(u.dm * dx), (float)imin, (u.d * dx) * (float)isum);
    } else {
        const float* sd = reinterpret_cast<const float*>(ss);
        const uint4 x0 = xs[0], x1 = xs[64];
        const uint32_t xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int dt = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) dt = kf_dot4(u.q[i], xv[i], dt);
        const int b = s * 64 + lane;
        return u.d * sd[b] * (float)dt;
    }
}

// ops::silu (crates/kf-backend-cpu/src/ops.rs): x / (1 + e^-x)
__device__ __forceinline__ float rw_silu(float x) { return x / (1.0f + expf(-x)); }

// Block (x, slot): weight rows [x * rpb, +rpb) of the slot's matrix (base + slot * expert_bytes) against the slot's
// pairs [offsets[slot], offsets[slot + 1]) of `order` (identity without order; one slot [0, pairs) without offsets),
// RMAX at a time. The activation row of pair p is p (per_slot) or p / n_used. Outputs y[p][o]: GLU ? silu(gate .
// x) * (up . x) : w . x + bias[o] + res[p][o].
// Threads of a block: wide rows (four register steps) stage large activation rows, so eight waves share them (four
// for the fused gate + up form, whose two rows of registers leave room for no more)
template <int STEPS, bool GLU>
constexpr int rw_threads() { return STEPS > 1 && !GLU ? 512 : 256; }

template <uint32_t TY, int RMAX, bool GLU, int STEPS>
__global__ void __launch_bounds__((rw_threads<STEPS, GLU>())) rows_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int64_t expert_bytes,
                                                         int64_t row_bytes, const int8_t* __restrict__ xq, const int32_t* __restrict__ xs32,
                                                         const float* __restrict__ xd32, int n, int n_out, const int32_t* __restrict__ order,
                                                         const int32_t* __restrict__ offsets, int pairs, int n_used, int per_slot,
                                                         const float* __restrict__ bias, const float* __restrict__ res, float* __restrict__ y,
                                                         int rpb) {
    using T = RwType<TY>;
    constexpr int THREADS = rw_threads<STEPS, GLU>(), WAVES = THREADS / 64;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = blockIdx.y;
    const int p0 = offsets ? offsets[slot] : 0;
    const int p1 = offsets ? offsets[slot + 1] : pairs;
    if (p0 >= p1) return;
    const int nblk = n / T::BLOCK;
    const int steps = (nblk + T::PER_STEP - 1) / T::PER_STEP;
    const int row_lds = rw_row_lds<TY>(n);
    const int o0 = blockIdx.x * rpb;
    const int o1 = min(o0 + rpb, n_out);
    const uint8_t* wbase = w + (int64_t)slot * expert_bytes;
    const uint8_t* ubase = GLU ? w2 + (int64_t)slot * expert_bytes : nullptr;
    const int nsum = n / 32, npc = n / 16;

    // staging registers: every thread moves at most KMAX 16-byte pieces and one sum/scale of each staged row
    constexpr int KMAX = (STEPS * T::STEP_PIECES + THREADS - 1) / THREADS;
    for (int c0 = p0; c0 < p1; c0 += RMAX) {
        const int R = min(RMAX, p1 - c0);
        RwLaneW ring[GLU ? 2 : 1][STEPS];
        auto load_row = [&](RwLaneW (&v)[GLU ? 2 : 1][STEPS], int orow) {  // every step of a row
            const uint8_t* gr = wbase + (int64_t)min(orow, n_out - 1) * row_bytes;
#pragma unroll
            for (int s2 = 0; s2 < STEPS; s2++)
                if (s2 < steps) rw_load<TY>(v[0][s2], gr, s2, nblk, lane);
            if constexpr (GLU) {
                const uint8_t* ur = ubase + (int64_t)min(orow, n_out - 1) * row_bytes;
#pragma unroll
                for (int s2 = 0; s2 < STEPS; s2++)
                    if (s2 < steps) rw_load<TY>(v[1][s2], ur, s2, nblk, lane);
            }
        };
        // the wave's first row of weights goes out before the activations are staged (it does not depend on them)
        int o = o0 + wave;
        if (o < o1) load_row(ring, o);
        // stage the chunk's activation rows: all loads first, then the stores (transposed int8 pieces, sums, scales)
        {
            typedef uint32_t v4u_ __attribute__((ext_vector_type(4)));
            v4u_ pv[RMAX][KMAX];
            int32_t sv[RMAX];
            float dv[RMAX];
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                if (r >= R) break;
                const int p = order ? order[c0 + r] : c0 + r;
                const int xrow = per_slot ? p : p / n_used;
                const v4u_* gq = reinterpret_cast<const v4u_*>(xq + (int64_t)xrow * n);
#pragma unroll
                for (int k = 0; k < KMAX; k++) pv[r][k] = gq[min((int)threadIdx.x + k * THREADS, npc - 1)];
                const int c = min((int)threadIdx.x, nsum - 1);
                if constexpr (TY == KF_TYPE_Q4_K) sv[r] = xs32[(int64_t)xrow * nsum + c];
                dv[r] = xd32[(int64_t)xrow * nsum + c];
            }
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                if (r >= R) break;
                uint8_t* xr = smem + r * row_lds;
#pragma unroll
                for (int k = 0; k < KMAX; k++) {
                    const int c = threadIdx.x + k * THREADS;
                    if (c >= npc) break;
                    int dst;
                    if constexpr (TY == KF_TYPE_Q4_K) {
                        const int sb = c >> 4, jj = (c >> 2) & 3, kk = c & 3;
                        dst = (((sb >> 4) * 4 + kk) << 6) + ((sb & 15) << 2) + jj;
                    } else {
                        const int bb = c >> 1, kk = c & 1;
                        dst = (((bb >> 6) * 2 + kk) << 6) + (bb & 63);
                    }
                    reinterpret_cast<v4u_*>(xr)[dst] = pv[r][k];
                }
                int32_t* ss = reinterpret_cast<int32_t*>(xr + steps * T::STEP_PIECES * 16);
                float* sd = reinterpret_cast<float*>(ss + (TY == KF_TYPE_Q4_K ? nsum : 0));
                if ((int)threadIdx.x < nsum) {
                    if constexpr (TY == KF_TYPE_Q4_K) ss[threadIdx.x] = sv[r];
                    sd[threadIdx.x] = dv[r];
                }
            }
        }
        __syncthreads();

        // each wave walks rows o0 + wave, + WAVES, ...; the next row's weights are requested before this row's
        // arithmetic (two register sets, STEPS steps of the row each)
        // a rolling ring: as soon as a step's weights are decoded, its registers take the same step of the wave's
        // next row, so that row's loads stream while this row's dots run
        auto compute_row = [&](RwLaneW (&v)[GLU ? 2 : 1][STEPS], int orow, int next) {
            float ag[RMAX], au[RMAX];
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                ag[r] = 0.0f;
                au[r] = 0.0f;
            }
            const uint8_t* gn = wbase + (int64_t)min(next, n_out - 1) * row_bytes;
            const uint8_t* un = GLU ? ubase + (int64_t)min(next, n_out - 1) * row_bytes : nullptr;
#pragma unroll
            for (int s2 = 0; s2 < STEPS; s2++) {
                if (s2 >= steps) break;
                const bool valid = s2 * T::PER_STEP + (TY == KF_TYPE_Q4_K ? (lane >> 2) : lane) < nblk;
                RwPrep pg, pu;
                rw_prep<TY>(pg, v[0][s2], lane);
                if constexpr (GLU) rw_prep<TY>(pu, v[1][s2], lane);
                if (next < o1) {  // uniform
                    rw_load<TY>(v[0][s2], gn, s2, nblk, lane);
                    if constexpr (GLU) rw_load<TY>(v[1][s2], un, s2, nblk, lane);
                }
#pragma unroll
                for (int r = 0; r < RMAX; r++) {
                    if (r >= R) break;
                    const uint8_t* xr = smem + r * row_lds;
                    if (valid) {
                        ag[r] += rw_dot<TY>(pg, xr, n, s2, lane);
                        if constexpr (GLU) au[r] += rw_dot<TY>(pu, xr, n, s2, lane);
                    }
                    if (KF_RW_PAIR_BARRIER) __builtin_amdgcn_sched_barrier(0);  // one pair's activations live at a time
                }
                if (STEPS > 1) __builtin_amdgcn_sched_barrier(0);  // one step's decoded weights live at a time
            }
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                if (r >= R) break;
                const float g = kf_wave_sum_dpp(ag[r]);
                float u = 0.0f;
                if constexpr (GLU) u = kf_wave_sum_dpp(au[r]);
                if (lane == 0) {
                    const int p = order ? order[c0 + r] : c0 + r;
                    float* yo = y + (int64_t)p * n_out + orow;
                    if constexpr (GLU)
                        *yo = rw_silu(g) * u;
                    else
                        *yo = g + (bias ? bias[orow] : 0.0f) + (res ? res[(int64_t)p * n_out + orow] : 0.0f);
                }
            }
        };
        for (; o < o1; o += WAVES) compute_row(ring, o, o + WAVES);
        __syncthreads();  // before the next chunk restages
    }
}

// Stable grouping of the routed pairs by slot, as a parallel counting sort in one block of KF_GROUP_WAVES waves with
// no atomics. The pairs are cut into one 64-aligned run per wave. Pass 1: each wave counts its run per slot into its
// own column of tab[slot][wave] (one ballot per distinct slot of a 64-pair window; only the window's leader lane
// writes). Scan: wave 0 turns tab into exclusive bases, slot-major and wave-minor (a shuffle prefix over 64 entries at
// a time plus a running carry), so slot s starts at offsets[s] and within it the runs follow wave order. Pass 2: each
// wave walks its run again and writes every pair at its slot's running base plus its ballot rank. Pair order is
// therefore kept within a slot, and the result does not depend on timing. Slots < 0 or >= n_slots are skipped.
constexpr int KF_GROUP_WAVES = 4;

template <bool PLACE>
__device__ __forceinline__ void moe_group_walk(const int32_t* __restrict__ slots, int b, int e, int n_slots, int* tab, int wave, int lane,
                                               int32_t* __restrict__ order) {
    for (int base = b; base < e; base += 64) {
        const int i = base + lane;
        const int s = i < e ? slots[i] : -1;
        const bool live = s >= 0 && s < n_slots;
        uint64_t left = __ballot(live);
        while (left) {
            const int leader = __builtin_ctzll(left);
            const int sv = __shfl(s, leader, 64);
            const uint64_t same = __ballot(live && s == sv);
            int* cell = tab + sv * KF_GROUP_WAVES + wave;
            const int at = *cell;
            if (PLACE && live && s == sv) order[at + __popcll(same & ((1ull << lane) - 1))] = i;
            if (lane == leader) *cell = at + __popcll(same);
            left &= ~same;
        }
    }
}

__global__ void __launch_bounds__(64 * KF_GROUP_WAVES) moe_group_kernel(const int32_t* __restrict__ slots, int total, int n_slots,
                                                                        int32_t* __restrict__ order, int32_t* __restrict__ offsets) {
    extern __shared__ int tab[];  // [n_slots][KF_GROUP_WAVES]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cells = n_slots * KF_GROUP_WAVES;
    for (int i = threadIdx.x; i < cells; i += blockDim.x) tab[i] = 0;
    __syncthreads();
    const int run = ((total + KF_GROUP_WAVES - 1) / KF_GROUP_WAVES + 63) & ~63;
    const int b = min(total, wave * run), e = min(total, b + run);
    moe_group_walk<false>(slots, b, e, n_slots, tab, wave, lane, order);
    __syncthreads();
    if (wave == 0) {
        int carry = 0;
        for (int c = 0; c < cells; c += 64) {
            const int k = c + lane;
            const int v = k < cells ? tab[k] : 0;
            int inc = v;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int up = __shfl_up(inc, d, 64);
                if (lane >= d) inc += up;
            }
            if (k < cells) {
                tab[k] = carry + inc - v;
                if (k % KF_GROUP_WAVES == 0) offsets[k / KF_GROUP_WAVES] = carry + inc - v;
            }
            carry += __shfl(inc, 63, 64);
        }
        if (lane == 0) offsets[n_slots] = carry;
    }
    __syncthreads();
    moe_group_walk<true>(slots, b, e, n_slots, tab, wave, lane, order);
}

// Weighted sum of each token's expert outputs: out[r][o] = sum over j = 0..n_used-1 (in that order) of
// (wts[r n_used + j] scale) part[r n_used + j][o] over the pairs whose slot is in [0, n_slots), plus host[r][o]
// (nullable). Block r chunks + c covers columns [c, c + 1) x 256 V of token r: the pair weights and slot checks are wave-uniform and
// read once per block; the columns move as V-wide vectors. Pairs outside the slots were skipped by the grouping, so
// their part rows were never written and are not read.
template <int V>
__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ part, const float* __restrict__ wts, const int32_t* __restrict__ slots,
                                                          const float* __restrict__ host, float* __restrict__ out, int n_used, int n_embd,
                                                          float scale, int n_slots, int chunks) {
    using vec = float __attribute__((ext_vector_type(V)));
    const int64_t r = blockIdx.x / chunks;
    const int o = ((blockIdx.x - (int)r * chunks) * 256 + threadIdx.x) * V;
    if (o >= n_embd) return;
    vec acc = (vec)0.0f;
    for (int j = 0; j < n_used; j++) {
        const int64_t p = r * n_used + j;
        const int sl = slots[p];
        if (sl < 0 || sl >= n_slots) continue;
        const float w = wts[p] * scale;
        acc += w * *reinterpret_cast<const vec*>(part + p * n_embd + o);
    }
    if (host) acc += *reinterpret_cast<const vec*>(host + r * n_embd + o);
    *reinterpret_cast<vec*>(out + r * n_embd + o) = acc;
}

template <uint32_t TY, int RMAX, bool GLU, int STEPS>
hipError_t rows_launch(const uint8_t* w, const uint8_t* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                       const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                       int per_slot, const float* bias, const float* res, float* y, hipStream_t s) {
    auto* fn = rows_kernel<TY, RMAX, GLU, STEPS>;
    const int lds = RMAX * rw_row_lds<TY>(n);
    if (lds > 65536) {
        const hipError_t e = kf_raise_lds(reinterpret_cast<const void*>(fn), lds);
        if (e != hipSuccess) return e;
    }
    constexpr int threads = rw_threads<STEPS, GLU>();
    constexpr int waves = threads / 64;
    // rows per block: enough blocks to fill the GPU (about 1024 over all slots), each wave walking at most 16 rows
    // (a block stages its activation rows once for all of them)
    const int slots = offsets ? n_slots : 1;
    int per_wave = (int)std::min<int64_t>(16, std::max<int64_t>(1, ((int64_t)n_out * slots / 1024 + waves - 1) / waves));
    const int rpb = per_wave * waves;
    dim3 grid((n_out + rpb - 1) / rpb, slots);
    fn<<<grid, threads, lds, s>>>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, pairs, n_used, per_slot, bias, res,
                                     y, rpb);
    return hipGetLastError();
}

// Pairs staged per chunk, at most 8: every chunk past the first streams the slot's weights again, so wide rows (one
// block of eight waves a CU) may take all of the CU's 160 KB of LDS; rows of one step keep within 96 KB so that
// several blocks share a CU
template <uint32_t TY>
int rows_rmax(int n) {
    const int per = rw_row_lds<TY>(n);
    const int steps = (n / RwType<TY>::BLOCK + RwType<TY>::PER_STEP - 1) / RwType<TY>::PER_STEP;
    const int budget = steps > 1 ? 160 * 1024 : 96 * 1024;
    return 8 * per <= budget ? 8 : 4 * per <= budget ? 4 : 2 * per <= budget ? 2 : 1;
}

template <uint32_t TY, bool GLU, int STEPS>
hipError_t rows_dispatch_steps(const uint8_t* w, const uint8_t* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                               const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                               int per_slot, const float* bias, const float* res, float* y, hipStream_t s) {
    switch (rows_rmax<TY>(n)) {
        case 8: return rows_launch<TY, 8, GLU, STEPS>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
        case 4: return rows_launch<TY, 4, GLU, STEPS>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
        case 2: return rows_launch<TY, 2, GLU, STEPS>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
        default: return rows_launch<TY, 1, GLU, STEPS>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
    }
}

// Register steps a row needs: one step when it covers the row (q4_K n <= 4096, q8_0 n <= 2048), else four
template <uint32_t TY, bool GLU>
hipError_t rows_dispatch(const uint8_t* w, const uint8_t* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                         const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                         int per_slot, const float* bias, const float* res, float* y, hipStream_t s) {
    const int steps = (n / RwType<TY>::BLOCK + RwType<TY>::PER_STEP - 1) / RwType<TY>::PER_STEP;
    if (steps <= 1)
        return rows_dispatch_steps<TY, GLU, 1>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
    return rows_dispatch_steps<TY, GLU, 4>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
}

}  // namespace

// Widest activation row of the multi-row product (four register steps per row)
int kf_rows_max_n(uint32_t ty) { return ty == KF_TYPE_Q4_K ? 4 * 16 * 256 : 4 * 64 * 32; }

// Host launcher of the multi-row / grouped product, validated by the caller (api.cpp). act is the activation scratch
// of act_rows rows of n columns (kind of the weight type). w2 non-null selects the fused gate + up form.
hipError_t kf_launch_rows(uint32_t ty, const void* w, const void* w2, int64_t expert_bytes, int64_t row_bytes, const void* act, int act_rows,
                          int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used, int per_slot,
                          const float* bias, const float* res, float* y, hipStream_t s) {
    if (n_out == 0) return hipSuccess;
    const kf_act_offsets o = kf_act_layout((size_t)act_rows, (size_t)n);
    const char* base = static_cast<const char*>(act);
    const auto* xq = reinterpret_cast<const int8_t*>(base + o.q);
    const auto* xs = reinterpret_cast<const int32_t*>(base + o.s32);
    const auto* xd = reinterpret_cast<const float*>(base + o.d32);
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* ub = static_cast<const uint8_t*>(w2);
    // q4_K: the matrix-core form (rows_mma.hip); KF_ROWS_VALU=1 keeps the per-lane dot form (a measurement switch)
    const bool valu = kf_knob_on(KF_KNOB_ROWS_VALU);
    // the activation rows a slot gets on average (grouped: every pair of act_rows x n_used, or one per row)
    const int slots = offsets ? n_slots : 1;
    const int avg_rows = offsets ? (per_slot ? act_rows : act_rows * n_used) / std::max(1, slots) : pairs;
    // one matrix (no slots, no fused up): K split over the waves of a block (rows_mma_1_kernel)
    if (ty == KF_TYPE_Q4_K && !valu && !offsets && !order && !w2 && per_slot == 1 && n_used == 1 &&
        kf_rows_mma_1_ok(ty, w, row_bytes, n, n_out, act_rows))
        return kf_launch_rows_mma_1(KF_TYPE_Q4_K, wb, row_bytes, xq, xs, xd, n, n_out, act_rows, bias, res, y, s);
    if (ty == KF_TYPE_Q4_K && !valu && kf_rows_mma_ok(n, n_out, slots, w2 != nullptr, avg_rows))
        return kf_launch_rows_mma(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, avg_rows, bias,
                                  res, y, s);
    if (ty == KF_TYPE_Q4_K)
        return w2 ? rows_dispatch<KF_TYPE_Q4_K, true>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s)
                  : rows_dispatch<KF_TYPE_Q4_K, false>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
    return w2 ? rows_dispatch<KF_TYPE_Q8_0, true>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s)
              : rows_dispatch<KF_TYPE_Q8_0, false>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
}

// The quantized activation rows of the routed pairs in group order, for the grouped GEMM: row p of dst is row
// order[p] / n_used (the pair's token) of src, for the pairs moe_group placed (p < offsets[n_slots]). Copies the sections
// the q4_K GEMM reads: q, the per-32 scales and the mins operands (xa). One block a pair row.
__global__ void __launch_bounds__(256) moe_gather_act_kernel(const int8_t* __restrict__ sq, const float* __restrict__ sd32,
                                                             const uint4* __restrict__ sxa, int8_t* __restrict__ dq,
                                                             float* __restrict__ dd32, uint4* __restrict__ dxa,
                                                             const int32_t* __restrict__ order, const int32_t* __restrict__ offsets,
                                                             int n_slots, int n_used, int n) {
    const int p = blockIdx.x;
    if (p >= offsets[n_slots]) return;
    const int64_t t = order[p] / n_used;
    const uint4* src = reinterpret_cast<const uint4*>(sq + t * n);
    uint4* dst = reinterpret_cast<uint4*>(dq + (int64_t)p * n);
    for (int i = threadIdx.x; i < n / 16; i += blockDim.x) dst[i] = src[i];
    for (int i = threadIdx.x; i < n / 32; i += blockDim.x) dd32[(int64_t)p * (n / 32) + i] = sd32[t * (n / 32) + i];
    for (int i = threadIdx.x; i < n / 256 * 2; i += blockDim.x) dxa[(int64_t)p * (n / 256) * 2 + i] = sxa[t * (n / 256) * 2 + i];
}

hipError_t kf_launch_moe_gather_act(const void* src, int src_rows, void* dst, int pairs, const int32_t* order, const int32_t* offsets,
                                    int n_slots, int n_used, int n, hipStream_t s) {
    if (pairs == 0) return hipSuccess;
    const kf_act_offsets so = kf_act_layout((size_t)src_rows, (size_t)n), dso = kf_act_layout((size_t)pairs, (size_t)n);
    const char* sb = static_cast<const char*>(src);
    char* db = static_cast<char*>(dst);
    moe_gather_act_kernel<<<pairs, 256, 0, s>>>(reinterpret_cast<const int8_t*>(sb + so.q), reinterpret_cast<const float*>(sb + so.d32),
                                                reinterpret_cast<const uint4*>(sb + so.xa), reinterpret_cast<int8_t*>(db + dso.q),
                                                reinterpret_cast<float*>(db + dso.d32), reinterpret_cast<uint4*>(db + dso.xa), order, offsets,
                                                n_slots, n_used, n);
    return hipGetLastError();
}

hipError_t kf_launch_moe_group(const int32_t* slots, int total, int n_slots, int32_t* order, int32_t* offsets, hipStream_t s) {
    moe_group_kernel<<<1, 64 * KF_GROUP_WAVES, (size_t)n_slots * KF_GROUP_WAVES * sizeof(int), s>>>(slots, total, n_slots, order, offsets);
    return hipGetLastError();
}

hipError_t kf_launch_moe_combine(const float* part, const float* wts, const int32_t* slots, const float* host, float* out, int rows, int n_used,
                                 int n_embd, float scale, int n_slots, hipStream_t s) {
    if (rows == 0 || n_embd == 0) return hipSuccess;
    // float4 columns when every row starts 16-byte aligned, else single columns
    const bool v4 = n_embd % 4 == 0 && reinterpret_cast<uintptr_t>(part) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(host) % 16 == 0;
    const int per = v4 ? 1024 : 256;
    const int chunks = (n_embd + per - 1) / per;
    const int64_t blocks = (int64_t)chunks * rows;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    if (v4)
        moe_combine_kernel<4><<<(unsigned)blocks, 256, 0, s>>>(part, wts, slots, host, out, n_used, n_embd, scale, n_slots, chunks);
    else
        moe_combine_kernel<1><<<(unsigned)blocks, 256, 0, s>>>(part, wts, slots, host, out, n_used, n_embd, scale, n_slots, chunks);
    return hipGetLastError();
}
