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
#include "kf_blocks.h"

#include <algorithm>

namespace {

constexpr int RW_THREADS = 256;
constexpr int RW_WAVES = RW_THREADS / 64;

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

// The lane's float contribution of one step against one staged activation row at xr (LDS)
template <uint32_t TY>
__device__ __forceinline__ float rw_dot(const RwLaneW& v, const uint8_t* xr, int n, int s, int lane) {
    using T = RwType<TY>;
    const uint4* xs = reinterpret_cast<const uint4*>(xr) + (s * T::STEP_PIECES) + lane;
    const int32_t* ss = reinterpret_cast<const int32_t*>(xr + (n / T::BLOCK + T::PER_STEP - 1) / T::PER_STEP * T::STEP_PIECES * 16);
    if constexpr (TY == KF_TYPE_Q4_K) {
        const float* sd = reinterpret_cast<const float*>(ss + n / 32);
        const int sb = s * 16 + (lane >> 2), j = lane & 3;
        const int2 bs = *reinterpret_cast<const int2*>(ss + sb * 8 + 2 * j);
        int isum, imin;
        kf_q4k_lane(v.a, v.b, v.c, j, xs[0], xs[64], xs[128], xs[192], bs.x, bs.y, isum, imin);
        const float dx = sd[sb * 8];
        const float d = kf_h2f(v.a.x & 0xffffu) * dx;
        const float dm = kf_h2f(v.a.x >> 16) * dx;
        return fmaf(-dm, (float)imin, d * (float)isum);
    } else {
        const float* sd = reinterpret_cast<const float*>(ss);
        const uint32_t wq[8] = {v.a.x, v.a.y, v.a.z, v.a.w, v.b.x, v.b.y, v.b.z, v.b.w};
        const int b = s * 64 + lane;
        const int dt = kf_q8_0_dot(wq, xs[0], xs[64]);
        return kf_h2f(v.c.x) * sd[b] * (float)dt;
    }
}

// ops::silu (crates/kf-backend-cpu/src/ops.rs): x / (1 + e^-x)
__device__ __forceinline__ float rw_silu(float x) { return x / (1.0f + expf(-x)); }

// Block (x, slot): weight rows [x * rpb, +rpb) of the slot's matrix (base + slot * expert_bytes) against the slot's
// pairs [offsets[slot], offsets[slot + 1]) of `order` (identity without order; one slot [0, pairs) without offsets),
// RMAX at a time. The activation row of pair p is p (per_slot) or p / n_used. Outputs y[p][o]: GLU ? silu(gate .
// x) * (up . x) : w . x + bias[o] + res[p][o].
template <uint32_t TY, int RMAX, bool GLU>
__global__ void __launch_bounds__(RW_THREADS) rows_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int64_t expert_bytes,
                                                         int64_t row_bytes, const int8_t* __restrict__ xq, const int32_t* __restrict__ xs32,
                                                         const float* __restrict__ xd32, int n, int n_out, const int32_t* __restrict__ order,
                                                         const int32_t* __restrict__ offsets, int pairs, int n_used, int per_slot,
                                                         const float* __restrict__ bias, const float* __restrict__ res, float* __restrict__ y,
                                                         int rpb) {
    using T = RwType<TY>;
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

    for (int c0 = p0; c0 < p1; c0 += RMAX) {
        const int R = min(RMAX, p1 - c0);
        // stage the chunk's activation rows: transposed int8 pieces, then sums and scales
        for (int r = 0; r < R; r++) {
            const int p = order ? order[c0 + r] : c0 + r;
            const int xrow = per_slot ? p : p / n_used;
            uint8_t* xr = smem + r * row_lds;
            const uint4* gq = reinterpret_cast<const uint4*>(xq + (int64_t)xrow * n);
            for (int c = threadIdx.x; c < npc; c += RW_THREADS) {
                int dst;
                if constexpr (TY == KF_TYPE_Q4_K) {
                    const int sb = c >> 4, jj = (c >> 2) & 3, k = c & 3;
                    dst = (((sb >> 4) * 4 + k) << 6) + ((sb & 15) << 2) + jj;
                } else {
                    const int bb = c >> 1, k = c & 1;
                    dst = (((bb >> 6) * 2 + k) << 6) + (bb & 63);
                }
                reinterpret_cast<uint4*>(xr)[dst] = gq[c];
            }
            int32_t* ss = reinterpret_cast<int32_t*>(xr + steps * T::STEP_PIECES * 16);
            float* sd = reinterpret_cast<float*>(ss + (TY == KF_TYPE_Q4_K ? nsum : 0));
            for (int c = threadIdx.x; c < nsum; c += RW_THREADS) {
                if constexpr (TY == KF_TYPE_Q4_K) ss[c] = xs32[(int64_t)xrow * nsum + c];
                sd[c] = xd32[(int64_t)xrow * nsum + c];
            }
        }
        __syncthreads();

        // each wave walks rows o0 + wave, + RW_WAVES, ...; the next row's weights are requested before this row's
        // arithmetic
        int o = o0 + wave;
        RwLaneW cw[4], cu[4];  // one register set per step of the row (n <= 16384 for q4_K, 8192 for q8_0)
        auto load_row = [&](int orow) {
            const uint8_t* gr = wbase + (int64_t)min(orow, n_out - 1) * row_bytes;
#pragma unroll
            for (int s = 0; s < 4; s++)
                if (s < steps) rw_load<TY>(cw[s], gr, s, nblk, lane);
            if constexpr (GLU) {
                const uint8_t* ur = ubase + (int64_t)min(orow, n_out - 1) * row_bytes;
#pragma unroll
                for (int s = 0; s < 4; s++)
                    if (s < steps) rw_load<TY>(cu[s], ur, s, nblk, lane);
            }
        };
        if (o < o1) load_row(o);
        for (; o < o1; o += RW_WAVES) {
            RwLaneW vw[4], vu[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                vw[s] = cw[s];
                if constexpr (GLU) vu[s] = cu[s];
            }
            if (o + RW_WAVES < o1) load_row(o + RW_WAVES);
            float ag[RMAX], au[RMAX];
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                ag[r] = 0.0f;
                au[r] = 0.0f;
            }
#pragma unroll
            for (int s = 0; s < 4; s++) {
                if (s >= steps) break;
                const bool valid = s * T::PER_STEP + (TY == KF_TYPE_Q4_K ? (lane >> 2) : lane) < nblk;
#pragma unroll
                for (int r = 0; r < RMAX; r++) {
                    if (r >= R) break;
                    const uint8_t* xr = smem + r * row_lds;
                    if (valid) {
                        ag[r] += rw_dot<TY>(vw[s], xr, n, s, lane);
                        if constexpr (GLU) au[r] += rw_dot<TY>(vu[s], xr, n, s, lane);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                if (r >= R) break;
                const float g = kf_wave_sum_dpp(ag[r]);
                float u = 0.0f;
                if constexpr (GLU) u = kf_wave_sum_dpp(au[r]);
                if (lane == 0) {
                    const int p = order ? order[c0 + r] : c0 + r;
                    float* yo = y + (int64_t)p * n_out + o;
                    if constexpr (GLU)
                        *yo = rw_silu(g) * u;
                    else
                        *yo = g + (bias ? bias[o] : 0.0f) + (res ? res[(int64_t)p * n_out + o] : 0.0f);
                }
            }
        }
        __syncthreads();  // before the next chunk restages
    }
}

// Pairs grouped by slot: counts by LDS atomics (order-free), offsets by one thread, then wave 0 places the pairs of
// each 64-pair window in pair order, slot by slot (ballot ranks), so the order is deterministic. Slots < 0 or
// >= n_slots are skipped.
__global__ void __launch_bounds__(256) moe_group_kernel(const int32_t* __restrict__ slots, int total, int n_slots, int32_t* __restrict__ order,
                                                        int32_t* __restrict__ offsets) {
    extern __shared__ int cnt[];
    for (int i = threadIdx.x; i < n_slots; i += blockDim.x) cnt[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        const int s = slots[i];
        if (s >= 0 && s < n_slots) atomicAdd(&cnt[s], 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int i = 0; i < n_slots; i++) {
            const int c = cnt[i];
            offsets[i] = run;
            cnt[i] = run;
            run += c;
        }
        offsets[n_slots] = run;
    }
    __syncthreads();
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    for (int base = 0; base < total; base += 64) {
        const int i = base + lane;
        const int s = i < total ? slots[i] : -1;
        bool todo = s >= 0 && s < n_slots;
        uint64_t left = __ballot(todo);
        while (left) {
            const int leader = __builtin_ctzll(left);
            const int sv = __shfl(s, leader, 64);
            const uint64_t m = __ballot(todo && s == sv);
            const int start = cnt[sv];
            if (todo && s == sv) {
                order[start + __popcll(m & ((1ull << lane) - 1))] = i;
                todo = false;
            }
            if (lane == leader) cnt[sv] = start + __popcll(m);
            left &= ~m;
        }
    }
}

// out[r][o] = sum over j of the row's pairs rj = r * n_used + j with slots[rj] >= 0 of wts[rj] * scale * part[rj][o]
// (+ host[r][o]), j in order
__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ part, const float* __restrict__ wts, const int32_t* __restrict__ slots,
                                                          const float* __restrict__ host, float* __restrict__ out, int rows, int n_used, int n_embd,
                                                          float scale) {
    const int64_t total = (int64_t)rows * n_embd;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / n_embd, o = i - r * n_embd;
        float acc = 0.0f;
        for (int j = 0; j < n_used; j++) {
            const int64_t rj = r * n_used + j;
            if (slots[rj] >= 0) acc += wts[rj] * scale * part[rj * n_embd + o];
        }
        out[i] = acc + (host ? host[i] : 0.0f);
    }
}

template <uint32_t TY, int RMAX, bool GLU>
hipError_t rows_launch(const uint8_t* w, const uint8_t* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                       const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                       int per_slot, const float* bias, const float* res, float* y, hipStream_t s) {
    auto* fn = rows_kernel<TY, RMAX, GLU>;
    const int lds = RMAX * rw_row_lds<TY>(n);
    static int lds_set = 0;
    if (lds > 65536 && lds_set < lds) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        lds_set = lds;
    }
    const int rpb = 16 * RW_WAVES;  // rows per block: 16 a wave
    dim3 grid((n_out + rpb - 1) / rpb, offsets ? n_slots : 1);
    fn<<<grid, RW_THREADS, lds, s>>>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, pairs, n_used, per_slot, bias, res,
                                     y, rpb);
    return hipGetLastError();
}

// Pairs staged per chunk: as many as fit 96 KB of LDS, at most 8
template <uint32_t TY>
int rows_rmax(int n) {
    const int per = rw_row_lds<TY>(n);
    return 8 * per <= 98304 ? 8 : 4 * per <= 98304 ? 4 : 2 * per <= 98304 ? 2 : 1;
}

template <uint32_t TY, bool GLU>
hipError_t rows_dispatch(const uint8_t* w, const uint8_t* w2, int64_t expert_bytes, int64_t row_bytes, const int8_t* xq, const int32_t* xs32,
                         const float* xd32, int n, int n_out, const int32_t* order, const int32_t* offsets, int n_slots, int pairs, int n_used,
                         int per_slot, const float* bias, const float* res, float* y, hipStream_t s) {
    switch (rows_rmax<TY>(n)) {
        case 8: return rows_launch<TY, 8, GLU>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
        case 4: return rows_launch<TY, 4, GLU>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
        case 2: return rows_launch<TY, 2, GLU>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
        default: return rows_launch<TY, 1, GLU>(w, w2, expert_bytes, row_bytes, xq, xs32, xd32, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
    }
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
    if (ty == KF_TYPE_Q4_K)
        return w2 ? rows_dispatch<KF_TYPE_Q4_K, true>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s)
                  : rows_dispatch<KF_TYPE_Q4_K, false>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
    return w2 ? rows_dispatch<KF_TYPE_Q8_0, true>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s)
              : rows_dispatch<KF_TYPE_Q8_0, false>(wb, ub, expert_bytes, row_bytes, xq, xs, xd, n, n_out, order, offsets, n_slots, pairs, n_used, per_slot, bias, res, y, s);
}

hipError_t kf_launch_moe_group(const int32_t* slots, int total, int n_slots, int32_t* order, int32_t* offsets, hipStream_t s) {
    moe_group_kernel<<<1, 256, (size_t)n_slots * sizeof(int), s>>>(slots, total, n_slots, order, offsets);
    return hipGetLastError();
}

hipError_t kf_launch_moe_combine(const float* part, const float* wts, const int32_t* slots, const float* host, float* out, int rows, int n_used,
                                 int n_embd, float scale, hipStream_t s) {
    const int64_t total = (int64_t)rows * n_embd;
    if (total == 0) return hipSuccess;
    const int grid = (int)std::min<int64_t>((total + 255) / 256, 4096);
    moe_combine_kernel<<<grid, 256, 0, s>>>(part, wts, slots, host, out, rows, n_used, n_embd, scale);
    return hipGetLastError();
}
