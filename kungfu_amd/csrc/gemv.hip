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
#include <type_traits>

#include "kf_knobs.h"
#include "kf_blocks.h"
#include "kf_host.h"
#include "kf_qa.h"

#include <algorithm>

namespace {

#ifndef KF_GV_THREADS
#define KF_GV_THREADS 512
#endif
// ablation builds for roofline evidence (0 = the product). Bits: 1 skips the activation staging, 2 replaces the
// arithmetic by a XOR of the parked bytes, 4 skips parking the weights in LDS (2 and 4 give wrong results by design)
#ifndef KF_GV_ABLATE
#define KF_GV_ABLATE 0
#endif
// rows a wave of the pipelined variant holds in flight (2, 3 or 4); KF_GEMV_DEPTH overrides it (a tuning knob)
#ifndef KF_GV_DEPTH
#define KF_GV_DEPTH 2
#endif
// row iterations a block holds in flight at once (1, 2 or 4)
#ifndef KF_GV_MAXIT
#define KF_GV_MAXIT 2
#endif

constexpr int GV_THREADS = KF_GV_THREADS;
constexpr int GV_WAVES = GV_THREADS / 64;

// Shape of one launch, computed on the host: S wave steps per row, WPR waves per row (each taking steps sp, sp+WPR,
// ...), RPB = GV_WAVES / WPR rows per block iteration, `iters` block iterations. A wave step is 16 q4_K super-blocks
// (2304 bytes, 4096 columns) or 64 q8_0 blocks (2176 bytes, 2048 columns).
//
// Weight bytes travel as contiguous 16-byte pieces (every wave load instruction reads 1 KB of consecutive bytes, the
// pattern that streams at the chip's read rate), land in the wave's own LDS buffer, and lanes read back the pieces
// their blocks need.
//
// LDS layout:
//   activations, wave-transposed so a wave's 16-byte reads are contiguous across lanes:
//     q4_K: step s, piece k (0..3), lane l -> activation bytes 64*l + 16*k of the step, at ((s*4 + k)*64 + l)*16
//     q8_0: step s, piece k (0..1), lane l -> activation bytes 32*l + 16*k of the step, at ((s*2 + k)*64 + l)*16
//   int32 sums per 32 (q4_K), f32 scales per 32
//   one GV_STEP_BYTES buffer per wave for its weight step
//   `iters * GV_WAVES` f32 partials when WPR > 1
constexpr int GV_STEP_BYTES = 2304;
constexpr int GV_PIECES = 3;  // 16-byte pieces per lane per step: 144 (q4_K) or 136 (q8_0) pieces over 64 lanes

struct GvLds {
    size_t xbytes, sums, scales, wbuf, part, total;
};

__host__ __device__ inline GvLds gv_lds(uint32_t ty, int n, int iters, int wpr) {
    GvLds l;
    const int steps = ty == KF_TYPE_Q4_K ? (n / 256 + 15) / 16 : (n / 32 + 63) / 64;
    l.xbytes = (size_t)steps * (ty == KF_TYPE_Q4_K ? 4096 : 2048);
    l.sums = l.xbytes;
    l.scales = l.sums + (ty == KF_TYPE_Q4_K ? (size_t)(n / 32) * 4 : 0);
    l.wbuf = l.scales + (size_t)(n / 32) * 4;
    l.wbuf = (l.wbuf + 15) / 16 * 16;
    l.part = l.wbuf + (size_t)GV_WAVES * GV_STEP_BYTES;
    l.total = l.part + (wpr > 1 ? (size_t)iters * GV_WAVES * 4 : 0);
    return l;
}

// The activation row of one block in flight: each thread loads at most GV_XC 16-byte pieces of int8 values and
// GV_SC per-32 sums and scales (n <= 32768 with 512 threads). The loads are issued before the weights are requested
// so that parking them in LDS waits only on them, not on the weights behind them.
constexpr int GV_XC = (32768 / 16 + GV_THREADS - 1) / GV_THREADS;
constexpr int GV_SC = (32768 / 32 + GV_THREADS - 1) / GV_THREADS;

struct GvStage {
    uint4 x[GV_XC];
    int32_t sum[GV_SC];
    float scale[GV_SC];
};

// Stacked row o of a grouped product (KfSegs; sg.n == 0: the single matrix w). The member is picked by unrolled
// selects on constant indices, so the table stays in kernel arguments (scalar registers when o is wave-uniform).
struct GvRow {
    const uint8_t* w;
    float* y;
    const float* bias;
    const float* res;
    int o;  // the row within its member
};

__device__ __forceinline__ GvRow gv_row(const KfSegs& sg, const uint8_t* w, float* y, const float* bias, const float* res, int o) {
    GvRow r{w, y, bias, res, o};
    if (sg.n > 0) {
        r = GvRow{sg.w[0], sg.y[0], sg.bias[0], sg.res[0], o};
#pragma unroll
        for (int k = 1; k < KF_MAX_SEGS; k++)
            if (k < sg.n && o >= sg.start[k]) r = GvRow{sg.w[k], sg.y[k], sg.bias[k], sg.res[k], o - sg.start[k]};
    }
    return r;
}

__device__ __forceinline__ const uint8_t* gv_row_ptr(const KfSegs& sg, const uint8_t* w, int64_t row_bytes, int o) {
    const GvRow r = gv_row(sg, w, nullptr, nullptr, nullptr, o);
    return r.w + (int64_t)r.o * row_bytes;
}

__device__ __forceinline__ void gv_store(const KfSegs& sg, float* y, const float* bias, const float* res, int o, float acc) {
    const GvRow r = gv_row(sg, nullptr, y, bias, res, o);
    r.y[r.o] = acc + (r.bias ? r.bias[r.o] : 0.0f) + (r.res ? r.res[r.o] : 0.0f);
}

template <uint32_t TY>
__device__ __forceinline__ void gv_stage_load(GvStage& st, const int8_t* __restrict__ xq, const int32_t* __restrict__ xs32,
                                              const float* __restrict__ xd32, int n) {
    // unpredicated loads (indices clamped into the row; the extra copies are not stored), so the compiler never
    // waits on one before issuing the next
    const uint4* gq = reinterpret_cast<const uint4*>(xq);
#pragma unroll
    for (int i = 0; i < GV_XC; i++) st.x[i] = gq[min((int)threadIdx.x + i * GV_THREADS, (n >> 4) - 1)];
#pragma unroll
    for (int i = 0; i < GV_SC; i++) {
        const int c = min((int)threadIdx.x + i * GV_THREADS, (n >> 5) - 1);
        if constexpr (TY == KF_TYPE_Q4_K) st.sum[i] = xs32[c];
        st.scale[i] = xd32[c];
    }
}

// Parks the activation row in LDS: int8 values in the wave-transposed order, per-32 sums (q4_K) and per-32 scales.
// Clamped duplicates write the same bytes to the same place, so no store is predicated either (a predicated store
// lets the compiler sink its load next to it, behind the weight loads).
template <uint32_t TY>
__device__ __forceinline__ void gv_stage_store(uint8_t* smem, size_t sums_at, size_t scales_at, const GvStage& st, int n) {
    uint4* sx = reinterpret_cast<uint4*>(smem);
#pragma unroll
    for (int i = 0; i < GV_XC; i++) {
        const int c = min((int)threadIdx.x + i * GV_THREADS, (n >> 4) - 1);
        int dst;
        if constexpr (TY == KF_TYPE_Q4_K) {
            const int sb = c >> 4, j = (c >> 2) & 3, k = c & 3;  // 16 pieces per super-block: pair j, piece k
            dst = (((sb >> 4) * 4 + k) << 6) + ((sb & 15) << 2) + j;
        } else {
            const int b = c >> 1, k = c & 1;  // 2 pieces per 32-block
            dst = (((b >> 6) * 2 + k) << 6) + (b & 63);
        }
        sx[dst] = st.x[i];
    }
#pragma unroll
    for (int i = 0; i < GV_SC; i++) {
        const int c = min((int)threadIdx.x + i * GV_THREADS, (n >> 5) - 1);
        if constexpr (TY == KF_TYPE_Q4_K) reinterpret_cast<int32_t*>(smem + sums_at)[c] = st.sum[i];
        reinterpret_cast<float*>(smem + scales_at)[c] = st.scale[i];
    }
}

// The fused variants (QX > 0) quantize the f32 activation row themselves, in place of a quant_act launch before the
// product: wave w owns the 256-column chunks w, w + GV_WAVES, ... (QX of them, n <= QX * GV_WAVES * 256). Its loads
// are issued before the weight requests, so quantizing waits on them alone; the integers, scales and sums are
// kf_qa_quant's, the same as the quant_act kernel writes, parked in the layout the staged variants fill.
template <int QX>
struct GvXf {
    float4 v[QX > 0 ? QX : 1];
    float4 w[QX > 0 ? QX : 1], b[QX > 0 ? QX : 1];  // the norm's weight and bias columns (the rms_norm variants)
};

// The rms_norm the fused variants apply before quantizing (NM = 1): weight and bias columns (either may be null) and
// eps; unused by the other variants
struct GvNorm {
    const float* w;
    const float* b;
    float eps;
};

template <int QX, int NM = 0>
__device__ __forceinline__ void gv_xf_load(GvXf<QX>& r, const float* __restrict__ x, int n, int wave, int lane, const GvNorm& nm = GvNorm{}) {
#pragma unroll
    for (int i = 0; i < QX; i++) {
        // unpredicated: a lane past the row's end reloads the row's last four columns, which it does not quantize
        const int c0 = min((wave + GV_WAVES * i) * 256 + 4 * lane, n - 4);
        r.v[i] = *reinterpret_cast<const float4*>(x + c0);
        if constexpr (NM) {
            r.w[i] = nm.w ? *reinterpret_cast<const float4*>(nm.w + c0) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            r.b[i] = nm.b ? *reinterpret_cast<const float4*>(nm.b + c0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
}

// rms_norm of the row the block's waves hold in their chunks (crates/kf-backend-cpu/src/ops.rs:222-239, as
// rms_norm_q8_kernel computes it): f32 squares summed in f64 (lane, then wave in a fixed tree, then the waves in
// order through LDS), ss / n rounded to f32, correctly rounded f32 square root and division, then (v * inv) * w + b
// unfused, in place. Every wave of the block calls it (one barrier, waiting on LDS only).
template <int QX>
__device__ __forceinline__ void gv_xf_norm(GvXf<QX>& r, double* part, int n, int wave, int lane, float eps) {
#pragma clang fp contract(off)
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < QX; i++) {
        const int ch = wave + GV_WAVES * i;
        if (ch * 256 < n && ch * 256 + 4 * lane < n) {
            const float4 t = r.v[i];
            const float a0 = t.x * t.x, a1 = t.y * t.y, a2 = t.z * t.z, a3 = t.w * t.w;
            s += (double)a0;
            s += (double)a1;
            s += (double)a2;
            s += (double)a3;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) part[wave] = s;
    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(63) & ~(15 << 8));
    __builtin_amdgcn_s_barrier();
    double t = 0.0;
#pragma unroll
    for (int k = 0; k < GV_WAVES; k++) t += part[k];
    const float ss = (float)(t / (double)n);
    const float rr = (float)sqrt((double)(ss + eps));
    const float inv = (float)(1.0 / (double)rr);
#pragma unroll
    for (int i = 0; i < QX; i++) {
        float4& v = r.v[i];
        const float4 w = r.w[i], b = r.b[i];
        float u;
        u = v.x * inv; u = u * w.x; v.x = u + b.x;
        u = v.y * inv; u = u * w.y; v.y = u + b.y;
        u = v.z * inv; u = u * w.z; v.z = u + b.z;
        u = v.w * inv; u = u * w.w; v.w = u + b.w;
    }
}

template <uint32_t TY, int QX>
__device__ __forceinline__ void gv_xf_quant(uint8_t* smem, size_t sums_at, size_t scales_at, const GvXf<QX>& r, int n, int wave, int lane) {
    constexpr int kind = TY == KF_TYPE_Q4_K ? KF_ACT_Q8K : KF_ACT_Q8_0;
#pragma unroll
    for (int i = 0; i < QX; i++) {
        const int ch = wave + GV_WAVES * i;
        if (ch * 256 >= n) break;  // wave-uniform
        const int c0 = ch * 256 + 4 * lane;
        const bool in = c0 < n;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (in) {
            v[0] = r.v[i].x;
            v[1] = r.v[i].y;
            v[2] = r.v[i].z;
            v[3] = r.v[i].w;
        }
        const KfQa q = kf_qa_quant(v, c0, in, kind);
        if (in) {
            const int c = c0 >> 4;  // the 16-column piece, placed as the staged variants place it
            int dst;
            if constexpr (TY == KF_TYPE_Q4_K) {
                const int sb = c >> 4, jj = (c >> 2) & 3, k = c & 3;
                dst = (((sb >> 4) * 4 + k) << 6) + ((sb & 15) << 2) + jj;
            } else {
                const int b = c >> 1, k = c & 1;
                dst = (((b >> 6) * 2 + k) << 6) + (b & 63);
            }
            *reinterpret_cast<uint32_t*>(smem + (size_t)dst * 16 + (c0 & 15)) = q.packed;
            if ((lane & 7) == 0) {
                if constexpr (TY == KF_TYPE_Q4_K) reinterpret_cast<int32_t*>(smem + sums_at)[c0 >> 5] = q.sum32;
                reinterpret_cast<float*>(smem + scales_at)[c0 >> 5] = q.d;
            }
        }
    }
}

// Per-lane constants of the weight pieces: lane l moves the 16-byte pieces l, l+64 and l+128 of a step
struct GvLane {
    int lane;
    uint32_t off[GV_PIECES];  // byte offsets of the lane's pieces within a step
};

// Loads one step's pieces (len bytes of the step starting at `step`, a wave-uniform address). Every lane loads all
// its pieces: a piece past the step's end is clamped onto the step's last 16 bytes, so no byte past the step is
// read and no load is predicated (predicated loads make the compiler wait for the ring before refilling it).
// Clamped pieces carry bytes another lane also holds; parking them writes the same bytes to the same place.
template <uint32_t TY>
__device__ __forceinline__ void gv_load_step(uint4* v, const uint8_t* step, int len, const GvLane& ln) {
#pragma unroll
    for (int i = 0; i < GV_PIECES; i++) {
        const uint32_t o = min(ln.off[i], (uint32_t)len - 16u);
        if constexpr (TY == KF_TYPE_Q4_K)
            v[i] = kf_load_stream_u4(step + o);
        else
            v[i] = kf_load_stream_u4_unaligned(step + o);
    }
}

// Parks the pieces in the wave's LDS buffer at the offsets they were loaded from
template <uint32_t TY>
__device__ __forceinline__ void gv_park(uint8_t* wb, const uint4* v, int len, const GvLane& ln) {
#pragma unroll
    for (int i = 0; i < GV_PIECES; i++) {
        const uint32_t o = min(ln.off[i], (uint32_t)len - 16u);
        if constexpr (TY == KF_TYPE_Q4_K)
            *reinterpret_cast<uint4*>(wb + o) = v[i];
        else
            *reinterpret_cast<kf_u32x4_a2*>(wb + o) = kf_u32x4_a2{v[i].x, v[i].y, v[i].z, v[i].w};
    }
}

// The lane's share of one q4_K step: super-block (lane >> 2) of the step, sub-block pair j = lane & 3. `sb` is the
// super-block's index in the row, `xs` the lane's first activation piece of the step in the transposed layout.
__device__ __forceinline__ float gv_q4k_lane(const uint8_t* wl, const uint4* xs, const int32_t* ss, const float* sd, int sb, int j) {
    const uint4 hdr = *reinterpret_cast<const uint4*>(wl);
    const uint4 qa = *reinterpret_cast<const uint4*>(wl + 16 + 32 * j);
    const uint4 qb = *reinterpret_cast<const uint4*>(wl + 32 + 32 * j);
    const int2 bs = *reinterpret_cast<const int2*>(ss + sb * 8 + 2 * j);
    int isum, imin;
    kf_q4k_lane(hdr, qa, qb, j, xs[0], xs[64], xs[128], xs[192], bs.x, bs.y, isum, imin);
    const float dx = sd[sb * 8];
    const float d = kf_h2f(hdr.x & 0xffffu) * dx;
    const float dm = kf_h2f(hdr.x >> 16) * dx;
    return fmaf(-dm, (float)imin, d * (float)isum);
}

// gv_q4k_lane with the activation side already in registers: x0..x3 the lane's four activation pieces, bs its two
// sub-block sums, dx the super-block's scale
__device__ __forceinline__ float gv_q4k_lane_r(const uint8_t* wl, const uint4 x0, const uint4 x1, const uint4 x2, const uint4 x3, const int2 bs,
                                               float dx, int j) {
    const uint4 hdr = *reinterpret_cast<const uint4*>(wl);
    const uint4 qa = *reinterpret_cast<const uint4*>(wl + 16 + 32 * j);
    const uint4 qb = *reinterpret_cast<const uint4*>(wl + 32 + 32 * j);
    int isum, imin;
    kf_q4k_lane(hdr, qa, qb, j, x0, x1, x2, x3, bs.x, bs.y, isum, imin);
    const float d = kf_h2f(hdr.x & 0xffffu) * dx;
    const float dm = kf_h2f(hdr.x >> 16) * dx;
    return fmaf(-dm, (float)imin, d * (float)isum);
}

// The lane's block of one q8_0 step: the 34 bytes at 34 * lane of the step; b is the block's index in the row
__device__ __forceinline__ float gv_q8_0_lane(const uint8_t* wl, const uint4* xs, const float* sd, int b) {
    const kf_u32x4_a2 q0 = *reinterpret_cast<const kf_u32x4_a2*>(wl + 2);
    const kf_u32x4_a2 q1 = *reinterpret_cast<const kf_u32x4_a2*>(wl + 18);
    const uint32_t wq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const int dt = kf_q8_0_dot(wq, xs[0], xs[64]);
    return kf_h2f(*reinterpret_cast<const uint16_t*>(wl)) * sd[b] * (float)dt;
}

// gv_q8_0_lane with the activation side in registers (x0, x1 the lane's pieces, dx its block's scale)
__device__ __forceinline__ float gv_q8_0_lane_r(const uint8_t* wl, const uint4 x0, const uint4 x1, float dx) {
    // the block's quants start 2 bytes past a dword boundary when its byte offset (34 x lane) is a multiple of 4: read
    // nine aligned dwords and realign (v_alignbyte_b32) rather than 2-byte aligned 16-byte LDS reads
    const uint32_t sh = (reinterpret_cast<uintptr_t>(wl) & 2u) ? 0u : 2u;
    const uint32_t* ap = reinterpret_cast<const uint32_t*>(wl + 2 - sh);
    uint32_t dw[9];
#pragma unroll
    for (int i = 0; i < 9; i++) dw[i] = ap[i];
    uint32_t wq[8];
#pragma unroll
    for (int i = 0; i < 8; i++) wq[i] = kf_alignbyte(dw[i + 1], dw[i], sh);
    const int dt = kf_q8_0_dot(wq, x0, x1);
    return kf_h2f(*reinterpret_cast<const uint16_t*>(wl)) * dx * (float)dt;
}

// Decode GEMV of one activation row. Block b, iteration it (< iters <= MAXIT), row group rg (= wave / WPR) owns row
// (it * gridDim.x + b) * RPB + rg; the WPR waves of a row group split its steps and meet in LDS at the end. A wave
// requests the weights of all its iterations before the activation row is staged, each into registers of its own,
// so nothing waits on a load before the last one is issued. Everything that depends only on the row or step is
// wave-uniform and lives in scalar registers.
template <uint32_t TY, int SPW, int WPR, int MAXIT>
__global__ void __launch_bounds__(GV_THREADS) gemv_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                          const int32_t* __restrict__ xs32, const float* __restrict__ xd32,
                                                          const float* __restrict__ bias, const float* __restrict__ res,
                                                          float* __restrict__ y, int n, int n_out, int iters, const KfSegs sg,
                                                          const float* __restrict__, const GvNorm) {
    constexpr int RPB = GV_WAVES / WPR;
    constexpr int STEP = TY == KF_TYPE_Q4_K ? 2304 : 2176;
    constexpr int PER_STEP = TY == KF_TYPE_Q4_K ? 16 : 64;  // blocks per step
    extern __shared__ __align__(16) uint8_t smem[];
    const GvLds L = gv_lds(TY, n, iters, WPR);
    GvLane ln;
    ln.lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < GV_PIECES; i++) ln.off[i] = 16u * (uint32_t)(ln.lane + 64 * i);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = wave / WPR, sp = wave % WPR;
    const int nblk = TY == KF_TYPE_Q4_K ? n >> 8 : n >> 5;
    const int B = gridDim.x;
    uint8_t* wb = smem + L.wbuf + wave * GV_STEP_BYTES;
    const int j = ln.lane & 3;
    const uint8_t* wl = TY == KF_TYPE_Q4_K ? wb + (ln.lane >> 2) * KF_Q4_K_BYTES : wb + 34 * ln.lane;
    const uint4* xl = reinterpret_cast<const uint4*>(smem) + ln.lane;
    const int32_t* ss = reinterpret_cast<const int32_t*>(smem + L.sums);
    const float* sd = reinterpret_cast<const float*>(smem + L.scales);
    const int blk_lane = TY == KF_TYPE_Q4_K ? (ln.lane >> 2) : ln.lane;

    GvStage st;
    if (!(KF_GV_ABLATE & 1)) gv_stage_load<TY>(st, xq, xs32, xd32, n);
    // keep the activation loads ahead of the weight loads: loads complete in issue order, so parking the
    // activations then waits only on them
    __builtin_amdgcn_sched_barrier(0);
    uint4 ring[MAXIT][SPW][GV_PIECES];
    const int64_t last_step = (row_bytes - 1) / STEP;
    int iw = iters;  // iterations whose row exists for this wave (see the pipelined variant)
    while (iw > 0 && ((iw - 1) * B + (int)blockIdx.x) * RPB + rg >= n_out) iw--;
    if (iw == 0) iw = 1;
#pragma unroll
    for (int it = 0; it < MAXIT; it++) {
        // unpredicated: an iteration or step past the end reloads a valid row or step whose result is never used
        const int o = min((min(it, iw - 1) * B + (int)blockIdx.x) * RPB + rg, n_out - 1);
        const uint8_t* row = gv_row_ptr(sg, w, row_bytes, o);
#pragma unroll
        for (int i = 0; i < SPW; i++) {
            const int64_t at = min((int64_t)(sp + i * WPR), last_step) * STEP;
            gv_load_step<TY>(ring[it][i], row + at, (int)min((int64_t)STEP, row_bytes - at), ln);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (!(KF_GV_ABLATE & 1)) gv_stage_store<TY>(smem, L.sums, L.scales, st, n);
    __syncthreads();
    float* part = reinterpret_cast<float*>(smem + L.part);
#pragma unroll
    for (int it = 0; it < MAXIT; it++) {
        const int o = (it * B + (int)blockIdx.x) * RPB + rg;
        if (it < iters && o < n_out) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < SPW; i++) {
                const int s = sp + i * WPR;
                const int64_t at = (int64_t)s * STEP;
                if (at < row_bytes) {
                    if (!(KF_GV_ABLATE & 4)) gv_park<TY>(wb, ring[it][i], (int)min((int64_t)STEP, row_bytes - at), ln);
                    __builtin_amdgcn_wave_barrier();
                    const int blk = s * PER_STEP + blk_lane;
                    if (KF_GV_ABLATE & 2) {
                        const uint4* q = reinterpret_cast<const uint4*>(wl);
                        acc += (KF_GV_ABLATE & 4) ? (float)(ring[it][i][0].x ^ ring[it][i][1].y ^ ring[it][i][2].z) : (float)(q->x ^ q->w);
                    } else if (blk < nblk) {
                        if constexpr (TY == KF_TYPE_Q4_K)
                            acc += gv_q4k_lane(wl, xl + ((s * 4) << 6), ss, sd, blk, j);
                        else
                            acc += gv_q8_0_lane(wl, xl + ((s * 2) << 6), sd, blk);
                    }
                    __builtin_amdgcn_wave_barrier();
                }
            }
            acc = kf_wave_sum_dpp(acc);
            if (ln.lane == 0) {
                if (WPR == 1) gv_store(sg, y, bias, res, o, acc);
                else part[it * GV_WAVES + wave] = acc;
            }
        }
    }
    if (WPR > 1) {
        __syncthreads();
        for (int t = threadIdx.x; t < iters * RPB; t += GV_THREADS) {
            const int it = t / RPB, g = t % RPB;
            const int o = (it * B + (int)blockIdx.x) * RPB + g;
            if (o >= n_out) continue;
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < WPR; q++) acc += part[it * GV_WAVES + g * WPR + q];
            gv_store(sg, y, bias, res, o, acc);
        }
    }
}

// ------------------------------------------------------------------------------------------------ DMA variant
// The same product with both the activation row and the weight steps fetched straight into LDS by
// global_load_lds_dwordx4 (gfx950): lane l of one instruction writes its 16 bytes at the instruction's LDS base
// + 16 * l. Nothing passes through registers, so the compiler cannot reorder the streams, and a wave's weights for
// all its row iterations are requested before the block waits on the (small, L2-resident) activation row.
// Requires 16-byte aligned rows (q4_K always; q8_0 when the row width is a multiple of 128).

__device__ __forceinline__ void gv_dma16(const void* src, void* lds_base) { kf_dma16(src, lds_base); }

__device__ __forceinline__ void gv_dma4(const void* src, void* lds_base) { kf_dma4(src, lds_base); }

struct GdLds {
    size_t sums, scales, wbuf, part, total;
};

// LDS of the DMA variant: transposed activations, sums, scales, then MAXIT * SPW step buffers per wave, partials
__host__ __device__ inline GdLds gd_lds(uint32_t ty, int n, int iters, int wpr, int maxit, int spw) {
    GdLds l;
    const int steps = ty == KF_TYPE_Q4_K ? (n / 256 + 15) / 16 : (n / 32 + 63) / 64;
    const size_t xbytes = (size_t)steps * (ty == KF_TYPE_Q4_K ? 4096 : 2048);
    const size_t n32 = (size_t)((n / 32 + 63) / 64 * 64);  // whole 64-entry DMA instructions
    l.sums = xbytes;
    l.scales = l.sums + (ty == KF_TYPE_Q4_K ? n32 * 4 : 0);
    l.wbuf = l.scales + n32 * 4;
    l.part = l.wbuf + (size_t)GV_WAVES * maxit * spw * GV_STEP_BYTES;
    l.total = l.part + (wpr > 1 ? (size_t)iters * GV_WAVES * 4 : 0);
    return l;
}

#ifdef KF_GV_TRACE
// timeline of every wave (variant builds only): entry, data in LDS, done, in 100 MHz ticks
__device__ uint64_t* kf_gv_trace;
#define KF_GV_STAMP(k)                                                                                                 \
    if (kf_gv_trace && (threadIdx.x & 63) == 0)                                                                        \
        kf_gv_trace[((size_t)blockIdx.x * GV_WAVES + (threadIdx.x >> 6)) * 4 + (k)] = __builtin_amdgcn_s_memrealtime();
#else
#define KF_GV_STAMP(k)
#endif

template <uint32_t TY, int SPW, int WPR, int MAXIT>
__global__ void __launch_bounds__(GV_THREADS) gemv_dma_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                              const int32_t* __restrict__ xs32, const float* __restrict__ xd32,
                                                              const float* __restrict__ bias, const float* __restrict__ res,
                                                              float* __restrict__ y, int n, int n_out, int iters, const KfSegs sg,
                                                              const float* __restrict__, const GvNorm) {
    constexpr int RPB = GV_WAVES / WPR;
    constexpr int STEP = TY == KF_TYPE_Q4_K ? 2304 : 2176;
    constexpr int PER_STEP = TY == KF_TYPE_Q4_K ? 16 : 64;  // blocks per step
    extern __shared__ __align__(16) uint8_t smem[];
    KF_GV_STAMP(0)
    const GdLds L = gd_lds(TY, n, iters, WPR, MAXIT, SPW);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = wave / WPR, sp = wave % WPR;
    const int nblk = TY == KF_TYPE_Q4_K ? n >> 8 : n >> 5;
    const int B = gridDim.x;
    const int steps = TY == KF_TYPE_Q4_K ? (nblk + 15) / 16 : (nblk + 63) / 64;
    const int64_t last_step = (row_bytes - 1) / STEP;

    // 1. the activation row, split over the block's waves: instruction q < steps*K4 moves piece k of step s (the 64
    //    lanes' 16-byte pieces of the transposed layout); then the per-32 sums and scales, 64 entries an instruction
    {
        constexpr int K4 = TY == KF_TYPE_Q4_K ? 4 : 2;
        const int nx = steps * K4;
        const int n32 = n >> 5, n32i = (n32 + 63) / 64;
        const int total = nx + (TY == KF_TYPE_Q4_K ? 2 : 1) * n32i;
        for (int q = wave; q < total; q += GV_WAVES) {
            if (q < nx) {
                const int st = q / K4, k = q % K4;
                // lane l of (step st, piece k) holds activation piece c = 256 st + 4 l + k (q4_K) or 128 st + 2 l + k
                int c = TY == KF_TYPE_Q4_K ? 256 * st + 4 * lane + k : 128 * st + 2 * lane + k;
                c = min(c, (n >> 4) - 1);  // lanes past the row's end fetch a valid piece nobody reads
                gv_dma16(xq + 16 * c, smem + (size_t)((st * K4 + k) << 10));
            } else {
                const int r = q - nx;
                const int which = TY == KF_TYPE_Q4_K ? r / n32i : 1;  // 0: sums, 1: scales
                const int i = (TY == KF_TYPE_Q4_K ? r % n32i : r) * 64;
                const int c = min(i + lane, n32 - 1);
                if (which == 0)
                    gv_dma4(xs32 + c, smem + L.sums + 4 * i);
                else
                    gv_dma4(xd32 + c, smem + L.scales + 4 * i);
            }
        }
    }
    // 2. the weights of every row iteration of the wave, one buffer per (iteration, step)
    uint8_t* wb = smem + L.wbuf + (size_t)wave * MAXIT * SPW * GV_STEP_BYTES;
    int iw = iters;  // iterations whose row exists for this wave (see the pipelined variant)
    while (iw > 0 && ((iw - 1) * B + (int)blockIdx.x) * RPB + rg >= n_out) iw--;
    if (iw == 0) iw = 1;
#pragma unroll
    for (int it = 0; it < MAXIT; it++) {
        const int o = min((min(it, iw - 1) * B + (int)blockIdx.x) * RPB + rg, n_out - 1);
        const uint8_t* row = gv_row_ptr(sg, w, row_bytes, o);
#pragma unroll
        for (int i = 0; i < SPW; i++) {
            const int64_t at = min((int64_t)(sp + i * WPR), last_step) * STEP;
            const int len = (int)min((int64_t)STEP, row_bytes - at);
            uint8_t* buf = wb + (it * SPW + i) * GV_STEP_BYTES;
            const uint8_t* src = row + at;
            gv_dma16(src + min(16 * lane, len - 16), buf);
            gv_dma16(src + min(16 * lane + 1024, len - 16), buf + 1024);
            if (lane < (GV_STEP_BYTES - 2048) / 16) gv_dma16(src + min(16 * lane + 2048, len - 16), buf + 2048);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    KF_GV_STAMP(1)
    __syncthreads();
    KF_GV_STAMP(2)

    // 3. the products, from LDS only
    const int j = lane & 3;
    const uint4* xl = reinterpret_cast<const uint4*>(smem) + lane;
    const int32_t* ss = reinterpret_cast<const int32_t*>(smem + L.sums);
    const float* sd = reinterpret_cast<const float*>(smem + L.scales);
    const int blk_lane = TY == KF_TYPE_Q4_K ? (lane >> 2) : lane;
    float* part = reinterpret_cast<float*>(smem + L.part);
#pragma unroll
    for (int it = 0; it < MAXIT; it++) {
        const int o = (it * B + (int)blockIdx.x) * RPB + rg;
        if (it < iters && o < n_out) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < SPW; i++) {
                const int s = sp + i * WPR;
                const int blk = s * PER_STEP + blk_lane;
                if (s < steps && blk < nblk) {
                    const uint8_t* buf = wb + (it * SPW + i) * GV_STEP_BYTES;
                    if constexpr (TY == KF_TYPE_Q4_K)
                        acc += gv_q4k_lane(buf + (lane >> 2) * KF_Q4_K_BYTES, xl + ((s * 4) << 6), ss, sd, blk, j);
                    else
                        acc += gv_q8_0_lane(buf + 34 * lane, xl + ((s * 2) << 6), sd, blk);
                }
            }
            acc = kf_wave_sum_dpp(acc);
            if (lane == 0) {
                if (WPR == 1) gv_store(sg, y, bias, res, o, acc);
                else part[it * GV_WAVES + wave] = acc;
            }
        }
    }
    KF_GV_STAMP(3)
    if (WPR > 1) {
        __syncthreads();
        for (int t = threadIdx.x; t < iters * RPB; t += GV_THREADS) {
            const int it = t / RPB, g = t % RPB;
            const int o = (it * B + (int)blockIdx.x) * RPB + g;
            if (o >= n_out) continue;
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < WPR; q++) acc += part[it * GV_WAVES + g * WPR + q];
            gv_store(sg, y, bias, res, o, acc);
        }
    }
}

// ------------------------------------------------------------------------------------------------ pipelined variant
// Persistent waves walk their rows with two register sets: while row i is parked in the wave's LDS buffer and
// multiplied, the loads of rows i+1 and i+2 are in flight, so the arithmetic of a wave overlaps its own weight stream
// (a wave that computes only after all its loads land holds its slot while the memory pipe idles). The activation
// row reaches LDS by DMA before any weight is requested.
template <uint32_t TY, int WPR, int D, int QX = 0, int NM = 0>
__global__ void __launch_bounds__(GV_THREADS) gemv_pipe_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                               const int32_t* __restrict__ xs32, const float* __restrict__ xd32,
                                                               const float* __restrict__ bias, const float* __restrict__ res,
                                                               float* __restrict__ y, int n, int n_out, int iters, const KfSegs sg,
                                                               const float* __restrict__ xf, const GvNorm nm) {
    constexpr int RPB = GV_WAVES / WPR;
    constexpr int STEP = TY == KF_TYPE_Q4_K ? 2304 : 2176;
    constexpr int PER_STEP = TY == KF_TYPE_Q4_K ? 16 : 64;
    extern __shared__ __align__(16) uint8_t smem[];
    KF_GV_STAMP(0)
    const GdLds L = gd_lds(TY, n, iters, WPR, 1, 1);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = wave / WPR, sp = wave % WPR;
    const int nblk = TY == KF_TYPE_Q4_K ? n >> 8 : n >> 5;
    const int B = gridDim.x;
    const int steps = TY == KF_TYPE_Q4_K ? (nblk + 15) / 16 : (nblk + 63) / 64;
    const int64_t at = (int64_t)min(sp, steps - 1) * STEP;  // the wave's step of every row
    const int len = (int)min((int64_t)STEP, row_bytes - at);
    const bool has_step = sp < steps;

    // the activation row is staged by the first waves only (256 pieces of 16 bytes and 128 sums and scales a wave,
    // all loads issued before the first wait), which then request their own weights; the other waves request theirs
    // at once, so most waves start streaming without waiting on the activation row. Fused: every wave loads its f32
    // chunks first and quantizes them once its first rows' weights are requested
    GvXf<QX> xr;
    if constexpr (QX > 0) {
        gv_xf_load<QX, NM>(xr, xf, n, wave, lane, nm);
        __builtin_amdgcn_sched_barrier(0);
    } else {
        const int nchunks = n >> 4, n32 = n >> 5;
        const int nsw = (nchunks + 255) / 256;
        if (!(KF_GV_ABLATE & 1) && wave < nsw) {
            const uint4* gq = reinterpret_cast<const uint4*>(xq);
            uint4 v[4];
            int32_t sv[2];
            float dv[2];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = gq[min(wave * 256 + i * 64 + lane, nchunks - 1)];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = min(wave * 128 + i * 64 + lane, n32 - 1);
                if constexpr (TY == KF_TYPE_Q4_K) sv[i] = xs32[c];
                dv[i] = xd32[c];
            }
            uint4* sx = reinterpret_cast<uint4*>(smem);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = min(wave * 256 + i * 64 + lane, nchunks - 1);
                int dst;
                if constexpr (TY == KF_TYPE_Q4_K) {
                    const int sb = c >> 4, jj = (c >> 2) & 3, k = c & 3;
                    dst = (((sb >> 4) * 4 + k) << 6) + ((sb & 15) << 2) + jj;
                } else {
                    const int bb = c >> 1, k = c & 1;
                    dst = (((bb >> 6) * 2 + k) << 6) + (bb & 63);
                }
                sx[dst] = v[i];
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = min(wave * 128 + i * 64 + lane, n32 - 1);
                if constexpr (TY == KF_TYPE_Q4_K) reinterpret_cast<int32_t*>(smem + L.sums)[c] = sv[i];
                reinterpret_cast<float*>(smem + L.scales)[c] = dv[i];
            }
        }
    }

    GvLane ln;
    ln.lane = lane;
#pragma unroll
    for (int i = 0; i < GV_PIECES; i++) ln.off[i] = 16u * (uint32_t)(lane + 64 * i);
    uint8_t* wb = smem + L.wbuf + (size_t)wave * GV_STEP_BYTES;
    const int j = lane & 3;
    const uint8_t* wl = TY == KF_TYPE_Q4_K ? wb + (lane >> 2) * KF_Q4_K_BYTES : wb + 34 * lane;
    const uint4* xl = reinterpret_cast<const uint4*>(smem) + lane + ((sp * (TY == KF_TYPE_Q4_K ? 4 : 2)) << 6);
    const int32_t* ss = reinterpret_cast<const int32_t*>(smem + L.sums);
    const float* sd = reinterpret_cast<const float*>(smem + L.scales);
    const int blk = sp * PER_STEP + (TY == KF_TYPE_Q4_K ? (lane >> 2) : lane);
    float* part = reinterpret_cast<float*>(smem + L.part);
    // the row group of iteration it: with one wave a row the grid sweeps the matrix (iteration it of every block is a
    // contiguous stretch), with split rows each block walks a contiguous range of its own (MI355X, q4_K down 14336 x
    // 4096: 7.42-7.47 against 7.56-7.59 us; gate+up at one wave a row 13.5 against 13.2-13.3 the other way)
    auto grp = [&](int it) { return WPR > 1 ? (int)blockIdx.x * iters + it : it * B + (int)blockIdx.x; };
    // iterations whose row exists for this wave; loads past them reload the wave's own last row (spread over the
    // chip, unlike a clamp to the matrix's last row, which would send every such wave to the same cache lines)
    int iw = iters;
    while (iw > 0 && grp(iw - 1) * RPB + rg >= n_out) iw--;
    if (iw == 0) iw = 1;  // a wave without rows still runs the barrier; it reloads row rg of the block's first group
    auto row_ptr = [&](int it) {
        const int o = min(grp(min(it, iw - 1)) * RPB + rg, n_out - 1);
        return gv_row_ptr(sg, w, row_bytes, o) + at;
    };
    // the wave's activation operands are the same for every row it walks (its step is fixed): read once from LDS,
    // after the barrier that publishes them
    uint4 xa4[4];
    int2 xbs = make_int2(0, 0);
    float xdx = 0.0f;
    auto load_act = [&]() {
        const int bb = min(blk, nblk - 1);
        if constexpr (TY == KF_TYPE_Q4_K) {
#pragma unroll
            for (int k = 0; k < 4; k++) xa4[k] = xl[64 * k];
            xbs = *reinterpret_cast<const int2*>(ss + bb * 8 + 2 * j);
            xdx = sd[bb * 8];
        } else {
            xa4[0] = xl[0];
            xa4[1] = xl[64];
            xa4[2] = xa4[3] = make_uint4(0u, 0u, 0u, 0u);
            xdx = sd[bb];
        }
    };
    uint4 ring[D][GV_PIECES];
    // Two schedules, both measured (one A/B session, us a launch):
    //   * split rows (WPR > 1): every load of the ring is unconditional, so the compiler's wait counts are exact and D
    //     rows stay in flight (a load skipped on some path makes the waits hold, on every path, for the fewest loads
    //     in flight). Rows past the wave's own read the activation row instead (small and cache-resident: no HBM
    //     traffic, never stored). Down: 7.6 against 7.8;
    //   * one wave a row: loads past the wave's rows are skipped and the store reads bias and residual itself; the
    //     compiler then waits at the store for every load in flight and, at the second row of the ring, for the row
    //     just requested, so a wave alternates between one row and none in flight. That measured faster than exact
    //     waits with two rows in flight (gate+up 13.1 against 13.6, QKV 5.0 against 5.05, O 4.2 against 4.26) and
    //     than exactly one row in flight behind an explicit wait (15.2).
    const uint8_t* spare = QX > 0 ? reinterpret_cast<const uint8_t*>(xf) : reinterpret_cast<const uint8_t*>(xq);
    const int spare_len = QX > 0 ? 4 * n : n;
    auto load_row = [&](int k, int it2) {
        if constexpr (WPR == 1) {
            if (it2 < iw) gv_load_step<TY>(ring[k], row_ptr(it2), len, ln);
        } else {
            const bool own = it2 < iw;
            gv_load_step<TY>(ring[k], own ? row_ptr(it2) : spare, own ? len : spare_len, ln);
        }
    };
    auto process = [&](const uint4* v, int it) {
        if (!(KF_GV_ABLATE & 4)) gv_park<TY>(wb, v, len, ln);
        __builtin_amdgcn_wave_barrier();
        float acc = 0.0f;
        if (KF_GV_ABLATE & 2) {
            acc = (KF_GV_ABLATE & 4) ? (float)(v[0].x ^ v[1].y ^ v[2].z) : (float)(*reinterpret_cast<const uint32_t*>(wl) ^ xl[0].x);
        } else if (has_step && blk < nblk) {
            if constexpr (TY == KF_TYPE_Q4_K)
                acc = gv_q4k_lane_r(wl, xa4[0], xa4[1], xa4[2], xa4[3], xbs, xdx, j);
            else
                acc = gv_q8_0_lane_r(wl, xa4[0], xa4[1], xdx);
        }
        __builtin_amdgcn_wave_barrier();
        acc = kf_wave_sum_dpp(acc);
        const int o = grp(it) * RPB + rg;
        if (lane == 0 && o < n_out) {
            if constexpr (WPR == 1)
                gv_store(sg, y, bias, res, o, acc);
            else
                part[it * GV_WAVES + wave] = acc;
        }
    };

    // the first D rows' weights go out before the block waits on its activation row; vmcnt counts loads in issue
    // order, so waiting until only those weight loads are outstanding means the activation loads have landed
#pragma unroll
    for (int k = 0; k < D; k++) {
        if constexpr (WPR == 1)
            gv_load_step<TY>(ring[k], row_ptr(k), len, ln);  // rows past the wave's own reload its last row
        else
            load_row(k, k);
    }
    if constexpr (QX > 0) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NM) {
            __shared__ double norm_part[GV_WAVES];
            gv_xf_norm<QX>(xr, norm_part, n, wave, lane, nm.eps);
        }
        gv_xf_quant<TY, QX>(smem, L.sums, L.scales, xr, n, wave, lane);
    }
    // the activation stores are LDS writes of this block only: waiting on lgkmcnt and a bare barrier order them
    // (__syncthreads would add a release fence that waits on the weight loads as well)
    __builtin_amdgcn_s_waitcnt(KF_WAITCNT_VM(63) & ~(15 << 8));
    __builtin_amdgcn_s_barrier();
    load_act();
    KF_GV_STAMP(1)
    // a ring of D rows in flight: row it is multiplied while rows it+1 .. it+D-1 stream, then its registers take row
    // it+D
    int it = 0;
    for (; it + D < iters; it += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            process(ring[k], it + k);
            load_row(k, it + k + D);
        }
    }
    KF_GV_STAMP(2)
#pragma unroll
    for (int k = 0; k < D; k++)
        if (it + k < iters) process(ring[k], it + k);
    KF_GV_STAMP(3)

    if (WPR > 1) {
        __syncthreads();
        for (int t = threadIdx.x; t < iters * RPB; t += GV_THREADS) {
            const int it2 = t / RPB, g = t % RPB;
            const int o = grp(it2) * RPB + g;
            if (o >= n_out) continue;
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < WPR; q++) acc += part[it2 * GV_WAVES + g * WPR + q];
            gv_store(sg, y, bias, res, o, acc);
        }
    }
}

// ------------------------------------------------------------------------------------------------ burst variant
// Every wave requests all R of its rows at launch (the pattern of the streaming-read probe, which reaches the chip's
// read rate: 10.4 us over the 66 MB gate+up rotation, one-shot) and multiplies them in order as they land. No block
// barrier: each lane loads its own activation operands (its four 16-byte pieces, two sub-block sums and a scale, or a
// q8_0 block's two pieces and scale) straight from global memory, where every block reads the same small row. A row
// travels as two 16-byte pieces and one dword a lane (2304 bytes: 1 KB, 1 KB and 256 B a wave instruction; q8_0's
// 2176-byte step the same with lanes past 32 reading a duplicate dword) and is parked in the wave's LDS buffer for the
// per-block lanes. Every load is unconditional (rows past the wave's own, absent bias and residual values read the
// activation row instead), so the compiler's wait before a row counts exactly the loads behind it.
template <uint32_t TY, int WPR, int R>
__global__ void __launch_bounds__(GV_THREADS) gemv_burst_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                                                const int32_t* __restrict__ xs32, const float* __restrict__ xd32,
                                                                const float* __restrict__ bias, const float* __restrict__ res,
                                                                float* __restrict__ y, int n, int n_out, int iters, const KfSegs sg,
                                                                const float* __restrict__, const GvNorm) {
    constexpr int RPB = GV_WAVES / WPR;
    constexpr int STEP = TY == KF_TYPE_Q4_K ? 2304 : 2176;
    constexpr int PER_STEP = TY == KF_TYPE_Q4_K ? 16 : 64;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = wave / WPR, sp = wave % WPR;
    const int nblk = TY == KF_TYPE_Q4_K ? n >> 8 : n >> 5;
    const int B = gridDim.x;
    const int steps = TY == KF_TYPE_Q4_K ? (nblk + 15) / 16 : (nblk + 63) / 64;
    const int64_t at = (int64_t)min(sp, steps - 1) * STEP;  // the wave's step of every row
    const int len = (int)min((int64_t)STEP, row_bytes - at);
    const bool has_step = sp < steps;
    const int j = lane & 3;
    const int blk = sp * PER_STEP + (TY == KF_TYPE_Q4_K ? (lane >> 2) : lane);
    const int bb = min(blk, nblk - 1);
    uint8_t* wb = smem + (size_t)wave * GV_STEP_BYTES;
    const uint8_t* wl = TY == KF_TYPE_Q4_K ? wb + (lane >> 2) * KF_Q4_K_BYTES : wb + 34 * lane;
    float* part = reinterpret_cast<float*>(smem + (size_t)GV_WAVES * GV_STEP_BYTES);
    int iw = iters;  // iterations whose row exists for this wave
    while (iw > 0 && ((iw - 1) * B + (int)blockIdx.x) * RPB + rg >= n_out) iw--;
    const uint8_t* spare = reinterpret_cast<const uint8_t*>(xq);

    // 1. the lane's activation operands, then the rows' bias and residual values
    uint4 xa4[4];
    int2 xbs = make_int2(0, 0);
    float xdx;
    if (KF_GV_ABLATE & 8) {
        xa4[0] = xa4[1] = xa4[2] = xa4[3] = make_uint4(lane, 1u, 2u, 3u);
        xdx = 1.0f;
    } else if constexpr (TY == KF_TYPE_Q4_K) {
        const uint4* xp = reinterpret_cast<const uint4*>(xq + (size_t)bb * 256 + 64 * j);
#pragma unroll
        for (int k = 0; k < 4; k++) xa4[k] = xp[k];
        xbs = *reinterpret_cast<const int2*>(xs32 + bb * 8 + 2 * j);
        xdx = xd32[bb * 8];
    } else {
        const uint4* xp = reinterpret_cast<const uint4*>(xq + (size_t)bb * 32);
        xa4[0] = xp[0];
        xa4[1] = xp[1];
        xa4[2] = xa4[3] = make_uint4(0u, 0u, 0u, 0u);
        xdx = xd32[bb];
    }
    auto row_of = [&](int it) { return min((min(it, max(iw, 1) - 1) * B + (int)blockIdx.x) * RPB + rg, n_out - 1); };
    float rb[R], rr[R];
    if constexpr (WPR == 1) {
#pragma unroll
        for (int it = 0; it < R; it++) {
            const GvRow r = gv_row(sg, nullptr, y, bias, res, row_of(it));
            rb[it] = *(r.bias ? r.bias + r.o : reinterpret_cast<const float*>(spare));
            rr[it] = *(r.res ? r.res + r.o : reinterpret_cast<const float*>(spare));
        }
    }
    // 2. every row of the wave
    uint4 va[R], vb[R];
    uint32_t vc[R];
    const uint32_t oa = min(16u * (uint32_t)lane, (uint32_t)len - 16u), ob = min(1024u + 16u * (uint32_t)lane, (uint32_t)len - 16u);
    const uint32_t oc = min(2048u + 4u * (uint32_t)lane, (uint32_t)len - 4u);
#pragma unroll
    for (int it = 0; it < R; it++) {
        const bool own = it < iw;
        const uint8_t* src = own ? gv_row_ptr(sg, w, row_bytes, row_of(it)) + at : spare;
        const uint32_t cap = own ? 0xffffffffu : (uint32_t)n - 16u;  // the activation row holds n bytes
        if constexpr (TY == KF_TYPE_Q4_K) {
            va[it] = kf_load_stream_u4(src + min(oa, cap));
            vb[it] = kf_load_stream_u4(src + min(ob, cap));
        } else {
            va[it] = kf_load_stream_u4_unaligned(src + min(oa, cap));
            vb[it] = kf_load_stream_u4_unaligned(src + min(ob, cap));
        }
        vc[it] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src + min(oc, cap)));
    }
    // 3. the rows in order as they land
#pragma unroll
    for (int it = 0; it < R; it++) {
        if (it < iters) {
            if (!(KF_GV_ABLATE & 4)) {
                *reinterpret_cast<uint4*>(wb + oa) = va[it];
                *reinterpret_cast<uint4*>(wb + ob) = vb[it];
                *reinterpret_cast<uint32_t*>(wb + oc) = vc[it];
            }
            __builtin_amdgcn_wave_barrier();
            float acc = 0.0f;
            if (KF_GV_ABLATE & 2) {
                acc = (KF_GV_ABLATE & 4) ? (float)(va[it].x ^ vb[it].y ^ vc[it]) : (float)(*reinterpret_cast<const uint32_t*>(wl) ^ xa4[0].x);
            } else if (has_step && blk < nblk) {
                if constexpr (TY == KF_TYPE_Q4_K)
                    acc = gv_q4k_lane_r(wl, xa4[0], xa4[1], xa4[2], xa4[3], xbs, xdx, j);
                else
                    acc = gv_q8_0_lane_r(wl, xa4[0], xa4[1], xdx);
            }
            __builtin_amdgcn_wave_barrier();
            acc = kf_wave_sum_dpp(acc);
            const int o = (it * B + (int)blockIdx.x) * RPB + rg;
            if (lane == 0 && o < n_out) {
                if constexpr (WPR == 1) {
                    const GvRow r = gv_row(sg, nullptr, y, bias, res, o);
                    r.y[r.o] = acc + (r.bias ? rb[it] : 0.0f) + (r.res ? rr[it] : 0.0f);
                } else {
                    part[it * GV_WAVES + wave] = acc;
                }
            }
        }
    }
    if constexpr (WPR > 1) {
        __syncthreads();
        for (int t = threadIdx.x; t < iters * RPB; t += GV_THREADS) {
            const int it2 = t / RPB, g = t % RPB;
            const int o = (it2 * B + (int)blockIdx.x) * RPB + g;
            if (o >= n_out) continue;
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < WPR; q++) acc += part[it2 * GV_WAVES + g * WPR + q];
            gv_store(sg, y, bias, res, o, acc);
        }
    }
}

// The unit loads of the per-block integer check: a q8_0 block read as its f16 scale and two unaligned 16-byte loads
struct Q8Unit {
    uint32_t dbits;
    uint4 q0, q1;

    __device__ __forceinline__ void load(const uint8_t* row, int b) {
        const uint8_t* blk = row + (int64_t)b * KF_Q8_0_BYTES;
        dbits = *reinterpret_cast<const uint16_t*>(blk);
        q0 = kf_load_stream_u4_unaligned(blk + 2);
        q1 = kf_load_stream_u4_unaligned(blk + 18);
    }
};

// Per-block integers of weight rows against activation rows, one thread per (weight row, activation row, block):
// q8_0 one int32 per 32-block, q4_K and q5_K (sumi, mins) per super-block, q6_K one int32 per super-block (dot minus
// the 32-offset bias). The check that pins the products' lane arithmetic.
__global__ void block_ints_kernel(uint32_t ty, const uint8_t* __restrict__ w, int64_t row_bytes, const int8_t* __restrict__ xq,
                                  const int32_t* __restrict__ xs16, const int32_t* __restrict__ xs32, int n, int n_out, int rows,
                                  int32_t* __restrict__ out) {
    const int per = ty == KF_TYPE_Q8_0 ? n / 32 : n / 256;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)n_out * rows * per) return;
    const int b = (int)(t % per);
    const int r = (int)((t / per) % rows);
    const int o = (int)(t / ((int64_t)per * rows));
    const uint8_t* row = w + (int64_t)o * row_bytes;
    const int8_t* x = xq + (int64_t)r * n;
    if (ty == KF_TYPE_Q6_K) {  // one int32 per super-block: the four lane units' sum
        const uint8_t* blk = row + (int64_t)b * KF_Q6_K_BYTES;
        int tot = 0;
        for (int j = 0; j < 4; j++) {
            KfQ6Lane u;
            u.load(blk, j);
            tot += u.dot(x + b * 256, xs16 + (int64_t)r * (n / 16) + b * 16, j);
        }
        out[t] = tot;
        return;
    }
    if (ty == KF_TYPE_Q5_K) {  // (sumi, mins) per super-block, as q4_K
        const uint8_t* blk = row + (int64_t)b * KF_Q5_K_BYTES;
        int sumi = 0, mins = 0;
        for (int j = 0; j < 4; j++) {
            KfQ5Lane u;
            u.load(blk, j);
            int isum, imin;
            u.dot(x + b * 256, xs32 + (int64_t)r * (n / 32) + b * 8, j, isum, imin);
            sumi += isum;
            mins += imin;
        }
        out[2 * t] = sumi;
        out[2 * t + 1] = mins;
        return;
    }
    if (ty == KF_TYPE_Q8_0) {
        Q8Unit u;
        u.load(row, b);
        const uint32_t wq[8] = {u.q0.x, u.q0.y, u.q0.z, u.q0.w, u.q1.x, u.q1.y, u.q1.z, u.q1.w};
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

// Compute units of the first device the process launches on (thread-safe static; the build targets one device model)
int cu_count() {
    static const int n = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = 256;
        return v;
    }();
    return n;
}

typedef void (*GvKernel)(const uint8_t*, int64_t, const int8_t*, const int32_t*, const float*, const float*, const float*, float*, int, int, int, const KfSegs,
                         const float*, const GvNorm);

// Most blocks of one kernel resident per CU at a dynamic LDS size, cached per (kernel, LDS)
int resident_blocks(GvKernel k, size_t smem) {
    struct Entry {
        GvKernel k;
        size_t smem;
        int v;
    };
    static std::mutex mu;  // launchers may run on several threads (one per stream)
    static Entry cache[64];
    static int used = 0;
    std::lock_guard<std::mutex> g(mu);
    for (int i = 0; i < used; i++)
        if (cache[i].k == k && cache[i].smem == smem) return cache[i].v;
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, reinterpret_cast<const void*>(k), GV_THREADS, smem) != hipSuccess || v < 1) v = 1;
    if (used < 64) cache[used++] = Entry{k, smem, v};
    return v;
}

// The fused variants of one (type, waves a row) for QX f32 chunks a wave (1, 2, 4 or 8): always the pipelined kernel,
// whose weights travel through registers, so the compiler waits on the activation loads alone (with the one-shot
// kernel's LDS DMA in flight it waits on everything before the quantization)
template <uint32_t TY, int WPR>
GvKernel gv_fused_pipe(int qx, bool norm) {
    switch (qx + (norm ? 2 : 0)) {
        case 1: return gemv_pipe_kernel<TY, WPR, KF_GV_DEPTH, 1>;
        case 2: return gemv_pipe_kernel<TY, WPR, KF_GV_DEPTH, 2>;
        case 3: return gemv_pipe_kernel<TY, WPR, KF_GV_DEPTH, 1, 1>;
        case 4: return gemv_pipe_kernel<TY, WPR, KF_GV_DEPTH, 2, 1>;
    }
    return nullptr;
}

// xf non-null: the fused variants, quantizing the f32 row xf themselves (qx chunks a wave); hipErrorNotSupported when
// neither fits (the caller then quantizes first)
template <uint32_t TY, int SPW, int WPR>
hipError_t launch_gemv(const uint8_t* w, int64_t row_bytes, const int8_t* xq, const int32_t* xs32, const float* xd32, const float* bias,
                       const float* res, float* y, int n, int n_out, int maxit_env, const KfSegs& sg, hipStream_t s, const float* xf = nullptr,
                       int qx = 0, const GvNorm* norm = nullptr) {
    const GvNorm nm = norm ? *norm : GvNorm{nullptr, nullptr, 0.0f};
    constexpr int RPB = GV_WAVES / WPR;
    const int groups = (n_out + RPB - 1) / RPB;
    const bool fused = xf != nullptr;
    // row iterations per block: enough blocks that the chip is full, each block's waves holding the loads of all
    // their rows at once
    const int want = maxit_env > 0 ? maxit_env : KF_GV_MAXIT;
    // the DMA variant needs 16-byte aligned rows and activation pieces
    const bool dma = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(fused ? static_cast<const void*>(xf) : xq) & 15) == 0 && !kf_knob_on(KF_KNOB_GEMV_NO_DMA);
    if (fused && (SPW != 1 || !dma)) return hipErrorNotSupported;
    // one-shot waves, each fetching its row straight into LDS, the whole matrix requested at launch (KF_GEMV_ONESHOT=1,
    // a comparison knob: one row a wave and every block resident at once). The persistent variant below measured
    // faster on q4_K QKV and O (5.34 / 4.25 us against 5.44 / 4.71) and level on q8_0, so it takes them too
    if (!fused && SPW == 1 && WPR == 1 && dma && maxit_env == 0 && kf_knob_on(KF_KNOB_GEMV_ONESHOT)) {
        const size_t smem = gd_lds(TY, n, 1, WPR, 1, 1).total;
        GvKernel k = gemv_dma_kernel<TY, 1, WPR, 1>;
        if (groups <= cu_count() * resident_blocks(k, smem) && smem <= 65536) {
            k<<<groups, GV_THREADS, smem, s>>>(w, row_bytes, xq, xs32, xd32, bias, res, y, n, n_out, 1, sg, xf, nm);
            return hipGetLastError();
        }
    }
    // the burst variant where every wave has one row, in a grid of at most four blocks a CU (O at 4096 x 4096, two
    // blocks a CU: 3.9 against 4.2 us for the pipelined kernel, which waits for its block's activation row first;
    // QKV at 4096 x 6144, three blocks a CU: 4.65 against 4.95; q8_0 at 4096 x 4096, two waves a row, four blocks a
    // CU: 5.04 against 5.11). With more rows a wave it measured slower than the pipelined kernel (gate+up, 7 rows a
    // wave: 14.4 against 13.1 us; 12.6 even without the arithmetic), so it takes one-row grids only;
    // KF_GEMV_BURST=n forces it up to n rows a wave (1, 2, 4, 7, 8) on a grid of two blocks a CU
    const int burst_rows = kf_knob_on(KF_KNOB_GEMV_BURST) ? kf_knob(KF_KNOB_GEMV_BURST) : 1;
    if (!fused && SPW == 1 && dma && maxit_env == 0 && !kf_knob_on(KF_KNOB_GEMV_NO_PIPE)) {
        const int bpc = kf_knob(KF_KNOB_GEMV_BPC);
        int grid = cu_count() * (bpc > 0 ? bpc : 2);
        if (!kf_knob_on(KF_KNOB_GEMV_BURST) && bpc <= 0 && groups <= 4 * cu_count()) grid = groups;  // one row a wave
        if (grid > groups) grid = groups;
        const int iters = (groups + grid - 1) / grid;
        const size_t smem = (size_t)GV_WAVES * GV_STEP_BYTES + (WPR > 1 ? (size_t)iters * GV_WAVES * 4 : 0);
        GvKernel k = iters > burst_rows ? nullptr
                     : iters == 1 ? gemv_burst_kernel<TY, WPR, 1>
                     : iters == 2 ? gemv_burst_kernel<TY, WPR, 2>
                     : iters <= 4 ? gemv_burst_kernel<TY, WPR, 4>
                     : iters == 7 ? gemv_burst_kernel<TY, WPR, 7>
                     : iters <= 8 ? gemv_burst_kernel<TY, WPR, 8>
                                  : nullptr;
        if (k && (int64_t)n <= 16 * 1024 * 1024) {
            k<<<grid, GV_THREADS, smem, s>>>(w, row_bytes, xq, xs32, xd32, bias, res, y, n, n_out, iters, sg, nullptr, nm);
            return hipGetLastError();
        }
    }
    // the pipelined persistent variant: a resident grid, every wave walking its rows two in flight
    if (SPW == 1 && dma && (fused || !kf_knob_on(KF_KNOB_GEMV_NO_PIPE))) {
        const int dv = kf_knob(KF_KNOB_GEMV_DEPTH);
        const int depth = dv >= 2 && dv <= 4 ? dv : KF_GV_DEPTH;
        GvKernel k = fused ? gv_fused_pipe<TY, WPR>(qx, norm != nullptr)
                           : depth == 4 ? gemv_pipe_kernel<TY, WPR, 4> : depth == 3 ? gemv_pipe_kernel<TY, WPR, 3> : gemv_pipe_kernel<TY, WPR, 2>;
        const size_t base_lds = gd_lds(TY, n, 0, WPR, 1, 1).total;
        // two blocks (16 waves) per CU measured best on MI355X (3.9-4.1 TB/s at 33 MB against 3.2-3.5 with every
        // resident slot filled, where waves contend for the memory pipe); KF_GEMV_BPC overrides it
        const int bpc = kf_knob(KF_KNOB_GEMV_BPC);
        const int per_cu = bpc > 0 ? bpc : std::min(2, resident_blocks(k, base_lds + (WPR > 1 ? 2048 : 0)));
        int grid = cu_count() * per_cu;
        if (grid > groups) grid = groups;
        const int iters = (groups + grid - 1) / grid;
        const size_t smem = gd_lds(TY, n, iters, WPR, 1, 1).total;
        if (k && smem <= 65536) {
            k<<<grid, GV_THREADS, smem, s>>>(w, row_bytes, xq, xs32, xd32, bias, res, y, n, n_out, iters, sg, xf, nm);
            return hipGetLastError();
        }
    }
    if (fused) return hipErrorNotSupported;
#define KF_GV_IT(M)                                                                                                      \
    if (want <= M) {                                                                                                     \
        const int grid = (groups + M - 1) / M;                                                                           \
        const int iters = (groups + grid - 1) / grid;                                                                    \
        if (dma && gd_lds(TY, n, iters, WPR, M, SPW).total <= 65536) {                                                   \
            const size_t smem = gd_lds(TY, n, iters, WPR, M, SPW).total;                                                 \
            gemv_dma_kernel<TY, SPW, WPR, M><<<grid, GV_THREADS, smem, s>>>(w, row_bytes, xq, xs32, xd32, bias, res, y, n, n_out, iters, sg, nullptr, nm); \
        } else {                                                                                                         \
            const size_t smem = gv_lds(TY, n, iters, WPR).total;                                                         \
            gemv_kernel<TY, SPW, WPR, M><<<grid, GV_THREADS, smem, s>>>(w, row_bytes, xq, xs32, xd32, bias, res, y, n, n_out, iters, sg, nullptr, nm); \
        }                                                                                                                \
        return hipGetLastError();                                                                                        \
    }
    KF_GV_IT(1)
    KF_GV_IT(2)
    KF_GV_IT(4)
#undef KF_GV_IT
    return hipErrorInvalidValue;
}

// Waves per row for a row of `steps` wave steps: the smallest power of two covering the steps, at most GV_WAVES
int gv_wpr(int steps) {
    int wpr = 1;
    while (wpr < steps && wpr < GV_WAVES) wpr *= 2;
    return wpr;
}

}  // namespace

#ifdef KF_GV_TRACE
extern "C" int kf_gv_set_trace(void* p) { return hipMemcpyToSymbol(HIP_SYMBOL(kf_gv_trace), &p, sizeof(p)) == hipSuccess ? 0 : -1; }
#endif

// Largest row width the single-row GEMV stages in LDS
int kf_gemv_max_n() { return 32768; }

// Host launcher for one activation row, validated by the caller (api.cpp): n a multiple of the type's block,
// n <= kf_gemv_max_n(). xq / xs32 / xd32 point at the row's int8 values, per-32 sums and per-32 scales. With segs
// non-null the n_out rows are the members' rows stacked (KfSegs) and w / y / bias / res are unused.
hipError_t kf_launch_gemv1(uint32_t ty, const void* wv, int64_t row_bytes, const int8_t* xq, const int32_t* xs32, const float* xd32,
                           const float* bias, const float* res, float* y, int n, int n_out, int maxit, const KfSegs* segs, hipStream_t s) {
    if (n_out == 0) return hipSuccess;
    KfSegs sg{};
    if (segs) sg = *segs;
    const uint8_t* w = static_cast<const uint8_t*>(wv);
    const int steps = ty == KF_TYPE_Q4_K ? (n / 256 + 15) / 16 : (n / 32 + 63) / 64;
    const int wpr = gv_wpr(steps);
    const int spw = (steps + wpr - 1) / wpr;
#define KF_GV(TY, SPW, WPR)                                                                                      \
    if (ty == TY && spw == SPW && wpr == WPR)                                                                    \
        return launch_gemv<TY, SPW, WPR>(w, row_bytes, xq, xs32, xd32, bias, res, y, n, n_out, maxit, sg, s);
    KF_GV(KF_TYPE_Q4_K, 1, 1)
    KF_GV(KF_TYPE_Q4_K, 1, 2)
    KF_GV(KF_TYPE_Q4_K, 1, 4)
    KF_GV(KF_TYPE_Q4_K, 1, 8)
    KF_GV(KF_TYPE_Q8_0, 1, 1)
    KF_GV(KF_TYPE_Q8_0, 1, 2)
    KF_GV(KF_TYPE_Q8_0, 1, 4)
    KF_GV(KF_TYPE_Q8_0, 1, 8)
    KF_GV(KF_TYPE_Q8_0, 2, 8)
#undef KF_GV
    return hipErrorInvalidValue;
}

// Largest row width the fused single-row GEMV quantizes itself: two 256-column chunks a wave. Every block quantizes
// the whole row (its waves multiply whole rows), so the quantization's VALU work is repeated in all 512 blocks; at two
// chunks a wave it hides under the first weight requests (4096 columns: 1.0 us saved against quant_act + GEMV), at
// seven (14336 columns) it measured 5.5 us slower than the two launches.
int kf_gemv_fused_max_n() { return 2 * GV_WAVES * 256; }

// The single-row GEMV quantizing its f32 activation row x itself (one launch in place of quant_act + GEMV; the same
// integers and scales, so the same outputs bit for bit). hipErrorNotSupported when no fused variant fits (n above
// kf_gemv_fused_max_n, rows or x not 16-byte aligned, a type other than q8_0 / q4_K): the caller quantizes first.
hipError_t kf_launch_gemv1_fused(uint32_t ty, const void* wv, int64_t row_bytes, const float* x, const float* bias, const float* res, float* y,
                                 int n, int n_out, const KfSegs* segs, hipStream_t s, const float* norm_w, const float* norm_b, float norm_eps,
                                 bool norm) {
    const GvNorm nmv{norm_w, norm_b, norm_eps};
    if (n_out == 0) return hipSuccess;
    if (n > kf_gemv_fused_max_n() || n % 4 != 0 || (ty != KF_TYPE_Q4_K && ty != KF_TYPE_Q8_0)) return hipErrorNotSupported;
    KfSegs sg{};
    if (segs) sg = *segs;
    const uint8_t* w = static_cast<const uint8_t*>(wv);
    const int steps = ty == KF_TYPE_Q4_K ? (n / 256 + 15) / 16 : (n / 32 + 63) / 64;
    const int wpr = gv_wpr(steps);
    const int spw = (steps + wpr - 1) / wpr;
    const int per_wave = ((n + 255) / 256 + GV_WAVES - 1) / GV_WAVES;
    const int qx = per_wave <= 1 ? 1 : 2;
#define KF_GVF(TY, WPR)                                                                                                    \
    if (ty == TY && spw == 1 && wpr == WPR)                                                                               \
        return launch_gemv<TY, 1, WPR>(w, row_bytes, nullptr, nullptr, nullptr, bias, res, y, n, n_out, 0, sg, s, x, qx, norm ? &nmv : nullptr);
    KF_GVF(KF_TYPE_Q4_K, 1)
    KF_GVF(KF_TYPE_Q4_K, 2)
    KF_GVF(KF_TYPE_Q4_K, 4)
    KF_GVF(KF_TYPE_Q4_K, 8)
    KF_GVF(KF_TYPE_Q8_0, 1)
    KF_GVF(KF_TYPE_Q8_0, 2)
    KF_GVF(KF_TYPE_Q8_0, 4)
    KF_GVF(KF_TYPE_Q8_0, 8)
#undef KF_GVF
    return hipErrorNotSupported;
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
        reinterpret_cast<const int32_t*>(base + off.s16), reinterpret_cast<const int32_t*>(base + off.s32), n, n_out, rows, out);
    return hipGetLastError();
}
