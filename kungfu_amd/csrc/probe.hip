// Streaming-read probe: the HBM read rate this box reaches with plain 16-byte loads, the measured peak that the
// benchmark reports beside the 8 TB/s spec peak (and, over the same bytes as a product launch, that launch's ceiling).
// No reference counterpart.
//
// One-shot grid: thread t of block b reads P consecutive-stride 16-byte pieces, ((b P + i) 256 + t) 16 for i < P, so
// every wave load instruction reads 1 KB of consecutive bytes and the whole buffer is requested at launch; the pieces
// are XOR-reduced and a lane writes its value only if it equals a key no data produces in practice, so the loads
// cannot be removed and the kernel writes (almost) nothing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kf_device.h"

namespace {

constexpr int PR_THREADS = 256;

template <int P>
__global__ void __launch_bounds__(PR_THREADS) stream_read_kernel(const uint4* __restrict__ buf, size_t pieces, uint32_t key,
                                                                 uint32_t* __restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * P * PR_THREADS + threadIdx.x;
    uint4 v[P];
#pragma unroll
    for (int i = 0; i < P; i++) {
        const size_t c = base + (size_t)i * PR_THREADS;
        v[i] = c < pieces ? kf_load_stream_u4(buf + c) : make_uint4(0, 0, 0, 0);
    }
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < P; i++) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (x == key) sink[0] = x;
}

}  // namespace

// Host launcher, validated by the caller: buf 16-byte aligned, bytes a multiple of 16, P in {4, 8, 16}
hipError_t kf_launch_stream_read(const void* buf, size_t bytes, int per_thread, uint32_t* sink, hipStream_t s) {
    const size_t pieces = bytes / 16;
    const size_t span = (size_t)per_thread * PR_THREADS;
    const unsigned blocks = (unsigned)((pieces + span - 1) / span);
    const auto* b = static_cast<const uint4*>(buf);
    const uint32_t key = 0x9e3779b9u;
    if (per_thread == 4)
        stream_read_kernel<4><<<blocks, PR_THREADS, 0, s>>>(b, pieces, key, sink);
    else if (per_thread == 16)
        stream_read_kernel<16><<<blocks, PR_THREADS, 0, s>>>(b, pieces, key, sink);
    else
        stream_read_kernel<8><<<blocks, PR_THREADS, 0, s>>>(b, pieces, key, sink);
    return hipGetLastError();
}
