// Host-side helpers shared by the launchers.
#pragma once
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>

// Raises a kernel's dynamic LDS limit on the current device to at least `bytes`. Launchers call it before every launch
// that needs more than the default 64 KB; the highest value set per (kernel, device) is remembered under a lock, so
// concurrent callers (one thread per stream) never lower a limit another launch relies on.
inline hipError_t kf_raise_lds(const void* fn, int bytes) {
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, int> set;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    std::lock_guard<std::mutex> g(mu);
    int& cur = set[{fn, dev}];
    if (cur >= bytes) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) cur = bytes;
    return e;
}

// Compute units of the current device, read once per device and remembered under a lock (256 if the query fails).
inline int kf_cu_count() {
    static std::mutex mu;
    static std::map<int, int> cus;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> g(mu);
    auto it = cus.find(dev);
    if (it != cus.end()) return it->second;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = 256;
    cus[dev] = v;
    return v;
}

// Device scratch of the split-K products (the few-row q8_0 split-K product, the tile GEMMs' tail splits): a static
// __device__ array of KF_SPLIT_SLOTS slots of KF_SPLIT_SCRATCH bytes per GPU (zero at load, never allocated). Slots
// 0 .. KF_SPLIT_STREAM_SLOTS - 1 go to (device, stream) pairs on first use and are held until kf_hip_release_stream;
// launches on one stream are ordered, so a slot is never used by two running products. The last slot belongs to
// products recorded under HIP graph capture (every captured product of a GPU shares it; direct launches never use
// it), so a replay never meets a direct product's tickets; two replays of graphs holding such products must not run
// at the same time. A slot starts with KF_SPLIT_TICKETS int32 tickets, which the kernels leave at zero when they end.
// Null (and the products take their scratch-free form) for a stream that finds every stream slot held by other
// streams, and under capture when KF_CAPTURE_NO_SPLIT is set.
constexpr size_t KF_SPLIT_SCRATCH = 40u << 20;
constexpr int KF_SPLIT_STREAM_SLOTS = 2;
constexpr int KF_SPLIT_SLOTS = KF_SPLIT_STREAM_SLOTS + 1;
constexpr int KF_SPLIT_TICKETS = 1 << 16;
void* kf_split_scratch(hipStream_t s);
