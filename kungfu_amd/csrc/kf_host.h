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
