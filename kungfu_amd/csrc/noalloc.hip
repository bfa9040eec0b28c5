// kf_hip_matmul_noalloc: kf_hip_matmul for callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc). The activation scratch that kf_hip_matmul takes as an
// argument is instead a file-scope device array of KF_NOALLOC_SCRATCH_BYTES, one copy per GPU, held until the process
// ends. No reference counterpart.
//
// In host code the array's name is only a host-side stand-in, not a device address: every host use goes through the
// device address that hipGetSymbolAddress returns, looked up once per device (with that device current) on the
// device's first call and kept per device.
#include "kf_host.h"
#include "kf_knobs.h"
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/kf_hip.h"
#include "kf_layout.h"

void kf_set_error(const char* fmt, ...);

namespace {

static __device__ __align__(256) uint8_t scratch[KF_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// The device address of `scratch` on `dev` (looked up on first use), or nullptr with the error recorded
void* scratch_ptr(int dev) {
    static std::mutex mu;
    static void* ptr[kMaxDevices] = {};
    if (dev < 0 || dev >= kMaxDevices) {
        kf_set_error("device %d: at most %d devices", dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> g(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            kf_set_error("hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
            (void)hipGetLastError();  // the failure is reported here, not by the next launch's error check
            return nullptr;
        }
        ptr[dev] = p;
    }
    return ptr[dev];
}

}  // namespace

extern "C" size_t kf_hip_noalloc_scratch_bytes(void) { return KF_NOALLOC_SCRATCH_BYTES; }

extern "C" int kf_hip_matmul_noalloc(uint32_t ty, const void* w, int n_in, int n_out, const float* x, int rows, const float* bias,
                                     const float* res, float* y, void* stream) {
    if (rows < 0 || n_in <= 0) {
        kf_set_error("%d rows of %d columns", rows, n_in);
        return KF_E_INVALID;
    }
    const size_t need = kf_hip_act_bytes(rows, n_in);
    if (need > KF_NOALLOC_SCRATCH_BYTES) {
        kf_set_error("%d rows of %d columns need %zu bytes of activation scratch, the no-allocation entry point holds %zu", rows, n_in, need,
                     (size_t)KF_NOALLOC_SCRATCH_BYTES);
        return KF_E_INVALID;
    }
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        kf_set_error("hipGetDevice: %s", hipGetErrorString(e));
        return KF_E_HIP;
    }
    void* act = scratch_ptr(dev);
    if (!act) return KF_E_HIP;
    // quant_act writes every byte of the scratch that the product reads, so nothing is cleared between calls
    return kf_hip_matmul(ty, w, n_in, n_out, x, rows, act, bias, res, y, stream);
}

// ------------------------------------------------------------------------------------------------ split-K scratch
// The split-K products' partial tiles and tickets (kf_host.h): static, so nothing is allocated and the addresses never
// change. Each device has its own copy, found with hipGetSymbolAddress once per device. Stream slots go to (device,
// stream) pairs on first use and come back through kf_hip_release_stream. A stream under graph capture gets the
// graph slot instead: a captured graph keeps the address it recorded and may be replayed on any stream, so it must
// never share a slot with direct launches, which hold stream slots only.
static __device__ __align__(256) uint8_t split_scratch[KF_SPLIT_SLOTS * KF_SPLIT_SCRATCH];

namespace {
std::mutex g_split_mu;
std::map<int, uint8_t*> g_split_base;                       // per device
std::map<std::pair<int, hipStream_t>, int> g_split_slot;    // per (device, stream)
std::map<int, unsigned> g_split_free;                       // per device: bit i set when slot i is free
}  // namespace

void* kf_split_scratch(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (capturing && kf_knob_on(KF_KNOB_CAPTURE_NO_SPLIT)) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> g(g_split_mu);
    auto b = g_split_base.find(dev);
    if (b == g_split_base.end()) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(split_scratch)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return nullptr;
        }
        b = g_split_base.emplace(dev, static_cast<uint8_t*>(p)).first;
        g_split_free[dev] = (1u << KF_SPLIT_STREAM_SLOTS) - 1;
    }
    if (capturing) return b->second + (size_t)KF_SPLIT_STREAM_SLOTS * KF_SPLIT_SCRATCH;
    auto it = g_split_slot.find({dev, s});
    if (it == g_split_slot.end()) {
        unsigned& fr = g_split_free[dev];
        if (fr == 0) return nullptr;  // every slot held by another stream: the scratch-free form
        const int i = __builtin_ctz(fr);
        fr &= ~(1u << i);
        it = g_split_slot.emplace(std::make_pair(dev, s), i).first;
    }
    return b->second + (size_t)it->second * KF_SPLIT_SCRATCH;
}

extern "C" int kf_hip_release_stream(void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        kf_set_error("hipGetDevice: %s", hipGetErrorString(e));
        return KF_E_HIP;
    }
    std::lock_guard<std::mutex> g(g_split_mu);
    auto it = g_split_slot.find({dev, s});
    if (it == g_split_slot.end()) return KF_OK;
    // the slot is free only once the stream's products that use it have ended
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        kf_set_error("hipStreamSynchronize: %s", hipGetErrorString(e));
        return KF_E_HIP;
    }
    g_split_free[dev] |= 1u << it->second;
    g_split_slot.erase(it);
    return KF_OK;
}
