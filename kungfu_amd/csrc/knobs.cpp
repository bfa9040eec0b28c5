// The launchers' knob table: environment read once per process, changed afterwards only through kf_hip_set_knob.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "kf_hip.h"
#include "kf_knobs.h"

namespace {
struct KnobName {
    const char* name;
    bool flag;
};
constexpr KnobName kNames[KF_KNOB_COUNT] = {
    {"KF_GEMV_MAXIT", false},  {"KF_GEMV_NO_DMA", true},  {"KF_GEMV_ONESHOT", true}, {"KF_GEMV_NO_PIPE", true},
    {"KF_GEMV_DEPTH", false},  {"KF_GEMV_BPC", false},    {"KF_MATMUL_NO_FUSE", true}, {"KF_ROWS_VALU", true},
    {"KF_RM_NB", false},       {"KF_RM_WHOLE", false},    {"KF_RM1_TILES", false},   {"KF_Q4K_KQ", false},
    {"KF_KQ_GEMM", false},     {"KF_MOE_KQ", false},      {"KF_GEMM_NO_TAIL", true}, {"KF_GEMM_TILE", true},
    {"KF_GEMM_SLICE", false},  {"KF_GEMM_SK", false},     {"KF_GEMM_SK_S", false},   {"KF_GEMM_SK_V", false},
    {"KF_GEMM_NO_MR", true},   {"KF_GEMM_MR", false},     {"KF_GEMM_SMALL_W", false}, {"KF_GEMM_SMALL_TN", false},
    {"KF_CAPTURE_NO_SPLIT", true}, {"KF_GEMV_BURST", false},
};
std::atomic<int> g_knob[KF_KNOB_COUNT];
std::once_flag g_once;

void load_env() {
    for (int i = 0; i < KF_KNOB_COUNT; i++) {
        const char* e = std::getenv(kNames[i].name);  // the library's one environment read
        int v = -1;
        if (e) v = kNames[i].flag ? 1 : std::max(0, std::atoi(e));
        g_knob[i].store(v, std::memory_order_relaxed);
    }
}

int find(const char* name) {
    if (!name) return -1;
    for (int i = 0; i < KF_KNOB_COUNT; i++)
        if (std::strcmp(kNames[i].name, name) == 0) return i;
    return -1;
}
}  // namespace

int kf_knob(KfKnob k) {
    std::call_once(g_once, load_env);
    return g_knob[k].load(std::memory_order_relaxed);
}

extern "C" int kf_hip_set_knob(const char* name, int value) {
    std::call_once(g_once, load_env);
    const int i = find(name);
    if (i < 0) return KF_E_INVALID;
    g_knob[i].store(value < 0 ? -1 : value, std::memory_order_relaxed);
    return KF_OK;
}

extern "C" int kf_hip_get_knob(const char* name) {
    std::call_once(g_once, load_env);
    const int i = find(name);
    return i < 0 ? -2 : g_knob[i].load(std::memory_order_relaxed);
}
