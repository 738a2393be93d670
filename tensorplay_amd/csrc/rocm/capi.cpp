// C-ABI plumbing shared by every entry point: thread-local last error,
// device facts, ABI version and the tuning hook.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <string>

#include "common.h"

namespace tpr {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int status, const std::string& msg) {
    g_last_error = msg;
    return status;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return fail(TPR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    }
    return TPR_OK;
}

DeviceInfo device_info() {
    // One atomic per device: 0 = not read yet.  Racing first callers each read
    // the attribute and store the same value, so no lock is needed.
    static constexpr int kMaxDev = 64;
    static std::atomic<int> cus_of[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) dev = 0;
    int cus = cus_of[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cus_of[dev].store(cus, std::memory_order_relaxed);
    }
    return DeviceInfo{cus};
}

DebugKnobs& knobs() {
    static DebugKnobs k;
    return k;
}

}  // namespace tpr

extern "C" {

const char* tpr_last_error(void) { return tpr::g_last_error.c_str(); }

int32_t tpr_abi_version(void) { return (1 << 16) | 4; }

int tpr_debug_set(const char* key, int64_t value) {
    if (!key) return tpr::fail(TPR_ERR_INVALID_ARG, "tpr_debug_set: null key");
    auto& k = tpr::knobs();
    if (!std::strcmp(key, "splits")) k.splits = value;
    else if (!std::strcmp(key, "lanes")) k.lanes = value;
    else if (!std::strcmp(key, "general")) k.general = value;
    else if (!std::strcmp(key, "topk_fallback")) k.topk_fallback = value;
    else if (!std::strcmp(key, "tx")) k.tx = value;
    else if (!std::strcmp(key, "topk_variant")) k.topk_variant = value;
    else if (!std::strcmp(key, "topk_waves")) k.topk_waves = value;
    else if (!std::strcmp(key, "unroll")) k.unroll = value;
    else if (!std::strcmp(key, "colblock")) k.colblock = value;
    else if (!std::strcmp(key, "nt")) k.nt = value;
    else if (!std::strcmp(key, "smx_two_pass")) k.smx_two_pass = value;
    else if (!std::strcmp(key, "smx_lanes")) k.smx_lanes = value;
    else if (!std::strcmp(key, "smx_split")) k.smx_split = value;
    else if (!std::strcmp(key, "smx_res")) k.smx_res = value;
    else if (!std::strcmp(key, "rowreg")) k.rowreg = value;
    else if (!std::strcmp(key, "topk_short")) k.topk_short = value;
    else if (!std::strcmp(key, "topk_radix")) k.topk_radix = value;
    else if (!std::strcmp(key, "topk_dyn")) k.topk_dyn = value;
    else return tpr::fail(TPR_ERR_INVALID_ARG, std::string("tpr_debug_set: unknown key ") + key);
    return TPR_OK;
}

}  // extern "C"
