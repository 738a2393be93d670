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

#ifdef TPR_DEBUG_KNOBS
DebugKnobs& knobs() {
    static DebugKnobs k;
    return k;
}
#endif

}  // namespace tpr

extern "C" {

const char* tpr_last_error(void) { return tpr::g_last_error.c_str(); }

int32_t tpr_abi_version(void) { return (1 << 16) | 4; }

#ifdef TPR_DEBUG_KNOBS
// Test builds only (libtpr_rocm_dev.so).
int tpr_debug_set(const char* key, int64_t value) {
    if (!key) return tpr::fail(TPR_ERR_INVALID_ARG, "tpr_debug_set: null key");
    auto& k = tpr::knobs();
#define TPR_KNOB_SET(name) if (!std::strcmp(key, #name)) { k.name = value; return TPR_OK; }
    TPR_KNOB_LIST(TPR_KNOB_SET)
#undef TPR_KNOB_SET
    return tpr::fail(TPR_ERR_INVALID_ARG, std::string("tpr_debug_set: unknown key ") + key);
}
#endif

}  // extern "C"
