// Shared device/host helpers for the gfx950 reduction + top-k kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "tpr_rocm.h"

namespace tpr {

constexpr int kWave = 64;  // CDNA wavefront width

// ---- error plumbing (host) -------------------------------------------------
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int check_launch(const char* what);

// Device facts used by the planners (cached per device, set on first use).
struct DeviceInfo {
    int cus;  // compute units (256 on MI355X)
};
const DeviceInfo& device_info();

// Process-wide tuning overrides (tpr_debug_set).
struct DebugKnobs {
    int64_t splits = 0;
    int64_t lanes = 0;
    int64_t general = 0;
    int64_t topk_fallback = 0;
    int64_t tx = 0;
    int64_t topk_variant = 0;
    int64_t topk_waves = 0;
    int64_t unroll = 0;
    int64_t colblock = 0;
    int64_t nt = 0;
    int64_t smx_two_pass = 0;
    int64_t smx_lanes = 0;
    int64_t smx_split = 0;
    int64_t smx_res = 0;
};
DebugKnobs& knobs();

// ---- device helpers ----------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace tpr
