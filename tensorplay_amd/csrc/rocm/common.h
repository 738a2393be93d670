// Shared device/host helpers for the gfx950 reduction + top-k kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <string>

#include "tpr_rocm.h"

namespace tpr {

constexpr int kWave = 64;  // CDNA wavefront width

// ---- error plumbing (host) -------------------------------------------------
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int check_launch(const char* what);

// Device facts used by the planners (read once per device, then cached).
struct DeviceInfo {
    int cus;  // compute units (256 on MI355X)
};
DeviceInfo device_info();

// Process-wide plan overrides for tests and tuning sweeps (tpr_debug_set).
// All zero in normal use.  Each knob is an atomic, so a thread that sets one
// while another plans a launch is not a data race; a launch reads each knob
// once, but a sweep that changes knobs while other threads launch gets plans
// that mix old and new values, so sweeps run single-threaded.
using Knob = std::atomic<int64_t>;
struct DebugKnobs {
    Knob splits{0};
    Knob lanes{0};
    Knob general{0};
    Knob topk_fallback{0};
    Knob tx{0};
    Knob topk_variant{0};
    Knob topk_waves{0};
    Knob unroll{0};
    Knob colblock{0};
    Knob nt{0};
    Knob smx_two_pass{0};
    Knob smx_lanes{0};
    Knob smx_split{0};
    Knob smx_res{0};
    Knob rowreg{0};
    Knob topk_short{0};
    Knob topk_radix{0};
    Knob topk_dyn{0};
};
DebugKnobs& knobs();

// ---- device helpers ----------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace tpr
