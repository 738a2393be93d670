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

// Plan overrides for tests and tuning sweeps.  The shipped library is built
// without TPR_DEBUG_KNOBS: every knob is then the constant 0, the planners fold
// it away, and the library holds no mutable plan state at all.  The test build
// (libtpr_rocm_dev.so, -DTPR_DEBUG_KNOBS) exports tpr_debug_set, which writes
// these process-wide atomics; a launch reads each knob once, but a sweep that
// changes knobs while other threads launch gets plans that mix old and new
// values, so sweeps run single-threaded.
#define TPR_KNOB_LIST(X) X(splits) X(lanes) X(general) X(topk_fallback) X(tx) X(topk_variant) X(topk_waves) \
    X(unroll) X(colblock) X(nt) X(smx_two_pass) X(smx_lanes) X(smx_split) X(smx_res) X(rowreg) X(topk_short) \
    X(topk_radix) X(topk_dyn) X(split_fin) X(smx_pieces) X(smx_spin) X(smx_fwd_pieces)
#ifdef TPR_DEBUG_KNOBS
using Knob = std::atomic<int64_t>;
struct DebugKnobs {
#define TPR_KNOB_FIELD(name) Knob name{0};
    TPR_KNOB_LIST(TPR_KNOB_FIELD)
#undef TPR_KNOB_FIELD
};
DebugKnobs& knobs();
#else
struct DebugKnobs {
#define TPR_KNOB_FIELD(name) static constexpr int64_t name = 0;
    TPR_KNOB_LIST(TPR_KNOB_FIELD)
#undef TPR_KNOB_FIELD
};
constexpr DebugKnobs knobs() { return DebugKnobs{}; }
#endif

// ---- device helpers ----------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace tpr
