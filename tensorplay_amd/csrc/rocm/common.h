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

// Lane lane ^ M's value, without LDS-pipe permutes: DPP quad permutes for
// M = 1, 2; for M = 4 quad_perm [3,2,1,0] (xor 3) then row_half_mirror
// (i -> 7 - i = i ^ 7 inside 8 lanes); row_ror:8 for M = 8 (rotating a
// 16-lane row by 8 is xor 8); for M = 16 and 32 the gfx950 permlane swaps of
// the value with itself (v_permlane16_swap: odd rows of the first operand
// with even rows of the second; v_permlane32_swap: upper half of the first
// with lower half of the second), each lane taking the copy that holds its
// partner's value.  Every lane of the wave must be active.
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (M == 1) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        const int t = __builtin_amdgcn_mov_dpp((int)v, 0x1B, 0xF, 0xF, false);  // quad_perm [3,2,1,0]
        return (uint32_t)__builtin_amdgcn_mov_dpp(t, 0x141, 0xF, 0xF, false);   // row_half_mirror
    } else if constexpr (M == 8) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16) ? r[0] : r[1];
    } else {
        static_assert(M == 32, "lane distance 1 .. 32");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32) ? r[0] : r[1];
    }
}

// Lane lane ^ m's float for a distance m known when the caller's loop unrolls
// (1 .. 32: the exchanges above; anything else: a shuffle).
__device__ __forceinline__ float xor_lane_f(float v, int m) {
    const uint32_t u = __float_as_uint(v);
    switch (m) {
        case 1: return __uint_as_float(xor_lane<1>(u));
        case 2: return __uint_as_float(xor_lane<2>(u));
        case 4: return __uint_as_float(xor_lane<4>(u));
        case 8: return __uint_as_float(xor_lane<8>(u));
        case 16: return __uint_as_float(xor_lane<16>(u));
        case 32: return __uint_as_float(xor_lane<32>(u));
        default: return __shfl_xor(v, m, 64);
    }
}

}  // namespace tpr
