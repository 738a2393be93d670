// gfx950 softmax / log_softmax along one dim, forward and backward, and the
// host planner behind tpr_softmax().
//
// Semantics follow TensorPlay's CPU composite
// (/root/reference/p10/src/backend/cpu/PointwiseKernels.cpp:519-545):
//   m = max over the dim (NaN ignored: strict compare from -inf), d = x - m,
//   softmax = exp(d) / sum(exp(d)), log_softmax = d - log(sum(exp(d))).
// So a NaN anywhere in a slice makes the whole slice NaN (it enters the sum),
// and a slice with no value above -inf (all -inf / NaN) is NaN everywhere.
// Backward follows the autograd formulas of config/derivatives.yaml:91-95:
//   softmax:     gx = (g - sum(g * y)) * y
//   log_softmax: gx = g - exp(y) * sum(g)
// with y the forward output.
//
// The reference materialises max, shifted, exp and sum tensors (five passes
// and three temporaries).  Here one kernel does it:
//   * rows shorter than 16384 floats (or a few long rows, up to 32768)
//     stay in registers: read once and written once -- k_smx_rows;
//   * forward rows of 16385..655360 floats with more rows than CUs and two
//     pieces or more per row, and every forward row of 153601..655360, are
//     cut into pieces held in registers by one workgroup each, (max, sum
//     exp) exchanged -- k_smx_fwd_pieces;
//   * rows of 16384..153600 floats, at least one per CU, stay on one CU in
//     registers plus LDS and are also read once -- k_smx_res (forward),
//     k_smx_res_bwd (gradients of rows the piece kernel does not take: g
//     held, y streamed);
//   * softmax and log_softmax gradients of rows of 16385..393216 floats are
//     cut into pieces, one workgroup each holding its g and y, with the
//     partial sums (g . y, or sum g) exchanged between the pieces --
//     k_smx_bwd_pieces (every input read once);
//   * longer rows stream twice: an online (max, sum-of-exp) pass, then the
//     output pass -- k_smx_rows2, or split over (row, chunk) workgroups when
//     the rows are fewer than the CUs -- k_smx_part / k_smx_apply;
//   * strided forward slices of 513..1024 rows with 16-byte columns: two row
//     pieces per 64-column group exchanging per-column statistics --
//     k_smx_cols4p;
//   * a strided softmax dim (inner extent > 1, or a non-unit dim stride)
//     keeps one column per lane, thread rows across the dim, an LDS merge of
//     the per-wave states, and also streams twice -- k_smx_cols.
// exp(d) is exp2(d * log2(e)); sums accumulate in fp32 per lane and combine in
// a fixed tree, so results are deterministic run to run.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <string>
#include <type_traits>

#include "common.h"

namespace tpr {
namespace {

constexpr float kL2E = 1.4426950408889634f;
enum { FWD = 0, FWD_LOG = 1, BWD = 2, BWD_LOG = 3 };

__device__ __forceinline__ float ex(float d) { return exp2f(d * kL2E); }
// Terms of a sum of exponentials: the bare hardware exp2 (no rescaling for
// results below 2^-126, which are below a sum's rounding anyway).
__device__ __forceinline__ float exs(float d) { return __builtin_amdgcn_exp2f(d * kL2E); }

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Row-segment loads / stores of VW floats; NT (nontemporal) is a template
// parameter because a runtime choice compiles to plain accesses only: the
// compiler merges the two branches' otherwise identical loads and stores and
// drops the nontemporal mark.
template <int VW, bool NT>
__device__ __forceinline__ void vld(float (&v)[VW], const float* p) {
    if constexpr (VW == 4) {
        f32x4 t;
        if constexpr (NT) t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
        else t = *reinterpret_cast<const f32x4*>(p);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
        if constexpr (NT) v[0] = __builtin_nontemporal_load(p);
        else v[0] = *p;
    }
}

template <int VW, bool NT>
__device__ __forceinline__ void vst(float* p, const float (&v)[VW]) {
    if constexpr (VW == 4) {
        const f32x4 t = {v[0], v[1], v[2], v[3]};
        if constexpr (NT) __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p));
        else *reinterpret_cast<f32x4*>(p) = t;
    } else {
        if constexpr (NT) __builtin_nontemporal_store(v[0], p);
        else *p = v[0];
    }
}

// Sum / max over G consecutive lanes (G <= 64: xor shuffles inside the wave;
// G > 64: one workgroup of G threads, via `sh` (G / 64 floats, private to this
// call site)).  The result is valid in every lane of the group.
template <int G, bool MAX>
__device__ __forceinline__ float grp(float v, float* sh) {
    constexpr int W = G < kWave ? G : kWave;
#pragma unroll
    for (int o = W / 2; o >= 1; o >>= 1) {
        const float t = xor_lane_f(v, o);
        v = MAX ? fmaxf(v, t) : v + t;
    }
    if constexpr (G > kWave) {
        if (__lane_id() == 0) sh[threadIdx.x / kWave] = v;
        __syncthreads();
        v = sh[0];
#pragma unroll
        for (int i = 1; i < G / kWave; ++i) v = MAX ? fmaxf(v, sh[i]) : v + sh[i];
    }
    return v;
}

// Online softmax state: running max m (never NaN) and s = sum exp(x - m).
// While m == -inf every element seen was -inf or NaN: s holds 0, or NaN once a
// NaN was seen, and is carried unscaled.
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
    const float M = fmaxf(m, m2);
    if (M == -INFINITY) {
        s += s2;
        return;
    }
    s = (m == -INFINITY ? s : s * exs(m - M)) + (m2 == -INFINITY ? s2 : s2 * exs(m2 - M));
    m = M;
}

// Add a chunk of K values to (m, s).
template <int K>
__device__ __forceinline__ void ms_add(float& m, float& s, const float* x) {
    float cm = x[0];
#pragma unroll
    for (int i = 1; i < K; ++i) cm = fmaxf(cm, x[i]);
    if (cm > m) {
        s = (m == -INFINITY) ? s : s * exs(m - cm);
        m = cm;
    }
    if (m == -INFINITY) {
#pragma unroll
        for (int i = 0; i < K; ++i) s += (x[i] != x[i]) ? x[i] : 0.0f;
    } else {
#pragma unroll
        for (int i = 0; i < K; ++i) s += exs(x[i] - m);
    }
}

template <int G>
__device__ __forceinline__ void grp_ms(float& m, float& s, float* shm, float* shs) {
    constexpr int W = G < kWave ? G : kWave;
#pragma unroll
    for (int o = W / 2; o >= 1; o >>= 1) ms_merge(m, s, __shfl_xor(m, o, kWave), __shfl_xor(s, o, kWave));
    if constexpr (G > kWave) {
        if (__lane_id() == 0) {
            shm[threadIdx.x / kWave] = m;
            shs[threadIdx.x / kWave] = s;
        }
        __syncthreads();
        m = shm[0];
        s = shs[0];
#pragma unroll
        for (int i = 1; i < G / kWave; ++i) ms_merge(m, s, shm[i], shs[i]);
    }
}

// Output of one element given the slice statistics.
//  FWD:     st0 = max, st1 = 1/sum       -> exp(x - max) * (1/sum)
//  FWD_LOG: st0 = max, st1 = log(sum)    -> (x - max) - log(sum)
//  BWD:     st0 = sum(g*y)               -> (g - st0) * y
//  BWD_LOG: st0 = sum(g)                 -> g - exp(y) * st0
template <int MODE>
__device__ __forceinline__ float outv(float a, float b, float st0, float st1) {
    if constexpr (MODE == FWD) return ex(a - st0) * st1;
    else if constexpr (MODE == FWD_LOG) return (a - st0) - st1;
    else if constexpr (MODE == BWD) return (a - st0) * b;
    else return a - ex(b) * st0;
}

struct SmxArgs {
    const float* a;  // x (forward) or g = dL/dy (backward)
    const float* b;  // y (backward only)
    float* out;      // dense [rows, n]
    long long rows, n;
    long long sa, sb;  // row strides of a and b (elements)
    int nt;            // nontemporal loads / stores
    int chunks;        // split rows: chunks per row
    float2* part;      // split rows: [rows, chunks] partial statistics
};

// ---------------------------------------------------------------------------
// Register-resident rows: G lanes per row, each lane holds V vectors of VW
// floats (vector j of lane l covers elements (j*G + l)*VW ...).  Read once,
// write once.  G <= 256: 256-thread workgroups holding 256/G rows; G > 256:
// one row per G-thread workgroup.
// ---------------------------------------------------------------------------
template <int MODE, int G, int V, int VW, bool NT>
__global__ __launch_bounds__(G > 256 ? G : 256) void k_smx_rows(SmxArgs p) {
    constexpr int BLK = G > 256 ? G : 256;
    constexpr int RPB = BLK / G;
    constexpr bool BW = MODE >= BWD;
    constexpr int NW = G > kWave ? G / kWave : 1;
    __shared__ float sh[2][NW];
    const int lane = threadIdx.x % G;
    const long long row = (long long)blockIdx.x * RPB + threadIdx.x / G;
    const bool live = row < p.rows;  // only G <= 64 can leave dead lanes (no barriers there)
    const float* pa = p.a + (live ? row : 0) * p.sa;
    const float* pb = BW ? p.b + (live ? row : 0) * p.sb : nullptr;
    float* po = p.out + (live ? row : 0) * p.n;

    float a[V][VW];
    float b[BW ? V : 1][VW];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const long long e = ((long long)j * G + lane) * VW;
        if (live && e < p.n) {
            vld<VW, NT>(a[j], pa + e);
            if constexpr (BW) vld<VW, NT>(b[j], pb + e);
        } else {
#pragma unroll
            for (int c = 0; c < VW; ++c) {
                a[j][c] = BW ? 0.0f : -INFINITY;
                if constexpr (BW) b[j][c] = 0.0f;
            }
        }
    }

    float st0, st1 = 0.0f;
    if constexpr (!BW) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < V; ++j)
#pragma unroll
            for (int c = 0; c < VW; ++c) m = fmaxf(m, a[j][c]);
        m = grp<G, true>(m, sh[0]);
        float s = 0.0f;
        if (m != -INFINITY) {
#pragma unroll
            for (int j = 0; j < V; ++j)
#pragma unroll
                for (int c = 0; c < VW; ++c) s += exs(a[j][c] - m);
        }
        s = grp<G, false>(s, sh[1]);
        if (m == -INFINITY) {  // no value above -inf in the slice: NaN, as the reference
            st0 = NAN;
            st1 = NAN;
        } else {
            st0 = m;
            st1 = (MODE == FWD) ? 1.0f / s : logf(s);
        }
    } else {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < V; ++j)
#pragma unroll
            for (int c = 0; c < VW; ++c) s += (MODE == BWD) ? a[j][c] * b[j][c] : a[j][c];
        st0 = grp<G, false>(s, sh[0]);
    }

    if (!live) return;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const long long e = ((long long)j * G + lane) * VW;
        if (e < p.n) {
            float o[VW];
#pragma unroll
            for (int c = 0; c < VW; ++c) o[c] = outv<MODE>(a[j][c], BW ? b[j][c] : 0.0f, st0, st1);
            vst<VW, NT>(po + e, o);
        }
    }
}

// ---------------------------------------------------------------------------
// Long rows: one 1024-thread workgroup per row, two streaming passes.  Pass 1
// accumulates the online (max, sum) state (forward) or the dot / sum
// (backward); pass 2 re-reads the row and writes the output.  Pass 1 uses
// ordinary loads so the row stays in the caches for pass 2.  Both passes keep
// two tiles in flight: the loads of tile t+1 are issued before tile t is
// consumed (one workgroup per CU has to cover the memory latency alone).
// ---------------------------------------------------------------------------
template <int MODE, int VW, int U, bool NT>
__global__ __launch_bounds__(1024) void k_smx_rows2(SmxArgs p) {
    constexpr int T = 1024;
    constexpr bool BW = MODE >= BWD;
    constexpr int UB = BW ? U : 1;
    constexpr long long TILE = (long long)T * VW * U;
    __shared__ float sh[2][T / kWave];
    const long long row = blockIdx.x;
    const long long n = p.n;
    const float* pa = p.a + row * p.sa;
    const float* pb = BW ? p.b + row * p.sb : nullptr;
    float* po = p.out + row * p.n;
    const int t = threadIdx.x;

    // wb: also load y (pass 1 of the log_softmax gradient needs g only)
    // ntc: std::bool_constant, nontemporal loads (pass 2 only: pass 1's data may
    // still be in the Infinity Cache when pass 2 re-reads it)
    auto load = [&](float (&xa)[U][VW], float (&xb)[UB][VW], long long base, auto ntc, bool wb) {
        constexpr bool L_NT = decltype(ntc)::value;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long e = base + ((long long)u * T + t) * VW;
            if (e < n) {
                vld<VW, L_NT>(xa[u], pa + e);
                if constexpr (BW) {
                    if (wb) vld<VW, L_NT>(xb[u], pb + e);
                }
            } else {
#pragma unroll
                for (int c = 0; c < VW; ++c) {
                    xa[u][c] = BW ? 0.0f : -INFINITY;
                    if constexpr (BW) xb[u][c] = 0.0f;
                }
            }
        }
    };

    float a0[U][VW], b0[UB][VW], a1[U][VW], b1[UB][VW];
    float m = -INFINITY, s = 0.0f;
    auto consume = [&](float (&xa)[U][VW], float (&xb)[UB][VW]) {
        if constexpr (!BW) {
            ms_add<U * VW>(m, s, &xa[0][0]);
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int c = 0; c < VW; ++c) s += (MODE == BWD) ? xa[u][c] * xb[u][c] : xa[u][c];
        }
    };
    constexpr bool WB1 = MODE == BWD;  // pass 1 reads y
    load(a0, b0, 0, std::false_type{}, WB1);
    for (long long base = 0;;) {
        if (base + TILE < n) load(a1, b1, base + TILE, std::false_type{}, WB1);
        consume(a0, b0);
        base += TILE;
        if (base >= n) break;
        if (base + TILE < n) load(a0, b0, base + TILE, std::false_type{}, WB1);
        consume(a1, b1);
        base += TILE;
        if (base >= n) break;
    }

    float st0, st1 = 0.0f;
    if constexpr (!BW) {
        grp_ms<T>(m, s, sh[0], sh[1]);
        if (m == -INFINITY) {
            st0 = NAN;
            st1 = NAN;
        } else {
            st0 = m;
            st1 = (MODE == FWD) ? 1.0f / s : logf(s);
        }
    } else {
        st0 = grp<T, false>(s, sh[0]);
    }

    auto emit = [&](float (&xa)[U][VW], float (&xb)[UB][VW], long long base) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long e = base + ((long long)u * T + t) * VW;
            if (e < n) {
                float o[VW];
#pragma unroll
                for (int c = 0; c < VW; ++c) o[c] = outv<MODE>(xa[u][c], BW ? xb[u][c] : 0.0f, st0, st1);
                vst<VW, NT>(po + e, o);
            }
        }
    };
    load(a0, b0, 0, std::bool_constant<NT>{}, true);
    for (long long base = 0;;) {
        if (base + TILE < n) load(a1, b1, base + TILE, std::bool_constant<NT>{}, true);
        emit(a0, b0, base);
        base += TILE;
        if (base >= n) break;
        if (base + TILE < n) load(a0, b0, base + TILE, std::bool_constant<NT>{}, true);
        emit(a1, b1, base);
        base += TILE;
        if (base >= n) break;
    }
}

// ---------------------------------------------------------------------------
// Rows of 16384 to 153600 floats (e.g. LLM vocabularies of 32K-152K), short
// enough for one CU: one 512-thread
// workgroup per row holds the row in registers (kResVR float4 per lane) plus
// LDS (the remaining vl float4 per lane, loaded straight from global memory
// into LDS without passing through registers).  Read once, write once, where
// the two-pass kernel reads twice.  Forward here; gradients k_smx_res_bwd.
//   vector v = j * 512 + t of the row is register r[j] of thread t for
//   j < kResVR, and lds[(j - kResVR) * 512 + t] after that.
// ---------------------------------------------------------------------------
constexpr int kResT = 512;
constexpr int kBufWord3 = 0x00020000;  // raw buffer resource, 32-bit data (gfx9 family)
constexpr int kResLdsMax = 160 * 1024;           // LDS of one gfx950 workgroup
constexpr int kResVLMax = kResLdsMax / (kResT * 16) - 1;  // float4 per lane in LDS (19; 4 KB spare)
// VR = float4 per lane in registers: 56 (224 VGPRs), 40, 24 or 8.  A kernel
// with VR takes rows of VR * 2048 .. (VR + 19) * 2048 floats; together they
// cover 16384 .. 153600 (the largest VR whose minimum the row reaches).
constexpr long long res_min(int vr) { return (long long)kResT * 4 * vr; }
constexpr long long res_max(int vr) { return (long long)kResT * 4 * (vr + kResVLMax); }
constexpr long long kResMax = res_max(56);       // 153600 floats

// Row loads and stores go through buffer resources spanning the row, with
// 32-bit offsets (no 64-bit address per vector).  The host sends only rows of
// at least res_min(kResVR) floats, so every register vector is inside the row; the
// LDS part is guarded.
template <int MODE, int NT, int kResVR>
__global__ __launch_bounds__(kResT) void k_smx_res(SmxArgs p, int vl) {
    extern __shared__ f32x4 lds[];
    __shared__ float sh[2][kResT / kWave];
    constexpr int aux = NT ? 2 : 0;  // cache policy: nontemporal
    const int t = threadIdx.x;
    const long long row = blockIdx.x;
    const float* ra = p.a + row * p.sa;
    float* ro = p.out + row * p.n;
    const int nb = (int)(p.n * 4);
    const __amdgpu_buffer_rsrc_t ba = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ra), (short)0, nb, kBufWord3);
    const __amdgpu_buffer_rsrc_t bo = __builtin_amdgcn_make_buffer_rsrc(ro, (short)0, nb, kBufWord3);
    const int q = (int)(p.n >> 2);  // float4 per row
    const f32x4 ninf = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};

    // LDS part first: the loads need no registers, so all of them are in
    // flight while the register part is issued behind them.
    const int wbase = t & ~(kWave - 1);
    const f32x4* pa = reinterpret_cast<const f32x4*>(ra);
    for (int j = 0; j < vl; ++j) {
        const int v = (kResVR + j) * kResT + t;
        if (v < q)
            __builtin_amdgcn_global_load_lds(
                (const void*)(pa + v),
                (__attribute__((address_space(3))) void*)(lds + j * kResT + wbase), 16, 0, 0);
    }
    f32x4 r[kResVR];
#pragma unroll
    for (int j = 0; j < kResVR; ++j) r[j] = __builtin_amdgcn_raw_buffer_load_b128(ba, (j * kResT + t) * 16, 0, aux);
    // vmcnt(kResVR): the LDS loads, issued first, have landed while the
    // register loads may still be in flight.  Each lane reads only the LDS
    // slots its own load filled, so no workgroup barrier.
    static_assert(kResVR < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((kResVR & 15) | ((kResVR >> 4) << 14) | 0x0F70);

    auto ldsv = [&](int j) -> f32x4 {
        return ((kResVR + j) * kResT + t < q) ? lds[j * kResT + t] : ninf;
    };
    // Online (max, sum exp) per lane, group by group in load order (the LDS
    // part, then register groups of 8 vectors as their loads land), so the
    // exponentials run under the remaining loads; one block merge at the end.
    auto group = [&](auto&& vec, int cnt, float& m, float& s) {
        float gm = -INFINITY;
        for (int j = 0; j < cnt; ++j) {
            const f32x4 x = vec(j);
            gm = fmaxf(fmaxf(gm, fmaxf(x.x, x.y)), fmaxf(x.z, x.w));
        }
        float gs = 0.0f;
        if (gm != -INFINITY) {
            for (int j = 0; j < cnt; ++j) {
                const f32x4 x = vec(j);
                gs += (exs(x.x - gm) + exs(x.y - gm)) + (exs(x.z - gm) + exs(x.w - gm));
            }
        } else {
            for (int j = 0; j < cnt; ++j) {  // only -inf and NaN: NaN stays
                const f32x4 x = vec(j);
                gs += ((x.x != x.x ? x.x : 0.0f) + (x.y != x.y ? x.y : 0.0f)) +
                      ((x.z != x.z ? x.z : 0.0f) + (x.w != x.w ? x.w : 0.0f));
            }
        }
        ms_merge(m, s, gm, gs);
    };
    float m = -INFINITY, s = 0.0f;
    group([&](int j) { return ldsv(j); }, vl, m, s);
    static_assert(kResVR % 8 == 0, "register vectors come in groups of 8");
#pragma unroll
    for (int g = 0; g < kResVR / 8; ++g) {
        float gm = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j) gm = fmaxf(fmaxf(gm, fmaxf(r[8 * g + j].x, r[8 * g + j].y)), fmaxf(r[8 * g + j].z, r[8 * g + j].w));
        float gs = 0.0f;
        if (gm != -INFINITY) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const f32x4 x = r[8 * g + j];
                gs += (exs(x.x - gm) + exs(x.y - gm)) + (exs(x.z - gm) + exs(x.w - gm));
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const f32x4 x = r[8 * g + j];
                gs += ((x.x != x.x ? x.x : 0.0f) + (x.y != x.y ? x.y : 0.0f)) +
                      ((x.z != x.z ? x.z : 0.0f) + (x.w != x.w ? x.w : 0.0f));
            }
        }
        ms_merge(m, s, gm, gs);
    }
    // block merge: the wave by lane swaps, then the waves through LDS
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) ms_merge(m, s, __shfl_xor(m, o, kWave), __shfl_xor(s, o, kWave));
    if (__lane_id() == 0) {
        sh[0][t / kWave] = m;
        sh[1][t / kWave] = s;
    }
    __syncthreads();
    m = sh[0][0];
    s = sh[1][0];
#pragma unroll
    for (int i = 1; i < kResT / kWave; ++i) ms_merge(m, s, sh[0][i], sh[1][i]);
    float st0, st1;
    if (m == -INFINITY) {  // no value above -inf in the slice: NaN, as the reference
        st0 = NAN;
        st1 = NAN;
    } else {
        st0 = m;
        st1 = (MODE == FWD) ? 1.0f / s : logf(s);
    }
    auto outq = [&](f32x4 x) -> f32x4 {
        return f32x4{outv<MODE>(x.x, 0.0f, st0, st1), outv<MODE>(x.y, 0.0f, st0, st1),
                     outv<MODE>(x.z, 0.0f, st0, st1), outv<MODE>(x.w, 0.0f, st0, st1)};
    };
#pragma unroll
    for (int j = 0; j < kResVR; ++j) __builtin_amdgcn_raw_buffer_store_b128(outq(r[j]), bo, (j * kResT + t) * 16, 0, aux);
    for (int j = 0; j < vl; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(outq(lds[j * kResT + t]), bo, ((kResVR + j) * kResT + t) * 16, 0, aux);
}

// The gradients on the same layout, with g held on chip (registers + LDS):
//   log_softmax (BWD_LOG): gx = g - exp(y) * sum(g): the sum comes from the
//     held g, then y streams past once: g, y and gx each cross HBM once;
//   softmax (BWD): gx = (g - sum(g * y)) * y: y streams past twice (the dot,
//     then the output), g once: four transfers where the two-pass kernel
//     makes five.
template <int MODE, int NT, int kResVR>
__global__ __launch_bounds__(kResT) void k_smx_res_bwd(SmxArgs p, int vl) {
    extern __shared__ f32x4 lds[];
    __shared__ float sh[kResT / kWave];
    constexpr int aux = NT ? 2 : 0;
    const int t = threadIdx.x;
    const long long row = blockIdx.x;
    const float* ra = p.a + row * p.sa;
    const float* rb = p.b + row * p.sb;
    float* ro = p.out + row * p.n;
    const int nb = (int)(p.n * 4);
    const __amdgpu_buffer_rsrc_t ba = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ra), (short)0, nb, kBufWord3);
    const __amdgpu_buffer_rsrc_t bb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(rb), (short)0, nb, kBufWord3);
    const __amdgpu_buffer_rsrc_t bo = __builtin_amdgcn_make_buffer_rsrc(ro, (short)0, nb, kBufWord3);
    const int q = (int)(p.n >> 2);
    const int wbase = t & ~(kWave - 1);
    const f32x4* pa = reinterpret_cast<const f32x4*>(ra);
    for (int j = 0; j < vl; ++j) {
        const int v = (kResVR + j) * kResT + t;
        if (v < q)
            __builtin_amdgcn_global_load_lds(
                (const void*)(pa + v),
                (__attribute__((address_space(3))) void*)(lds + j * kResT + wbase), 16, 0, 0);
    }
    f32x4 r[kResVR];
#pragma unroll
    for (int j = 0; j < kResVR; ++j) r[j] = __builtin_amdgcn_raw_buffer_load_b128(ba, (j * kResT + t) * 16, 0, aux);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the LDS loads have landed
    __syncthreads();
    auto vs = [](f32x4 x) { return (x.x + x.y) + (x.z + x.w); };
    auto vd = [](f32x4 x, f32x4 y) { return (x.x * y.x + x.y * y.y) + (x.z * y.z + x.w * y.w); };
    float s = 0.0f;
    // BWD: the dot's y loads go in blocks of YB vectors per lane, each block in
    // its own basic block behind an opaque always-true test, so the compiler
    // cannot hoist every y load next to the held g (that spills)
    constexpr int YB = kResVR >= 56 ? 2 : 4;
    int live = 1;
    if constexpr (MODE == BWD) asm volatile("s_mov_b32 %0, 1" : "=s"(live));
#pragma unroll
    for (int g = 0; g < kResVR / 8; ++g) {
        float gs = 0.0f;
#pragma unroll
        for (int h = 0; h < 8 / YB; ++h) {
            if constexpr (MODE == BWD_LOG) {
#pragma unroll
                for (int j = 0; j < YB; ++j) gs += vs(r[8 * g + YB * h + j]);
            } else if (live) {
                f32x4 y[YB];
#pragma unroll
                for (int j = 0; j < YB; ++j)
                    y[j] = __builtin_amdgcn_raw_buffer_load_b128(bb, ((8 * g + YB * h + j) * kResT + t) * 16, 0, 0);
#pragma unroll
                for (int j = 0; j < YB; ++j) gs += vd(r[8 * g + YB * h + j], y[j]);
                asm volatile("" : "+v"(gs));
            }
        }
        s += gs;
    }
    float sl = 0.0f;
    for (int j = 0; j < vl; ++j) {
        const int v = (kResVR + j) * kResT + t;
        if (v < q) {
            if constexpr (MODE == BWD_LOG) sl += vs(lds[j * kResT + t]);
            else sl += vd(lds[j * kResT + t], __builtin_amdgcn_raw_buffer_load_b128(bb, v * 16, 0, 0));
        }
    }
    s = grp<kResT, false>(s + sl, sh);
    // an opaque zero soffset for the output pass's y loads: otherwise the
    // compiler reuses the dot pass's loads (and products) and keeps them live
    // next to g, which spills
    int z0 = 0;
    if constexpr (MODE == BWD) asm volatile("s_mov_b32 %0, 0" : "=s"(z0));
    auto outq = [&](f32x4 g, f32x4 y) -> f32x4 {
        return f32x4{outv<MODE>(g.x, y.x, s, 0.0f), outv<MODE>(g.y, y.y, s, 0.0f),
                     outv<MODE>(g.z, y.z, s, 0.0f), outv<MODE>(g.w, y.w, s, 0.0f)};
    };
#pragma unroll
    for (int j = 0; j < kResVR; ++j) {
        const f32x4 y = __builtin_amdgcn_raw_buffer_load_b128(bb, (j * kResT + t) * 16, z0, aux);
        __builtin_amdgcn_raw_buffer_store_b128(outq(r[j], y), bo, (j * kResT + t) * 16, 0, aux);
    }
    for (int j = 0; j < vl; ++j) {
        const int off = ((kResVR + j) * kResT + t) * 16;
        const f32x4 y = __builtin_amdgcn_raw_buffer_load_b128(bb, off, z0, aux);
        __builtin_amdgcn_raw_buffer_store_b128(outq(lds[j * kResT + t], y), bo, off, 0, aux);
    }
}

// ---------------------------------------------------------------------------
// Gradients with g AND y held on chip: softmax gx = (g - sum(g * y)) * y and
// log_softmax gx = g - exp(y) * sum(g) need the whole row's statistic (the
// "dot" below: sum(g * y) or sum(g)) before any output, and a long row's g and y together
// exceed one CU, so a row is cut into NS pieces of at most kPcVR * 512
// float4 of each, one 512-thread workgroup per piece holding its g and y in
// registers: every input crosses HBM once (k_smx_res_bwd streams y twice).
// The pieces of a row exchange their partial dots through device memory:
//   * each piece's workgroup writes (epoch << 32 | partial bits) to its slot
//     with a device-scope atomic exchange (epoch: a per-launch tag from the
//     host, never 0, so no clearing is needed);
//   * thread 0 polls the other pieces' slots (device-scope atomic ors of 0)
//     until each carries this launch's epoch or `spin` ticks of the 100 MHz
//     real-time counter have passed;
//   * a piece still missing then is recomputed by this workgroup from HBM
//     (its g and y read again, summed in the same order, so the bits equal
//     the owner's): the wait is bounded and the result never depends on
//     whether a partner was resident.  Pieces of a row are adjacent in the
//     grid, so they normally run together.
// The row's dot is the sum of the NS partials in piece order in every
// workgroup, so all pieces use the same value.
// ---------------------------------------------------------------------------
constexpr int kPcMax = 16;                     // most pieces per row
constexpr int kFwdPcVR = 20;                   // forward pieces: float4 of x per lane
constexpr int kSmxSlots = 1 << 18;             // exchange slots (2 MiB); a launch never needs more

}  // namespace
}  // namespace tpr

static __device__ unsigned long long smx_slots[tpr::kSmxSlots];

namespace tpr {
namespace {

template <int MODE, int NT, int PT, int kPcVR>
__global__ __launch_bounds__(PT) void k_smx_bwd_pieces(SmxArgs p, int ns, int pv, unsigned epoch, int spin) {
    static_assert(MODE == BWD || MODE == BWD_LOG, "gradients only");
    __shared__ float sh[PT / kWave];
    __shared__ float parts[kPcMax];
    __shared__ unsigned missing;
    constexpr int aux = NT ? 2 : 0;
    const int t = threadIdx.x;
    const long long row = blockIdx.x / ns;
    const int pc = (int)(blockIdx.x % ns);
    const int q = (int)(p.n >> 2);
    const float* ra = p.a + row * p.sa;
    const float* rb = p.b + row * p.sb;
    auto rsrc = [&](const float* base, int i) {
        const int v0 = i * pv;
        const int len = max(0, min(q, v0 + pv) - v0);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base + 4LL * v0), (short)0, len * 16, kBufWord3);
    };
    // the row statistic's term of one vector pair: softmax g . y, log_softmax sum(g)
    auto vd = [](f32x4 x, f32x4 y) {
        if constexpr (MODE == BWD_LOG) return (x.x + x.y) + (x.z + x.w);
        else return (x.x * y.x + x.y * y.y) + (x.z * y.z + x.w * y.w);
    };
    const __amdgpu_buffer_rsrc_t bg = rsrc(ra, pc), by = rsrc(rb, pc);
    f32x4 g[kPcVR], y[kPcVR];
#pragma unroll
    for (int j = 0; j < kPcVR; ++j) g[j] = __builtin_amdgcn_raw_buffer_load_b128(bg, (j * PT + t) * 16, 0, aux);
#pragma unroll
    for (int j = 0; j < kPcVR; ++j) y[j] = __builtin_amdgcn_raw_buffer_load_b128(by, (j * PT + t) * 16, 0, aux);
    float s = 0.0f;  // vectors past the piece read 0 (buffer range check) and add nothing
#pragma unroll
    for (int j = 0; j < kPcVR; ++j) s += vd(g[j], y[j]);
    s = grp<PT, false>(s, sh);
    if (t == 0) {
        parts[pc] = s;
        unsigned need = 0;
        if (ns > 1) {
            unsigned long long* slot = smx_slots;
            const long long base = row * ns;
            __hip_atomic_exchange(slot + ((base + pc) & (kSmxSlots - 1)),
                                  ((unsigned long long)epoch << 32) | __float_as_uint(s), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
            need = ((1u << ns) - 1u) & ~(1u << pc);
            const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                for (int i = 0; i < ns; ++i) {
                    if (!((need >> i) & 1u)) continue;
                    const unsigned long long v = __hip_atomic_fetch_or(slot + ((base + i) & (kSmxSlots - 1)), 0ull,
                                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((unsigned)(v >> 32) == epoch) {
                        parts[i] = __uint_as_float((unsigned)v);
                        need &= ~(1u << i);
                    }
                }
                if (need == 0 || __builtin_amdgcn_s_memrealtime() - t0 > (unsigned long long)spin) break;
                __builtin_amdgcn_s_sleep(2);
            }
        }
        missing = need;
    }
    __syncthreads();
    const unsigned miss = missing;
    for (int i = 0; i < ns; ++i) {
        if (!((miss >> i) & 1u)) continue;  // uniform
        const __amdgpu_buffer_rsrc_t mg = rsrc(ra, i), my = rsrc(rb, i);
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < kPcVR; ++j) {
            const f32x4 gm = __builtin_amdgcn_raw_buffer_load_b128(mg, (j * PT + t) * 16, 0, 0);
            if constexpr (MODE == BWD_LOG) s2 += vd(gm, gm);
            else s2 += vd(gm, __builtin_amdgcn_raw_buffer_load_b128(my, (j * PT + t) * 16, 0, 0));
        }
        s2 = grp<PT, false>(s2, sh);
        if (t == 0) parts[i] = s2;
        __syncthreads();
    }
    float dot = parts[0];
    for (int i = 1; i < ns; ++i) dot += parts[i];
    const __amdgpu_buffer_rsrc_t bo = rsrc(p.out + row * p.n, pc);
#pragma unroll
    for (int j = 0; j < kPcVR; ++j) {
        const f32x4 r = {outv<MODE>(g[j].x, y[j].x, dot, 0.0f), outv<MODE>(g[j].y, y[j].y, dot, 0.0f),
                         outv<MODE>(g[j].z, y[j].z, dot, 0.0f), outv<MODE>(g[j].w, y[j].w, dot, 0.0f)};
        __builtin_amdgcn_raw_buffer_store_b128(r, bo, (j * PT + t) * 16, 0, aux);  // past the piece: dropped
    }
}

// ---------------------------------------------------------------------------
// Forward softmax / log_softmax by row pieces: the same cut and exchange as
// k_smx_bwd_pieces, each 512-thread workgroup holding its piece of x in
// registers (kPcVR float4 per lane, few enough registers for two workgroups
// per CU, so one loads while the other writes).  A piece's statistic is its
// (max, sum of exp(x - max)) pair, two slots of (epoch << 32 | bits) each;
// a missing piece is recomputed from HBM by the same per-lane code and the
// same block merge, so its bits equal the owner's.  Every workgroup merges
// the pieces' pairs in piece order.  NaN and -inf follow k_smx_res: max
// ignores NaN, a lane or piece with no value above -inf carries its NaNs in
// the sum, a row with no value above -inf is NaN.
// ---------------------------------------------------------------------------
// One lane's (max, sum exp) over its vectors j < nv of a piece, then the block
// merge.  STREAM (the recompute of another piece): one vector loaded at a
// time in a rolled loop over j < nv; else the held vectors, unrolled over
// kPcVR, which the caller has set to -inf past nv.  The two give the same
// bits: a -inf vector leaves the max alone and adds exp2(-inf) = +0 to a sum
// that starts at +0.
template <int PT, int kPcVR, bool STREAM, class V>
__device__ __forceinline__ void piece_stats(V&& vec, int nv, float (&sh)[2][PT / kWave], float& m, float& s) {
    const f32x4 ninf = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    (void)ninf;
    auto at = [&](int j) -> f32x4 { return vec(j); };  // held vectors: -inf past nv already
    const int n = STREAM ? nv : kPcVR;
    float gm = -INFINITY;
#pragma unroll
    for (int j = 0; j < (STREAM ? 1 : kPcVR); ++j) {
        for (int jj = j; jj < (STREAM ? n : j + 1); ++jj) {
            const f32x4 x = at(jj);
            gm = fmaxf(fmaxf(gm, fmaxf(x.x, x.y)), fmaxf(x.z, x.w));
        }
    }
    float gs = 0.0f;
    if (gm != -INFINITY) {
#pragma unroll
        for (int j = 0; j < (STREAM ? 1 : kPcVR); ++j) {
            for (int jj = j; jj < (STREAM ? n : j + 1); ++jj) {
                const f32x4 x = at(jj);
                gs += (exs(x.x - gm) + exs(x.y - gm)) + (exs(x.z - gm) + exs(x.w - gm));
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < (STREAM ? 1 : kPcVR); ++j) {
            for (int jj = j; jj < (STREAM ? n : j + 1); ++jj) {  // only -inf and NaN: NaN stays
                const f32x4 x = at(jj);
                gs += ((x.x != x.x ? x.x : 0.0f) + (x.y != x.y ? x.y : 0.0f)) +
                      ((x.z != x.z ? x.z : 0.0f) + (x.w != x.w ? x.w : 0.0f));
            }
        }
    }
    m = gm;
    s = gs;
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) ms_merge(m, s, __shfl_xor(m, o, kWave), __shfl_xor(s, o, kWave));
    const int t = threadIdx.x;
    __syncthreads();  // sh may still be read from an earlier merge
    if (__lane_id() == 0) {
        sh[0][t / kWave] = m;
        sh[1][t / kWave] = s;
    }
    __syncthreads();
    m = sh[0][0];
    s = sh[1][0];
#pragma unroll
    for (int i = 1; i < PT / kWave; ++i) ms_merge(m, s, sh[0][i], sh[1][i]);
}

template <int MODE, int NT, int PT, int kPcVR>
__global__ __launch_bounds__(PT) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_smx_fwd_pieces(SmxArgs p, int ns, int pv, unsigned epoch, int spin) {
    static_assert(MODE == FWD || MODE == FWD_LOG, "forward only");
    __shared__ float sh[2][PT / kWave];
    __shared__ float pm[kPcMax], ps[kPcMax];
    __shared__ unsigned missing;
    constexpr int aux = NT ? 2 : 0;
    const int t = threadIdx.x;
    const long long row = blockIdx.x / ns;
    const int pc = (int)(blockIdx.x % ns);
    const int q = (int)(p.n >> 2);
    const float* ra = p.a + row * p.sa;
    auto plen = [&](int i) { return max(0, min(q, i * pv + pv) - i * pv); };  // float4 of piece i
    auto rsrc = [&](const float* base, int i) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base + 4LL * i * pv), (short)0, plen(i) * 16,
                                                 kBufWord3);
    };
    // vectors j of this lane: piece vector j * PT + t, inside the piece for j < nv
    auto nv_of = [&](int i) { return (plen(i) - t + PT - 1) / PT; };
    const __amdgpu_buffer_rsrc_t bx = rsrc(ra, pc);
    f32x4 x[kPcVR];
#pragma unroll
    for (int j = 0; j < kPcVR; ++j) x[j] = __builtin_amdgcn_raw_buffer_load_b128(bx, (j * PT + t) * 16, 0, aux);
    float m, s;
    {
        const int nv = nv_of(pc);  // the rest read 0 (buffer range) and are never stored
        const f32x4 ninf = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int j = 0; j < kPcVR; ++j) x[j] = j < nv ? x[j] : ninf;
    }
    piece_stats<PT, kPcVR, false>([&](int j) { return x[j]; }, kPcVR, sh, m, s);
    if (t == 0) {
        pm[pc] = m;
        ps[pc] = s;
        unsigned need = 0;
        if (ns > 1) {
            unsigned long long* slot = smx_slots;
            const long long base = 2 * row * ns;
            const unsigned long long tag = (unsigned long long)epoch << 32;
            __hip_atomic_exchange(slot + ((base + 2 * pc) & (kSmxSlots - 1)), tag | __float_as_uint(m),
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_exchange(slot + ((base + 2 * pc + 1) & (kSmxSlots - 1)), tag | __float_as_uint(s),
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            need = ((1u << ns) - 1u) & ~(1u << pc);
            const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                for (int i = 0; i < ns; ++i) {
                    if (!((need >> i) & 1u)) continue;
                    const unsigned long long vm = __hip_atomic_fetch_or(
                        slot + ((base + 2 * i) & (kSmxSlots - 1)), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const unsigned long long vs = __hip_atomic_fetch_or(
                        slot + ((base + 2 * i + 1) & (kSmxSlots - 1)), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((unsigned)(vm >> 32) == epoch && (unsigned)(vs >> 32) == epoch) {
                        pm[i] = __uint_as_float((unsigned)vm);
                        ps[i] = __uint_as_float((unsigned)vs);
                        need &= ~(1u << i);
                    }
                }
                if (need == 0 || __builtin_amdgcn_s_memrealtime() - t0 > (unsigned long long)spin) break;
                __builtin_amdgcn_s_sleep(2);
            }
        }
        missing = need;
    }
    __syncthreads();
    const unsigned miss = missing;
    for (int i = 0; i < ns; ++i) {
        if (!((miss >> i) & 1u)) continue;  // uniform
        const __amdgpu_buffer_rsrc_t mx = rsrc(ra, i);
        float m2, s2;
        piece_stats<PT, kPcVR, true>(
            [&](int j) { return __builtin_amdgcn_raw_buffer_load_b128(mx, (j * PT + t) * 16, 0, 0); }, nv_of(i), sh,
            m2, s2);
        if (t == 0) {
            pm[i] = m2;
            ps[i] = s2;
        }
    }
    __syncthreads();
    float M = pm[0], S = ps[0];
    for (int i = 1; i < ns; ++i) ms_merge(M, S, pm[i], ps[i]);
    float st0, st1;
    if (M == -INFINITY) {  // no value above -inf in the row: NaN, as the reference
        st0 = NAN;
        st1 = NAN;
    } else {
        st0 = M;
        st1 = (MODE == FWD) ? 1.0f / S : logf(S);
    }
    float* ro = p.out + row * p.n;
    const __amdgpu_buffer_rsrc_t bo = rsrc(ro, pc);
#pragma unroll
    for (int j = 0; j < kPcVR; ++j) {
        const f32x4 r = {outv<MODE>(x[j].x, 0.0f, st0, st1), outv<MODE>(x[j].y, 0.0f, st0, st1),
                         outv<MODE>(x[j].z, 0.0f, st0, st1), outv<MODE>(x[j].w, 0.0f, st0, st1)};
        __builtin_amdgcn_raw_buffer_store_b128(r, bo, (j * PT + t) * 16, 0, aux);  // past the piece: dropped
    }
}

// ---------------------------------------------------------------------------
// Split long rows (few rows, e.g. LLM vocabulary logits): each row is cut into
// kChunk-element chunks, one 256-thread workgroup per (row, chunk) in both
// kernels, so the chip is full however few rows there are.
//   k_smx_part:  partial statistics of the chunk -> part[row, chunk]
//                (forward: online (max, sum); backward: sum(g*y) or sum(g));
//   k_smx_apply: every thread merges the row's partials in chunk order (the
//                same result in every workgroup of the row), then re-reads its
//                chunk and writes the output.
// ---------------------------------------------------------------------------
constexpr int kChunk = 8192;

template <int MODE, int VW>
__global__ __launch_bounds__(256) void k_smx_part(SmxArgs p) {
    constexpr bool BW = MODE >= BWD;
    constexpr int U = 8 / VW;                 // 8 floats per thread per step
    constexpr int STEP = 256 * VW * U;        // 2048 floats
    __shared__ float sh[2][256 / kWave];
    const long long row = blockIdx.x / p.chunks;
    const long long c0 = (long long)(blockIdx.x - row * p.chunks) * kChunk;
    const float* pa = p.a + row * p.sa;
    const float* pb = BW ? p.b + row * p.sb : nullptr;
    const int t = threadIdx.x;
    float m = -INFINITY, s = 0.0f;
#pragma unroll
    for (int it = 0; it < kChunk / STEP; ++it) {
        float x[U][VW], y[BW ? U : 1][VW];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long e = c0 + it * STEP + ((long long)u * 256 + t) * VW;
            if (e < p.n) {
                vld<VW, false>(x[u], pa + e);
                if constexpr (MODE == BWD) vld<VW, false>(y[u], pb + e);  // BWD_LOG: sum(g) needs no y
            } else {
#pragma unroll
                for (int c = 0; c < VW; ++c) {
                    x[u][c] = BW ? 0.0f : -INFINITY;
                    if constexpr (BW) y[u][c] = 0.0f;
                }
            }
        }
        if constexpr (!BW) {
            ms_add<U * VW>(m, s, &x[0][0]);
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int c = 0; c < VW; ++c) s += (MODE == BWD) ? x[u][c] * y[u][c] : x[u][c];
        }
    }
    if constexpr (!BW) grp_ms<256>(m, s, sh[0], sh[1]);
    else s = grp<256, false>(s, sh[0]);
    if (t == 0) p.part[blockIdx.x] = make_float2(m, s);
}

template <int MODE, int VW, bool NT>
__global__ __launch_bounds__(256) void k_smx_apply(SmxArgs p) {
    constexpr bool BW = MODE >= BWD;
    constexpr int U = 8 / VW;
    constexpr int STEP = 256 * VW * U;
    const long long row = blockIdx.x / p.chunks;
    const long long c0 = (long long)(blockIdx.x - row * p.chunks) * kChunk;
    const float* pa = p.a + row * p.sa;
    const float* pb = BW ? p.b + row * p.sb : nullptr;
    float* po = p.out + row * p.n;
    const int t = threadIdx.x;
    const float2* pp = p.part + row * p.chunks;
    float st0, st1 = 0.0f;
    if constexpr (!BW) {
        float m = pp[0].x, s = pp[0].y;
        for (int k = 1; k < p.chunks; ++k) ms_merge(m, s, pp[k].x, pp[k].y);
        if (m == -INFINITY) {
            st0 = NAN;
            st1 = NAN;
        } else {
            st0 = m;
            st1 = (MODE == FWD) ? 1.0f / s : logf(s);
        }
    } else {
        float s = pp[0].y;
        for (int k = 1; k < p.chunks; ++k) s += pp[k].y;
        st0 = s;
    }
#pragma unroll
    for (int it = 0; it < kChunk / STEP; ++it) {
        float x[U][VW], y[BW ? U : 1][VW];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long e = c0 + it * STEP + ((long long)u * 256 + t) * VW;
            if (e < p.n) {
                vld<VW, NT>(x[u], pa + e);
                if constexpr (BW) vld<VW, NT>(y[u], pb + e);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long e = c0 + it * STEP + ((long long)u * 256 + t) * VW;
            if (e < p.n) {
                float o[VW];
#pragma unroll
                for (int c = 0; c < VW; ++c) o[c] = outv<MODE>(x[u][c], BW ? y[u][c] : 0.0f, st0, st1);
                vst<VW, NT>(po + e, o);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Strided dim: [outer, n, inner] with any strides.  One column (o, i) per
// lane, 64 columns per workgroup, BY waves splitting the dim (wave w takes
// r = w, w + BY, ...).  Per-wave states merge through LDS in a fixed order.
// The output is dense [outer, n, inner].
// ---------------------------------------------------------------------------
struct SmxColArgs {
    const float* a;
    const float* b;
    float* out;
    long long outer, n, inner;
    long long a_so, a_sn, a_si;
    long long b_so, b_sn, b_si;
    int nt;  // nontemporal second-pass loads and stores
};

template <int MODE, int BY>
__global__ __launch_bounds__(kWave * BY) void k_smx_cols(SmxColArgs p) {
    constexpr bool BW = MODE >= BWD;
    constexpr int U = 4;
    __shared__ float shm[BY][kWave];
    __shared__ float shs[BY][kWave];
    const int lane = threadIdx.x % kWave;
    const int w = threadIdx.x / kWave;
    const long long cols = p.outer * p.inner;
    const long long col = (long long)blockIdx.x * kWave + lane;
    const bool live = col < cols;
    const long long o = live ? col / p.inner : 0;
    const long long i = live ? col - o * p.inner : 0;
    const float* pa = p.a + o * p.a_so + i * p.a_si;
    const float* pb = BW ? p.b + o * p.b_so + i * p.b_si : nullptr;
    float* po = p.out + o * p.n * p.inner + i;
    const long long n = live ? p.n : 0;

    float m = -INFINITY, s = 0.0f;
    long long r = w;
    for (; r + (U - 1) * BY < n; r += U * BY) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long rr = r + (long long)u * BY;
            if constexpr (!BW) x[u] = pa[rr * p.a_sn];
            else x[u] = (MODE == BWD) ? pa[rr * p.a_sn] * pb[rr * p.b_sn] : pa[rr * p.a_sn];
        }
        if constexpr (!BW) ms_add<U>(m, s, x);
        else
#pragma unroll
            for (int u = 0; u < U; ++u) s += x[u];
    }
    for (; r < n; r += BY) {
        float x[1];
        if constexpr (!BW) {
            x[0] = pa[r * p.a_sn];
            ms_add<1>(m, s, x);
        } else {
            s += (MODE == BWD) ? pa[r * p.a_sn] * pb[r * p.b_sn] : pa[r * p.a_sn];
        }
    }
    shm[w][lane] = m;
    shs[w][lane] = s;
    __syncthreads();
    float st0, st1 = 0.0f;
    if constexpr (!BW) {
        m = shm[0][lane];
        s = shs[0][lane];
#pragma unroll
        for (int k = 1; k < BY; ++k) ms_merge(m, s, shm[k][lane], shs[k][lane]);
        if (m == -INFINITY) {
            st0 = NAN;
            st1 = NAN;
        } else {
            st0 = m;
            st1 = (MODE == FWD) ? 1.0f / s : logf(s);
        }
    } else {
        s = shs[0][lane];
#pragma unroll
        for (int k = 1; k < BY; ++k) s += shs[k][lane];
        st0 = s;
    }
    for (r = w; r < n; r += BY) {
        const float y = BW ? pb[r * p.b_sn] : 0.0f;
        po[r * p.inner] = outv<MODE>(pa[r * p.a_sn], y, st0, st1);
    }
}

// Strided dim with a contiguous, 16-byte aligned inner dim (inner % 4 == 0):
// a wave covers 4 rows x 64 columns (16 lanes of float4 per row, 256 bytes
// contiguous), BY waves split the dim, 64 columns per workgroup.  Per-thread
// online states per float4 component, merged across the wave's 4 row lanes by
// shuffles and across waves through LDS in a fixed order.
template <int MODE, int BY>
__global__ __launch_bounds__(kWave * BY) void k_smx_cols4(SmxColArgs p) {
    constexpr bool BW = MODE >= BWD;
    constexpr int U = 4;
    constexpr int RS = 4 * BY;  // rows per step
    __shared__ float shm[BY][16][4];
    __shared__ float shs[BY][16][4];
    const int lane = threadIdx.x % kWave;
    const int w = threadIdx.x / kWave;
    const int cl = lane % 16, rl = lane / 16;
    const long long ncg = (p.inner + 63) / 64;
    const long long o = blockIdx.x / ncg;
    const long long c = (blockIdx.x - o * ncg) * 64 + 4 * cl;  // first column of this lane
    const bool live = c < p.inner;
    const float* pa = p.a + o * p.a_so + (live ? c : 0);
    const float* pb = BW ? p.b + o * p.b_so + (live ? c : 0) : nullptr;
    float* po = p.out + o * p.n * p.inner + (live ? c : 0);
    const long long n = live ? p.n : 0;

    float m[4], sm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        m[q] = -INFINITY;
        sm[q] = 0.0f;
    }
    long long r = rl + 4 * w;
    for (; r + (U - 1) * RS < n; r += U * RS) {
        float x[U][4], y[BW ? U : 1][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            vld<4, false>(x[u], pa + (r + (long long)u * RS) * p.a_sn);
            if constexpr (MODE == BWD) vld<4, false>(y[u], pb + (r + (long long)u * RS) * p.b_sn);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (!BW) {
                float v[U];
#pragma unroll
                for (int u = 0; u < U; ++u) v[u] = x[u][q];
                ms_add<U>(m[q], sm[q], v);
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) sm[q] += (MODE == BWD) ? x[u][q] * y[u][q] : x[u][q];
            }
        }
    }
    for (; r < n; r += RS) {
        float x[4], y[4];
        vld<4, false>(x, pa + r * p.a_sn);
        if constexpr (MODE == BWD) vld<4, false>(y, pb + r * p.b_sn);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (!BW) ms_add<1>(m[q], sm[q], &x[q]);
            else sm[q] += (MODE == BWD) ? x[q] * y[q] : x[q];
        }
    }
    // merge the wave's 4 row lanes (xor 16, 32), then the BY waves via LDS
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float m2 = xor_lane_f(m[q], off), s2 = xor_lane_f(sm[q], off);
            if constexpr (!BW) ms_merge(m[q], sm[q], m2, s2);
            else sm[q] += s2;
        }
    }
    if (rl == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            shm[w][cl][q] = m[q];
            shs[w][cl][q] = sm[q];
        }
    }
    __syncthreads();
    float st0[4], st1[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float M = shm[0][cl][q], S = shs[0][cl][q];
#pragma unroll
        for (int k = 1; k < BY; ++k) {
            if constexpr (!BW) ms_merge(M, S, shm[k][cl][q], shs[k][cl][q]);
            else S += shs[k][cl][q];
        }
        if constexpr (!BW) {
            if (M == -INFINITY) {
                st0[q] = NAN;
                st1[q] = NAN;
            } else {
                st0[q] = M;
                st1[q] = (MODE == FWD) ? 1.0f / S : logf(S);
            }
        } else {
            st0[q] = S;
            st1[q] = 0.0f;
        }
    }
    for (r = rl + 4 * w; r < n; r += RS) {
        float x[4], y[4], out[4];
        vld<4, false>(x, pa + r * p.a_sn);
        if constexpr (BW) vld<4, false>(y, pb + r * p.b_sn);
#pragma unroll
        for (int q = 0; q < 4; ++q) out[q] = outv<MODE>(x[q], BW ? y[q] : 0.0f, st0[q], st1[q]);
        vst<4, false>(po + r * p.inner, out);  // plain: nontemporal was slower here (dim 0 of [64, 1024, 1024]: 143 vs 129 us)
    }
}

// Strided dim held in registers: like k_smx_cols4, but a wave covers 64/CW
// rows x 4*CW columns (CW lanes of float4 per row: 16 -> 256 contiguous bytes,
// 8 -> 128), BY waves, and each lane keeps its V rows (r = rl + (64/CW) w +
// i * RS) in registers, so the slice is read once and written from registers.
// For n <= RS * V.
template <int MODE, int BY, int V, int CW, bool NT>
__global__ __launch_bounds__(kWave * BY) void k_smx_cols4r(SmxColArgs p) {
    constexpr bool BW = MODE >= BWD;
    constexpr int RW = kWave / CW;  // rows per wave step
    constexpr int RS = RW * BY;      // rows per workgroup step
    // per-wave (max, sum) of each column as whole float4 per lane: one 16-byte
    // LDS store / load per lane, consecutive lanes on consecutive banks
    __shared__ f32x4 shm[BY][CW];
    __shared__ f32x4 shs[BY][CW];
    const int lane = threadIdx.x % kWave;
    const int w = threadIdx.x / kWave;
    const int cl = lane % CW, rl = lane / CW;
    const long long ncg = (p.inner + 4 * CW - 1) / (4 * CW);
    const long long o = blockIdx.x / ncg;
    const long long c = (blockIdx.x - o * ncg) * (4 * CW) + 4 * cl;  // first column of this lane
    const bool live = c < p.inner;
    const float* pa = p.a + o * p.a_so + (live ? c : 0);
    const float* pb = BW ? p.b + o * p.b_so + (live ? c : 0) : nullptr;
    float* po = p.out + o * p.n * p.inner + (live ? c : 0);
    const int n = live ? (int)p.n : 0;
    const int r0 = rl + RW * w;

    float x[V][4], y[BW ? V : 1][4];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int r = r0 + i * RS;
        if (r < n) {
            vld<4, NT>(x[i], pa + r * p.a_sn);
            if constexpr (BW) vld<4, NT>(y[i], pb + r * p.b_sn);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                x[i][q] = BW ? 0.0f : -INFINITY;
                if constexpr (BW) y[i][q] = 0.0f;
            }
        }
    }
    float m[4], sm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if constexpr (!BW) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < V; ++i) mx = fmaxf(mx, x[i][q]);
            float sv = 0.0f;
            if (mx != -INFINITY) {
#pragma unroll
                for (int i = 0; i < V; ++i) sv += exs(x[i][q] - mx);
            } else {
#pragma unroll
                for (int i = 0; i < V; ++i) sv += (x[i][q] != x[i][q]) ? x[i][q] : 0.0f;  // NaN stays
            }
            m[q] = mx;
            sm[q] = sv;
        } else {
            float sv = 0.0f;
#pragma unroll
            for (int i = 0; i < V; ++i) sv += (MODE == BWD) ? x[i][q] * y[i][q] : x[i][q];
            m[q] = 0.0f;
            sm[q] = sv;
        }
    }
    // merge the wave's RW row lanes (xor CW .. 32), then the BY waves via LDS
#pragma unroll
    for (int off = CW; off <= 32; off <<= 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float m2 = xor_lane_f(m[q], off), s2 = xor_lane_f(sm[q], off);
            if constexpr (!BW) ms_merge(m[q], sm[q], m2, s2);
            else sm[q] += s2;
        }
    }
    if (rl == 0) {
        shm[w][cl] = f32x4{m[0], m[1], m[2], m[3]};
        shs[w][cl] = f32x4{sm[0], sm[1], sm[2], sm[3]};
    }
    __syncthreads();
    // merge the waves one float4 pair at a time (few live registers: the
    // slice values are still held)
    f32x4 Mv = shm[0][cl], Sv = shs[0][cl];
    for (int k = 1; k < BY; ++k) {
        const f32x4 mk = shm[k][cl], sk = shs[k][cl];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (!BW) {
                float M = Mv[q], S = Sv[q];
                ms_merge(M, S, mk[q], sk[q]);
                Mv[q] = M;
                Sv[q] = S;
            } else {
                Sv[q] += sk[q];
            }
        }
    }
    float st0[4], st1[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float M = Mv[q], S = Sv[q];
        if constexpr (!BW) {
            if (M == -INFINITY) {
                st0[q] = NAN;
                st1[q] = NAN;
            } else {
                st0[q] = M;
                st1[q] = (MODE == FWD) ? 1.0f / S : logf(S);
            }
        } else {
            st0[q] = S;
            st1[q] = 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int r = r0 + i * RS;
        if (r < n) {
            float out[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) out[q] = outv<MODE>(x[i][q], BW ? y[i][q] : 0.0f, st0[q], st1[q]);
            vst<4, NT>(po + (long long)r * p.inner, out);
        }
    }
}


// ---------------------------------------------------------------------------
// Strided forward softmax by row pieces: a 64-column group of a slice of
// 513..1024 rows is cut into two pieces of <= 512 rows, one 8-wave workgroup
// each holding its rows in registers (16 per lane, as k_smx_cols4r with 16
// waves holds the whole slice), so two workgroups share a CU and one loads
// while the other writes.  The pieces exchange their per-column (max, sum exp)
// through the slot array with the launch's epoch (lanes of wave 0 with rl = 0
// own 4 columns each: 8 slots), waiting a bounded time; a piece not seen in
// time is recomputed from HBM by the same per-lane code (rows streamed in the
// same order) and the same merges, so its bits equal the owner's.  Every
// workgroup merges the two pieces in piece order.
// ---------------------------------------------------------------------------
template <int BY, int V, bool STREAM, class L>
__device__ __forceinline__ void col_piece_stats(L&& row, f32x4 (&shm)[BY][16], f32x4 (&shs)[BY][16], f32x4& Mv,
                                                f32x4& Sv) {
    constexpr int CW = 16;
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave, cl = lane % CW, rl = lane / CW;
    float m[4], sm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) m[q] = -INFINITY;
    auto max_step = [&](const f32x4 x) {
        m[0] = fmaxf(m[0], x.x);
        m[1] = fmaxf(m[1], x.y);
        m[2] = fmaxf(m[2], x.z);
        m[3] = fmaxf(m[3], x.w);
    };
    // the same steps in the same order either way: the held rows unrolled,
    // the streamed ones one row at a time (few registers next to the held x);
    // the -inf test per column outside the row loop (inside it, the selects
    // kept both results of every element live)
    if constexpr (STREAM) {
#pragma nounroll
        for (int i = 0; i < V; ++i) max_step(row(i));
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) max_step(row(i));
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float acc = 0.0f;
        if (m[q] != -INFINITY) {
            if constexpr (STREAM) {
#pragma nounroll
                for (int i = 0; i < V; ++i) acc += exs(row(i)[q] - m[q]);
            } else {
#pragma unroll
                for (int i = 0; i < V; ++i) acc += exs(row(i)[q] - m[q]);
            }
        } else {  // only -inf and NaN: NaN stays
            if constexpr (STREAM) {
#pragma nounroll
                for (int i = 0; i < V; ++i) {
                    const float v = row(i)[q];
                    acc += (v != v) ? v : 0.0f;
                }
            } else {
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const float v = row(i)[q];
                    acc += (v != v) ? v : 0.0f;
                }
            }
        }
        sm[q] = acc;
    }
#pragma unroll
    for (int off = CW; off <= 32; off <<= 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float m2 = xor_lane_f(m[q], off), s2 = xor_lane_f(sm[q], off);
            ms_merge(m[q], sm[q], m2, s2);
        }
    }
    __syncthreads();  // shm / shs may still be read from an earlier call
    if (rl == 0) {
        shm[w][cl] = f32x4{m[0], m[1], m[2], m[3]};
        shs[w][cl] = f32x4{sm[0], sm[1], sm[2], sm[3]};
    }
    __syncthreads();
    Mv = shm[0][cl];
    Sv = shs[0][cl];
    for (int k = 1; k < BY; ++k) {
        const f32x4 mk = shm[k][cl], sk = shs[k][cl];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float M = Mv[q], S = Sv[q];
            ms_merge(M, S, mk[q], sk[q]);
            Mv[q] = M;
            Sv[q] = S;
        }
    }
}

template <int MODE, int BY, int V, bool NT>
__global__ __launch_bounds__(kWave * BY) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_smx_cols4p(SmxColArgs p, unsigned epoch, int spin) {
    static_assert(MODE == FWD || MODE == FWD_LOG, "forward only");
    constexpr int CW = 16, RW = kWave / CW, RS = RW * BY, PR = RS * V;  // PR rows per piece
    __shared__ f32x4 shm[BY][CW];
    __shared__ f32x4 shs[BY][CW];
    __shared__ f32x4 pm[2][CW], ps[2][CW];
    __shared__ int missing;
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave, cl = lane % CW, rl = lane / CW;
    const long long ncg = (p.inner + 4 * CW - 1) / (4 * CW);
    const long long gi = blockIdx.x / 2;  // column group
    const int pc = (int)(blockIdx.x % 2);
    const long long o = gi / ncg;
    const long long c = (gi - o * ncg) * (4 * CW) + 4 * cl;
    const bool live = c < p.inner;
    const float* pa = p.a + o * p.a_so + (live ? c : 0);
    float* po = p.out + o * p.n * p.inner + (live ? c : 0);
    const int n = live ? (int)p.n : 0;
    const f32x4 ninf = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    auto rows_of = [&](int piece, int i) { return piece * PR + rl + RW * w + i * RS; };
    auto load = [&](int piece, int i) -> f32x4 {
        const int r = rows_of(piece, i);
        if (r >= min(n, (piece + 1) * PR)) return ninf;
        float v[4];
        vld<4, false>(v, pa + (long long)r * p.a_sn);
        return f32x4{v[0], v[1], v[2], v[3]};
    };
    f32x4 x[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int r = rows_of(pc, i);
        if (r < min(n, (pc + 1) * PR)) {
            float v[4];
            vld<4, NT>(v, pa + (long long)r * p.a_sn);
            x[i] = f32x4{v[0], v[1], v[2], v[3]};
        } else {
            x[i] = ninf;
        }
    }
    f32x4 Mv, Sv;
    col_piece_stats<BY, V, false>([&](int i) { return x[i]; }, shm, shs, Mv, Sv);
    const int other = pc ^ 1;
    if (w == 0 && rl == 0) {
        pm[pc][cl] = Mv;
        ps[pc][cl] = Sv;
        unsigned long long* slot = smx_slots;
        const unsigned long long tag = (unsigned long long)epoch << 32;
        const long long mine = ((gi * 2 + pc) * CW + cl) * 8, theirs = ((gi * 2 + other) * CW + cl) * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            __hip_atomic_exchange(slot + ((mine + q) & (kSmxSlots - 1)), tag | __float_as_uint(Mv[q]),
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_exchange(slot + ((mine + 4 + q) & (kSmxSlots - 1)), tag | __float_as_uint(Sv[q]),
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        unsigned need = 0xffu;  // bit j: slot j of the other piece not seen yet
        float got[8];
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        for (;;) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (!((need >> j) & 1u)) continue;
                const unsigned long long v = __hip_atomic_fetch_or(slot + ((theirs + j) & (kSmxSlots - 1)), 0ull,
                                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((unsigned)(v >> 32) == epoch) {
                    got[j] = __uint_as_float((unsigned)v);
                    need &= ~(1u << j);
                }
            }
            if (need == 0 || __builtin_amdgcn_s_memrealtime() - t0 > (unsigned long long)spin) break;
            __builtin_amdgcn_s_sleep(2);
        }
        if (need == 0) {
            pm[other][cl] = f32x4{got[0], got[1], got[2], got[3]};
            ps[other][cl] = f32x4{got[4], got[5], got[6], got[7]};
        }
        // any of the 16 owner lanes short: the whole workgroup recomputes
        const bool short_any = __ballot(need != 0) != 0ull;
        if (lane == 0) missing = short_any ? 1 : 0;
    }
    __syncthreads();
    if (missing) {  // uniform
        f32x4 Mo, So;
        col_piece_stats<BY, V, true>([&](int i) { return load(other, i); }, shm, shs, Mo, So);
        if (w == 0 && rl == 0) {
            pm[other][cl] = Mo;
            ps[other][cl] = So;
        }
        __syncthreads();
    }
    float st0[4], st1[4];
    {
        const f32x4 m0 = pm[0][cl], s0 = ps[0][cl], m1 = pm[1][cl], s1 = ps[1][cl];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float M = m0[q], S = s0[q];
            ms_merge(M, S, m1[q], s1[q]);
            if (M == -INFINITY) {
                st0[q] = NAN;
                st1[q] = NAN;
            } else {
                st0[q] = M;
                st1[q] = (MODE == FWD) ? 1.0f / S : logf(S);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int r = rows_of(pc, i);
        if (r < min(n, (pc + 1) * PR)) {
            float out[4];
            const float xv[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) out[q] = outv<MODE>(xv[q], 0.0f, st0[q], st1[q]);
            vst<4, NT>(po + (long long)r * p.inner, out);
        }
    }
}

// ---------------------------------------------------------------------------
// Float64 inputs (the reference's composite runs in the input dtype, so a
// Float64 tensor gives a Float64 softmax).  Same semantics as the float32
// kernels, computed in double with exp / log: two passes over a slice.
//   k_smx_f64_rows: one 256-thread workgroup per slice: unit-stride slices,
//                   and strided ones when there are fewer than 64 per CU;
//   k_smx_f64_cols: any other layout, one thread per (outer, inner) slice
//                   (consecutive threads take consecutive inner indices).
// ---------------------------------------------------------------------------
struct SmxF64Args {
    const double* a;
    const double* b;
    double* out;  // dense [outer, n, inner]
    long long outer, n, inner;
    long long a_so, a_sn, a_si;
    long long b_so, b_sn, b_si;
};

__device__ __forceinline__ void ms_merge_d(double& m, double& s, double m2, double s2) {
    const double M = fmax(m, m2);
    if (M == -INFINITY) {
        s += s2;
        return;
    }
    s = (m == -INFINITY ? s : s * exp(m - M)) + (m2 == -INFINITY ? s2 : s2 * exp(m2 - M));
    m = M;
}

__device__ __forceinline__ void ms_add_d(double& m, double& s, double x) {
    if (x > m) {  // a NaN x never raises m
        s = (m == -INFINITY) ? s : s * exp(m - x);
        m = x;
    }
    if (m == -INFINITY) s += (x != x) ? x : 0.0;
    else s += exp(x - m);
}

template <int MODE>
__device__ __forceinline__ double outv_d(double a, double b, double st0, double st1) {
    if constexpr (MODE == FWD) return exp(a - st0) * st1;
    else if constexpr (MODE == FWD_LOG) return (a - st0) - st1;
    else if constexpr (MODE == BWD) return (a - st0) * b;
    else return a - exp(b) * st0;
}

template <int MODE>
__device__ __forceinline__ void fin_d(double m, double s, double& st0, double& st1) {
    if constexpr (MODE < BWD) {
        if (m == -INFINITY) {
            st0 = NAN;
            st1 = NAN;
        } else {
            st0 = m;
            st1 = (MODE == FWD) ? 1.0 / s : log(s);
        }
    } else {
        st0 = s;
        st1 = 0.0;
    }
}

// One 256-thread workgroup per slice.  UNIT: unit-stride slices (rows);
// otherwise slice blockIdx.x = (outer, inner) walked with its strides, which
// keeps few long strided slices (softmax over dim 0 of [1e6, 2]) on many
// threads.
template <int MODE, bool UNIT>
__global__ __launch_bounds__(256) void k_smx_f64_rows(SmxF64Args p) {
    constexpr bool BW = MODE >= BWD;
    __shared__ double shm[4], shs[4];
    const long long c = blockIdx.x;
    const long long o = UNIT ? c : c / p.inner, i = UNIT ? 0 : c - o * p.inner;
    const long long sa = UNIT ? 1 : p.a_sn, sb = UNIT ? 1 : p.b_sn, so = UNIT ? 1 : p.inner;
    const double* pa = p.a + o * p.a_so + i * p.a_si;
    const double* pb = BW ? p.b + o * p.b_so + i * p.b_si : nullptr;
    double* po = p.out + o * p.n * p.inner + i;
    const int t = threadIdx.x;
    double m = -INFINITY, s = 0.0;
    for (long long e = t; e < p.n; e += 256) {
        if constexpr (!BW) ms_add_d(m, s, pa[e * sa]);
        else s += (MODE == BWD) ? pa[e * sa] * pb[e * sb] : pa[e * sa];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const double m2 = __shfl_xor(m, o, kWave), s2 = __shfl_xor(s, o, kWave);
        if constexpr (!BW) ms_merge_d(m, s, m2, s2);
        else s += s2;
    }
    if (__lane_id() == 0) {
        shm[t / kWave] = m;
        shs[t / kWave] = s;
    }
    __syncthreads();
    m = shm[0];
    s = shs[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) {
        if constexpr (!BW) ms_merge_d(m, s, shm[i], shs[i]);
        else s += shs[i];
    }
    double st0, st1;
    fin_d<MODE>(m, s, st0, st1);
    for (long long e = t; e < p.n; e += 256)
        po[e * so] = outv_d<MODE>(pa[e * sa], BW ? pb[e * sb] : 0.0, st0, st1);
}

template <int MODE>
__global__ __launch_bounds__(256) void k_smx_f64_cols(SmxF64Args p) {
    constexpr bool BW = MODE >= BWD;
    const long long cols = p.outer * p.inner;
    for (long long c = (long long)blockIdx.x * 256 + threadIdx.x; c < cols; c += (long long)gridDim.x * 256) {
        const long long o = c / p.inner, i = c - o * p.inner;
        const double* pa = p.a + o * p.a_so + i * p.a_si;
        const double* pb = BW ? p.b + o * p.b_so + i * p.b_si : nullptr;
        double* po = p.out + o * p.n * p.inner + i;
        double m = -INFINITY, s = 0.0;
        for (long long r = 0; r < p.n; ++r) {
            if constexpr (!BW) ms_add_d(m, s, pa[r * p.a_sn]);
            else s += (MODE == BWD) ? pa[r * p.a_sn] * pb[r * p.b_sn] : pa[r * p.a_sn];
        }
        double st0, st1;
        fin_d<MODE>(m, s, st0, st1);
        for (long long r = 0; r < p.n; ++r)
            po[r * p.inner] = outv_d<MODE>(pa[r * p.a_sn], BW ? pb[r * p.b_sn] : 0.0, st0, st1);
    }
}

template <int MODE>
int run_f64(const SmxF64Args& a, hipStream_t st) {
    const long long cols = a.outer * a.inner;
    if (a.inner == 1 && a.a_sn == 1 && (MODE < BWD || a.b_sn == 1)) {
        hipLaunchKernelGGL((k_smx_f64_rows<MODE, true>), dim3((unsigned)a.outer), dim3(256), 0, st, a);
    } else if (cols < 64LL * device_info().cus && a.n >= 256) {
        // fewer slices than 64 per CU: a workgroup per slice instead of a thread
        hipLaunchKernelGGL((k_smx_f64_rows<MODE, false>), dim3((unsigned)cols), dim3(256), 0, st, a);
    } else {
        const long long blocks = std::max(1LL, std::min((cols + 255) / 256, (long long)device_info().cus * 16));
        hipLaunchKernelGGL((k_smx_f64_cols<MODE>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    return check_launch("tpr_softmax (float64)");
}

// ---------------------------------------------------------------------------
// Host planner
// ---------------------------------------------------------------------------
template <int MODE, int G, int V, int VW>
int launch_rows(const SmxArgs& a, hipStream_t st) {
    constexpr int BLK = G > 256 ? G : 256;
    constexpr int RPB = BLK / G;
    const long long blocks = (a.rows + RPB - 1) / RPB;
    if (a.nt) hipLaunchKernelGGL((k_smx_rows<MODE, G, V, VW, true>), dim3((unsigned)blocks), dim3(BLK), 0, st, a);
    else hipLaunchKernelGGL((k_smx_rows<MODE, G, V, VW, false>), dim3((unsigned)blocks), dim3(BLK), 0, st, a);
    return check_launch("tpr_softmax (rows)");
}

// Single-pass variants: VW = 4 -> G in {16, 64, 256, 1024}, V in {1, 2, 4, 8},
// and forward rows of 16385..32768 floats on 512 lanes with V = 16 (two
// workgroups per CU, so one loads while the other reduces: 67% vs 55% of the
// HBM peak with one 1024-lane workgroup per CU); VW = 1 -> G in {64, 256, 1024},
// V in {4, 16} (backward: 4).  Returns -1 when the row is too long.
template <int MODE>
int rows_single(const SmxArgs& a, int vw, hipStream_t st) {
    constexpr bool BW = MODE >= BWD;
    const long long n = a.n;
    if (vw == 4) {
        const long long q = (n + 3) / 4;  // vectors per row
        const int vmax = 8;
        auto pick = [&](int g) -> int {  // smallest V with g*V >= q, or 0
            for (int v = 1; v <= vmax; v *= 2)
                if ((long long)g * v >= q) return v;
            return 0;
        };
        // fewest lanes that keep V <= 4, else the widest workgroup with V = 8
        if constexpr (!BW) {
            if (knobs().smx_lanes != 1024 && q > 4096 && q <= 8192) return launch_rows<MODE, 512, 16, 4>(a, st);
        }
        for (int g : {16, 64, 256, 1024}) {
            const int v = pick(g);
            if (v == 0 || (v > 4 && g < 1024)) continue;
#define TPR_SMX_V(GG)                                                              \
    switch (v) {                                                                   \
        case 1: return launch_rows<MODE, GG, 1, 4>(a, st);                         \
        case 2: return launch_rows<MODE, GG, 2, 4>(a, st);                         \
        case 4: return launch_rows<MODE, GG, 4, 4>(a, st);                         \
        default: return launch_rows<MODE, GG, 8, 4>(a, st);                        \
    }
            switch (g) {
                case 16: TPR_SMX_V(16)
                case 64: TPR_SMX_V(64)
                case 256: TPR_SMX_V(256)
                default: TPR_SMX_V(1024)
            }
#undef TPR_SMX_V
        }
        return -1;
    }
    for (int g : {64, 256, 1024}) {
        if ((long long)g * 4 >= n) {
            switch (g) {
                case 64: return launch_rows<MODE, 64, 4, 1>(a, st);
                case 256: return launch_rows<MODE, 256, 4, 1>(a, st);
                default: return launch_rows<MODE, 1024, 4, 1>(a, st);
            }
        }
    }
    if constexpr (!BW) {
        if (n <= 1024LL * 16) return launch_rows<MODE, 1024, 16, 1>(a, st);
    }
    return -1;
}

long long split_chunks(long long n) { return (n + kChunk - 1) / kChunk; }

// Rows too long for registers: split over (row, chunk) workgroups when the rows
// alone cannot fill the chip, else one 1024-thread workgroup per row.
bool use_split(long long rows, long long n) {
    const long long force = knobs().smx_split;
    if (force) return force > 0;
    (void)n;
    return rows < device_info().cus;
}

template <int MODE, int NT, int VR>
int launch_res_vr(const SmxArgs& a, hipStream_t st) {
    const long long q = a.n / 4;
    const long long jl = (q + kResT - 1) / kResT;  // float4 per lane
    const int vl = (int)std::max(0LL, jl - VR);
    const size_t lds_bytes = (size_t)vl * kResT * 16;
    constexpr bool BW = MODE >= BWD;
    const void* fn = BW ? reinterpret_cast<const void*>(&k_smx_res_bwd<BW ? MODE : BWD, NT, VR>)
                        : reinterpret_cast<const void*>(&k_smx_res<BW ? FWD : MODE, NT, VR>);
    if (lds_bytes > 65536) {
        // once per device for this kernel: allow the largest dynamic LDS it
        // ever takes (kResVLMax float4 per lane)
        static std::atomic<unsigned long long> done{0};
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) dev = 0;
        const unsigned long long bit = 1ull << (dev & 63);
        if (!(done.load(std::memory_order_acquire) & bit)) {
            const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     kResVLMax * kResT * 16);
            if (e != hipSuccess)
                return fail(TPR_ERR_HIP, std::string("tpr_softmax: LDS attribute: ") + hipGetErrorString(e));
            done.fetch_or(bit, std::memory_order_acq_rel);
        }
    }
    if constexpr (BW)
        hipLaunchKernelGGL((k_smx_res_bwd<MODE, NT, VR>), dim3((unsigned)a.rows), dim3(kResT), lds_bytes, st, a, vl);
    else
        hipLaunchKernelGGL((k_smx_res<MODE, NT, VR>), dim3((unsigned)a.rows), dim3(kResT), lds_bytes, st, a, vl);
    return check_launch("tpr_softmax (rows in registers + LDS)");
}

// Rows of res_min(vr) .. res_max(vr) floats, vr in {56, 40, 24, 8}.
template <int MODE>
int launch_res(const SmxArgs& a, int vr, hipStream_t st) {
    if (a.n < res_min(vr) || a.n > res_max(vr))
        return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: row length outside the resident kernel's range");
#define TPR_RES(V) \
    case V: return a.nt ? launch_res_vr<MODE, 1, V>(a, st) : launch_res_vr<MODE, 0, V>(a, st);
    switch (vr) {
        TPR_RES(56)
        TPR_RES(40)
        TPR_RES(24)
        TPR_RES(8)
        default: return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: no resident kernel with that register count");
    }
#undef TPR_RES
}

// Pieces per row for k_smx_bwd_pieces with PT-thread workgroups (0: not
// taken): softmax gradients of rows of 16384 .. kPcMax * PT * kPcVR * 4
// floats, 16-byte vectors.
int bwd_pieces(long long n, int vw, int pt, int vr) {
    if (vw != 4 || n <= 16384 || knobs().smx_pieces < 0 || knobs().smx_two_pass) return 0;
    const long long q = n / 4;
    const long long per = (long long)pt * vr;
    const long long ns = (q + per - 1) / per;
    return ns <= kPcMax ? (int)ns : 0;
}

// Per-launch tag of the partial slots, one counter for every instantiation of
// the piece kernel: they share the slots, so a tag may never repeat across them.
std::atomic<unsigned> smx_epoch_ctr{0};

template <int MODE, int PT, int VR>
int launch_bwd_pieces(const SmxArgs& a, int ns, hipStream_t st) {
    const long long grid = a.rows * ns;
    if (grid > 0x7fffffffLL) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: too many row pieces");
    const long long q = a.n / 4;
    const int pv = (int)((q + ns - 1) / ns);
    // per-launch tag of the partial-dot slots: never 0 (the slots' initial value)
    unsigned ep = smx_epoch_ctr.fetch_add(1, std::memory_order_relaxed) + 1u;
    if (ep == 0) ep = smx_epoch_ctr.fetch_add(1, std::memory_order_relaxed) + 1u;
    // wait for the row's other pieces up to 40 us (100 MHz ticks); the test
    // knob smx_spin = -1 makes every piece recompute the others instead
    const int spin = knobs().smx_spin < 0 ? 0 : 4000;
    if (a.nt) hipLaunchKernelGGL((k_smx_bwd_pieces<MODE, 1, PT, VR>), dim3((unsigned)grid), dim3(PT), 0, st, a, ns, pv, ep, spin);
    else hipLaunchKernelGGL((k_smx_bwd_pieces<MODE, 0, PT, VR>), dim3((unsigned)grid), dim3(PT), 0, st, a, ns, pv, ep, spin);
    return check_launch("tpr_softmax (gradient, row pieces)");
}

template <int MODE, int PT, int VR>
int launch_fwd_pieces(const SmxArgs& a, int ns, hipStream_t st) {
    const long long grid = a.rows * ns;
    if (grid > 0x7fffffffLL) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: too many row pieces");
    const long long q = a.n / 4;
    const int pv = (int)((q + ns - 1) / ns);
    unsigned ep = smx_epoch_ctr.fetch_add(1, std::memory_order_relaxed) + 1u;
    if (ep == 0) ep = smx_epoch_ctr.fetch_add(1, std::memory_order_relaxed) + 1u;
    const int spin = knobs().smx_spin < 0 ? 0 : 4000;
    if (a.nt) hipLaunchKernelGGL((k_smx_fwd_pieces<MODE, 1, PT, VR>), dim3((unsigned)grid), dim3(PT), 0, st, a, ns, pv, ep, spin);
    else hipLaunchKernelGGL((k_smx_fwd_pieces<MODE, 0, PT, VR>), dim3((unsigned)grid), dim3(PT), 0, st, a, ns, pv, ep, spin);
    return check_launch("tpr_softmax (row pieces)");
}

template <int MODE>
int run_rows(const SmxArgs& a0, int vw, hipStream_t st) {
    SmxArgs a = a0;
    const int two_pass = knobs().smx_two_pass;
    // gradients: g and y both held (row pieces over workgroups), each read once
    if constexpr (MODE >= BWD) {
        // 512-thread pieces of 24 float4 per lane; measured on MI355X (us):
        // [256, 151936] 84.8 against 90.4 (256-thread pieces), 90.9 (12 float4
        // per lane, two workgroups per CU) and 96.0 (g held, y read twice);
        // [1024, 32768] 67.2 against 74.2 (g held)
        // (one slot per piece: a launch whose pieces outnumber the slots would
        // reuse a slot under the same epoch, so it takes the kernels below)
        const int ns = bwd_pieces(a.n, vw, 512, 24);
        if (ns > 0 && a.rows * ns <= kSmxSlots) return launch_bwd_pieces<MODE, 512, 24>(a, ns, st);
    } else if (knobs().smx_fwd_pieces >= 0) {
        // forward: x held by row pieces when the one-row-per-CU kernel below
        // would take more than one round and a row makes two pieces or more;
        // measured on MI355X (us, resident -> pieces): [512, 65536] 56.7 ->
        // 48.4 (log 54.5 -> 44.8), [2048, 50260] 165 -> 159 (log 164 -> 151),
        // [1024, 128256] 197 -> 189, but C5 [256, 151936] 57.1 -> 60.8 (one
        // round: every CU loads, then every CU writes, at full rate anyway)
        // and [1024, 32768] (one piece per row) 43.9 -> 48.3.  Rows longer than
        // one CU holds (> 153600 floats) take them at any row count instead of
        // streaming twice: [64, 262144] 44.4 -> 28.6, [32, 500000] 45.9 ->
        // 33.9, [512, 163840] 153 -> 120, [8, 655360] 25.0 -> 20.8.  The test
        // knob smx_fwd_pieces = 1 takes every row the pieces can hold.
        const int ns = bwd_pieces(a.n, vw, 512, kFwdPcVR);
        if (ns > 0 && a.rows * ns * 2 <= kSmxSlots &&  // two slots per piece, none reused in a launch
            (knobs().smx_fwd_pieces > 0 || (ns >= 2 && a.rows > device_info().cus) ||
             (a.n > kResMax && knobs().smx_fwd_pieces == 0)))
            return launch_fwd_pieces<MODE, 512, kFwdPcVR>(a, ns, st);
    }
    // rows of 16384..153600 floats, at least one per CU: one row per CU in
    // registers + LDS (forward: x held; gradients: g held, y streamed).
    // Measured on MI355X at [1024, 32768] against the register-only kernels:
    // softmax 44.6 vs 48.8 us, log_softmax 43.6 vs 50.7 us, their gradients
    // 74.6 / 68.0 vs 79.2 / 80.9 us.  Fewer rows than CUs take the split
    // (row, chunk) kernels below, which use the whole chip.
    if (!two_pass && knobs().smx_res >= 0 && !a.part && vw == 4 && a.n >= res_min(8) && a.n <= kResMax) {
        int vr = 0;
        for (int c : {56, 40, 24, 8})
            if (vr == 0 && a.n >= res_min(c)) vr = c;
        return launch_res<MODE>(a, vr, st);
    }
    if (!two_pass) {
        const int rc = rows_single<MODE>(a, vw, st);
        if (rc >= 0) return rc;
    }
    constexpr bool BW = MODE >= BWD;
    if (a.part) {
        const long long blocks = a.rows * a.chunks;
        if (vw == 4) {
            hipLaunchKernelGGL((k_smx_part<MODE, 4>), dim3((unsigned)blocks), dim3(256), 0, st, a);
            if (a.nt) hipLaunchKernelGGL((k_smx_apply<MODE, 4, true>), dim3((unsigned)blocks), dim3(256), 0, st, a);
            else hipLaunchKernelGGL((k_smx_apply<MODE, 4, false>), dim3((unsigned)blocks), dim3(256), 0, st, a);
        } else {
            hipLaunchKernelGGL((k_smx_part<MODE, 1>), dim3((unsigned)blocks), dim3(256), 0, st, a);
            if (a.nt) hipLaunchKernelGGL((k_smx_apply<MODE, 1, true>), dim3((unsigned)blocks), dim3(256), 0, st, a);
            else hipLaunchKernelGGL((k_smx_apply<MODE, 1, false>), dim3((unsigned)blocks), dim3(256), 0, st, a);
        }
        return check_launch("tpr_softmax (split rows)");
    }
    if (vw == 4 && a.nt) hipLaunchKernelGGL((k_smx_rows2<MODE, 4, BW ? 2 : 4, true>), dim3((unsigned)a.rows), dim3(1024), 0, st, a);
    else if (vw == 4) hipLaunchKernelGGL((k_smx_rows2<MODE, 4, BW ? 2 : 4, false>), dim3((unsigned)a.rows), dim3(1024), 0, st, a);
    else if (a.nt) hipLaunchKernelGGL((k_smx_rows2<MODE, 1, BW ? 8 : 16, true>), dim3((unsigned)a.rows), dim3(1024), 0, st, a);
    else hipLaunchKernelGGL((k_smx_rows2<MODE, 1, BW ? 8 : 16, false>), dim3((unsigned)a.rows), dim3(1024), 0, st, a);
    return check_launch("tpr_softmax (long rows)");
}

template <int MODE>
int run_cols(const SmxColArgs& a, hipStream_t st) {
    constexpr bool BW = MODE >= BWD;
    auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const bool v4 = a.a_si == 1 && a.inner % 4 == 0 && a.inner >= 16 && al(a.a) && al(a.out) && a.a_so % 4 == 0 &&
                    a.a_sn % 4 == 0 && (!BW || (a.b_si == 1 && al(a.b) && a.b_so % 4 == 0 && a.b_sn % 4 == 0)) &&
                    knobs().general == 0;
    if (v4) {
        const long long blocks = a.outer * ((a.inner + 63) / 64);
        if (blocks <= 0x7fffffffLL) {
            // more waves along longer dims (measured at [64, 1024, 1024] dim 1: 16 waves 150 us,
            // 8 waves 160 us; at [16, 256, 8192] dim 1: 8 waves 70 us, 16 waves 92 us)
            // slices of 65..1024 rows (backward, two inputs: ..256) stay in
            // registers: read once
            // forward slices of 513..1024 rows: two row pieces per 64-column
            // group (8-wave workgroups, two per CU) while the grid's slots fit
            if constexpr (!BW) {
                const long long gp = 2 * blocks;
                if (a.n > 512 && a.n <= 1024 && knobs().smx_res >= 0 && knobs().smx_two_pass == 0 &&
                    knobs().smx_fwd_pieces >= 0 && knobs().smx_pieces >= 0 && gp * 128 <= kSmxSlots) {
                    unsigned ep = smx_epoch_ctr.fetch_add(1, std::memory_order_relaxed) + 1u;
                    if (ep == 0) ep = smx_epoch_ctr.fetch_add(1, std::memory_order_relaxed) + 1u;
                    const int spin = knobs().smx_spin < 0 ? 0 : 4000;
                    if (a.nt) hipLaunchKernelGGL((k_smx_cols4p<MODE, 8, 16, true>), dim3((unsigned)gp), dim3(kWave * 8), 0, st, a, ep, spin);
                    else hipLaunchKernelGGL((k_smx_cols4p<MODE, 8, 16, false>), dim3((unsigned)gp), dim3(kWave * 8), 0, st, a, ep, spin);
                    return check_launch("tpr_softmax (strided dim, row pieces)");
                }
            }
            if (a.n > 64 && a.n <= (BW ? 256 : 1024) && knobs().smx_res >= 0 && knobs().smx_two_pass == 0) {
                // 64-column groups (CW = 16); 32-column groups (CW = 8, two
                // workgroups per CU) measured slower: 143 vs 131 us at [64, 1024,
                // 1024] dim 1, 193 vs 111 us at [2048, 128, 256]
                const unsigned g = (unsigned)(a.outer * ((a.inner + 63) / 64));
#define TPR_C4R(BYV, VV)                                                                                          \
    {                                                                                                             \
        if (a.nt) hipLaunchKernelGGL((k_smx_cols4r<MODE, BYV, VV, 16, true>), dim3(g), dim3(kWave * BYV), 0, st, a); \
        else hipLaunchKernelGGL((k_smx_cols4r<MODE, BYV, VV, 16, false>), dim3(g), dim3(kWave * BYV), 0, st, a); \
    }
                if (a.n <= 128) TPR_C4R(8, 4)
                else if (a.n <= 256) TPR_C4R(8, 8)
                else if constexpr (!BW) {
                    if (a.n <= 512) TPR_C4R(16, 8)
                    else TPR_C4R(16, 16)
                }
#undef TPR_C4R
                return check_launch("tpr_softmax (strided dim, in registers)");
            }
            int by = a.n >= 1024 ? 16 : (a.n >= 128 ? 8 : 4);
            if (knobs().colblock == 256 || knobs().colblock == 512 || knobs().colblock == 1024) by = (int)knobs().colblock / 64;
            if (by == 16) hipLaunchKernelGGL((k_smx_cols4<MODE, 16>), dim3((unsigned)blocks), dim3(kWave * 16), 0, st, a);
            else if (by == 8) hipLaunchKernelGGL((k_smx_cols4<MODE, 8>), dim3((unsigned)blocks), dim3(kWave * 8), 0, st, a);
            else hipLaunchKernelGGL((k_smx_cols4<MODE, 4>), dim3((unsigned)blocks), dim3(kWave * 4), 0, st, a);
            return check_launch("tpr_softmax (strided dim, vectors)");
        }
    }
    const long long cols = a.outer * a.inner;
    const long long blocks = (cols + kWave - 1) / kWave;
    if (blocks > 0x7fffffffLL) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: too many slices");
    if (a.n >= 256) hipLaunchKernelGGL((k_smx_cols<MODE, 8>), dim3((unsigned)blocks), dim3(kWave * 8), 0, st, a);
    else hipLaunchKernelGGL((k_smx_cols<MODE, 4>), dim3((unsigned)blocks), dim3(kWave * 4), 0, st, a);
    return check_launch("tpr_softmax (strided dim)");
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace tpr

namespace tpr {
namespace {
bool rows_path(const tpr_softmax_desc* d) {
    const bool bw = d->mode >= TPR_SOFTMAX_BWD;
    return d->inner == 1 && d->a_strides[1] == 1 && (!bw || d->b_strides[1] == 1) && d->outer <= 0x7fffffffLL &&
           knobs().general == 0;
}

// Workspace of the split-row kernels (zero when they are not used): one float2
// per (row, chunk).  Independent of pointer alignment: it assumes the scalar
// single-pass capacity (16384 floats forward, 4096 backward).
size_t smx_workspace(const tpr_softmax_desc* d) {
    if (d->dtype == TPR_FLOAT64 || !rows_path(d) || d->outer == 0 || d->n == 0) return 0;
    const bool bw = d->mode >= TPR_SOFTMAX_BWD;
    const long long cap1 = bw ? 4096 : 16384;
    if (!(knobs().smx_two_pass || d->n > cap1)) return 0;
    if (!use_split(d->outer, d->n)) return 0;
    const long long blocks = d->outer * split_chunks(d->n);
    if (blocks > 0x7fffffffLL) return 0;
    return (size_t)blocks * sizeof(float2);
}
}  // namespace
}  // namespace tpr

extern "C" size_t tpr_softmax_workspace_bytes(const tpr_softmax_desc* d) {
    if (!d || d->mode < TPR_SOFTMAX_FWD || d->mode > TPR_LOG_SOFTMAX_BWD || d->outer < 0 || d->n < 0 || d->inner < 0)
        return 0;
    return tpr::smx_workspace(d);
}

extern "C" int tpr_softmax(const tpr_softmax_desc* d, const void* a, const void* b, void* out, void* workspace,
                           size_t workspace_bytes, void* stream) {
    using namespace tpr;
    if (!d) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: null descriptor");
    if (d->mode < TPR_SOFTMAX_FWD || d->mode > TPR_LOG_SOFTMAX_BWD)
        return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: unknown mode");
    if (d->dtype != TPR_FLOAT32 && d->dtype != TPR_FLOAT64)
        return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_softmax: float32 and float64 only");
    if (d->outer < 0 || d->n < 0 || d->inner < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: negative extent");
    if (d->outer == 0 || d->n == 0 || d->inner == 0) return TPR_OK;
    const bool bw = d->mode >= TPR_SOFTMAX_BWD;
    if (!a || !out || (bw && !b)) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (d->dtype == TPR_FLOAT64) {
        if (d->outer > 0x7fffffffLL) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: too many slices");
        SmxF64Args f{static_cast<const double*>(a), static_cast<const double*>(b), static_cast<double*>(out),
                     d->outer, d->n, d->inner, d->a_strides[0], d->a_strides[1], d->a_strides[2],
                     bw ? d->b_strides[0] : 0, bw ? d->b_strides[1] : 0, bw ? d->b_strides[2] : 0};
        switch (d->mode) {
            case TPR_SOFTMAX_FWD: return run_f64<FWD>(f, st);
            case TPR_LOG_SOFTMAX_FWD: return run_f64<FWD_LOG>(f, st);
            case TPR_SOFTMAX_BWD: return run_f64<BWD>(f, st);
            default: return run_f64<BWD_LOG>(f, st);
        }
    }
    const float* pa = static_cast<const float*>(a);
    const float* pb = static_cast<const float*>(b);
    float* po = static_cast<float*>(out);

    if (rows_path(d)) {
        SmxArgs r{pa, pb, po, d->outer, d->n, d->a_strides[0], bw ? d->b_strides[0] : 0, 0, 0, nullptr};
        const size_t wsn = smx_workspace(d);
        if (wsn) {
            if (!workspace || workspace_bytes < wsn)
                return fail(TPR_ERR_WORKSPACE, "tpr_softmax: workspace smaller than tpr_softmax_workspace_bytes");
            r.part = static_cast<float2*>(workspace);
            r.chunks = (int)split_chunks(d->n);
        }
        const long long bytes = d->outer * d->n * 4LL * (bw ? 3 : 2);
        r.nt = knobs().nt ? (knobs().nt > 0) : (bytes >= (256LL << 20));
        const bool v4 = d->n % 4 == 0 && al16(pa) && al16(po) && (d->outer == 1 || r.sa % 4 == 0) &&
                        (!bw || (al16(pb) && (d->outer == 1 || r.sb % 4 == 0)));
        const int vw = v4 ? 4 : 1;
        switch (d->mode) {
            case TPR_SOFTMAX_FWD: return run_rows<FWD>(r, vw, st);
            case TPR_LOG_SOFTMAX_FWD: return run_rows<FWD_LOG>(r, vw, st);
            case TPR_SOFTMAX_BWD: return run_rows<BWD>(r, vw, st);
            default: return run_rows<BWD_LOG>(r, vw, st);
        }
    }
    SmxColArgs c{pa, pb, po, d->outer, d->n, d->inner,
                 d->a_strides[0], d->a_strides[1], d->a_strides[2],
                 bw ? d->b_strides[0] : 0, bw ? d->b_strides[1] : 0, bw ? d->b_strides[2] : 0, 0};
    c.nt = knobs().nt ? (knobs().nt > 0 ? 1 : 0) : (d->outer * d->n * d->inner * 4LL >= (256LL << 20) ? 1 : 0);
    switch (d->mode) {
        case TPR_SOFTMAX_FWD: return run_cols<FWD>(c, st);
        case TPR_LOG_SOFTMAX_FWD: return run_cols<FWD_LOG>(c, st);
        case TPR_SOFTMAX_BWD: return run_cols<BWD>(c, st);
        default: return run_cols<BWD_LOG>(c, st);
    }
}
