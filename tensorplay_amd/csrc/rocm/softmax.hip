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
//   * rows that fit in registers (up to 32768 floats per 1024-thread
//     workgroup) are read once and written once -- k_smx_rows;
//   * longer rows stream twice: an online (max, sum-of-exp) pass, then the
//     output pass -- k_smx_rows2;
//   * a strided softmax dim (inner extent > 1, or a non-unit dim stride)
//     keeps one column per lane, thread rows across the dim, an LDS merge of
//     the per-wave states, and also streams twice -- k_smx_cols.
// exp(d) is exp2(d * log2(e)); sums accumulate in fp32 per lane and combine in
// a fixed tree, so results are deterministic run to run.

#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "common.h"

namespace tpr {
namespace {

constexpr float kL2E = 1.4426950408889634f;
enum { FWD = 0, FWD_LOG = 1, BWD = 2, BWD_LOG = 3 };

__device__ __forceinline__ float ex(float d) { return exp2f(d * kL2E); }

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int VW>
struct Vec;
template <>
struct Vec<4> {
    __device__ static void load(float (&v)[4], const float* p, int nt) {
        f32x4 t;
        if (nt) t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
        else t = *reinterpret_cast<const f32x4*>(p);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
    __device__ static void store(float* p, const float (&v)[4], int nt) {
        f32x4 t = {v[0], v[1], v[2], v[3]};
        if (nt) __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p));
        else *reinterpret_cast<f32x4*>(p) = t;
    }
};
template <>
struct Vec<1> {
    __device__ static void load(float (&v)[1], const float* p, int nt) {
        v[0] = nt ? __builtin_nontemporal_load(p) : *p;
    }
    __device__ static void store(float* p, const float (&v)[1], int nt) {
        if (nt) __builtin_nontemporal_store(v[0], p);
        else *p = v[0];
    }
};

// Sum / max over G consecutive lanes (G <= 64: xor shuffles inside the wave;
// G > 64: one workgroup of G threads, via `sh` (G / 64 floats, private to this
// call site)).  The result is valid in every lane of the group.
template <int G, bool MAX>
__device__ __forceinline__ float grp(float v, float* sh) {
    constexpr int W = G < kWave ? G : kWave;
#pragma unroll
    for (int o = W / 2; o >= 1; o >>= 1) {
        const float t = __shfl_xor(v, o, kWave);
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
    s = (m == -INFINITY ? s : s * ex(m - M)) + (m2 == -INFINITY ? s2 : s2 * ex(m2 - M));
    m = M;
}

// Add a chunk of K values to (m, s).
template <int K>
__device__ __forceinline__ void ms_add(float& m, float& s, const float* x) {
    float cm = x[0];
#pragma unroll
    for (int i = 1; i < K; ++i) cm = fmaxf(cm, x[i]);
    if (cm > m) {
        s = (m == -INFINITY) ? s : s * ex(m - cm);
        m = cm;
    }
    if (m == -INFINITY) {
#pragma unroll
        for (int i = 0; i < K; ++i) s += (x[i] != x[i]) ? x[i] : 0.0f;
    } else {
#pragma unroll
        for (int i = 0; i < K; ++i) s += ex(x[i] - m);
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
};

// ---------------------------------------------------------------------------
// Register-resident rows: G lanes per row, each lane holds V vectors of VW
// floats (vector j of lane l covers elements (j*G + l)*VW ...).  Read once,
// write once.  G <= 256: 256-thread workgroups holding 256/G rows; G > 256:
// one row per G-thread workgroup.
// ---------------------------------------------------------------------------
template <int MODE, int G, int V, int VW>
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
            Vec<VW>::load(a[j], pa + e, p.nt);
            if constexpr (BW) Vec<VW>::load(b[j], pb + e, p.nt);
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
                for (int c = 0; c < VW; ++c) s += ex(a[j][c] - m);
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
            Vec<VW>::store(po + e, o, p.nt);
        }
    }
}

// ---------------------------------------------------------------------------
// Long rows: one 1024-thread workgroup per row, two streaming passes.  Pass 1
// accumulates the online (max, sum) state (forward) or the dot / sum
// (backward); pass 2 re-reads the row and writes the output.  Pass 1 uses
// ordinary loads so the row stays in the caches for pass 2.
// ---------------------------------------------------------------------------
template <int MODE, int VW, int U>
__global__ __launch_bounds__(1024) void k_smx_rows2(SmxArgs p) {
    constexpr int T = 1024;
    constexpr bool BW = MODE >= BWD;
    constexpr long long TILE = (long long)T * VW * U;
    __shared__ float sh[2][T / kWave];
    const long long row = blockIdx.x;
    const float* pa = p.a + row * p.sa;
    const float* pb = BW ? p.b + row * p.sb : nullptr;
    float* po = p.out + row * p.n;
    const int t = threadIdx.x;

    float st0, st1 = 0.0f;
    if constexpr (!BW) {
        float m = -INFINITY, s = 0.0f;
        for (long long base = 0; base < p.n; base += TILE) {
            float x[U][VW];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long long e = base + ((long long)u * T + t) * VW;
                if (e < p.n) {
                    Vec<VW>::load(x[u], pa + e, 0);
                } else {
#pragma unroll
                    for (int c = 0; c < VW; ++c) x[u][c] = -INFINITY;
                }
            }
            ms_add<U * VW>(m, s, &x[0][0]);
        }
        grp_ms<T>(m, s, sh[0], sh[1]);
        if (m == -INFINITY) {
            st0 = NAN;
            st1 = NAN;
        } else {
            st0 = m;
            st1 = (MODE == FWD) ? 1.0f / s : logf(s);
        }
    } else {
        float s = 0.0f;
        for (long long base = 0; base < p.n; base += TILE) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long long e = base + ((long long)u * T + t) * VW;
                if (e < p.n) {
                    float g[VW], y[VW];
                    Vec<VW>::load(g, pa + e, 0);
                    Vec<VW>::load(y, pb + e, 0);
#pragma unroll
                    for (int c = 0; c < VW; ++c) s += (MODE == BWD) ? g[c] * y[c] : g[c];
                }
            }
        }
        st0 = grp<T, false>(s, sh[0]);
    }

    for (long long base = 0; base < p.n; base += TILE) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long e = base + ((long long)u * T + t) * VW;
            if (e < p.n) {
                float x[VW], y[VW], o[VW];
                Vec<VW>::load(x, pa + e, p.nt);
                if constexpr (BW) Vec<VW>::load(y, pb + e, p.nt);
#pragma unroll
                for (int c = 0; c < VW; ++c) o[c] = outv<MODE>(x[c], BW ? y[c] : 0.0f, st0, st1);
                Vec<VW>::store(po + e, o, p.nt);
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

// ---------------------------------------------------------------------------
// Host planner
// ---------------------------------------------------------------------------
template <int MODE, int G, int V, int VW>
int launch_rows(const SmxArgs& a, hipStream_t st) {
    constexpr int BLK = G > 256 ? G : 256;
    constexpr int RPB = BLK / G;
    const long long blocks = (a.rows + RPB - 1) / RPB;
    hipLaunchKernelGGL((k_smx_rows<MODE, G, V, VW>), dim3((unsigned)blocks), dim3(BLK), 0, st, a);
    return check_launch("tpr_softmax (rows)");
}

// Single-pass variants: VW = 4 -> G in {16, 64, 256, 1024}, V in {1, 2, 4, 8}
// (backward: V <= 4, two loaded operands); VW = 1 -> G in {64, 256, 1024},
// V in {4, 16} (backward: 4).  Returns -1 when the row is too long.
template <int MODE>
int rows_single(const SmxArgs& a, int vw, hipStream_t st) {
    constexpr bool BW = MODE >= BWD;
    const long long n = a.n;
    if (vw == 4) {
        const long long q = (n + 3) / 4;  // vectors per row
        const int vmax = BW ? 4 : 8;
        auto pick = [&](int g) -> int {  // smallest V with g*V >= q, or 0
            for (int v = 1; v <= vmax; v *= 2)
                if ((long long)g * v >= q) return v;
            return 0;
        };
        // fewest lanes that keep V <= 4, else the widest workgroup with V = 8
        for (int g : {16, 64, 256, 1024}) {
            const int v = pick(g);
            if (v == 0 || (v > 4 && g < 1024)) continue;
#define TPR_SMX_V(GG)                                                              \
    switch (v) {                                                                   \
        case 1: return launch_rows<MODE, GG, 1, 4>(a, st);                         \
        case 2: return launch_rows<MODE, GG, 2, 4>(a, st);                         \
        case 4: return launch_rows<MODE, GG, 4, 4>(a, st);                         \
        default: if constexpr (!BW) return launch_rows<MODE, GG, 8, 4>(a, st);     \
                 return -1;                                                        \
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

template <int MODE>
int run_rows(const SmxArgs& a, int vw, hipStream_t st) {
    const int two_pass = knobs().smx_two_pass;
    if (!two_pass) {
        const int rc = rows_single<MODE>(a, vw, st);
        if (rc >= 0) return rc;
    }
    if (vw == 4) hipLaunchKernelGGL((k_smx_rows2<MODE, 4, 4>), dim3((unsigned)a.rows), dim3(1024), 0, st, a);
    else hipLaunchKernelGGL((k_smx_rows2<MODE, 1, 8>), dim3((unsigned)a.rows), dim3(1024), 0, st, a);
    return check_launch("tpr_softmax (long rows)");
}

template <int MODE>
int run_cols(const SmxColArgs& a, hipStream_t st) {
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

extern "C" int tpr_softmax(const tpr_softmax_desc* d, const void* a, const void* b, void* out, void* stream) {
    using namespace tpr;
    if (!d) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: null descriptor");
    if (d->mode < TPR_SOFTMAX_FWD || d->mode > TPR_LOG_SOFTMAX_BWD)
        return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: unknown mode");
    if (d->dtype != TPR_FLOAT32) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_softmax: float32 only");
    if (d->outer < 0 || d->n < 0 || d->inner < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: negative extent");
    if (d->outer == 0 || d->n == 0 || d->inner == 0) return TPR_OK;
    const bool bw = d->mode >= TPR_SOFTMAX_BWD;
    if (!a || !out || (bw && !b)) return fail(TPR_ERR_INVALID_ARG, "tpr_softmax: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const float* pa = static_cast<const float*>(a);
    const float* pb = static_cast<const float*>(b);
    float* po = static_cast<float*>(out);

    const bool rows = d->inner == 1 && d->a_strides[1] == 1 && (!bw || d->b_strides[1] == 1) &&
                      d->outer <= 0x7fffffffLL && knobs().general == 0;
    if (rows) {
        SmxArgs r{pa, pb, po, d->outer, d->n, d->a_strides[0], bw ? d->b_strides[0] : 0, 0};
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
                 bw ? d->b_strides[0] : 0, bw ? d->b_strides[1] : 0, bw ? d->b_strides[2] : 0};
    switch (d->mode) {
        case TPR_SOFTMAX_FWD: return run_cols<FWD>(c, st);
        case TPR_LOG_SOFTMAX_FWD: return run_cols<FWD_LOG>(c, st);
        case TPR_SOFTMAX_BWD: return run_cols<BWD>(c, st);
        default: return run_cols<BWD_LOG>(c, st);
    }
}
