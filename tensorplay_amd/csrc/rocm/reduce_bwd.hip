// gfx950 gradients of sum / mean / var / std (full and along dims), behind
// tpr_reduce_backward().
//
// Formulas of /root/reference/config/derivatives.yaml:82-86 and :182-186,
// evaluated in float32 in the order TensorPlay's autograd composes them:
//   sum:  gx = g                                    (grad.expand(self.shape()))
//   mean: gx = (float)((double)g / count)           (grad.expand(...) / self.numel(),
//                                                    div.Scalar in double,
//                                                    ArithmeticKernels.cpp:1502-1532)
//   var:  gx = (float)((double)((g * 2) * (x - mean)) / (count - correction))
//   std:  gx = (g * (x - mean)) / (result * (float)(count - correction))
// where g, mean and result are the per-output values broadcast over the reduced
// dims (mean = the same reduction's MEAN, computed here by tpr_reduce into the
// workspace).  The reference builds each formula from four to six separate
// elementwise kernels and temporaries of the input's size; here it is one
// streaming pass (plus the mean's reduction pass for var / std).
//
// The output is dense row-major over the input's shape.  The host merges
// adjacent dims that are contiguous in the input and share reduce status, so
// the common cases (a full reduction, a reduction over a trailing or leading
// block of dims) index one or two dims; the kernel handles up to eight.

#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "common.h"

namespace tpr {
namespace {

// Division of a 32-bit index by an invariant divisor d >= 1 as a multiply-high
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, unsigned case): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (umulhi(n, m) + n) >> l for every
// n < 2^32 (the sum is formed in 64 bits).
struct FastDiv {
    unsigned m;
    unsigned l;
};

FastDiv make_fastdiv(unsigned long long d) {
    unsigned l = 0;
    while ((1ULL << l) < d) ++l;
    const unsigned long long m = (((1ULL << 32) * ((1ULL << l) - d)) / d) + 1;
    return FastDiv{(unsigned)m, l};
}

__device__ __forceinline__ unsigned fastdiv(unsigned n, FastDiv f) {
    return (unsigned)(((unsigned long long)__umulhi(n, f.m) + n) >> f.l);
}

struct RbArgs {
    int nd;
    FastDiv fd[TPR_MAX_DIMS];
    long long sizes[TPR_MAX_DIMS];
    long long xs[TPR_MAX_DIMS];  // input strides (elements)
    long long os[TPR_MAX_DIMS];  // per-output value strides (0 on reduced dims)
    long long total;
    const float* g;
    const float* x;
    const float* mean;
    const float* res;
    float* gi;
    double count;   // element count of one reduction (mean's divisor)
    double denom;   // count - correction (var)
    float denom_f;  // (float)(count - correction) (std: result * Scalar)
    double inv_denom;  // 1 / denom (the row kernel multiplies instead of dividing)
};

enum { B_SUM = 0, B_MEAN = 1, B_VAR = 2, B_STD = 3 };

template <int OP>
__device__ __forceinline__ float bwd_value(const RbArgs& a, long long xo, long long so) {
    const float g = a.g[so];
    if constexpr (OP == B_SUM) {
        return g;
    } else if constexpr (OP == B_MEAN) {
        return g;  // divided by count per output beforehand (k_mean_scale)
    } else if constexpr (OP == B_VAR) {
        const float t = (g * 2.0f) * (a.x[xo] - a.mean[so]);
        return (float)((double)t / a.denom);
    } else {
        const float t = g * (a.x[xo] - a.mean[so]);
        return t / (a.res[so] * a.denom_f);
    }
}

// VEC consecutive outputs per thread (VEC = 4: the innermost merged dim has a
// size divisible by 4, so a vector never crosses it); IdxT: 32-bit index math
// when the element count allows.
template <int OP, int VEC, class IdxT>
__global__ __launch_bounds__(256) void k_red_bwd(RbArgs a) {
    const IdxT nvec = (IdxT)(a.total / VEC);
    const int last = a.nd - 1;
    for (IdxT v = (IdxT)blockIdx.x * 256 + threadIdx.x; v < nvec; v += (IdxT)gridDim.x * 256) {
        IdxT e = v * VEC;
        long long xo = 0, so = 0;
        for (int d = last; d >= 0; --d) {
            const IdxT sz = (IdxT)a.sizes[d];
            IdxT q;
            if constexpr (sizeof(IdxT) == 4) q = fastdiv(e, a.fd[d]);
            else q = e / sz;
            const IdxT c = e - q * sz;
            e = q;
            xo += (long long)c * a.xs[d];
            so += (long long)c * a.os[d];
        }
        float o[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[k] = bwd_value<OP>(a, xo + k * a.xs[last], so + k * a.os[last]);
        float* dst = a.gi + (long long)v * VEC;
        if constexpr (VEC == 4) {
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            f32x4 t = {o[0], o[1], o[2], o[3]};
            __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(dst));
        } else {
            __builtin_nontemporal_store(o[0], dst);
        }
    }
}

// Rows of the innermost merged dim (at least 1024 elements): a workgroup
// covers 256 * VEC * U consecutive outputs of one row (long rows, split in
// `chunks` pieces) or of rpb = CH / L whole rows (short rows).  The first rpb
// threads find the rows' offsets once (into LDS); every thread then issues the
// loads of its U vectors before any store, so short rows do not serialise on
// load latency.  U = 4 for var / std (they read x), 2 for sum / mean over
// rows shorter than 4096 elements (a workgroup then covers one or two rows)
// and 1 for sum / mean over long rows, which only write: one 16-byte store per
// thread over a grid covering the whole output writes faster than several per
// thread (measured on MI355X, a 256 MiB broadcast: 40 us against 45-52 us with
// 2-8 stores per thread).  INNER: 0 = the innermost dim is reduced (g / mean / result
// are one value per row), 1 = it is kept with unit stride in the per-output
// arrays (loaded as vectors beside x).
template <int OP, int VEC, int INNER, int U>
__global__ __launch_bounds__(256) void k_red_bwd_rows(RbArgs a, long long chunks, int rpb, long long rows) {
    constexpr int CH = 256 * VEC * U;
    constexpr bool XS = OP == B_VAR || OP == B_STD;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __shared__ long long sxo[4], sso[4];  // rpb <= CH / 1024 <= 4
    const int last = a.nd - 1;
    const long long L = a.sizes[last];
    const long long grp = blockIdx.x / chunks;
    const long long c0 = (blockIdx.x - grp * chunks) * (long long)CH;
    const int t = threadIdx.x;
    if (t < rpb) {
        long long xo = 0, so = 0, r = grp * rpb + t;
        if (r < rows) {
            for (int d = last - 1; d >= 0; --d) {
                const long long c = r % a.sizes[d];
                r /= a.sizes[d];
                xo += c * a.xs[d];
                so += c * a.os[d];
            }
        }
        sxo[t] = xo;
        sso[t] = so;
    }
    __syncthreads();
    const long long xs = a.xs[last];

    float gv[U][VEC], mv[U][VEC], rv[U][VEC], xv[U][VEC];
    long long oo[U];  // output offset of each vector, -1 = none
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long e = c0 + ((long long)u * 256 + t) * VEC;
        const long long rr = e / L;
        const long long i = e - rr * L;
        const long long row = grp * rpb + rr;
        oo[u] = -1;
        if (rr >= rpb || row >= rows) continue;
        oo[u] = row * L + i;
        const long long xo = sxo[rr], so = sso[rr];
        if constexpr (INNER == 0) {
            const float g1 = a.g[so];
            const float m1 = XS ? a.mean[so] : 0.0f;
            const float r1 = OP == B_STD ? a.res[so] : 0.0f;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                gv[u][k] = g1;
                mv[u][k] = m1;
                rv[u][k] = r1;
            }
        } else if constexpr (VEC == 4) {
            const f32x4 q = *reinterpret_cast<const f32x4*>(a.g + so + i);
            gv[u][0] = q.x; gv[u][1] = q.y; gv[u][2] = q.z; gv[u][3] = q.w;
            if constexpr (XS) {
                const f32x4 w = *reinterpret_cast<const f32x4*>(a.mean + so + i);
                mv[u][0] = w.x; mv[u][1] = w.y; mv[u][2] = w.z; mv[u][3] = w.w;
            }
            if constexpr (OP == B_STD) {
                const f32x4 w = *reinterpret_cast<const f32x4*>(a.res + so + i);
                rv[u][0] = w.x; rv[u][1] = w.y; rv[u][2] = w.z; rv[u][3] = w.w;
            }
        } else {
            gv[u][0] = a.g[so + i];
            if constexpr (XS) mv[u][0] = a.mean[so + i];
            if constexpr (OP == B_STD) rv[u][0] = a.res[so + i];
        }
        if constexpr (XS) {
            if (VEC == 4 && xs == 1) {
                const f32x4 w = *reinterpret_cast<const f32x4*>(a.x + xo + i);
                xv[u][0] = w.x; xv[u][1] = w.y; xv[u][2] = w.z; xv[u][3] = w.w;
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) xv[u][k] = a.x[xo + (i + k) * xs];
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (oo[u] < 0) continue;
        float o[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            if constexpr (OP == B_SUM || OP == B_MEAN) {
                o[k] = gv[u][k];  // MEAN: g was divided by count per output beforehand
            } else if constexpr (OP == B_VAR) {
                const float tt = (gv[u][k] * 2.0f) * (xv[u][k] - mv[u][k]);
                o[k] = (float)((double)tt / a.denom);
            } else {
                const float tt = gv[u][k] * (xv[u][k] - mv[u][k]);
                o[k] = tt / (rv[u][k] * a.denom_f);
            }
        }
        if constexpr (VEC == 4) {
            f32x4 w = {o[0], o[1], o[2], o[3]};
            __builtin_nontemporal_store(w, reinterpret_cast<f32x4*>(a.gi + oo[u]));
        } else {
            __builtin_nontemporal_store(o[0], a.gi + oo[u]);
        }
    }
}

// VAR / STD over one innermost reduced run (unit stride in x, 16-byte
// aligned, length L % 4 == 0, L <= 256 * V, every other dim kept): one wave per
// row holds the row in registers (V float4 per lane), forms the row's mean
// itself (fp32 lane sums combined in fp64, then / count as tpr_reduce's MEAN)
// and writes the gradient from registers, so x is read once instead of twice
// (the MEAN pass and the gradient pass).
template <int OP, int V>
__global__ __launch_bounds__(256) void k_vs_bwd_rows(RbArgs a, long long rows) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // uniform per wave; no barriers below
    const int last = a.nd - 1;
    const int q = (int)(a.sizes[last] >> 2);  // float4 per row
    long long xo = 0, so = 0, r = row;
    if (last == 1) {  // one kept dim (the usual case after merging): no 64-bit divisions
        xo = row * a.xs[0];
        so = row * a.os[0];
    } else {
        for (int d = last - 1; d >= 0; --d) {
            const long long c = r % a.sizes[d];
            r /= a.sizes[d];
            xo += c * a.xs[d];
            so += c * a.os[d];
        }
    }
    const f32x4* px = reinterpret_cast<const f32x4*>(a.x + xo);
    f32x4 v[V];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int e = j * 64 + lane;
        if (e < q) {
            v[j] = __builtin_nontemporal_load(px + e);
            s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
        }
    }
    double sd = s;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sd += __shfl_xor(sd, o, 64);
    const float mean = (float)(sd / a.count);
    const float g = a.g[so];
    const float rs = OP == B_STD ? a.res[so] : 0.0f;
    f32x4* po = reinterpret_cast<f32x4*>(a.gi + row * (long long)a.sizes[last]);
    // one reciprocal per row instead of a divide per element: the double
    // product rounds to the same float as the quotient except within ~2^-52 of
    // a rounding boundary (one ulp then)
    const double inv = OP == B_VAR ? a.inv_denom : 1.0 / (double)(rs * a.denom_f);
    auto f = [&](float x) -> float {
        const float tt = OP == B_VAR ? (g * 2.0f) * (x - mean) : g * (x - mean);
        return (float)((double)tt * inv);
    };
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int e = j * 64 + lane;
        if (e < q) {
            const f32x4 o = {f(v[j].x), f(v[j].y), f(v[j].z), f(v[j].w)};
            __builtin_nontemporal_store(o, po + e);
        }
    }
}

// VAR / STD over a reduced dim of R <= 1024 rows followed by a kept,
// contiguous inner dim ([outer, R, inner] after merging; inner % 4 == 0):
// a workgroup takes 64 columns of one outer index (16 lanes x float4 per row,
// a wave covers 4 rows, BY waves), each lane keeps its V rows in registers,
// the column sums combine across lanes and waves (LDS), and the gradient is
// written from registers: x read once.
template <int OP, int BY, int V>
__global__ __launch_bounds__(64 * BY) void k_vs_bwd_cols(RbArgs a, long long outer, int R, long long inner,
                                                       long long ncg) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    constexpr int RS = 4 * BY;
    __shared__ float shs[BY][16][4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int cl = lane & 15, rl = lane >> 4;
    const long long o = blockIdx.x / ncg;
    const long long c = (blockIdx.x - o * ncg) * 64 + 4 * cl;
    const bool live = c < inner;
    const int nrow = live ? R : 0;
    const float* px = a.x + o * a.xs[0] + (live ? c : 0);
    const long long xr = a.xs[1];
    f32x4 v[V];
    float sm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int r0 = rl + 4 * w;
    const f32x4* qx = reinterpret_cast<const f32x4*>(px + r0 * xr);  // advanced by RS rows per vector
    const long long qstep = RS * xr / 4;
#pragma unroll
    for (int i = 0; i < V; ++i, qx += qstep) {
        const int r = r0 + i * RS;
        if (r < nrow) {
            v[i] = __builtin_nontemporal_load(qx);
            sm[0] += v[i].x;
            sm[1] += v[i].y;
            sm[2] += v[i].z;
            sm[3] += v[i].w;
        }
    }
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1)
#pragma unroll
        for (int k = 0; k < 4; ++k) sm[k] += __shfl_xor(sm[k], off, 64);
    if (rl == 0)
#pragma unroll
        for (int k = 0; k < 4; ++k) shs[w][cl][k] = sm[k];
    __syncthreads();
    float mean[4], g[4];
    double inv[4];  // a reciprocal per column instead of a divide per element (as k_vs_bwd_rows)
    const long long so = o * a.os[0] + (live ? c : 0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        double S = 0.0;
#pragma unroll
        for (int b = 0; b < BY; ++b) S += shs[b][cl][k];
        mean[k] = (float)(S / a.count);
        g[k] = live ? a.g[so + k] : 0.0f;
        const float rs = (OP == B_STD && live) ? a.res[so + k] : 0.0f;
        inv[k] = OP == B_VAR ? a.inv_denom : 1.0 / (double)(rs * a.denom_f);
    }
    auto f = [&](float x, int k) -> float {
        const float tt = OP == B_VAR ? (g[k] * 2.0f) * (x - mean[k]) : g[k] * (x - mean[k]);
        return (float)((double)tt * inv[k]);
    };
    f32x4* qo = reinterpret_cast<f32x4*>(a.gi + o * (long long)R * inner + (live ? c : 0) + r0 * inner);
    const long long ostep = RS * inner / 4;
#pragma unroll
    for (int i = 0; i < V; ++i, qo += ostep) {
        const int r = r0 + i * RS;
        if (r < nrow) {
            const f32x4 y = {f(v[i].x, 0), f(v[i].y, 1), f(v[i].z, 2), f(v[i].w, 3)};
            __builtin_nontemporal_store(y, qo);
        }
        __builtin_amdgcn_sched_barrier(0);  // store as computed (no register build-up)
    }
}

template <int OP>
bool launch_vs_cols(const RbArgs& a, hipStream_t st) {
    // [outer?, R, inner]: inner kept with unit stride in x and out, R reduced,
    // outer (if present) kept
    if (knobs().general != 0 || (a.nd != 2 && a.nd != 3)) return false;
    RbArgs b = a;
    if (a.nd == 2) {  // no outer dim: shift so that index 0 is a size-1 outer
        b.sizes[2] = a.sizes[1]; b.xs[2] = a.xs[1]; b.os[2] = a.os[1];
        b.sizes[1] = a.sizes[0]; b.xs[1] = a.xs[0]; b.os[1] = a.os[0];
        b.sizes[0] = 1; b.xs[0] = 0; b.os[0] = 0;
    } else if (a.os[0] == 0) {
        return false;  // outer reduced as well
    }
    const long long outer = b.sizes[0], R = b.sizes[1], inner = b.sizes[2];
    if (b.os[1] != 0 || b.os[2] != 1 || b.xs[2] != 1 || inner % 4 != 0 || R > 1024 || R < 1) return false;
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (!al(a.x) || !al(a.gi) || b.xs[1] % 4 != 0 || b.xs[0] % 4 != 0) return false;
    const long long ncg = (inner + 63) / 64;
    const long long blocks = outer * ncg;
    if (blocks > 0x7fffffffLL) return false;
    const dim3 gr((unsigned)blocks);
    if (R <= 128) hipLaunchKernelGGL((k_vs_bwd_cols<OP, 8, 4>), gr, dim3(512), 0, st, b, outer, (int)R, inner, ncg);
    else if (R <= 256) hipLaunchKernelGGL((k_vs_bwd_cols<OP, 8, 8>), gr, dim3(512), 0, st, b, outer, (int)R, inner, ncg);
    else if (R <= 512) hipLaunchKernelGGL((k_vs_bwd_cols<OP, 16, 8>), gr, dim3(1024), 0, st, b, outer, (int)R, inner, ncg);
    // 513..1024 rows: 16 waves x 16 vectors per lane (a few VGPRs spill at the
    // 128-register cap; 8 waves x 32 vectors measured slower: 134 vs 125 us
    // for var over dim 1 of [64, 1024, 1024])
    else hipLaunchKernelGGL((k_vs_bwd_cols<OP, 16, 16>), gr, dim3(1024), 0, st, b, outer, (int)R, inner, ncg);
    return true;
}

// Rows of one fused VAR / STD gradient (k_vs_bwd_rows); false when the layout
// does not fit it.
template <int OP>
bool launch_vs_rows(const RbArgs& a, hipStream_t st) {
    const int last = a.nd - 1;
    const long long L = a.sizes[last];
    if (a.os[last] != 0 || a.xs[last] != 1 || L % 4 != 0 || L > 4096 || knobs().general != 0) return false;
    for (int d = 0; d < last; ++d)
        if (a.os[d] == 0) return false;  // another reduced dim: the mean spans more than one run
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (!al(a.x) || !al(a.gi)) return false;
    for (int d = 0; d < last; ++d)
        if (a.xs[d] % 4 != 0) return false;  // every row start 16-byte aligned
    const long long rows = a.total / L;
    const long long blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffffLL) return false;
    const int v = L <= 256 ? 1 : L <= 512 ? 2 : L <= 1024 ? 4 : L <= 2048 ? 8 : 16;
    const dim3 gr((unsigned)blocks), bl(256);
    switch (v) {
        case 1: hipLaunchKernelGGL((k_vs_bwd_rows<OP, 1>), gr, bl, 0, st, a, rows); break;
        case 2: hipLaunchKernelGGL((k_vs_bwd_rows<OP, 2>), gr, bl, 0, st, a, rows); break;
        case 4: hipLaunchKernelGGL((k_vs_bwd_rows<OP, 4>), gr, bl, 0, st, a, rows); break;
        case 8: hipLaunchKernelGGL((k_vs_bwd_rows<OP, 8>), gr, bl, 0, st, a, rows); break;
        default: hipLaunchKernelGGL((k_vs_bwd_rows<OP, 16>), gr, bl, 0, st, a, rows); break;
    }
    return true;
}

// MEAN: q[o] = (float)((double)g[o] / count) once per output (the gradient is
// then a broadcast of q, as for SUM).
__global__ __launch_bounds__(256) void k_mean_scale(const float* g, float* q, long long n, double count) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
        q[i] = (float)((double)g[i] / count);
}

template <int OP>
int launch_bwd(const RbArgs& a, hipStream_t st) {
    const long long L = a.sizes[a.nd - 1];
    const long long os = a.os[a.nd - 1];
    if (L >= 1024 && (os == 0 || os == 1) && knobs().general == 0) {
        auto al = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        // vectors: whole 16-byte groups on every side that is read or written per element
        const bool v4 = L % 4 == 0 && al(a.gi) && (a.xs[a.nd - 1] != 1 || al(a.x)) &&
                        (os == 0 || (al(a.g) && al(a.mean) && al(a.res)));
        // vectors per thread: 4 when x is read (var / std), else 2 for rows
        // shorter than 4096 (measured on MI355X at [64, 1024, 1024]: mean / sum
        // backward over dim 1, rows of 1024, 43-45 us against 50 us with 4 and
        // 51-58 us with 1) and 1 for long rows
        int u = (OP == B_VAR || OP == B_STD) ? 4 : (L < 4096 ? 2 : 1);
        if (knobs().unroll == 1 || knobs().unroll == 2 || knobs().unroll == 4) u = (int)knobs().unroll;
        const long long ch = 256LL * (v4 ? 4 : 1) * u;
        const long long chunks = (L + ch - 1) / ch;
        const long long rows = a.total / L;
        const int rpb = L < ch ? (int)(ch / L) : 1;  // short rows: several per workgroup
        const long long blocks = (rows + rpb - 1) / rpb * chunks;
        if (blocks <= 0x7fffffffLL) {
            const dim3 gr((unsigned)blocks), bl(256);
#define TPR_RB_ROWS(VV, II)                                                                                 \
    if (u == 4) hipLaunchKernelGGL((k_red_bwd_rows<OP, VV, II, 4>), gr, bl, 0, st, a, chunks, rpb, rows);     \
    else if (u == 2) hipLaunchKernelGGL((k_red_bwd_rows<OP, VV, II, 2>), gr, bl, 0, st, a, chunks, rpb, rows); \
    else hipLaunchKernelGGL((k_red_bwd_rows<OP, VV, II, 1>), gr, bl, 0, st, a, chunks, rpb, rows);
            if (os == 0) {
                if (v4) { TPR_RB_ROWS(4, 0) } else { TPR_RB_ROWS(1, 0) }
            } else {
                if (v4) { TPR_RB_ROWS(4, 1) } else { TPR_RB_ROWS(1, 1) }
            }
#undef TPR_RB_ROWS
            return check_launch("tpr_reduce_backward");
        }
    }
    const bool v4 = a.sizes[a.nd - 1] % 4 == 0 && (reinterpret_cast<uintptr_t>(a.gi) & 15) == 0;
    const long long nvec = a.total / (v4 ? 4 : 1);
    long long blocks = (nvec + 255) / 256;
    const long long cap = (long long)device_info().cus * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    const bool small = a.total < (1LL << 31);
    RbArgs b = a;
    for (int d = 0; d < a.nd; ++d) b.fd[d] = make_fastdiv((unsigned long long)a.sizes[d]);
    if (v4) {
        if (small) hipLaunchKernelGGL((k_red_bwd<OP, 4, unsigned>), dim3((unsigned)blocks), dim3(256), 0, st, b);
        else hipLaunchKernelGGL((k_red_bwd<OP, 4, long long>), dim3((unsigned)blocks), dim3(256), 0, st, b);
    } else {
        if (small) hipLaunchKernelGGL((k_red_bwd<OP, 1, unsigned>), dim3((unsigned)blocks), dim3(256), 0, st, b);
        else hipLaunchKernelGGL((k_red_bwd<OP, 1, long long>), dim3((unsigned)blocks), dim3(256), 0, st, b);
    }
    return check_launch("tpr_reduce_backward");
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// The MEAN reduction descriptor the var / std gradient needs.
tpr_reduce_desc mean_desc(const tpr_reduce_desc* d) {
    tpr_reduce_desc m = *d;
    m.op = TPR_MEAN;
    m.in_dtype = TPR_FLOAT32;
    m.out_dtype = TPR_FLOAT32;
    return m;
}

long long kept_count(const tpr_reduce_desc* d) {
    long long n = 1;
    for (int i = 0; i < d->ndim; ++i)
        if (!((d->reduce_mask >> i) & 1u)) n *= d->sizes[i];
    return n;
}

uint32_t full_mask(const tpr_reduce_desc* d) { return d->ndim == 0 ? 0u : ((1u << d->ndim) - 1u); }

}  // namespace
}  // namespace tpr

extern "C" size_t tpr_reduce_backward_workspace_bytes(const tpr_reduce_desc* d) {
    using namespace tpr;
    if (!d || d->ndim < 0 || d->ndim > TPR_MAX_DIMS) return 0;
    if (d->op == TPR_MEAN) return align256((size_t)kept_count(d) * sizeof(float));
    if (d->op != TPR_VAR && d->op != TPR_STD) return 0;
    const tpr_reduce_desc m = mean_desc(d);
    return align256((size_t)kept_count(d) * sizeof(float)) + tpr_reduce_workspace_bytes(&m);
}

extern "C" int tpr_reduce_backward(const tpr_reduce_desc* d, const void* grad_out, const void* in,
                                   const void* result, void* grad_in, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    using namespace tpr;
    if (!d) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce_backward: null descriptor");
    if (d->ndim < 0 || d->ndim > TPR_MAX_DIMS)
        return fail(TPR_ERR_INVALID_ARG, "tpr_reduce_backward: ndim out of range");
    if (d->op != TPR_SUM && d->op != TPR_MEAN && d->op != TPR_VAR && d->op != TPR_STD)
        return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce_backward: sum, mean, var and std only");
    if (d->in_dtype != TPR_FLOAT32 || (d->out_dtype != TPR_FLOAT32))
        return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce_backward: float32 only");
    if (d->reduce_mask & ~full_mask(d)) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce_backward: bad reduce_mask");
    long long total = 1, rcount = 1;
    for (int i = 0; i < d->ndim; ++i) {
        if (d->sizes[i] < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce_backward: negative size");
        total *= d->sizes[i];
        if ((d->reduce_mask >> i) & 1u) rcount *= d->sizes[i];
    }
    if (total == 0) return TPR_OK;
    if (!grad_out || !grad_in || ((d->op == TPR_VAR || d->op == TPR_STD) && !in) || (d->op == TPR_STD && !result))
        return fail(TPR_ERR_INVALID_ARG, "tpr_reduce_backward: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const long long count = d->count_override > 0 ? d->count_override : rcount;

    RbArgs a;
    std::memset(&a, 0, sizeof(a));
    a.g = static_cast<const float*>(grad_out);
    a.x = static_cast<const float*>(in);
    a.res = static_cast<const float*>(result);
    a.gi = static_cast<float*>(grad_in);
    a.total = total;
    a.count = (double)count;
    a.denom = (double)(count - d->correction);
    a.denom_f = (float)(count - d->correction);
    a.inv_denom = 1.0 / a.denom;

    if (d->op == TPR_MEAN) {
        const size_t need = tpr_reduce_backward_workspace_bytes(d);
        if (!workspace || workspace_bytes < need)
            return fail(TPR_ERR_WORKSPACE, "tpr_reduce_backward: workspace smaller than tpr_reduce_backward_workspace_bytes");
        const long long nout = kept_count(d);
        long long blocks = (nout + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        float* q = static_cast<float*>(workspace);
        hipLaunchKernelGGL(k_mean_scale, dim3((unsigned)blocks), dim3(256), 0, st, a.g, q, nout, a.count);
        const int rc = check_launch("tpr_reduce_backward (mean scale)");
        if (rc != TPR_OK) return rc;
        a.g = q;
    }
    if (d->op == TPR_VAR || d->op == TPR_STD) {
        const size_t need = tpr_reduce_backward_workspace_bytes(d);
        if (!workspace || workspace_bytes < need)
            return fail(TPR_ERR_WORKSPACE, "tpr_reduce_backward: workspace smaller than tpr_reduce_backward_workspace_bytes");
    }

    // per-output strides: dense row-major over the kept dims
    long long ostr[TPR_MAX_DIMS] = {0};
    {
        long long acc = 1;
        for (int i = d->ndim - 1; i >= 0; --i) {
            if ((d->reduce_mask >> i) & 1u) continue;
            ostr[i] = acc;
            acc *= d->sizes[i];
        }
    }
    // merge dims (outer into inner) that are contiguous in the input and share reduce status
    int nd = 0;
    for (int i = 0; i < d->ndim; ++i) {
        const long long sz = d->sizes[i];
        if (sz == 1) continue;
        const bool red = (d->reduce_mask >> i) & 1u;
        const long long xs = (d->op == TPR_VAR || d->op == TPR_STD) ? d->strides[i] : 0;
        if (nd > 0) {
            const int j = nd - 1;
            const bool jred = a.os[j] == 0;
            // j is the previous (outer) kept entry; merging i into it keeps the outer's strides
            if (jred == red && a.xs[j] == xs * sz && a.os[j] == ostr[i] * sz) {
                a.sizes[j] *= sz;
                a.xs[j] = xs;
                a.os[j] = red ? 0 : ostr[i];
                continue;
            }
        }
        a.sizes[nd] = sz;
        a.xs[nd] = xs;
        a.os[nd] = red ? 0 : ostr[i];
        ++nd;
    }
    if (nd == 0) {  // a single element
        a.sizes[0] = 1;
        nd = 1;
    }
    a.nd = nd;
    if (d->op == TPR_VAR || d->op == TPR_STD) {
        // one pass when the reduced run (innermost) or the reduced column
        // slice (middle dim) fits in registers, else the MEAN reduction into
        // the workspace and the streaming gradient pass
        const bool fused = d->op == TPR_VAR ? (launch_vs_rows<B_VAR>(a, st) || launch_vs_cols<B_VAR>(a, st))
                                            : (launch_vs_rows<B_STD>(a, st) || launch_vs_cols<B_STD>(a, st));
        if (fused) return check_launch("tpr_reduce_backward (var/std rows)");
        const tpr_reduce_desc m = mean_desc(d);
        float* mean = static_cast<float*>(workspace);
        const size_t moff = align256((size_t)kept_count(d) * sizeof(float));
        const int rc = tpr_reduce(&m, in, mean, static_cast<char*>(workspace) + moff, workspace_bytes - moff, stream);
        if (rc != TPR_OK) return rc;
        a.mean = mean;
    }
    switch (d->op) {
        case TPR_SUM: return launch_bwd<B_SUM>(a, st);
        case TPR_MEAN: return launch_bwd<B_MEAN>(a, st);
        case TPR_VAR: return launch_bwd<B_VAR>(a, st);
        default: return launch_bwd<B_STD>(a, st);
    }
}
