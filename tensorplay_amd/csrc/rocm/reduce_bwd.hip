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

struct RbArgs {
    int nd;
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
};

enum { B_SUM = 0, B_MEAN = 1, B_VAR = 2, B_STD = 3 };

template <int OP>
__device__ __forceinline__ float bwd_value(const RbArgs& a, long long xo, long long so) {
    const float g = a.g[so];
    if constexpr (OP == B_SUM) {
        return g;
    } else if constexpr (OP == B_MEAN) {
        return (float)((double)g / a.count);
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
            const IdxT c = e % sz;
            e /= sz;
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

template <int OP>
int launch_bwd(const RbArgs& a, hipStream_t st) {
    const bool v4 = a.sizes[a.nd - 1] % 4 == 0 && (reinterpret_cast<uintptr_t>(a.gi) & 15) == 0;
    const long long nvec = a.total / (v4 ? 4 : 1);
    long long blocks = (nvec + 255) / 256;
    const long long cap = (long long)device_info().cus * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    const bool small = a.total < (1LL << 31);
    if (v4) {
        if (small) hipLaunchKernelGGL((k_red_bwd<OP, 4, unsigned>), dim3((unsigned)blocks), dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_red_bwd<OP, 4, long long>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    } else {
        if (small) hipLaunchKernelGGL((k_red_bwd<OP, 1, unsigned>), dim3((unsigned)blocks), dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_red_bwd<OP, 1, long long>), dim3((unsigned)blocks), dim3(256), 0, st, a);
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

    if (d->op == TPR_VAR || d->op == TPR_STD) {
        const size_t need = tpr_reduce_backward_workspace_bytes(d);
        if (!workspace || workspace_bytes < need)
            return fail(TPR_ERR_WORKSPACE, "tpr_reduce_backward: workspace smaller than tpr_reduce_backward_workspace_bytes");
        const tpr_reduce_desc m = mean_desc(d);
        float* mean = static_cast<float*>(workspace);
        const size_t moff = align256((size_t)kept_count(d) * sizeof(float));
        const int rc = tpr_reduce(&m, in, mean, static_cast<char*>(workspace) + moff, workspace_bytes - moff, stream);
        if (rc != TPR_OK) return rc;
        a.mean = mean;
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
    switch (d->op) {
        case TPR_SUM: return launch_bwd<B_SUM>(a, st);
        case TPR_MEAN: return launch_bwd<B_MEAN>(a, st);
        case TPR_VAR: return launch_bwd<B_VAR>(a, st);
        default: return launch_bwd<B_STD>(a, st);
    }
}
