// gfx950 nll_loss forward and backward, behind tpr_nll_loss() and
// tpr_nll_loss_backward().
//
// Forward follows the CPU kernel
// (/root/reference/p10/src/backend/cpu/LossKernels.cpp:12-55):
//   loss_i = -x[i, t_i] * w[t_i] (float32), 0 for ignored samples;
//   total_weight = sum of w[t_i] over samples that are not ignored;
//   mean = sum(loss_i) / total_weight when total_weight > 0, sum = sum(loss_i).
// The reference sums the losses in double (as here) and the weights in float
// sequentially (here in double, then rounded once to float: identical for
// unit weights, and within one rounding otherwise).  The CUDA path
// (LossKernels.cu:38-61) instead does float atomicAdds, whose order varies run
// to run; here partial sums per workgroup are combined in a fixed order by a
// second one-workgroup kernel, so results are deterministic.
// Backward writes grad_input in one pass (zeros plus the target element),
// instead of the reference's zeros() then scatter.

#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace tpr {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kNllBlock = 256;
constexpr int kNllMaxBlocks = 1024;

struct NllPart {
    double loss;
    double weight;
    int bad;
    int pad;
};

struct NllArgs {
    const float* x;
    long long n, c, s0, s1;
    const long long* t;
    long long ts;
    const float* w;
    long long reduction, ignore;
    float* out;       // [n] for reduction none
    NllPart* part;    // one per workgroup
};

template <class T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__global__ __launch_bounds__(kNllBlock) void k_nll_part(NllArgs a) {
    __shared__ double sl[kNllBlock / kWave], sw[kNllBlock / kWave];
    __shared__ int sb[kNllBlock / kWave];
    double loss = 0.0, wsum = 0.0;
    int bad = 0;
    for (long long i = (long long)blockIdx.x * kNllBlock + threadIdx.x; i < a.n;
         i += (long long)gridDim.x * kNllBlock) {
        const long long t = a.t[i * a.ts];
        float li = 0.0f;
        if (t != a.ignore) {
            if (t < 0 || t >= a.c) {
                bad = 1;
            } else {
                const float w = a.w ? a.w[t] : 1.0f;
                li = -a.x[i * a.s0 + t * a.s1] * w;
                loss += (double)li;
                wsum += (double)w;
            }
        }
        if (a.reduction == 0) a.out[i] = li;
    }
    loss = wave_sum(loss);
    wsum = wave_sum(wsum);
    bad = wave_sum(bad);
    const int w = threadIdx.x / kWave;
    if (__lane_id() == 0) {
        sl[w] = loss;
        sw[w] = wsum;
        sb[w] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        NllPart p{0.0, 0.0, 0, 0};
        for (int k = 0; k < kNllBlock / kWave; ++k) {
            p.loss += sl[k];
            p.weight += sw[k];
            p.bad |= sb[k] != 0;
        }
        a.part[blockIdx.x] = p;
    }
}

struct NllFin {
    const NllPart* part;
    int nparts;
    long long reduction;
    float* out;
    float* total_weight;
    int* status;
};

__global__ __launch_bounds__(kNllBlock) void k_nll_fin(NllFin f) {
    __shared__ double sl[kNllBlock / kWave], sw[kNllBlock / kWave];
    __shared__ int sb[kNllBlock / kWave];
    double loss = 0.0, wsum = 0.0;
    int bad = 0;
    for (int k = threadIdx.x; k < f.nparts; k += kNllBlock) {
        loss += f.part[k].loss;
        wsum += f.part[k].weight;
        bad |= f.part[k].bad;
    }
    loss = wave_sum(loss);
    wsum = wave_sum(wsum);
    bad = wave_sum(bad);
    const int w = threadIdx.x / kWave;
    if (__lane_id() == 0) {
        sl[w] = loss;
        sw[w] = wsum;
        sb[w] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double l = 0.0, ws = 0.0;
        int b = 0;
        for (int k = 0; k < kNllBlock / kWave; ++k) {
            l += sl[k];
            ws += sw[k];
            b |= sb[k] != 0;
        }
        const float tw = (float)ws;
        if (f.reduction == 1 && tw > 0.0f) l /= (double)tw;
        if (f.reduction != 0) f.out[0] = (float)l;
        f.total_weight[0] = tw;
        if (f.status) f.status[0] = b;
    }
}

// ---- backward ---------------------------------------------------------------
struct NllBwdArgs {
    const float* g;
    long long gs;
    const long long* t;
    long long ts;
    const float* w;
    const float* tw;
    long long n, c, reduction, ignore;
    float* gi;
    long long chunks;  // workgroups per row (row kernel)
};

__device__ __forceinline__ float nll_grad_value(const NllBwdArgs& a, long long i, long long t) {
    float g = a.reduction == 0 ? a.g[i * a.gs] : a.g[0];
    if (a.reduction == 1 && a.tw) {
        const double tw = (double)a.tw[0];
        if (tw > 0.0) g = (float)((double)g / tw);
    }
    const float w = a.w ? a.w[t] : 1.0f;
    return -w * g;
}

// Rows of at least 1024 elements: workgroup (row, chunk) writes 256 * kNllU
// 16-byte vectors (VW = 4) or scalars (VW = 1) of one row.
// Vectors each thread of the row kernel writes: one (a write-only kernel runs
// fastest with one 16-byte store per thread over a grid covering the output:
// measured on MI355X, a 256 MiB fill takes 40 us against 45-52 us with 2-8
// stores per thread).
constexpr int kNllU = 1;

template <int VW>
__global__ __launch_bounds__(kNllBlock) void k_nll_bwd_rows(NllBwdArgs a) {
    constexpr long long CH = (long long)kNllBlock * kNllU * VW;
    const long long row = blockIdx.x / a.chunks;
    const long long base = (blockIdx.x - row * a.chunks) * CH;
    const long long t = a.t[row * a.ts];
    const bool hit = t != a.ignore && t >= 0 && t < a.c;
    const float v = hit ? nll_grad_value(a, row, t) : 0.0f;
    float* out = a.gi + row * a.c;
#pragma unroll
    for (int u = 0; u < kNllU; ++u) {
        const long long e = base + ((long long)u * kNllBlock + threadIdx.x) * VW;
        if (e >= a.c) break;
        if constexpr (VW == 4) {
            f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
            if (hit && t >= e && t < e + 4) z[t - e] = v;
            __builtin_nontemporal_store(z, reinterpret_cast<f32x4_t*>(out + e));
        } else {
            __builtin_nontemporal_store((hit && t == e) ? v : 0.0f, out + e);
        }
    }
}

// Short rows: one element per thread over the flat [n, c] output.
__global__ __launch_bounds__(kNllBlock) void k_nll_bwd_flat(NllBwdArgs a) {
    const long long total = a.n * a.c;
    for (long long e = (long long)blockIdx.x * kNllBlock + threadIdx.x; e < total;
         e += (long long)gridDim.x * kNllBlock) {
        const long long row = e / a.c;
        const long long col = e - row * a.c;
        const long long t = a.t[row * a.ts];
        float v = 0.0f;
        if (t == col && t != a.ignore) v = nll_grad_value(a, row, t);
        a.gi[e] = v;
    }
}

}  // namespace
}  // namespace tpr

extern "C" size_t tpr_nll_loss_workspace_bytes(int64_t n) {
    using namespace tpr;
    if (n <= 0) return sizeof(NllPart);
    long long blocks = (n + kNllBlock - 1) / kNllBlock;
    if (blocks > kNllMaxBlocks) blocks = kNllMaxBlocks;
    return (size_t)blocks * sizeof(NllPart);
}

extern "C" int tpr_nll_loss(const void* input, int32_t dtype, int64_t n, int64_t c, int64_t s0, int64_t s1,
                            const int64_t* target, int64_t ts, const void* weight, int64_t reduction,
                            int64_t ignore_index, void* out, void* total_weight, int32_t* status,
                            void* workspace, size_t workspace_bytes, void* stream) {
    using namespace tpr;
    if (dtype != TPR_FLOAT32) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_nll_loss: float32 input only");
    if (n < 0 || c < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_nll_loss: negative extent");
    if (reduction < 0 || reduction > 2) return fail(TPR_ERR_INVALID_ARG, "tpr_nll_loss: invalid reduction mode");
    if (!total_weight || (!out && (reduction != 0 || n > 0)) || (n > 0 && (!input || !target)))
        return fail(TPR_ERR_INVALID_ARG, "tpr_nll_loss: null pointer");
    const size_t need = tpr_nll_loss_workspace_bytes(n);
    if (!workspace || workspace_bytes < need)
        return fail(TPR_ERR_WORKSPACE, "tpr_nll_loss: workspace smaller than tpr_nll_loss_workspace_bytes");
    hipStream_t st = static_cast<hipStream_t>(stream);
    NllPart* part = static_cast<NllPart*>(workspace);
    long long blocks = (n + kNllBlock - 1) / kNllBlock;
    if (blocks > kNllMaxBlocks) blocks = kNllMaxBlocks;
    if (blocks < 1) blocks = 1;
    NllArgs a{static_cast<const float*>(input), n, c, s0, s1,
              reinterpret_cast<const long long*>(target), ts, static_cast<const float*>(weight),
              reduction, ignore_index, static_cast<float*>(out), part};
    hipLaunchKernelGGL(k_nll_part, dim3((unsigned)blocks), dim3(kNllBlock), 0, st, a);
    int rc = check_launch("tpr_nll_loss");
    if (rc) return rc;
    NllFin f{part, (int)blocks, reduction, static_cast<float*>(out), static_cast<float*>(total_weight),
             reinterpret_cast<int*>(status)};
    hipLaunchKernelGGL(k_nll_fin, dim3(1), dim3(kNllBlock), 0, st, f);
    return check_launch("tpr_nll_loss (finalize)");
}

extern "C" int tpr_nll_loss_backward(const void* grad_output, int64_t gs, const int64_t* target, int64_t ts,
                                     const void* weight, const void* total_weight, int64_t n, int64_t c,
                                     int64_t reduction, int64_t ignore_index, void* grad_input, void* stream) {
    using namespace tpr;
    if (n < 0 || c < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_nll_loss_backward: negative extent");
    if (reduction < 0 || reduction > 2)
        return fail(TPR_ERR_INVALID_ARG, "tpr_nll_loss_backward: invalid reduction mode");
    if (n == 0 || c == 0) return TPR_OK;
    if (!grad_output || !target || !grad_input) return fail(TPR_ERR_INVALID_ARG, "tpr_nll_loss_backward: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    NllBwdArgs a{static_cast<const float*>(grad_output), gs, reinterpret_cast<const long long*>(target), ts,
                 static_cast<const float*>(weight), static_cast<const float*>(total_weight),
                 n, c, reduction, ignore_index, static_cast<float*>(grad_input), 0};
    if (c >= 1024) {
        const bool v4 = c % 4 == 0 && (reinterpret_cast<uintptr_t>(grad_input) & 15) == 0;
        const long long ch = (long long)kNllBlock * kNllU * (v4 ? 4 : 1);
        a.chunks = (c + ch - 1) / ch;
        const long long blocks = n * a.chunks;
        if (blocks > 0x7fffffffLL) return fail(TPR_ERR_INVALID_ARG, "tpr_nll_loss_backward: too large");
        if (v4) hipLaunchKernelGGL((k_nll_bwd_rows<4>), dim3((unsigned)blocks), dim3(kNllBlock), 0, st, a);
        else hipLaunchKernelGGL((k_nll_bwd_rows<1>), dim3((unsigned)blocks), dim3(kNllBlock), 0, st, a);
    } else {
        long long blocks = (n * c + kNllBlock - 1) / kNllBlock;
        const long long cap = (long long)device_info().cus * 32;
        if (blocks > cap) blocks = cap;
        hipLaunchKernelGGL(k_nll_bwd_flat, dim3((unsigned)blocks), dim3(kNllBlock), 0, st, a);
    }
    return check_launch("tpr_nll_loss_backward");
}
