// gfx950 top-k / top-p (nucleus) sampling over rows of logits, behind
// tpr_sample().  A consumer of the top-k path: tpr_topk selects the k largest
// logits of every row (sorted, ties to the lowest index) into the workspace,
// then k_sample turns each row's k candidates into one token id.
//
// TensorPlay has no sampler; the definition here (documented in the header) is
// the usual temperature -> top-k -> softmax -> top-p -> inverse-CDF draw:
//   z_j = v_j / T for the sorted candidates v_0 >= v_1 >= ... >= v_{k-1};
//   p_j = exp(z_j - z_0);  c_j = p_0 + ... + p_j;
//   m   = the first j with c_j >= top_p * c_{k-1}  (the nucleus is 0..m);
//   id  = index of the first j <= m with c_j > u * c_m  (u in [0, 1) given per row).
// T <= 0 is greedy: the id of v_0.  One 64-lane wave per row; each lane owns a
// contiguous block of candidates, so the inclusive scan is a per-lane serial
// sum plus a wave scan of the block totals.

#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace tpr {
namespace {

constexpr int kSampleWaves = 4;  // rows per 256-thread workgroup

struct SampleArgs {
    const float* vals;      // [rows, k] sorted descending
    const long long* idx;   // [rows, k]
    const float* u;         // [rows]
    long long* out;         // [rows]
    long long rows;
    int k;
    float temperature;
    float top_p;
};

__global__ __launch_bounds__(64 * kSampleWaves) void k_sample(SampleArgs a) {
    const int lane = threadIdx.x % kWave;
    const long long row = (long long)blockIdx.x * kSampleWaves + threadIdx.x / kWave;
    if (row >= a.rows) return;  // whole waves exit together; no barriers below
    const float* v = a.vals + row * a.k;
    const long long* ix = a.idx + row * a.k;
    if (!(a.temperature > 0.0f)) {
        if (lane == 0) a.out[row] = ix[0];
        return;
    }
    const int per = (a.k + kWave - 1) / kWave;  // candidates per lane (<= 16)
    const int j0 = lane * per;
    const float z0 = v[0] / a.temperature;
    float p[16];
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int j = j0 + q;
        p[q] = 0.0f;
        if (q < per && j < a.k) {
            p[q] = expf(v[j] / a.temperature - z0);
            s += p[q];
        }
    }
    // exclusive scan of the lane totals across the wave
    float incl = s;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const float t = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += t;
    }
    const float excl = incl - s;
    const float total = __shfl(incl, kWave - 1, kWave);
    const float cut = a.top_p * total;
    // m: first j with c_j >= cut (the last candidate if none, e.g. NaN)
    int m_lane = 0x7fffffff;
    {
        float c = excl;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int j = j0 + q;
            if (q < per && j < a.k) {
                c += p[q];
                if (c >= cut && m_lane == 0x7fffffff) m_lane = j;
            }
        }
    }
    int m = m_lane;
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) m = min(m, __shfl_xor(m, o, kWave));
    if (m == 0x7fffffff) m = a.k - 1;
    // c_m: the inclusive sum at m, held by the lane that owns m
    float cm_lane = 0.0f;
    {
        float c = excl;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int j = j0 + q;
            if (q < per && j < a.k) {
                c += p[q];
                if (j == m) cm_lane = c;
            }
        }
    }
    const float cm = __shfl(cm_lane, m / per, kWave);
    const float thr = a.u[row] * cm;
    int pick_lane = 0x7fffffff;
    {
        float c = excl;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int j = j0 + q;
            if (q < per && j <= m) {
                c += p[q];
                if (c > thr && pick_lane == 0x7fffffff) pick_lane = j;
            }
        }
    }
    int pick = pick_lane;
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) pick = min(pick, __shfl_xor(pick, o, kWave));
    if (pick > m) pick = m;
    if (lane == 0) a.out[row] = ix[pick];
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace
}  // namespace tpr

extern "C" size_t tpr_sample_workspace_bytes(int32_t dtype, int64_t rows, int64_t cols, int64_t k) {
    using namespace tpr;
    if (rows <= 0 || k <= 0) return 0;
    const size_t cand = align256((size_t)rows * k * sizeof(float)) + align256((size_t)rows * k * sizeof(long long));
    return cand + tpr_topk_workspace_bytes(dtype, rows, cols, k);
}

extern "C" int tpr_sample(const void* logits, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride,
                          int64_t k, float temperature, float top_p, const float* uniforms, int64_t* out_ids,
                          void* workspace, size_t workspace_bytes, void* stream) {
    using namespace tpr;
    if (dtype != TPR_FLOAT32) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_sample: float32 logits only");
    if (rows < 0 || cols < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: negative shape");
    if (k < 1 || k > cols) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: k must be in [1, cols]");
    if (k > 1024) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_sample: k > 1024 is not implemented");
    if (!(top_p > 0.0f) || top_p > 1.0f) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: top_p must be in (0, 1]");
    if (rows == 0) return TPR_OK;
    if (!logits || !uniforms || !out_ids) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: null pointer");
    const size_t need = tpr_sample_workspace_bytes(dtype, rows, cols, k);
    if (!workspace || workspace_bytes < need)
        return fail(TPR_ERR_WORKSPACE, "tpr_sample: workspace smaller than tpr_sample_workspace_bytes");
    char* ws = static_cast<char*>(workspace);
    float* vals = reinterpret_cast<float*>(ws);
    const size_t o1 = align256((size_t)rows * k * sizeof(float));
    long long* idx = reinterpret_cast<long long*>(ws + o1);
    const size_t o2 = o1 + align256((size_t)rows * k * sizeof(long long));
    int rc = tpr_topk(logits, dtype, rows, cols, row_stride, k, 1, 1, vals, idx, ws + o2, workspace_bytes - o2, stream);
    if (rc != TPR_OK) return rc;
    SampleArgs a{vals, idx, uniforms, reinterpret_cast<long long*>(out_ids), rows, (int)k, temperature, top_p};
    const long long blocks = (rows + kSampleWaves - 1) / kSampleWaves;
    hipLaunchKernelGGL(k_sample, dim3((unsigned)blocks), dim3(64 * kSampleWaves), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("tpr_sample");
}
