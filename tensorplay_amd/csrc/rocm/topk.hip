// gfx950 top-k along the last dim of a [rows, cols] float32 view.
//
// TensorPlay has no topk (grep of /root/reference finds no schema, kernel or
// test); this implements the definition in tpr_rocm.h: order by a 32-bit
// sortable key (value order, -0.0 == +0.0, NaN above everything; inverted for
// largest=0), then by lowest index.  Each (key, index) pair is packed into one
// 64-bit "composite" key  (key << 32) | (0xffffffff - index)  so every element
// of a row has a distinct composite and larger composite == ranks earlier.
//
// One 1024-thread workgroup per row, row streamed once from HBM in chunks of
// 1024 x 4*V floats (128-bit loads, next chunk prefetched into registers):
//  1. Chunk 0 gives a lower bound T on the row's k-th key: each wave takes the
//     r-th largest of its 64 per-lane maxima (r = ceil(k/16)), and the minimum
//     over the 16 waves has >= 16*r >= k distinct elements at or above it.
//  2. Every element with key >= T is appended to an LDS candidate list
//     (wave-aggregated slot reservation: one LDS atomic per wave per chunk).
//  3. When the list grows past a limit it is compacted to its exact top k
//     (rank selection below) and T rises to the k-th key kept.
//  4. At the end the exact top k of the list is ranked and written in order.
// Rank selection: rank(c) = #{candidates with a larger composite}; composites
// are distinct, so the ranks 0..k-1 are a permutation and give the sorted
// output directly.  The work is split over all 1024 threads (partial counts
// accumulated in LDS).
// If the list would overflow (adversarial rows: all-equal values, long runs of
// the threshold value), the workgroup switches to an exact multi-pass path:
// 4-pass 8-bit radix select over the row in global memory finds the k-th key,
// then an index-ordered gather takes every larger key plus the lowest-index
// elements equal to it.

#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace tpr {
namespace {

constexpr int kT = 1024;         // threads per workgroup (one row)
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kB = 2048;         // candidate list capacity
constexpr int kKMax = 1024;      // largest k this kernel handles

__device__ __forceinline__ uint32_t f2key(float f, int largest) {
    uint32_t u = __float_as_uint(f);
    u = ((u & 0x7fffffffu) > 0x7f800000u) ? 0x7fc00000u : u;  // canonical NaN
    u = (u == 0x80000000u) ? 0u : u;                          // -0 -> +0
    uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return largest ? k : ~k;  // valid keys are never 0: 0 marks "no element"
}

__device__ __forceinline__ unsigned long long comp_key(uint32_t key, uint32_t idx) {
    return ((unsigned long long)key << 32) | (unsigned long long)(0xffffffffu - idx);
}

__device__ __forceinline__ uint32_t comp_index(unsigned long long c) {
    return 0xffffffffu - (uint32_t)(c & 0xffffffffull);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = max(v, (uint32_t)__shfl_xor((int)v, m, 64));
    return v;
}

__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = __lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        int t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    return v;
}

struct TopkArgs {
    const float* in;
    long long rows;
    int cols;
    long long row_stride;
    int k;
    int largest;
    int force_fallback;
    float* out_v;
    long long* out_i;
};

struct TopkShared {
    unsigned long long cand[kB];
    unsigned long long sel[kKMax];
    int rank[kB];
    uint32_t wave_val[kW];
    int wave_cnt[kW];
    uint32_t hist[256];
    int count;
    int over;
    uint32_t thresh;
    int digit;
    int kk;
    int eq_taken;
};

// Exact top-k of sh.cand[0..m) into sh.sel[0..k) (sorted).  m >= k.
// Work split: candidate i gets G = kT / m' groups of threads, each counting a
// slice of the list; partial counts land in sh.rank[i] by LDS atomics.
__device__ void rank_select(TopkShared& sh, int m, int k) {
    const int tid = threadIdx.x;
    for (int i = tid; i < m; i += kT) sh.rank[i] = 0;
    __syncthreads();
    int groups = kT / max(m, 1);
    groups = max(1, min(groups, 64));
    const int slice = (m + groups - 1) / groups;
    for (int w = tid; w < m * groups; w += kT) {
        const int i = w % m;
        const int g = w / m;
        const unsigned long long ci = sh.cand[i];
        const int j0 = g * slice;
        const int j1 = min(m, j0 + slice);
        int r = 0;
        for (int j = j0; j < j1; ++j) r += (sh.cand[j] > ci) ? 1 : 0;
        if (groups == 1) sh.rank[i] = r;
        else if (r) atomicAdd(&sh.rank[i], r);
    }
    __syncthreads();
    for (int i = tid; i < m; i += kT) {
        const int r = sh.rank[i];
        if (r < k) sh.sel[r] = sh.cand[i];
    }
    __syncthreads();
}

template <bool VEC>
__device__ __forceinline__ float4 load4(const float* p, long long e, int n) {
    if (VEC && e + 3 < n) return *reinterpret_cast<const float4*>(p + e);
    float4 t;
    t.x = (e + 0 < n) ? p[e + 0] : 0.0f;
    t.y = (e + 1 < n) ? p[e + 1] : 0.0f;
    t.z = (e + 2 < n) ? p[e + 2] : 0.0f;
    t.w = (e + 3 < n) ? p[e + 3] : 0.0f;
    return t;
}

// Exact multi-pass path (any data).  Leaves the k selected composites in
// sh.cand[0..k) (unordered).
__device__ void exact_select(TopkShared& sh, const float* p, int n, int k, int largest) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    uint32_t prefix = 0, pmask = 0;
    int kk = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) sh.hist[tid] = 0;
        __syncthreads();
        for (int e = tid; e < n; e += kT) {
            const uint32_t key = f2key(p[e], largest);
            if ((key & pmask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            int cum = 0, d = 0;
            for (int b = 255; b >= 0; --b) {
                const int h = (int)sh.hist[b];
                if (cum + h >= kk) { d = b; break; }
                cum += h;
            }
            sh.digit = d;
            sh.kk = kk - cum;
        }
        __syncthreads();
        prefix |= (uint32_t)sh.digit << shift;
        pmask |= 0xffu << shift;
        kk = sh.kk;
        __syncthreads();
    }
    const uint32_t T = prefix;  // exact k-th key; kk = how many keys == T to take
    if (tid == 0) { sh.count = 0; sh.eq_taken = 0; }
    __syncthreads();
    for (int base = 0; base < n; base += kT) {
        const int e = base + tid;
        const uint32_t key = (e < n) ? f2key(p[e], largest) : 0u;
        const bool gt = (e < n) && key > T;
        const bool eq = (e < n) && key == T;
        if (gt) sh.cand[atomicAdd(&sh.count, 1)] = comp_key(key, (uint32_t)e);
        const unsigned long long bal = __ballot(eq);
        const int before = __popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) sh.wave_cnt[w] = __popcll(bal);
        __syncthreads();
        int wbase = sh.eq_taken;
        int total = 0;
        for (int i = 0; i < kW; ++i) {
            if (i < w) wbase += sh.wave_cnt[i];
            total += sh.wave_cnt[i];
        }
        if (eq && wbase + before < kk) sh.cand[atomicAdd(&sh.count, 1)] = comp_key(key, (uint32_t)e);
        __syncthreads();
        if (tid == 0) sh.eq_taken += total;
        __syncthreads();
    }
    __syncthreads();
}

template <int V, bool VEC>
__global__ __launch_bounds__(kT) void k_topk(TopkArgs a) {
    __shared__ TopkShared sh;
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    const long long row = blockIdx.x;
    const float* p = a.in + row * a.row_stride;
    const int n = a.cols;
    const int k = a.k;
    const int largest = a.largest;
    constexpr int CH = kT * 4 * V;
    const int nchunks = (n + CH - 1) / CH;
    const int r = (k + kW - 1) / kW;                 // per-wave rank for the bound
    const int compact_at = max(2 * k, 256);          // list size that triggers compaction

    if (tid == 0) { sh.count = 0; sh.over = 0; }
    __syncthreads();

    bool over = a.force_fallback != 0;
    uint32_t T = 1;  // admit every valid key until the bound is known
    float4 cur[V], nxt[V];
#pragma unroll
    for (int j = 0; j < V; ++j) cur[j] = load4<VEC>(p, 4LL * (j * kT + tid), n);

    for (int c = 0; c < nchunks && !over; ++c) {
        const long long cbase = (long long)c * CH;
        if (c + 1 < nchunks) {
#pragma unroll
            for (int j = 0; j < V; ++j) nxt[j] = load4<VEC>(p, cbase + CH + 4LL * (j * kT + tid), n);
        }
        uint32_t key[4 * V];
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const long long e = cbase + 4LL * (j * kT + tid);
            key[4 * j + 0] = (e + 0 < n) ? f2key(cur[j].x, largest) : 0u;
            key[4 * j + 1] = (e + 1 < n) ? f2key(cur[j].y, largest) : 0u;
            key[4 * j + 2] = (e + 2 < n) ? f2key(cur[j].z, largest) : 0u;
            key[4 * j + 3] = (e + 3 < n) ? f2key(cur[j].w, largest) : 0u;
        }
        if (c == 0) {
            uint32_t m = 0;
#pragma unroll
            for (int q = 0; q < 4 * V; ++q) m = max(m, key[q]);
            uint32_t rth = 0;
            for (int i = 0; i < r; ++i) {
                const uint32_t wm = wave_max_u32(m);
                rth = wm;
                if (wm == 0) break;
                const unsigned long long bal = __ballot(m == wm);
                if (lane == __ffsll((long long)bal) - 1) m = 0;
            }
            if (lane == 0) sh.wave_val[w] = rth;
            __syncthreads();
            uint32_t tb = 0xffffffffu;
#pragma unroll
            for (int i = 0; i < kW; ++i) tb = min(tb, sh.wave_val[i]);
            T = max(T, tb);
        }
        // filter
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < 4 * V; ++q) cnt += (key[q] >= T) ? 1 : 0;
        const int incl = wave_incl_scan(cnt);
        int base = 0;
        if (lane == 63 && incl > 0) base = atomicAdd(&sh.count, incl);
        base = __shfl(base, 63, 64);
        int pos = base + incl - cnt;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const long long e = cbase + 4LL * (j * kT + tid);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (key[4 * j + q] >= T) {
                    if (pos < kB) sh.cand[pos] = comp_key(key[4 * j + q], (uint32_t)(e + q));
                    else sh.over = 1;
                    ++pos;
                }
            }
        }
        __syncthreads();
        // read the shared verdicts, then fence them off from the next chunk's atomics
        over = sh.over != 0;
        const int m = sh.count;
        __syncthreads();
        if (over) break;
        if (m > compact_at) {
            rank_select(sh, m, k);
            for (int i = tid; i < k; i += kT) sh.cand[i] = sh.sel[i];
            if (tid == 0) {
                sh.count = k;
                sh.thresh = (uint32_t)(sh.sel[k - 1] >> 32);
            }
            __syncthreads();
            // Later chunks hold only larger indices, so an equal key there ranks
            // below the k-th kept element: admit strictly larger keys only.
            const uint32_t th = sh.thresh;
            T = (th == 0xffffffffu) ? th : th + 1u;
            __syncthreads();
        }
#pragma unroll
        for (int j = 0; j < V; ++j) cur[j] = nxt[j];
    }
    __syncthreads();

    int m = sh.count;
    if (over) {
        exact_select(sh, p, n, k, largest);
        m = k;
    }
    rank_select(sh, m, k);
    for (int i = tid; i < k; i += kT) {
        const uint32_t idx = comp_index(sh.sel[i]);
        a.out_v[row * k + i] = p[idx];
        a.out_i[row * k + i] = (long long)idx;
    }
}

}  // namespace
}  // namespace tpr

extern "C" {

size_t tpr_topk_workspace_bytes(int32_t dtype, int64_t rows, int64_t cols, int64_t k) {
    (void)dtype; (void)rows; (void)cols; (void)k;
    return 0;
}

int tpr_topk(const void* in, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride,
             int64_t k, int32_t largest, int32_t sorted, void* out_values, void* out_indices,
             void* workspace, size_t workspace_bytes, void* stream) {
    using namespace tpr;
    (void)sorted; (void)workspace; (void)workspace_bytes;
    if (dtype != TPR_FLOAT32) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_topk: only float32 is implemented");
    if (rows < 0 || cols < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: negative shape");
    if (k < 0 || k > cols) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: selected index k out of range");
    if (rows == 0 || k == 0) return TPR_OK;
    if (cols > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: rows longer than 2^31-1");
    if (k > kKMax) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: k > 1024 is not implemented");
    if (rows > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: more than 2^31-1 rows");
    if (!in || !out_values || !out_indices) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: null pointer");
    TopkArgs a;
    a.in = static_cast<const float*>(in);
    a.rows = rows;
    a.cols = (int)cols;
    a.row_stride = row_stride;
    a.k = (int)k;
    a.largest = largest ? 1 : 0;
    a.force_fallback = knobs().topk_fallback ? 1 : 0;
    a.out_v = static_cast<float*>(out_values);
    a.out_i = static_cast<long long*>(out_indices);
    const bool vec = ((reinterpret_cast<uintptr_t>(in) & 15u) == 0) && (rows == 1 || row_stride % 4 == 0);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (vec) hipLaunchKernelGGL((k_topk<4, true>), dim3(rows), dim3(kT), 0, st, a);
    else hipLaunchKernelGGL((k_topk<4, false>), dim3(rows), dim3(kT), 0, st, a);
    return check_launch("k_topk");
}

}  // extern "C"
