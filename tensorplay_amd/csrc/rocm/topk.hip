// gfx950 top-k along the last dim of a [rows, cols] float32 view.
//
// TensorPlay has no topk (grep of /root/reference finds no schema, kernel or
// test); this implements the definition in tpr_rocm.h: order by a 32-bit
// sortable key (value order, -0.0 == +0.0, NaN above everything; inverted for
// largest=0), then by lowest index.  Each (key, index) pair is packed into one
// 64-bit "composite" key  (key << 32) | (0xffffffff - index)  so every element
// of a row has a distinct composite and larger composite == ranks earlier.
//
// Pass 1 (k_topk_seg): one 512-thread workgroup per (row, segment); rows are
// cut into segments so that the grid holds several workgroups per CU (memory
// latency is hidden by occupancy, not by register double-buffering).  Each
// workgroup streams its segment once from HBM in chunks of 512 x 16 floats
// (four 128-bit loads per thread) and keeps the exact top k of the segment:
//  1. The first chunk gives a lower bound T on the segment's k-th key: each
//     wave takes the r-th largest of its 64 per-lane maxima (r = ceil(k/8)); the
//     minimum over the 8 waves has >= 8*r >= k distinct elements at or above it.
//  2. Every element with key >= T is appended to an LDS candidate list
//     (wave-aggregated slot reservation: one LDS atomic per wave per chunk).
//  3. When the list grows past max(2k, 256) it is compacted to its exact top k
//     (rank selection below) and T rises past the k-th key kept.
//  4. The exact top k of the list is ranked; with one segment per row it is the
//     answer, otherwise its k composites go to the workspace.
// Pass 2 (k_topk_merge, only when rows are split): per row, rank the
// segments' candidates and write the final top k.
// Rank selection: rank(c) = #{candidates with a larger composite}; composites
// are distinct, so the ranks 0..k-1 are a permutation and give the sorted
// output directly.  The work is split over all threads (partial counts summed
// in LDS).
// If the list would overflow (adversarial rows: all-equal values, long runs of
// the threshold value), the workgroup switches to an exact multi-pass path over
// its segment: 4-pass 8-bit radix select in global memory finds the k-th key,
// then an index-ordered gather takes every larger key plus the lowest-index
// elements equal to it.

#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace tpr {
namespace {

constexpr int kT = 512;          // threads per segment workgroup
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kV = 4;            // float4 loads per thread per chunk
constexpr int kCH = kT * 4 * kV; // elements per chunk (8192)
constexpr int kB = 2048;         // candidate list capacity
constexpr int kKMax = 1024;      // largest k
constexpr int kMergeT = 256;     // merge workgroup
constexpr int kMergeMax = 4096;  // candidates a merge workgroup ranks (nseg * k)

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

// DPP wave reductions from the device library (no LDS round trips).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return __ockl_wfred_max_u32(v); }

__device__ __forceinline__ unsigned long long lanemask_lt() {
    return (1ull << __lane_id()) - 1ull;
}

struct TopkArgs {
    const float* in;
    long long rows;
    int cols;
    long long row_stride;
    int k;
    int largest;
    int force_fallback;
    int nseg;
    int seg_len;                 // multiple of kCH
    unsigned long long* part;    // [rows][nseg][k] composites when nseg > 1
    float* out_v;
    long long* out_i;
};

// Two candidate lists (ping-pong for compaction).  The final ranking reuses the
// idle list for its rank counters and sorted output.
struct TopkShared {
    unsigned long long list[2][kB];
    uint32_t wave_val[kW];
    int wave_cnt[kW];
    uint32_t hist[256];
    int count;
    int count2;
    int over;
    uint32_t thresh;
    uint32_t hi;
    int digit;
    int kk;
    int eq_taken;
};
static_assert(sizeof(int) * kB + sizeof(unsigned long long) * kKMax <= sizeof(unsigned long long) * kB,
              "rank + sel must fit in one idle list");

// Exact top-k of cand[0..m) into sel[0..k) (sorted).  m >= k.  Candidate i is
// counted by `groups` threads, each over a slice of the list; partial counts
// are summed in rank[i] with LDS atomics.
template <int NT>
__device__ void rank_select(const unsigned long long* cand, int* rank, unsigned long long* sel, int m, int k) {
    const int tid = threadIdx.x;
    for (int i = tid; i < m; i += NT) rank[i] = 0;
    __syncthreads();
    int groups = NT / max(m, 1);
    groups = max(1, min(groups, 64));
    const int slice = (m + groups - 1) / groups;
    for (int w = tid; w < m * groups; w += NT) {
        const int i = w % m;
        const int g = w / m;
        const unsigned long long ci = cand[i];
        const int j0 = g * slice;
        const int j1 = min(m, j0 + slice);
        int r0 = 0, r1 = 0, r2 = 0, r3 = 0;
        int j = j0;
        for (; j + 4 <= j1; j += 4) {
            const unsigned long long c0 = cand[j], c1 = cand[j + 1], c2 = cand[j + 2], c3 = cand[j + 3];
            r0 += (c0 > ci) ? 1 : 0;
            r1 += (c1 > ci) ? 1 : 0;
            r2 += (c2 > ci) ? 1 : 0;
            r3 += (c3 > ci) ? 1 : 0;
        }
        for (; j < j1; ++j) r0 += (cand[j] > ci) ? 1 : 0;
        const int r = r0 + r1 + r2 + r3;
        if (groups == 1) rank[i] = r;
        else if (r) atomicAdd(&rank[i], r);
    }
    __syncthreads();
    for (int i = tid; i < m; i += NT) {
        const int r = rank[i];
        if (r < k) sel[r] = cand[i];
    }
    __syncthreads();
}

// Loads one chunk (kV float4 per thread).  The bounds test is uniform across the
// workgroup, so a full chunk is kV unconditional 128-bit loads; the tail chunk
// uses clamped (always valid) scalar addresses and a select, so no divergent
// branch sits between a load and its use.
template <bool VEC>
__device__ __forceinline__ void load_chunk(float4 (&dst)[kV], const float* p, int cbase, int n) {
    const int tid = threadIdx.x;
    if (VEC && cbase + kCH <= n) {
#pragma unroll
        for (int j = 0; j < kV; ++j)
            dst[j] = *reinterpret_cast<const float4*>(p + cbase + 4 * (j * kT + tid));
    } else {
#pragma unroll
        for (int j = 0; j < kV; ++j) {
            const int e = cbase + 4 * (j * kT + tid);
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int eq = e + q;
                const float x = p[eq < n ? eq : n - 1];
                v[q] = (eq < n) ? x : 0.0f;
            }
            dst[j] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
}

// Exact multi-pass path over p[lo, hi) (any data).  Leaves the k selected
// composites in sh.list[0][0..k) (unordered).  hi - lo >= k.
__device__ void exact_select(TopkShared& sh, const float* p, int lo, int hi, int k, int largest) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    unsigned long long* cand = sh.list[0];
    uint32_t prefix = 0, pmask = 0;
    int kk = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) sh.hist[tid] = 0;
        __syncthreads();
        for (int e = lo + tid; e < hi; e += kT) {
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
    for (int base = lo; base < hi; base += kT) {
        const int e = base + tid;
        const uint32_t key = (e < hi) ? f2key(p[e], largest) : 0u;
        const bool gt = (e < hi) && key > T;
        const bool eq = (e < hi) && key == T;
        if (gt) cand[atomicAdd(&sh.count, 1)] = comp_key(key, (uint32_t)e);
        const unsigned long long bal = __ballot(eq);
        const int before = __popcll(bal & lanemask_lt());
        if (lane == 0) sh.wave_cnt[w] = __popcll(bal);
        __syncthreads();
        int wbase = sh.eq_taken;
        int total = 0;
        for (int i = 0; i < kW; ++i) {
            if (i < w) wbase += sh.wave_cnt[i];
            total += sh.wave_cnt[i];
        }
        if (eq && wbase + before < kk) cand[atomicAdd(&sh.count, 1)] = comp_key(key, (uint32_t)e);
        __syncthreads();
        if (tid == 0) sh.eq_taken += total;
        __syncthreads();
    }
    __syncthreads();
}

// Raises the bound T using the candidate list src[0..m) (all keys >= T) and
// moves the survivors to dst.  A 256-bin histogram of (key - T) >> shift, with
// shift chosen so the bins span [T, max key], locates the bin where the count
// from the top first reaches k; its lower edge T' has >= k candidates at or
// above it, so it is a valid bound.  Returns T'; sh.count2 = survivors.
__device__ uint32_t compact(TopkShared& sh, const unsigned long long* src, unsigned long long* dst, int m,
                            int k, uint32_t T) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    uint32_t mx = 0;
    for (int i = tid; i < m; i += kT) mx = max(mx, (uint32_t)(src[i] >> 32));
    mx = wave_max_u32(mx);
    if (lane == 0) sh.wave_val[w] = mx;
    if (tid < 256) sh.hist[tid] = 0;
    if (tid == 0) sh.count2 = 0;
    __syncthreads();
    uint32_t hi = 0;
#pragma unroll
    for (int i = 0; i < kW; ++i) hi = max(hi, sh.wave_val[i]);
    const uint32_t range = hi - T;
    const int shift = (range < 256u) ? 0 : (32 - __clz((int)range)) - 8;
    for (int i = tid; i < m; i += kT) atomicAdd(&sh.hist[((uint32_t)(src[i] >> 32) - T) >> shift], 1u);
    __syncthreads();
    if (w == 0) {
        // lane l owns bins 4l..4l+3; suffix sums from the top bin downwards
        const uint32_t h0 = sh.hist[4 * lane], h1 = sh.hist[4 * lane + 1];
        const uint32_t h2 = sh.hist[4 * lane + 2], h3 = sh.hist[4 * lane + 3];
        const int own = (int)(h0 + h1 + h2 + h3);
        // inclusive suffix sum over lanes >= lane
        int suf = own;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int t = __shfl_down(suf, d, 64);
            if (lane + d < 64) suf += t;
        }
        const unsigned long long ok = __ballot(suf >= k);
        const int L = 63 - __clzll((long long)ok);  // highest lane whose suffix reaches k
        if (lane == L) {
            int cum = suf - own;  // count strictly above this lane's bins
            int b = 3;
            const uint32_t hs[4] = {h0, h1, h2, h3};
            for (; b > 0; --b) {
                if (cum + (int)hs[b] >= k) break;
                cum += (int)hs[b];
            }
            sh.thresh = T + ((uint32_t)(4 * lane + b) << shift);
        }
    }
    __syncthreads();
    const uint32_t Tn = sh.thresh;
    for (int i0 = 0; i0 < m; i0 += kT) {
        const int i = i0 + tid;
        const unsigned long long c = (i < m) ? src[i] : 0ull;
        const bool keep = (i < m) && (uint32_t)(c >> 32) >= Tn;
        const unsigned long long bal = __ballot(keep);
        int base = 0;
        if (lane == 0 && bal) base = atomicAdd(&sh.count2, __popcll(bal));
        base = __shfl(base, 0, 64);
        if (keep) dst[base + __popcll(bal & lanemask_lt())] = c;
    }
    __syncthreads();
    return Tn;
}

template <bool VEC>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_topk_seg(TopkArgs a) {
    __shared__ TopkShared sh;
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    const long long row = blockIdx.x / a.nseg;
    const int seg = blockIdx.x % a.nseg;
    const float* p = a.in + row * a.row_stride;
    const int k = a.k;
    const int largest = a.largest;
    const int lo = seg * a.seg_len;
    const int hi = min(a.cols, lo + a.seg_len);
    const int n = hi;  // loads are bounded by the segment end
    const int nchunks = (hi - lo + kCH - 1) / kCH;
    const int r = (k + kW - 1) / kW;                 // per-wave rank for the bound
    const int compact_at = max(2 * k, 256);          // list size that triggers compaction

    if (tid == 0) { sh.count = 0; sh.over = 0; }
    __syncthreads();

    int cur_list = 0;
    bool over = a.force_fallback != 0 || r > 64;
    uint32_t T = 1;  // admit every valid key until the bound is known
    for (int c = 0; c < nchunks && !over; ++c) {
        const int cbase = lo + c * kCH;
        float4 cur[kV];
        load_chunk<VEC>(cur, p, cbase, n);
        uint32_t key[4 * kV];
#pragma unroll
        for (int j = 0; j < kV; ++j) {
            const int e = cbase + 4 * (j * kT + tid);
            key[4 * j + 0] = (e + 0 < n) ? f2key(cur[j].x, largest) : 0u;
            key[4 * j + 1] = (e + 1 < n) ? f2key(cur[j].y, largest) : 0u;
            key[4 * j + 2] = (e + 2 < n) ? f2key(cur[j].z, largest) : 0u;
            key[4 * j + 3] = (e + 3 < n) ? f2key(cur[j].w, largest) : 0u;
        }
        if (c == 0) {
            uint32_t m = 0;
#pragma unroll
            for (int q = 0; q < 4 * kV; ++q) m = max(m, key[q]);
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
        // filter: per-slot ballots give each passing element its wave offset
        unsigned long long* cand = sh.list[cur_list];
        unsigned long long bal[4 * kV];
        int total = 0;
#pragma unroll
        for (int q = 0; q < 4 * kV; ++q) {
            bal[q] = __ballot(key[q] >= T);
            total += __popcll(bal[q]);
        }
        if (total) {
            int base = 0;
            if (lane == 0) base = atomicAdd(&sh.count, total);
            base = __shfl(base, 0, 64);
            const unsigned long long lt = lanemask_lt();
#pragma unroll
            for (int q = 0; q < 4 * kV; ++q) {
                if (bal[q] & (1ull << lane)) {
                    const int pos = base + __popcll(bal[q] & lt);
                    const int e = cbase + 4 * ((q >> 2) * kT + tid) + (q & 3);
                    if (pos < kB) cand[pos] = comp_key(key[q], (uint32_t)e);
                    else sh.over = 1;
                }
                base += __popcll(bal[q]);
            }
        }
        __syncthreads();
        // read the shared verdicts, then fence them off from the next chunk's atomics
        over = sh.over != 0;
        const int m = sh.count;
        __syncthreads();
        if (over) break;
        if (m > compact_at) {
            T = compact(sh, sh.list[cur_list], sh.list[cur_list ^ 1], m, k, T);
            cur_list ^= 1;
            if (tid == 0) sh.count = sh.count2;
            __syncthreads();
        }
    }
    __syncthreads();

    int m = sh.count;
    if (over) {
        exact_select(sh, p, lo, hi, k, largest);
        m = k;
        cur_list = 0;
    }
    const unsigned long long* cand = sh.list[cur_list];
    int* rank = reinterpret_cast<int*>(sh.list[cur_list ^ 1]);
    unsigned long long* sel = sh.list[cur_list ^ 1] + kB / 2;
    rank_select<kT>(cand, rank, sel, m, k);
    if (a.nseg == 1) {
        for (int i = tid; i < k; i += kT) {
            const uint32_t idx = comp_index(sel[i]);
            a.out_v[row * k + i] = p[idx];
            a.out_i[row * k + i] = (long long)idx;
        }
    } else {
        unsigned long long* dst = a.part + ((long long)row * a.nseg + seg) * k;
        for (int i = tid; i < k; i += kT) dst[i] = sel[i];
    }
}

struct MergeShared {
    unsigned long long cand[kMergeMax];
    int rank[kMergeMax];
    unsigned long long sel[kKMax];
};

// Pass 2: exact top k of a row's nseg * k segment winners.
__global__ __launch_bounds__(kMergeT) void k_topk_merge(TopkArgs a) {
    __shared__ MergeShared sh;
    const long long row = blockIdx.x;
    const int k = a.k;
    const int m = a.nseg * k;
    const unsigned long long* src = a.part + row * (long long)m;
    for (int i = threadIdx.x; i < m; i += kMergeT) sh.cand[i] = src[i];
    __syncthreads();
    rank_select<kMergeT>(sh.cand, sh.rank, sh.sel, m, k);
    const float* p = a.in + row * a.row_stride;
    for (int i = threadIdx.x; i < k; i += kMergeT) {
        const uint32_t idx = comp_index(sh.sel[i]);
        a.out_v[row * k + i] = p[idx];
        a.out_i[row * k + i] = (long long)idx;
    }
}

struct TopkPlan {
    int nseg;
    int seg_len;
    size_t ws;
};

TopkPlan plan_topk(long long rows, long long cols, long long k) {
    TopkPlan pl{1, 0, 0};
    const long long chunks = (cols + kCH - 1) / kCH;
    // aim for >= 4 segment workgroups per CU, >= 2 chunks per segment, and a
    // merge list that fits one merge workgroup
    const long long want = 4LL * device_info().cus;
    long long nseg = 1;
    if (rows < want) nseg = (want + rows - 1) / rows;
    nseg = std::min(nseg, std::max(1LL, chunks / 2));
    nseg = std::min(nseg, std::max(1LL, (long long)kMergeMax / std::max(1LL, k)));
    if (knobs().splits > 0) nseg = std::min<long long>(knobs().splits, std::max(1LL, (long long)kMergeMax / std::max(1LL, k)));
    const long long seg_chunks = (chunks + nseg - 1) / nseg;
    pl.seg_len = (int)std::max<long long>(kCH, seg_chunks * kCH);
    pl.nseg = (int)((cols + pl.seg_len - 1) / pl.seg_len);
    if (pl.nseg < 1) pl.nseg = 1;
    // a segment shorter than k cannot hold k winners: do not split such rows
    if (pl.nseg > 1 && (cols - (long long)(pl.nseg - 1) * pl.seg_len) < k) {
        pl.nseg = 1;
        pl.seg_len = (int)std::max<long long>(kCH, chunks * kCH);
    }
    pl.ws = pl.nseg > 1 ? (size_t)rows * pl.nseg * k * sizeof(unsigned long long) : 0;
    return pl;
}

}  // namespace
}  // namespace tpr

extern "C" {

size_t tpr_topk_workspace_bytes(int32_t dtype, int64_t rows, int64_t cols, int64_t k) {
    (void)dtype;
    if (rows <= 0 || cols <= 0 || k <= 0 || k > cols || k > tpr::kKMax || cols > 0x7fffffffLL) return 0;
    return tpr::plan_topk(rows, cols, k).ws;
}

int tpr_topk(const void* in, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride,
             int64_t k, int32_t largest, int32_t sorted, void* out_values, void* out_indices,
             void* workspace, size_t workspace_bytes, void* stream) {
    using namespace tpr;
    (void)sorted;
    if (dtype != TPR_FLOAT32) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_topk: only float32 is implemented");
    if (rows < 0 || cols < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: negative shape");
    if (k < 0 || k > cols) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: selected index k out of range");
    if (rows == 0 || k == 0) return TPR_OK;
    if (cols > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: rows longer than 2^31-1");
    if (k > kKMax) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: k > 1024 is not implemented");
    if (!in || !out_values || !out_indices) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: null pointer");
    const TopkPlan pl = plan_topk(rows, cols, k);
    if (rows * (long long)pl.nseg > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: grid too large");
    if (pl.ws > 0 && (workspace == nullptr || workspace_bytes < pl.ws))
        return fail(TPR_ERR_WORKSPACE, "tpr_topk: workspace too small (need " + std::to_string(pl.ws) + " bytes)");
    TopkArgs a;
    a.in = static_cast<const float*>(in);
    a.rows = rows;
    a.cols = (int)cols;
    a.row_stride = row_stride;
    a.k = (int)k;
    a.largest = largest ? 1 : 0;
    a.force_fallback = knobs().topk_fallback ? 1 : 0;
    a.nseg = pl.nseg;
    a.seg_len = pl.seg_len;
    a.part = static_cast<unsigned long long*>(workspace);
    a.out_v = static_cast<float*>(out_values);
    a.out_i = static_cast<long long*>(out_indices);
    const bool vec = ((reinterpret_cast<uintptr_t>(in) & 15u) == 0) && (rows == 1 || row_stride % 4 == 0);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const long long grid = rows * pl.nseg;
    if (vec) hipLaunchKernelGGL((k_topk_seg<true>), dim3(grid), dim3(kT), 0, st, a);
    else hipLaunchKernelGGL((k_topk_seg<false>), dim3(grid), dim3(kT), 0, st, a);
    int rc = check_launch("k_topk_seg");
    if (rc != TPR_OK || pl.nseg == 1) return rc;
    hipLaunchKernelGGL(k_topk_merge, dim3(rows), dim3(kMergeT), 0, st, a);
    return check_launch("k_topk_merge");
}

}  // extern "C"
