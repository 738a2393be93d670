// gfx950 top-k along the last dim of a [rows, cols] view (float32, int32 and
// uint32 through the filter kernels below, 1- and 2-byte integers through the
// lane-group one; every dtype through the radix-select kernels).
//
// TensorPlay has no topk (grep of /root/reference finds no schema, kernel or
// test); this implements the definition in tpr_rocm.h: order by a 32-bit
// sortable key (value order, -0.0 == +0.0, NaN above everything; inverted for
// largest=0), then by lowest index.  Each (key, index) pair is packed into one
// 64-bit "composite" key  (key << 32) | (0xffffffff - index)  so every element
// of a row has a distinct composite and larger composite == ranks earlier.
//
// A row is cut into segments so the grid holds several workgroups per CU; each
// 512-thread workgroup keeps the exact top k of its segment.  With one segment
// per row it writes the answer, otherwise k_topk_merge ranks the segments'
// winners.  The segment kernel is a threshold filter over one HBM pass:
//   * Bound.  In a first slice every wave takes the r-th largest of its 64
//     per-lane maxima (r = ceil(k/8)); the minimum T0 over the 8 waves has
//     >= 8r >= k distinct elements at or above it, so no element below T0 can
//     be in the top k.
//   * Filter.  Elements with key >= T are appended to an LDS candidate list.
//   * Compaction.  A long list is cut with a 256-bin histogram of
//     (key - T) >> shift spanning [T, max key]: the lower edge of the bin where
//     the count from the top reaches k has >= k candidates at or above it and
//     becomes the new T.  Cost O(list), no sorting.
//   * Ranking.  rank(c) = #{candidates with a larger composite}; composites are
//     distinct, so ranks 0..k-1 are a permutation and give the sorted output.
//   * Exact path.  If a list would overflow (adversarial rows: all-equal values,
//     long runs of one value) the workgroup switches to a 4-pass 8-bit radix
//     select over its segment in global memory, then an index-ordered gather
//     takes every larger key plus the lowest-index elements equal to the k-th.
// Kernels:
//   k_topk_wave  (k <= 256: 256-entry wave lists up to k = 128, 512 above;
//     segments >= 8192, or >= 4096 with 4-wave workgroups): every wave streams
//     its own 1024-element slices (w, w+NW, ... or handed out by an LDS
//     counter) into a wave-private list with no workgroup barrier in the loop,
//     so one wave's filtering overlaps the other waves' loads.  Waves share a
//     monotone threshold through an LDS atomicMax; a published value always
//     has >= k candidates at or above it in the publishing wave's list, so it
//     bounds every wave.
//   k_topk_short (rows <= 4096, k <= 64, or k <= 128 on many rows <= 2048):
//     16/32/64 lanes per row, the row in registers, no workgroup barrier;
//     also 1- and 2-byte integers and bool on 16-byte aligned rows.
//   k_topk_rsel  (rows <= 32768 of <= 4-byte elements, large k or any dtype;
//     longer rows in segments of <= 32768 plus the merge): the row in
//     registers, an exact radix select, a bitonic sort of the k.
//   k_topk_radix (8-byte elements, or rows too long for the above): the same
//     select streaming over the row in memory.
//   k_topk_block (k <= 1024 on rows the others do not take): workgroup-wide
//     chunks with one shared list.
//   k_topk_merge: the k winners of a row's segments (radix cut, then ranking
//     or a bitonic sort).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <type_traits>
#include <string>

#include "common.h"

#ifdef TPR_DEBUG_KNOBS
// Test build only: merge outputs whose row index had to be clamped into the
// row (a segment that left its workspace slice unwritten, against the segment
// contract); read and cleared through tpr_debug_get("topk_merge_clamped").
static __device__ unsigned int topk_merge_clamped;
#endif

namespace tpr {
namespace {

constexpr int kT = 512;          // threads per segment workgroup
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kMaxW = 16;        // most waves of any top-k workgroup (1024 threads)
constexpr int kV = 4;            // float4 loads per thread per chunk (block kernel)
constexpr int kCH = kT * 4 * kV; // elements per block-kernel chunk (8192)
constexpr int kB = 2048;         // block candidate list capacity
constexpr int kKMax = 1024;      // largest k of the segment kernels (larger k: k_topk_radix)
constexpr int kMergeT = 256;     // merge workgroup
constexpr int kMergeMax = 8192;  // candidates a merge workgroup ranks (nseg * k)

constexpr int kWaveK = 256;                   // largest k of the wave kernel (129..256: 512-entry lists)
constexpr int kShortK2 = 128;                 // largest k of the lane-group kernel (64 lanes, two keys each)
// Rows shorter than 16384 with k above this take the register radix select:
// the wave kernel has too few slices per wave there (MI355X, us, k = 256:
// [1024, 8192] 4 waves 118, 8 waves 42, radix 35; [4096, 4096] 4 waves 155,
// radix 55), while up to it the 4-wave kernel mostly wins (k = 150:
// [1024, 8192] 23 against 35, [4096, 8192] 76 against 110).
constexpr int kWave4K = 192;
constexpr int kWaveSmallK = 128;              // largest k of the wave kernel on 1- / 2-byte rows
constexpr int kWB = 256;                      // per-wave list capacity
constexpr int kWaveCompact = 192;             // per-wave list size that always triggers compaction
constexpr int kSlice = 64 * 16;               // elements per wave slice (4 float4 per lane)
constexpr int kWaveMinSeg = kW * kSlice;      // every wave has a full first slice (8192)
constexpr long long kWaveMaxSeg = 1LL << 28;  // longest wave-kernel segment (32-bit byte offsets)

// Order-preserving float -> uint32 map: non-negative u -> u | 2^31, negative
// u -> ~u + 1 (two's-complement negate of the magnitude's image), so -0.0 and
// +0.0 land on the same key 2^31; every NaN is first made 0x7fc00000 (above
// +inf).  lmask = 0 keeps the order (largest), ~0 reverses it (smallest).
// Valid keys are never 0: 0 marks "no element".  Branch-free: one NaN compare
// (f != f) and select, an arithmetic shift, xor, subtract, xor.
__device__ __forceinline__ uint32_t f2key_sel(float f, uint32_t lmask) {
    const uint32_t u = (f != f) ? 0x7fc00000u : __float_as_uint(f);
    const uint32_t m = (uint32_t)((int32_t)u >> 31);
    return ((u ^ (m | 0x80000000u)) - m) ^ lmask;
}

__device__ __forceinline__ uint32_t f2key(float f, int largest) {
    return f2key_sel(f, largest ? 0u : 0xffffffffu);
}

// Inverse of f2key.  Exact except for the two canonicalised cases (-0.0 comes
// back as +0.0, any NaN as 0x7fc00000); callers re-read the input for those.
__device__ __forceinline__ uint32_t key2bits(uint32_t key, int largest) {
    const uint32_t k = largest ? key : ~key;
    return (k & 0x80000000u) ? (k & 0x7fffffffu) : (0u - k);
}

// Output value of a selected element: from its key, or from the input row when
// the key cannot tell (+-0.0, NaN payloads).
__device__ __forceinline__ float selected_value(const float* p, uint32_t key, uint32_t idx, int largest) {
    const uint32_t u = key2bits(key, largest);
    return (u == 0u || u == 0x7fc00000u) ? p[idx] : __uint_as_float(u);
}

// Order-preserving key of a 32-bit integer (its bits in f): int32 flips the
// sign bit, uint32 is its own key; lmask as for floats.  Unlike float keys an
// integer key can be 0 (INT_MIN / 0 largest, INT_MAX / UINT_MAX smallest),
// the key of padding past a row's end.
__device__ __forceinline__ uint32_t i2key_sel(float f, uint32_t smask, uint32_t lmask) {
    return __float_as_uint(f) ^ smask ^ lmask;
}

// Key of one element of a float32 (ikind 0), int32 (1) or uint32 (2) row.
__device__ __forceinline__ uint32_t elem_key(float f, int largest, int ikind) {
    const uint32_t lm = largest ? 0u : 0xffffffffu;
    return ikind ? i2key_sel(f, ikind == 1 ? 0x80000000u : 0u, lm) : f2key_sel(f, lm);
}

// Ascending sortable key of an element of any dtype, as an unsigned integer of
// the element's width (32 bits for elements of at most 4 bytes): floats as
// f2key (-0.0 == +0.0, every NaN above +inf), signed integers with the sign
// bit flipped, unsigned integers and bool as they are; inverted for
// largest = 0.
template <class T>
struct SortKey {
    using K = typename std::conditional<(sizeof(T) > 4), unsigned long long, uint32_t>::type;
    static constexpr int kBits = 8 * (int)sizeof(T);
    __device__ static K of(T x, int largest) {
        K k;
        if constexpr (std::is_same<T, float>::value) {
            return f2key(x, largest);
        } else if constexpr (std::is_same<T, double>::value) {
            const unsigned long long b = (unsigned long long)__double_as_longlong(x);
            const unsigned long long u =
                ((b & 0x7fffffffffffffffull) > 0x7ff0000000000000ull) ? 0x7ff8000000000000ull : b;
            const unsigned long long m = (unsigned long long)((long long)u >> 63);
            k = (u ^ (m | 0x8000000000000000ull)) - m;
        } else if constexpr (std::is_signed<T>::value) {
            using U = typename std::make_unsigned<T>::type;
            k = (K)(U)((U)x ^ (U)((U)1 << (kBits - 1)));
        } else {
            k = (K)x;
        }
        if (!largest) k = ~k & (kBits == 64 ? ~(K)0 : (K)(((unsigned long long)1 << kBits) - 1));
        return k;
    }
};

// Bits of an integer element (ikind 1 signed, 2 unsigned / bool; em = the
// element's mask) from its sortable key: the key is the element with the sign
// bit flipped (signed) and complemented for largest = 0, so this is exact and
// the selected values need no second read of the input (which the row's
// nontemporal loads have not left in the cache).
__device__ __forceinline__ uint32_t int_key_bits(uint32_t key, int ikind, int largest, uint32_t em) {
    const uint32_t sm = ikind == 1 ? (em >> 1) + 1u : 0u;
    return (key ^ (largest ? 0u : 0xffffffffu) ^ sm) & em;
}

// 64-bit sortable key of an 8-byte element given by its bits: float64 (ikind
// 0), int64 (1) or uint64 (2), as SortKey.
__device__ __forceinline__ unsigned long long key64_of(unsigned long long bits, int largest, int ikind) {
    if (ikind == 0) return SortKey<double>::of(__longlong_as_double((long long)bits), largest);
    if (ikind == 1) return SortKey<long long>::of((long long)bits, largest);
    return SortKey<unsigned long long>::of(bits, largest);
}

__device__ __forceinline__ unsigned long long comp_key(uint32_t key, uint32_t idx) {
    return ((unsigned long long)key << 32) | (unsigned long long)(0xffffffffu - idx);
}

__device__ __forceinline__ uint32_t comp_index(unsigned long long c) {
    return 0xffffffffu - (uint32_t)(c & 0xffffffffull);
}

// DPP wave reduction from the device library (no LDS round trips).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return __ockl_wfred_max_u32(v); }

// Inclusive prefix sum over the wave's 64 lanes (every lane active): DPP row
// shifts by 1, 2, 4, 8 (lanes whose source is outside the row add the 0 passed
// as `old`), then row_bcast:15 and row_bcast:31 carry the row totals upward.
// No LDS round trips.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

__device__ __forceinline__ unsigned long long lanemask_lt() { return (1ull << __lane_id()) - 1ull; }

struct TopkArgs {
    const float* in;
    long long rows;
    int cols;
    long long row_stride;
    int k;
    int largest;
    int ikind;  // k_topk_short: 0 float32, 1 int32, 2 uint32 (the elements' bits, loaded as floats)
    int force_fallback;
    int nseg;
    int seg_len;
    unsigned long long* part;  // [rows][nseg][k] composites when nseg > 1
    float* out_v;
    long long* out_i;
    // sampling (tpr_sample): instead of writing values / indices, draw one id
    // per row from the sorted top k (see sample_from_sel)
    int sample;
    int dyn;  // wave kernel: slices after the first ones handed out by an LDS counter
    int* flags;  // 8-byte rows in the wave kernel: per row, 1 = finish in k_topk_radix (else null)
    float temperature, top_p;
    const float* u;
    long long* ids;
};

// Top-k / top-p draw from a row's sorted selection (composites in rank order),
// run by one wave (threads 0..63):  p_j = exp(v_j/T - v_0/T), c_j = p_0 + .. +
// p_j, m = first j with c_j >= top_p * c_{k-1}, id = index of the first j <= m
// with c_j > u * c_m; T <= 0 takes the first.  Each lane owns a contiguous
// block of <= 16 candidates: serial sums inside the block, a wave scan of the
// block totals, ballots for the two searches.
__device__ void sample_from_sel(const TopkArgs& a, long long row, const float* p, const unsigned long long* sel,
                                int k) {
    const int lane = __lane_id();
    if (!(a.temperature > 0.0f)) {
        if (lane == 0) a.ids[row] = (long long)comp_index(sel[0]);
        return;
    }
    const int per = (k + 63) / 64;
    const int j0 = lane * per;
    const float z0 = selected_value(p, (uint32_t)(sel[0] >> 32), comp_index(sel[0]), a.largest) / a.temperature;
    float pr[16];
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int j = j0 + q;
        pr[q] = 0.0f;
        if (q < per && j < k) {
            const float v = selected_value(p, (uint32_t)(sel[j] >> 32), comp_index(sel[j]), a.largest);
            pr[q] = expf(v / a.temperature - z0);
            s += pr[q];
        }
    }
    // inclusive scan of the block totals by DPP (row shifts, then the row
    // broadcasts), no LDS round trips; lane 63's total read directly
    float incl = s;
#define TPR_DPP_ADD(CTRL, ROWS) \
    incl += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(incl), CTRL, ROWS, 0xf, false))
    TPR_DPP_ADD(0x111, 0xf);  // row_shr:1
    TPR_DPP_ADD(0x112, 0xf);  // row_shr:2
    TPR_DPP_ADD(0x114, 0xf);  // row_shr:4
    TPR_DPP_ADD(0x118, 0xf);  // row_shr:8
    TPR_DPP_ADD(0x142, 0xa);  // row_bcast:15
    TPR_DPP_ADD(0x143, 0xc);  // row_bcast:31
#undef TPR_DPP_ADD
    const float excl = incl - s;
    const float cut = a.top_p * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), 63));
    int mj = 0x7fffffff;
    float c = excl;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int j = j0 + q;
        if (q < per && j < k) {
            c += pr[q];
            if (c >= cut && mj == 0x7fffffff) mj = j;
        }
    }
    mj = __ockl_wfred_min_i32(mj);
    const int m = (mj == 0x7fffffff) ? k - 1 : mj;
    float cm_l = 0.0f;
    c = excl;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int j = j0 + q;
        if (q < per && j < k) {
            c += pr[q];
            if (j == m) cm_l = c;
        }
    }
    const float thr = a.u[row] * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cm_l), m / per));
    int pj = 0x7fffffff;
    c = excl;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int j = j0 + q;
        if (q < per && j <= m) {
            c += pr[q];
            if (c > thr && pj == 0x7fffffff) pj = j;
        }
    }
    pj = __ockl_wfred_min_i32(pj);
    if (pj > m) pj = m;
    if (lane == 0) a.ids[row] = (long long)comp_index(sel[pj]);
}

// Sampling with k > kKMax: the draw of sample_from_sel over a row's sorted top
// k that tpr_topk has already written (vals[row][k] in rank order, idx[row][k]
// their indices), one workgroup of NT threads per row.  Thread t owns the
// contiguous positions [t*per, (t+1)*per): serial sums inside its block, a
// workgroup scan of the block totals, workgroup minima for the nucleus end m
// and the drawn position.  p_j is formed with explicit roundings (no
// contraction), so the three passes over a block see bit-identical c_j.
constexpr int kDrawNT = 1024;

__device__ __forceinline__ float draw_weight(float v, float temperature, float z0) {
    return expf(__fsub_rn(__fdiv_rn(v, temperature), z0));
}

template <int W>
__device__ __forceinline__ int block_min_i32(int v, int* sh) {
    v = __ockl_wfred_min_i32(v);
    if (__lane_id() == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = sh[0];
#pragma unroll
    for (int q = 1; q < W; ++q) r = min(r, sh[q]);
    return r;
}

template <int NT>
__global__ __launch_bounds__(NT) void k_sample_sorted(const float* vals, const long long* idx, int k,
                                                      float temperature, float top_p, const float* u,
                                                      long long* ids) {
    constexpr int W = NT / 64;
    __shared__ float wsum[W];
    __shared__ int wmin[2][W];
    __shared__ float cm_sh;
    const long long row = blockIdx.x;
    const float* v = vals + row * k;
    const int tid = threadIdx.x, w = tid >> 6;
    if (!(temperature > 0.0f)) {
        if (tid == 0) ids[row] = idx[row * k];
        return;
    }
    const int per = (k + NT - 1) / NT;
    const int j0 = min(k, tid * per), j1 = min(k, j0 + per);
    const float z0 = __fdiv_rn(v[0], temperature);
    float s = 0.0f;
    for (int j = j0; j < j1; ++j) s += draw_weight(v[j], temperature, z0);
    float incl = s;
#define TPR_DPP_ADD(CTRL, ROWS) \
    incl += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(incl), CTRL, ROWS, 0xf, false))
    TPR_DPP_ADD(0x111, 0xf);  // row_shr:1
    TPR_DPP_ADD(0x112, 0xf);  // row_shr:2
    TPR_DPP_ADD(0x114, 0xf);  // row_shr:4
    TPR_DPP_ADD(0x118, 0xf);  // row_shr:8
    TPR_DPP_ADD(0x142, 0xa);  // row_bcast:15
    TPR_DPP_ADD(0x143, 0xc);  // row_bcast:31
#undef TPR_DPP_ADD
    if (__lane_id() == 63) wsum[w] = incl;
    __syncthreads();
    float before = 0.0f, total = 0.0f;
#pragma unroll
    for (int q = 0; q < W; ++q) {
        const float t = wsum[q];
        if (q < w) before += t;
        total += t;
    }
    const float excl = before + (incl - s);
    const float cut = top_p * total;
    int mj = 0x7fffffff;
    float c = excl;
    for (int j = j0; j < j1; ++j) {
        c += draw_weight(v[j], temperature, z0);
        if (c >= cut) {
            mj = j;
            break;
        }
    }
    mj = block_min_i32<W>(mj, wmin[0]);
    const int m = (mj == 0x7fffffff) ? k - 1 : mj;
    if (m >= j0 && m < j1) {
        c = excl;
        for (int j = j0; j <= m; ++j) c += draw_weight(v[j], temperature, z0);
        cm_sh = c;
    }
    __syncthreads();
    const float thr = u[row] * cm_sh;
    int pj = 0x7fffffff;
    c = excl;
    for (int j = j0; j < j1 && j <= m; ++j) {
        c += draw_weight(v[j], temperature, z0);
        if (c > thr) {
            pj = j;
            break;
        }
    }
    pj = block_min_i32<W>(pj, wmin[1]);
    if (pj > m) pj = m;
    if (tid == 0) ids[row] = idx[row * k + pj];
}

// Workspace of tpr_sample with k > kKMax: tpr_topk's own workspace, then the
// sorted values [rows][k] (float32) and indices [rows][k] (int64), each part
// starting on a 256-byte boundary.
struct SampleSortedLayout {
    size_t topk_ws, vals_off, idx_off, total;
};

inline size_t round_up_256(size_t b) { return (b + 255) & ~(size_t)255; }

inline SampleSortedLayout sample_sorted_layout(int64_t rows, int64_t cols, int64_t k) {
    SampleSortedLayout l;
    l.topk_ws = tpr_topk_workspace_bytes(TPR_FLOAT32, rows, cols, k);
    l.vals_off = round_up_256(l.topk_ws);
    l.idx_off = l.vals_off + round_up_256((size_t)rows * (size_t)k * sizeof(float));
    l.total = l.idx_off + (size_t)rows * (size_t)k * sizeof(long long);
    return l;
}

// Small shared state of the workgroup-level helpers.
struct BlockScratch {
    uint32_t wave_val[kMaxW];
    uint32_t wave_t[kMaxW];  // wave kernel: per-wave final bounds (see k_topk_wave)
    int wave_cnt[kMaxW];
    uint32_t hist[256];
    int count;
    int count2;
    int over;
    uint32_t thresh;
    uint32_t tshared;
    int digit;
    int kk;
    int eq_taken;
    int next_slice;  // wave kernel: next slice to hand out (dynamic assignment)
};

// r-th largest of the wave's per-lane maxima of `key` (0 if fewer than r lanes
// hold valid keys).
__device__ __forceinline__ uint32_t wave_rth_of_lane_max(const uint32_t* key, int nkeys, int r) {
    const int lane = __lane_id();
    uint32_t m = 0;
    for (int q = 0; q < nkeys; ++q) m = max(m, key[q]);
    uint32_t rth = 0;
    for (int i = 0; i < r; ++i) {
        const uint32_t wm = wave_max_u32(m);
        rth = wm;
        if (wm == 0) break;
        const unsigned long long bal = __ballot(m == wm);
        if (lane == __ffsll((long long)bal) - 1) m = 0;
    }
    return rth;
}

// Exact top-k of cand[0..m) into sel[0..k) (sorted).  m >= k.  Candidate i is
// counted by `groups` threads, each over a slice of the list; partial counts
// are summed in rank[i] with LDS atomics.
// W8: the composites carry the high half of 64-bit keys; lo[i] is the low
// half of candidate i's key, which orders equal high halves before the index.
template <int NT, bool W8 = false>
__device__ void rank_select(const unsigned long long* cand, int* rank, unsigned long long* sel, int m, int k,
                            const uint32_t* lo = nullptr) {
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
        if constexpr (W8) {
            // d ranks above c: larger high half, or equal high halves and a
            // larger low half, or both equal and a lower index
            const uint32_t chi = (uint32_t)(ci >> 32), clo = lo[i];
            for (; j < j1; ++j) {
                const unsigned long long d = cand[j];
                const uint32_t dhi = (uint32_t)(d >> 32), dlo = lo[j];
                r0 += (dhi > chi || (dhi == chi && (dlo > clo || (dlo == clo && d > ci)))) ? 1 : 0;
            }
        } else {
            for (; j + 4 <= j1; j += 4) {
                const unsigned long long c0 = cand[j], c1 = cand[j + 1], c2 = cand[j + 2], c3 = cand[j + 3];
                r0 += (c0 > ci) ? 1 : 0;
                r1 += (c1 > ci) ? 1 : 0;
                r2 += (c2 > ci) ? 1 : 0;
                r3 += (c3 > ci) ? 1 : 0;
            }
            for (; j < j1; ++j) r0 += (cand[j] > ci) ? 1 : 0;
        }
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

// Threshold from a 256-bin histogram whose bins span [T, T + 256 << shift):
// lane l of one wave owns bins 4l..4l+3.  Returns the lower edge of the bin
// where the count from the top first reaches k (valid in every lane).
__device__ __forceinline__ uint32_t hist_threshold(const uint32_t* hist, int k, uint32_t T, int shift) {
    const int lane = __lane_id();
    const uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
    const int own = (int)(h0 + h1 + h2 + h3);
    // inclusive suffix sum over lanes >= lane = total - exclusive prefix: the
    // prefix by DPP row shifts and row broadcasts (every lane active), the
    // total read from lane 63, no LDS round trips
    int pre = own;
#define TPR_DPP_ADD(CTRL, ROWS) pre += __builtin_amdgcn_update_dpp(0, pre, CTRL, ROWS, 0xf, false)
    TPR_DPP_ADD(0x111, 0xf);  // row_shr:1
    TPR_DPP_ADD(0x112, 0xf);  // row_shr:2
    TPR_DPP_ADD(0x114, 0xf);  // row_shr:4
    TPR_DPP_ADD(0x118, 0xf);  // row_shr:8
    TPR_DPP_ADD(0x142, 0xa);  // row_bcast:15
    TPR_DPP_ADD(0x143, 0xc);  // row_bcast:31
#undef TPR_DPP_ADD
    const int suf = __builtin_amdgcn_readlane(pre, 63) - pre + own;
    const unsigned long long ok = __ballot(suf >= k);
    if (ok == 0) return T;                      // fewer than k entries: no raise
    const int L = 63 - __clzll((long long)ok);  // highest lane whose suffix reaches k
    uint32_t tn = 0;
    if (lane == L) {
        int cum = suf - own;
        const uint32_t hs[4] = {h0, h1, h2, h3};
        int b = 3;
        for (; b > 0; --b) {
            if (cum + (int)hs[b] >= k) break;
            cum += (int)hs[b];
        }
        tn = T + ((uint32_t)(4 * lane + b) << shift);
    }
    return (uint32_t)__builtin_amdgcn_readlane((int)tn, L);
}

__device__ __forceinline__ int hist_shift(uint32_t hi, uint32_t T) {
    const uint32_t range = hi - T;
    return (range < 256u) ? 0 : (32 - __clz((int)range)) - 8;
}

// Workgroup-level compaction: raises T using src[0..m) (all keys >= T) and moves
// the survivors to dst.  Returns the new T; bs.count2 = survivors.
template <int NT>
__device__ uint32_t block_compact(BlockScratch& bs, const unsigned long long* src, unsigned long long* dst, int m,
                                  int k, uint32_t T) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    uint32_t mx = 0;
    for (int i = tid; i < m; i += NT) mx = max(mx, (uint32_t)(src[i] >> 32));
    mx = wave_max_u32(mx);
    if (lane == 0) bs.wave_val[w] = mx;
    if (tid < 256) bs.hist[tid] = 0;
    if (tid == 0) bs.count2 = 0;
    __syncthreads();
    uint32_t hi = 0;
    for (int i = 0; i < NT / 64; ++i) hi = max(hi, bs.wave_val[i]);
    const int shift = hist_shift(hi, T);
    for (int i = tid; i < m; i += NT) atomicAdd(&bs.hist[((uint32_t)(src[i] >> 32) - T) >> shift], 1u);
    __syncthreads();
    if (w == 0) {
        const uint32_t tn = hist_threshold(bs.hist, k, T, shift);
        if (lane == 0) bs.thresh = tn;
    }
    __syncthreads();
    const uint32_t Tn = bs.thresh;
    for (int i0 = 0; i0 < m; i0 += NT) {
        const int i = i0 + tid;
        const unsigned long long c = (i < m) ? src[i] : 0ull;
        const bool keep = (i < m) && (uint32_t)(c >> 32) >= Tn;
        const unsigned long long bal = __ballot(keep);
        int base = 0;
        if (lane == 0 && bal) base = atomicAdd(&bs.count2, __popcll(bal));
        base = __builtin_amdgcn_readlane(base, 0);
        if (keep) dst[base + __popcll(bal & lanemask_lt())] = c;
    }
    __syncthreads();
    return Tn;
}

// Wave-level compaction of list[0..m) in place; m is updated.  Entries below T
// (admitted before another wave raised the shared bound) are dropped.  If more
// than k entries are >= T, the threshold is raised by the histogram rule and
// the survivors are those >= the new threshold (>= k of them); otherwise T is
// returned unchanged.
__device__ uint32_t wave_compact(unsigned long long* list, uint32_t* hist, int& m, int k, uint32_t T) {
    const int lane = __lane_id();
    uint32_t mx = 0;
    int ge = 0;
    for (int i = lane; i < m; i += 64) {
        const uint32_t key = (uint32_t)(list[i] >> 32);
        if (key >= T) {
            mx = max(mx, key);
            ++ge;
        }
    }
    mx = wave_max_u32(mx);
    ge = (int)__ockl_wfred_add_u32((uint32_t)ge);
    uint32_t tn = T;
    if (ge > k) {
        const int shift = hist_shift(mx, T);
#pragma unroll
        for (int b = 0; b < 4; ++b) hist[4 * lane + b] = 0;
        __builtin_amdgcn_wave_barrier();
        for (int i = lane; i < m; i += 64) {
            const uint32_t key = (uint32_t)(list[i] >> 32);
            if (key >= T) atomicAdd(&hist[(key - T) >> shift], 1u);
        }
        __builtin_amdgcn_wave_barrier();
        tn = hist_threshold(hist, k, T, shift);
    }
    // a write position never passes the read position, so in place is safe
    int out = 0;
    for (int i0 = 0; i0 < m; i0 += 64) {
        const int i = i0 + lane;
        const unsigned long long c = (i < m) ? list[i] : 0ull;
        const bool keep = (i < m) && (uint32_t)(c >> 32) >= tn;
        const unsigned long long b = __ballot(keep);
        __builtin_amdgcn_wave_barrier();
        if (keep) list[out + __popcll(b & lanemask_lt())] = c;
        out += __popcll(b);
        __builtin_amdgcn_wave_barrier();
    }
    m = out;
    return tn;
}

// A key with at least kw entries of list[0..m) at or above it (T when fewer
// than kw entries are >= T): the lower edge of the histogram bin over
// [T, list max] where the count from the top reaches kw.  The list is not
// changed.
__device__ uint32_t wave_kth_bound(const unsigned long long* list, uint32_t* hist, int m, int kw, uint32_t T) {
    const int lane = __lane_id();
    uint32_t mx = 0;
    int ge = 0;
    for (int i = lane; i < m; i += 64) {
        const uint32_t key = (uint32_t)(list[i] >> 32);
        if (key >= T) {
            mx = max(mx, key);
            ++ge;
        }
    }
    mx = wave_max_u32(mx);
    ge = (int)__ockl_wfred_add_u32((uint32_t)ge);
    if (ge < kw) return T;
    const int shift = hist_shift(mx, T);
#pragma unroll
    for (int b = 0; b < 4; ++b) hist[4 * lane + b] = 0;
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < m; i += 64) {
        const uint32_t key = (uint32_t)(list[i] >> 32);
        if (key >= T) atomicAdd(&hist[(key - T) >> shift], 1u);
    }
    __builtin_amdgcn_wave_barrier();
    return hist_threshold(hist, kw, T, shift);
}

// Exact multi-pass path over p[lo, hi) (any data): leaves the k selected
// composites in cand[0..k) (unordered).  hi - lo >= k.
// Sortable 32-bit key of element e of a row of EB-byte elements (EB = 4:
// float32 / int32 / uint32 by ikind; EB = 1, 2: 8- and 16-bit integers and
// bool, key = the element with its sign bit flipped when signed, complemented
// for largest = 0: the lane-group kernel's key).
template <int EB>
__device__ __forceinline__ uint32_t row_key(const void* p, int e, int largest, int ikind) {
    if constexpr (EB == 4) {
        return elem_key(static_cast<const float*>(p)[e], largest, ikind);
    } else {
        constexpr uint32_t em = EB == 1 ? 0xffu : 0xffffu;
        const uint32_t v = EB == 1 ? static_cast<const uint8_t*>(p)[e] : static_cast<const uint16_t*>(p)[e];
        const uint32_t sm = ikind == 1 ? (em >> 1) + 1u : 0u;
        return (v ^ sm ^ (largest ? 0u : 0xffffffffu)) & em;
    }
}

template <int NT, int EB = 4>
__device__ void exact_select(BlockScratch& bs, unsigned long long* cand, const void* p, int lo, int hi, int k,
                             int largest, int ikind) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    uint32_t prefix = 0, pmask = 0;
    int kk = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) bs.hist[tid] = 0;
        __syncthreads();
        for (int e = lo + tid; e < hi; e += NT) {
            const uint32_t key = row_key<EB>(p, e, largest, ikind);
            if ((key & pmask) == prefix) atomicAdd(&bs.hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            int cum = 0, d = 0;
            for (int b = 255; b >= 0; --b) {
                const int h = (int)bs.hist[b];
                if (cum + h >= kk) { d = b; break; }
                cum += h;
            }
            bs.digit = d;
            bs.kk = kk - cum;
        }
        __syncthreads();
        prefix |= (uint32_t)bs.digit << shift;
        pmask |= 0xffu << shift;
        kk = bs.kk;
        __syncthreads();
    }
    const uint32_t T = prefix;  // exact k-th key; kk = how many keys == T to take
    if (tid == 0) { bs.count = 0; bs.eq_taken = 0; }
    __syncthreads();
    for (int base = lo; base < hi; base += NT) {
        const int e = base + tid;
        const uint32_t key = (e < hi) ? row_key<EB>(p, e, largest, ikind) : 0u;
        const bool gt = (e < hi) && key > T;
        const bool eq = (e < hi) && key == T;
        if (gt) cand[atomicAdd(&bs.count, 1)] = comp_key(key, (uint32_t)e);
        const unsigned long long bal = __ballot(eq);
        const int before = __popcll(bal & lanemask_lt());
        if (lane == 0) bs.wave_cnt[w] = __popcll(bal);
        __syncthreads();
        int wbase = bs.eq_taken;
        int total = 0;
        for (int i = 0; i < NW; ++i) {
            if (i < w) wbase += bs.wave_cnt[i];
            total += bs.wave_cnt[i];
        }
        if (eq && wbase + before < kk) cand[atomicAdd(&bs.count, 1)] = comp_key(key, (uint32_t)e);
        __syncthreads();
        if (tid == 0) bs.eq_taken += total;
        __syncthreads();
    }
    __syncthreads();
}

// Writes the ranked top k of one segment: the final values/indices when the row
// is not split, else the k composites for the merge pass.
template <int EB = 4>
__device__ __forceinline__ void write_segment(const TopkArgs& a, long long row, int seg, const float* p,
                                              const unsigned long long* sel, int k) {
    if (a.nseg == 1 && a.sample) {
        if (threadIdx.x < 64) sample_from_sel(a, row, p, sel, k);
    } else if (a.nseg == 1) {
        for (int i = threadIdx.x; i < k; i += blockDim.x) {
            const uint32_t idx = comp_index(sel[i]);
            const uint32_t key = (uint32_t)(sel[i] >> 32);
            if constexpr (EB == 8) {  // the element itself (the composite carries half its key)
                reinterpret_cast<unsigned long long*>(a.out_v)[row * k + i] =
                    reinterpret_cast<const unsigned long long*>(p)[idx];
            } else if constexpr (EB == 1) {
                reinterpret_cast<uint8_t*>(a.out_v)[row * k + i] = (uint8_t)int_key_bits(key, a.ikind, a.largest, 0xffu);
            } else if constexpr (EB == 2) {
                reinterpret_cast<uint16_t*>(a.out_v)[row * k + i] =
                    (uint16_t)int_key_bits(key, a.ikind, a.largest, 0xffffu);
            } else {
                a.out_v[row * k + i] = a.ikind ? __uint_as_float(int_key_bits(key, a.ikind, a.largest, 0xffffffffu))
                                               : selected_value(p, key, idx, a.largest);
            }
            a.out_i[row * k + i] = (long long)idx;
        }
    } else {
        unsigned long long* dst = a.part + ((long long)row * a.nseg + seg) * k;
        for (int i = threadIdx.x; i < k; i += blockDim.x) dst[i] = sel[i];
    }
}

// ---------------------------------------------------------------------------
// Wave-independent segment kernel.
// ---------------------------------------------------------------------------
template <int NW, int KWB>
struct WaveShared {
    unsigned long long wl[NW][KWB];    // per-wave candidate lists (2 or 4 KiB per wave)
    union {
        uint32_t hist[NW][256];        // per-wave histograms while streaming
        unsigned long long un[NW * KWB];  // gathered list afterwards
    };
    BlockScratch bs;
};
// After the gather the per-wave list area (NW * KWB composites) is idle: rank
// (m <= NW * KWB ints) takes its first half and sel (k composites) its second;
// lists of KWB hold k <= KWB / 2 (kWB = 256 for k <= 128, 512 above).
static_assert(kWaveK <= 4 * 512 / 2, "sel fits in the second half of the list area");

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufWord3 = 0x00020000;  // raw buffer resource, 32-bit data (gfx9 family)
constexpr int kNT = 2;                 // cache policy bit: nontemporal (the row is read once)

// One float through a buffer resource (the 32-bit buffer load returns the raw
// bits as an unsigned int: reinterpret, never convert).
__device__ __forceinline__ float buf_ld_f32(__amdgpu_buffer_rsrc_t r, int off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kNT));
}

// Segment loads go through a buffer resource whose range is the segment: the
// hardware range check is per dword, so a load past the segment end returns 0
// and moves no data.  Slice loads are therefore unconditional (a prefetch past
// the last slice is free), which keeps the compiler's wait counts exact.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t segment_rsrc(const float* seg, int n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(seg), (short)0, n * 4, kBufWord3);
}

// Loads slice elements [rel, rel + 256*SV) of the segment: lane l, vector j
// gets elements rel + 4*(j*64 + l) .. +3.  VEC: 128-bit loads (16-byte aligned
// segment); otherwise four 32-bit loads per vector.
template <bool VEC, int SV>
__device__ __forceinline__ void load_slice(float4 (&cur)[SV], __amdgpu_buffer_rsrc_t r, int rel) {
    const int lane = __lane_id();
#pragma unroll
    for (int j = 0; j < SV; ++j) {
        const int off = 4 * (rel + 4 * (j * 64 + lane));
        if constexpr (VEC) {
            const f32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT);
            cur[j] = make_float4(v.x, v.y, v.z, v.w);
        } else {
            cur[j] = make_float4(buf_ld_f32(r, off), buf_ld_f32(r, off + 4), buf_ld_f32(r, off + 8),
                                 buf_ld_f32(r, off + 12));
        }
    }
}


// Sortable keys of one slice; elements at or past `hi` get key 0 (below every
// threshold).  A slice wholly inside the segment (every one but the last; the
// test is wave-uniform) takes no bounds test at all.
template <int SV>
__device__ __forceinline__ void slice_keys(const float4 (&cur)[SV], int base, int hi, int largest, int ikind,
                                           uint32_t (&key)[4 * SV]) {
    if (ikind) {  // 32-bit integers (a wave-uniform branch around the float conversion)
        const int lim = hi - base - 4 * (int)__lane_id();
#pragma unroll
        for (int j = 0; j < SV; ++j) {
            key[4 * j + 0] = (256 * j + 0 < lim) ? elem_key(cur[j].x, largest, ikind) : 0u;
            key[4 * j + 1] = (256 * j + 1 < lim) ? elem_key(cur[j].y, largest, ikind) : 0u;
            key[4 * j + 2] = (256 * j + 2 < lim) ? elem_key(cur[j].z, largest, ikind) : 0u;
            key[4 * j + 3] = (256 * j + 3 < lim) ? elem_key(cur[j].w, largest, ikind) : 0u;
        }
        return;
    }
    if (hi - base >= 256 * SV) {
        const uint32_t lm = largest ? 0u : 0xffffffffu;
#pragma unroll
        for (int j = 0; j < SV; ++j) {
            key[4 * j + 0] = f2key_sel(cur[j].x, lm);
            key[4 * j + 1] = f2key_sel(cur[j].y, lm);
            key[4 * j + 2] = f2key_sel(cur[j].z, lm);
            key[4 * j + 3] = f2key_sel(cur[j].w, lm);
        }
        return;
    }
    const int lim = hi - base - 4 * (int)__lane_id();  // element e = base + 4*lane + 256*j + q is valid iff 256*j + q < lim
#pragma unroll
    for (int j = 0; j < SV; ++j) {
        key[4 * j + 0] = (256 * j + 0 < lim) ? f2key(cur[j].x, largest) : 0u;
        key[4 * j + 1] = (256 * j + 1 < lim) ? f2key(cur[j].y, largest) : 0u;
        key[4 * j + 2] = (256 * j + 2 < lim) ? f2key(cur[j].z, largest) : 0u;
        key[4 * j + 3] = (256 * j + 3 < lim) ? f2key(cur[j].w, largest) : 0u;
    }
}

// Keys of one slice of EB-byte elements: slice_keys for 4-byte rows; for 1-
// and 2-byte integer rows each lane's SV = EB vectors hold 16 elements (lane
// l, vector j: elements (j*64 + l)*(16/EB) .. +16/EB-1 of the slice, byte order
// inside a vector = element order), keyed as the lane-group kernel does.
template <int EB, int SV>
__device__ __forceinline__ void slice_keys_eb(const float4 (&cur)[SV], int base, int hi, int largest, int ikind,
                                              uint32_t (&key)[16 * SV / EB]) {
    if constexpr (EB == 4) {
        slice_keys(cur, base, hi, largest, ikind, key);
    } else if constexpr (EB == 8) {
        // the high 32 bits of each element's 64-bit key (two elements per vector)
        const int lim = hi - base;
        const int lane = __lane_id();
#pragma unroll
        for (int j = 0; j < SV; ++j) {
            const unsigned long long b0 =
                ((unsigned long long)__float_as_uint(cur[j].y) << 32) | __float_as_uint(cur[j].x);
            const unsigned long long b1 =
                ((unsigned long long)__float_as_uint(cur[j].w) << 32) | __float_as_uint(cur[j].z);
            const int e = (j * 64 + lane) * 2;
            key[2 * j] = e < lim ? (uint32_t)(key64_of(b0, largest, ikind) >> 32) : 0u;
            key[2 * j + 1] = e + 1 < lim ? (uint32_t)(key64_of(b1, largest, ikind) >> 32) : 0u;
        }
    } else {
        constexpr int EPV = 16 / EB, EPW = 4 / EB;
        constexpr uint32_t em = EB == 1 ? 0xffu : 0xffffu;
        const uint32_t sm = ikind == 1 ? (em >> 1) + 1u : 0u;
        const uint32_t lm = largest ? 0u : 0xffffffffu;
        const int lim = hi - base;
        const int lane = __lane_id();
#pragma unroll
        for (int j = 0; j < SV; ++j) {
            const uint32_t wv[4] = {__float_as_uint(cur[j].x), __float_as_uint(cur[j].y), __float_as_uint(cur[j].z),
                                    __float_as_uint(cur[j].w)};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
#pragma unroll
                for (int t = 0; t < EPW; ++t) {
                    const int q = j * EPV + c * EPW + t;
                    const uint32_t kv = (((wv[c] >> (8 * EB * t)) & em) ^ sm ^ lm) & em;
                    key[q] = ((j * 64 + lane) * EPV + c * EPW + t < lim) ? kv : 0u;
                }
            }
        }
    }
}

template <bool VEC, int SV, int OCC, int PD, int NW, int KWB = kWB, int EB = 4>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(OCC, 8))) void k_topk_wave(TopkArgs a) {
    static_assert(EB == 4 || (EB == 8 && SV == 4 && VEC) || (SV == EB && VEC),
                  "1- / 2-byte rows: SV = EB float4 per lane; 8-byte rows: SV = 4; both 16-byte aligned");
    constexpr int kSlF = 256 * SV;         // 4-byte words per wave slice
    constexpr int kSl = kSlF * 4 / EB;     // elements per wave slice (1024)
    constexpr int kNK = 16 * SV / EB;      // keys per lane per slice (16)
    constexpr int kEPV = 16 / EB;          // elements per 16-byte vector
    constexpr int kW = NW;         // waves of this workgroup
    constexpr int kT = NW * 64;
    constexpr int kB = NW * KWB;   // gathered-list capacity
    __shared__ WaveShared<NW, KWB> sh;
    BlockScratch& bs = sh.bs;
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);  // wave-uniform: scalar loop control
    const long long row = blockIdx.x / a.nseg;
    const int seg = blockIdx.x % a.nseg;
    const char* pr = reinterpret_cast<const char*>(a.in) + row * a.row_stride * EB;
    const float* p = reinterpret_cast<const float*>(pr);
    const int k = a.k;
    const int largest = a.largest;
    const int lo = seg * a.seg_len;
    const int hi = min(a.cols, lo + a.seg_len);
    const int nsl = (hi - lo + kSl - 1) / kSl;
    const int r = (k + kW - 1) / kW;
    const int compact_at = min(KWB == kWB ? kWaveCompact : KWB - 64, max(2 * k, 64));  // per-wave list length that triggers compaction
    unsigned long long* list = sh.wl[w];
    uint32_t* hist = sh.hist[w];

    if (tid == 0) {
        bs.tshared = 1;
        bs.count = 0;
        bs.over = a.force_fallback;
        bs.next_slice = 2 * kW;  // slices w and w + kW (prefetched) are static
    }

    // Wave slices are w, w+8, w+16, ...  PD = slices whose loads are in flight
    // while the current one is filtered (0: load, wait, filter; 1: the next
    // slice's load is issued as soon as the current one has become keys; 2: two
    // register buffers alternate, so two slices are in flight).
    float4 bufA[SV];
    float4 bufB[PD == 2 ? SV : 1];
    uint32_t key[kNK];
    // (1- / 2-byte rows: the range is rounded up to whole dwords; elements past
    // the segment's end inside the last dword are masked in the keys)
    const __amdgpu_buffer_rsrc_t rs =
        EB == 4 ? segment_rsrc(p + lo, hi - lo)
                : __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(pr + (long long)lo * EB), (short)0,
                                                    ((hi - lo) * EB + 3) & ~3, kBufWord3);
    load_slice<VEC, SV>(bufA, rs, w * kSlF);
    if constexpr (PD == 2) load_slice<VEC, SV>(bufB, rs, (w + kW) * kSlF);
    slice_keys_eb<EB>(bufA, lo + w * kSl, hi, largest, a.ikind, key);
    if constexpr (PD == 1) load_slice<VEC, SV>(bufA, rs, (w + kW) * kSlF);
    if constexpr (PD == 2) load_slice<VEC, SV>(bufA, rs, (w + 2 * kW) * kSlF);
    // the first slice of every wave gives the workgroup bound T0
    const uint32_t rth = wave_rth_of_lane_max(key, kNK, r);
    if (lane == 0) bs.wave_val[w] = rth;
    __syncthreads();
    uint32_t T = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < kW; ++i) T = min(T, bs.wave_val[i]);
    T = max(T, 1u);
    bool over = bs.over != 0;
    int cnt = 0;  // this wave's list length (wave-uniform)

    // Appends the slice's keys >= T to the wave list; false when the list
    // cannot take them (the workgroup then takes the exact path).
    auto filter = [&](int base) -> bool {
        T = max(T, __atomic_load_n(&bs.tshared, __ATOMIC_RELAXED));
        int total = 0;
#pragma unroll
        for (int q = 0; q < kNK; ++q) total += __popcll(__ballot(key[q] >= T));
        while (total > 0 && cnt + total > KWB) {  // no room: drop stale entries / raise T first
            const int before = cnt;
            const uint32_t tn = wave_compact(list, hist, cnt, k, T);
            if (tn > T) {
                if (lane == 0) atomicMax(&bs.tshared, tn);
                T = tn;
                total = 0;
#pragma unroll
                for (int q = 0; q < kNK; ++q) total += __popcll(__ballot(key[q] >= T));
            } else if (cnt == before) {
                return false;  // nothing could be dropped
            }
        }
        if (total) {
            const unsigned long long lt = lanemask_lt();
            int pos = cnt;
#pragma unroll
            for (int q = 0; q < kNK; ++q) {
                const bool pass = key[q] >= T;
                const unsigned long long b = __ballot(pass);
                if (b == 0ull) continue;  // uniform: most slots hold no candidate
                if (pass)
                    list[pos + __popcll(b & lt)] =
                        comp_key(key[q], (uint32_t)(base + ((q / kEPV) * 64 + lane) * kEPV + (q % kEPV)));
                pos += __popcll(b);
            }
            cnt = pos;
        }
        if (cnt > compact_at) {
            const uint32_t tn = wave_compact(list, hist, cnt, k, T);
            if (tn > T) {
                if (lane == 0) atomicMax(&bs.tshared, tn);
                T = tn;
            }
        }
        return __atomic_load_n(&bs.over, __ATOMIC_RELAXED) == 0;
    };

    // streaming loop: no workgroup barriers
    if (!over) {
        int c = w;
        if constexpr (PD == 2) {
            for (;;) {
                if (!filter(lo + c * kSl)) { over = true; break; }
                c += kW;
                if (c >= nsl) break;
                slice_keys_eb<EB>(bufB, lo + c * kSl, hi, largest, a.ikind, key);
                load_slice<VEC, SV>(bufB, rs, (c + 2 * kW) * kSlF);
                if (!filter(lo + c * kSl)) { over = true; break; }
                c += kW;
                if (c >= nsl) break;
                slice_keys_eb<EB>(bufA, lo + c * kSl, hi, largest, a.ikind, key);
                load_slice<VEC, SV>(bufA, rs, (c + 2 * kW) * kSlF);
            }
        } else if (PD == 1 && NW == 16 && a.dyn) {
            // Slices past the first two of each wave go to whichever wave asks
            // next (an LDS counter), so the waves of a workgroup finish their
            // streaming together instead of waiting at the gather for the ones
            // that drew an extra slice or more candidates.  Only the 16-wave
            // kernel (one workgroup per CU, 128 VGPRs): in the 8-wave kernels
            // the extra code path made them spill.
            auto grab = [&]() -> int {
                int v = 0;
                if (lane == 0) v = atomicAdd(&bs.next_slice, 1);
                return __builtin_amdgcn_readfirstlane(v);
            };
            int nx = w + kW;  // already loading into bufA
            while (c < nsl) {
                if (c != w) {
                    slice_keys_eb<EB>(bufA, lo + c * kSl, hi, largest, a.ikind, key);
                    nx = grab();
                    load_slice<VEC, SV>(bufA, rs, nx * kSlF);  // past the segment: reads 0, no traffic
                }
                if (!filter(lo + c * kSl)) { over = true; break; }
                c = nx;
            }
        } else {
            for (; c < nsl; c += kW) {
                const int base = lo + c * kSl;
                if (c != w) {
                    if constexpr (PD == 0) load_slice<VEC, SV>(bufA, rs, c * kSlF);
                    slice_keys_eb<EB>(bufA, base, hi, largest, a.ikind, key);
                    if constexpr (PD == 1) {
                        load_slice<VEC, SV>(bufA, rs, (c + kW) * kSlF);
                    }
                }
                if (!filter(base)) { over = true; break; }
            }
        }
    }
    // Final per-wave bounds: t_w has >= ceil(k / NW) entries of wave w's list
    // at or above it, and the lists hold distinct elements, so the minimum
    // over the waves has >= k elements at or above it: a bound for the whole
    // workgroup, far tighter than one wave's k-th.  Measured on MI355X:
    // [1024, 32768] k = 64 29.6 -> 28.6 us, k = 8 29.9 -> 27.9 us.
    if (!over) {
        T = max(T, __atomic_load_n(&bs.tshared, __ATOMIC_RELAXED));
        const uint32_t tw = wave_kth_bound(list, hist, cnt, (k + kW - 1) / kW, T);
        if (lane == 0) bs.wave_t[w] = tw;
    } else if (lane == 0) {
        bs.wave_t[w] = 0;
    }
    if (over && lane == 0) __atomic_store_n(&bs.over, 1, __ATOMIC_RELAXED);
    __syncthreads();

    // gather: each wave keeps the entries at or above the final shared threshold
    const bool any_over = bs.over != 0;
    uint32_t Tf = max(T, bs.tshared);
    if (!any_over) {
        uint32_t tm = 0xffffffffu;
#pragma unroll
        for (int i = 0; i < kW; ++i) tm = min(tm, bs.wave_t[i]);
        Tf = max(Tf, tm);
    }
    __syncthreads();  // the histogram area is reused as the gathered list below
    if (!any_over) {
        for (int i0 = 0; i0 < cnt; i0 += 64) {
            const int i = i0 + lane;
            const unsigned long long c = (i < cnt) ? list[i] : 0ull;
            const bool keep = (i < cnt) && (uint32_t)(c >> 32) >= Tf;
            const unsigned long long b = __ballot(keep);
            int gbase = 0;
            if (lane == 0 && b) gbase = atomicAdd(&bs.count, __popcll(b));
            gbase = __builtin_amdgcn_readlane(gbase, 0);
            if (keep) sh.un[gbase + __popcll(b & lanemask_lt())] = c;  // sum of lists <= kW * KWB == kB
        }
    }
    __syncthreads();
    unsigned long long* cand = sh.un;
    unsigned long long* other = &sh.wl[0][0];
    int m = bs.count;
    // fewer than k gathered: the segment has keys of 0 (integers only; the
    // filter keeps keys >= 1), which the exact select takes
    if (any_over || m < k) {
        if constexpr (EB == 8) {
            // no 64-bit exact path here: the row is finished by k_topk_radix
            if (threadIdx.x == 0) a.flags[row] = 1;
            return;
        } else {
            exact_select<kT, EB>(bs, cand, pr, lo, hi, k, largest, a.ikind);
            m = k;
        }
    } else if (m > (k >= 128 ? k + max(k / 4, 32) : max(2 * k, 256))) {
        // (large k: cut close to k before the O(m^2) ranking; MI355X, us:
        // [256, 151936] k = 256 40.9 -> 37.4, [1024, 32768] k = 200 53.9 -> 47.9,
        // [4096, 8192] k = 128 55.4 -> 54.6; at k = 64 the cut cost more than it
        // saved, C3 29.5 -> 30.7)
        block_compact<kT>(bs, cand, other, m, k, Tf);
        m = bs.count2;
        unsigned long long* t = cand;
        cand = other;
        other = t;
    }
    int* rank = reinterpret_cast<int*>(other);
    unsigned long long* sel = other + kB / 2;
    if constexpr (EB == 8) {
        // The candidates hold every element whose key's high half reaches Tf, a
        // superset of the top k; ties of the high half are ordered by the low
        // half, read back for each candidate (rank and low halves fit below sel
        // while m <= kB / 2, else k_topk_radix finishes the row).
        if (m > kB / 2) {
            if (threadIdx.x == 0) a.flags[row] = 1;
            return;
        }
        uint32_t* lo32 = reinterpret_cast<uint32_t*>(rank + m);
        const unsigned long long* p8 = reinterpret_cast<const unsigned long long*>(pr);
        for (int i = threadIdx.x; i < m; i += kT)
            lo32[i] = (uint32_t)key64_of(p8[comp_index(cand[i])], largest, a.ikind);
        rank_select<kT, true>(cand, rank, sel, m, k, lo32);
        if (threadIdx.x == 0) a.flags[row] = 0;
    } else {
        rank_select<kT>(cand, rank, sel, m, k);
    }
    write_segment<EB>(a, row, seg, p, sel, k);
}

// ---------------------------------------------------------------------------
// Workgroup-level segment kernel (large k, short rows).
// ---------------------------------------------------------------------------
struct BlockShared {
    unsigned long long list[2][kB];
    BlockScratch bs;
};

// Loads one chunk (kV float4 per thread).  The bounds test is uniform across the
// workgroup, so a full chunk is kV unconditional 128-bit loads; the tail chunk
// uses clamped (always valid) scalar addresses and a select.
template <bool VEC>
__device__ __forceinline__ void load_chunk(float4 (&dst)[kV], const float* p, int cbase, int n) {
    const int tid = threadIdx.x;
    if (VEC && cbase + kCH <= n) {
#pragma unroll
        for (int j = 0; j < kV; ++j) dst[j] = *reinterpret_cast<const float4*>(p + cbase + 4 * (j * kT + tid));
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

template <bool VEC>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(6, 8))) void k_topk_block(TopkArgs a) {
    __shared__ BlockShared sh;
    BlockScratch& bs = sh.bs;
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
    const int nchunks = (hi - lo + kCH - 1) / kCH;
    const int r = (k + kW - 1) / kW;
    const int compact_at = max(2 * k, 256);

    if (tid == 0) { bs.count = 0; bs.over = 0; }
    __syncthreads();

    int cur_list = 0;
    bool over = a.force_fallback != 0 || r > 64;
    uint32_t T = 1;  // admit every valid key until the bound is known
    for (int c = 0; c < nchunks && !over; ++c) {
        const int cbase = lo + c * kCH;
        float4 cur[kV];
        load_chunk<VEC>(cur, p, cbase, hi);
        uint32_t key[4 * kV];
        if (a.ikind) {  // 32-bit integers
#pragma unroll
            for (int j = 0; j < kV; ++j) {
                const int e = cbase + 4 * (j * kT + tid);
                key[4 * j + 0] = (e + 0 < hi) ? elem_key(cur[j].x, largest, a.ikind) : 0u;
                key[4 * j + 1] = (e + 1 < hi) ? elem_key(cur[j].y, largest, a.ikind) : 0u;
                key[4 * j + 2] = (e + 2 < hi) ? elem_key(cur[j].z, largest, a.ikind) : 0u;
                key[4 * j + 3] = (e + 3 < hi) ? elem_key(cur[j].w, largest, a.ikind) : 0u;
            }
        } else if (cbase + kCH <= hi) {  // whole chunk inside the segment (uniform): no bounds tests
            const uint32_t lm = largest ? 0u : 0xffffffffu;
#pragma unroll
            for (int j = 0; j < kV; ++j) {
                key[4 * j + 0] = f2key_sel(cur[j].x, lm);
                key[4 * j + 1] = f2key_sel(cur[j].y, lm);
                key[4 * j + 2] = f2key_sel(cur[j].z, lm);
                key[4 * j + 3] = f2key_sel(cur[j].w, lm);
            }
        } else {
#pragma unroll
            for (int j = 0; j < kV; ++j) {
                const int e = cbase + 4 * (j * kT + tid);
                key[4 * j + 0] = (e + 0 < hi) ? f2key(cur[j].x, largest) : 0u;
                key[4 * j + 1] = (e + 1 < hi) ? f2key(cur[j].y, largest) : 0u;
                key[4 * j + 2] = (e + 2 < hi) ? f2key(cur[j].z, largest) : 0u;
                key[4 * j + 3] = (e + 3 < hi) ? f2key(cur[j].w, largest) : 0u;
            }
        }
        if (c == 0) {
            const uint32_t rth = wave_rth_of_lane_max(key, 4 * kV, r);
            if (lane == 0) bs.wave_val[w] = rth;
            __syncthreads();
            uint32_t tb = 0xffffffffu;
#pragma unroll
            for (int i = 0; i < kW; ++i) tb = min(tb, bs.wave_val[i]);
            T = max(T, tb);
        }
        // filter: per-slot ballots give each passing element its wave offset
        unsigned long long* cand = sh.list[cur_list];
        int total = 0;
#pragma unroll
        for (int q = 0; q < 4 * kV; ++q) total += __popcll(__ballot(key[q] >= T));
        if (total) {
            int base = 0;
            if (lane == 0) base = atomicAdd(&bs.count, total);
            base = __builtin_amdgcn_readlane(base, 0);
            const unsigned long long lt = lanemask_lt();
#pragma unroll
            for (int q = 0; q < 4 * kV; ++q) {
                const bool pass = key[q] >= T;
                const unsigned long long b = __ballot(pass);
                if (pass) {
                    const int pos = base + __popcll(b & lt);
                    const int e = cbase + 4 * ((q >> 2) * kT + tid) + (q & 3);
                    if (pos < kB) cand[pos] = comp_key(key[q], (uint32_t)e);
                    else bs.over = 1;
                }
                base += __popcll(b);
            }
        }
        __syncthreads();
        // read the shared verdicts, then fence them off from the next chunk's atomics
        over = bs.over != 0;
        const int m = bs.count;
        __syncthreads();
        if (over) break;
        if (m > compact_at) {
            T = block_compact<kT>(bs, sh.list[cur_list], sh.list[cur_list ^ 1], m, k, T);
            cur_list ^= 1;
            if (tid == 0) bs.count = bs.count2;
            __syncthreads();
        }
    }
    __syncthreads();

    int m = bs.count;
    if (over || m < k) {  // m < k: keys of 0 in an integer segment (see k_topk_wave)
        exact_select<kT>(bs, sh.list[0], p, lo, hi, k, largest, a.ikind);
        m = k;
        cur_list = 0;
    }
    const unsigned long long* cand = sh.list[cur_list];
    int* rank = reinterpret_cast<int*>(sh.list[cur_list ^ 1]);
    unsigned long long* sel = sh.list[cur_list ^ 1] + kB / 2;
    rank_select<kT>(cand, rank, sel, m, k);
    write_segment(a, row, seg, p, sel, k);
}

// ---------------------------------------------------------------------------
// Short rows (cols <= 4096, k <= 64): L lanes per row, G = 64 / L rows per
// wave, 4 waves per workgroup and no workgroup barrier.  Each lane holds E4
// float4 of its row in registers (lane sl, vector j: elements
// 4*(j*L + sl) .. +3, so the L lanes of a row read 16*L contiguous bytes per
// vector), so the row is read from HBM exactly once and selected without
// touching memory again:
//   * bound: a bitonic sort of the L per-lane maxima inside the row's lane
//     group gives their k-th largest T0 (k <= L), which has >= k elements at
//     or above it;
//   * candidates: the elements >= T0 (usually a few times k) go to a
//     row-private LDS list at positions from a group prefix scan of the lanes'
//     counts;
//   * ranking: rank = number of candidates with a larger composite
//     (composites are distinct), ranks < k are written in order;
//   * exact path, when more than 8L elements tie at or above T0 (all-equal
//     rows, long runs): the exact k-th key T* by a 32-step bit search over the
//     keys in registers, every key > T* plus the lowest-index keys == T*
//     (index order: vector j, then lane, then component), then the ranking.
// ---------------------------------------------------------------------------
constexpr int kShortT = 256;  // threads per short-row workgroup (4 waves)
constexpr int kShortMaxCols = 4096;
constexpr int kShortMaxK = 64;
// Many rows of <= 2048 elements also take k of 65..128 in the lane-group
// kernel (64 lanes; the bound is the k-th largest of the lanes' two largest
// keys).  MI355X, us, register radix select -> lane groups: [16384, 1024]
// k = 100 94.3 -> 55.8; [65536, 256] k = 100 324 -> 89; [4096, 2048] k = 100
// 37.5 -> 22.6; [16384, 2048] k = 80 114 -> 38.7; but [8192, 3000] k = 128
// 83 -> 125 and [512, 2000] k = 100 13.5 -> 15.7, so rows of <= 2048 and >= 8
// rows per CU.  topk_short = 1 (debug knob) takes every row below 4096.
__host__ inline bool short_exact(long long rows, long long cols, long long k);

// Float max / min of three without the canonicalising moves the compiler adds
// to fmaxf / fminf in IEEE mode: v_max3_f32 / v_min3_f32 return the largest /
// smallest non-NaN operand (NaN only when all three are NaN).
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float min3_f32(float a, float b, float c) {
    float r;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

template <int L>
__device__ __forceinline__ int group_sum(int v) {
#pragma unroll
    for (int o = 1; o < L; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Inclusive prefix sum over the lanes of an L-lane group (L = 16, 32 or 64;
// sl = lane in group): DPP row shifts by 1, 2, 4, 8 inside each 16-lane row
// (lanes whose source is outside the row add the 0 passed as `old`), then
// row_bcast:15 carries row 0's total into row 1 and row 2's into row 3, and
// row_bcast:31 the total of rows 0-1 into rows 2-3.  No LDS round trips.
template <int L>
__device__ __forceinline__ int group_scan(int v, int sl) {
    static_assert(L == 16 || L == 32 || L == 64, "lane groups of 16, 32 or 64");
    (void)sl;
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    if constexpr (L >= 32) v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    if constexpr (L == 64) v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

// Largest value over the lanes of an L-lane group (every lane of the group
// active; groups are whole 16-lane rows, so the exchanges stay inside them).
template <int L>
__device__ __forceinline__ uint32_t group_max(uint32_t v) {
    v = max(v, xor_lane<1>(v));
    v = max(v, xor_lane<2>(v));
    v = max(v, xor_lane<4>(v));
    v = max(v, xor_lane<8>(v));
    if constexpr (L >= 32) v = max(v, xor_lane<16>(v));
    if constexpr (L == 64) v = max(v, xor_lane<32>(v));
    return v;
}

template <int M, int P>
__device__ __forceinline__ void sort_lane_stage(unsigned long long (&x)[P], bool keep_max) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t lo = xor_lane<M>((uint32_t)x[p]);
        const uint32_t hi = xor_lane<M>((uint32_t)(x[p] >> 32));
        const unsigned long long y = ((unsigned long long)hi << 32) | lo;
        x[p] = ((x[p] > y) == keep_max) ? x[p] : y;
    }
}

// Descending bitonic sort of 64 * P composites held P per lane across one
// wave (lane l holds positions l*P .. l*P+P-1): lane permutes for distances of
// at least P, compare-exchanges in registers below.
template <int P>
__device__ __forceinline__ void wave_sort_desc(unsigned long long (&x)[P]) {
    const int lane = __lane_id();
#pragma unroll
    for (int s = 2; s <= 64 * P; s <<= 1) {
#pragma unroll
        for (int d = s >> 1; d >= P; d >>= 1) {
            const int m = d / P;  // partner lane lane ^ m
            const bool keep_max = ((lane & m) == 0) == (((lane * P) & s) == 0);
            switch (m) {
                case 1: sort_lane_stage<1, P>(x, keep_max); break;
                case 2: sort_lane_stage<2, P>(x, keep_max); break;
                case 4: sort_lane_stage<4, P>(x, keep_max); break;
                case 8: sort_lane_stage<8, P>(x, keep_max); break;
                case 16: sort_lane_stage<16, P>(x, keep_max); break;
                default: sort_lane_stage<32, P>(x, keep_max); break;
            }
        }
#pragma unroll
        for (int dd = P / 2; dd >= 1; dd >>= 1) {
            if (dd < s) {
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    if ((q & dd) == 0) {
                        const bool desc = ((lane * P + q) & s) == 0;
                        const unsigned long long u = x[q], v = x[q + dd];
                        const bool sw = (u > v) != desc;
                        x[q] = sw ? v : u;
                        x[q + dd] = sw ? u : v;
                    }
                }
            }
        }
    }
}

// Bitonic sort (ascending) of the values m held by the L lanes of each group:
// lane sl of the group returns the sl-th smallest.
template <int L>
__device__ __forceinline__ uint32_t group_sort_asc(uint32_t m, int sl) {
    uint32_t v = m;
#pragma unroll
    for (int size = 2; size <= L; size <<= 1) {
#pragma unroll
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            uint32_t o;
            switch (stride) {
                case 1: o = xor_lane<1>(v); break;
                case 2: o = xor_lane<2>(v); break;
                case 4: o = xor_lane<4>(v); break;
                case 8: o = xor_lane<8>(v); break;
                case 16: o = xor_lane<16>(v); break;
                default: o = xor_lane<32>(v); break;
            }
            const bool asc = (sl & size) == 0;
            const bool lower = (sl & stride) == 0;
            v = (lower == asc) ? min(v, o) : max(v, o);
        }
    }
    return v;
}

// The r-th largest (r >= 1) of the wave's 64 * NV values v[] (the multiset
// over every lane), all below 2^BITS: a BITS-step bit search, one compare per
// value and a ballot count per step (the prefix stays in scalar registers).
template <int NV, int BITS = 32>
__device__ __forceinline__ uint32_t wave_rth_largest(const uint32_t (&v)[NV], int r) {
    uint32_t pre = 0;
#pragma unroll 4
    for (int b = BITS - 1; b >= 0; --b) {
        const uint32_t cand = pre | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) cnt += __popcll(__ballot(v[i] >= cand));
        if (cnt >= r) pre = cand;
    }
    return pre;
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// hist_threshold for one L-lane group: bins [T, T + 256 << shift), lane sl of
// the group owns bins sl*NB .. sl*NB + NB-1.  Returns the lower edge of the bin
// where the count from the top first reaches k (T when it never does).
template <int L>
__device__ __forceinline__ uint32_t group_hist_threshold(const uint32_t* hist, int k, uint32_t T, int shift,
                                                         int sl, int grp) {
    constexpr int NB = 256 / L;
    uint32_t h[NB];
    int own = 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        h[b] = hist[sl * NB + b];
        own += (int)h[b];
    }
    int suf = own;  // inclusive suffix sum over the group's lanes >= sl
#pragma unroll
    for (int o = 1; o < L; o <<= 1) {
        const int t = __shfl_down(suf, o, 64);
        if (sl + o < L) suf += t;
    }
    const unsigned long long gmask = (L == 64) ? ~0ull : ((1ull << L) - 1ull);
    const unsigned long long ok = (__ballot(suf >= k) >> (grp * L)) & gmask;
    if (ok == 0ull) return T;
    const int hl = 63 - __clzll((long long)ok);  // highest lane of the group whose suffix reaches k
    uint32_t tn = 0;
    if (sl == hl) {
        int cum = suf - own;
        int b = NB - 1;
        for (; b > 0; --b) {
            if (cum + (int)h[b] >= k) break;
            cum += (int)h[b];
        }
        tn = T + ((uint32_t)(sl * NB + b) << shift);
    }
    return __shfl(tn, grp * L + hl, 64);
}

// Output r of a row: the value (exact, from the key or the input, in the
// input's dtype of EB bytes) and index.
template <int EB>
__device__ __forceinline__ void write_ranked(const TopkArgs& a, long long row, int k, const float* p, int largest,
                                             int r, unsigned long long c) {
    const uint32_t idx = comp_index(c);
    const uint32_t key = (uint32_t)(c >> 32);
    if constexpr (EB == 1) {
        reinterpret_cast<uint8_t*>(a.out_v)[row * k + r] = (uint8_t)int_key_bits(key, a.ikind, largest, 0xffu);
    } else if constexpr (EB == 2) {
        reinterpret_cast<uint16_t*>(a.out_v)[row * k + r] = (uint16_t)int_key_bits(key, a.ikind, largest, 0xffffu);
    } else {
        a.out_v[row * k + r] = a.ikind ? __uint_as_float(int_key_bits(key, a.ikind, largest, 0xffffffffu))
                                       : selected_value(p, key, idx, largest);
    }
    a.out_i[row * k + r] = (long long)idx;
}

// Element index of key q of lane sl in the lane-group kernel: keys run over the
// lane's 16-byte vectors j, their dwords c and, for elements of EB < 4 bytes,
// the 4 / EB elements of a dword (element order inside a lane's vector).
template <int L, int EB>
__device__ __forceinline__ int short_elem(int q, int sl) {
    constexpr int EPW = 4 / EB;
    const int w = q / EPW;
    return (4 * ((w >> 2) * L + sl) + (w & 3)) * EPW + q % EPW;
}

template <int L, int E4, bool VEC, bool LG, int EB = 4>
__global__ __launch_bounds__(kShortT) void k_topk_short(TopkArgs a) {
    static_assert(EB == 4 || VEC, "1- and 2-byte rows: 16-byte aligned rows only");
    constexpr int G = 64 / L;
    constexpr int EPW = 4 / EB;     // elements per dword
    constexpr int E = 4 * E4 * EPW;  // keys per lane
    constexpr int C = 8 * L;  // candidate capacity of one row
    constexpr int RPB = (kShortT / 64) * G;
    __shared__ unsigned long long cl[RPB][C];  // C * 8 >= 1 KiB: also the row's histogram (see below)
    const int lane = __lane_id();
    const int grp = lane / L;
    const int sl = lane % L;
    const int slot = (threadIdx.x / 64) * G + grp;
    const long long row = (long long)blockIdx.x * RPB + slot;
    const bool live = row < a.rows;
    const int cols = a.cols;
    const int k = a.k;
    constexpr int largest = LG ? 1 : 0;
    const float* p = reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.in) +
                                                    (live ? row * a.row_stride * EB : 0));
    // One buffer resource per wave (a per-lane resource would make every load
    // a loop over the wave's distinct rows): it spans the wave's live rows, the
    // lane group's row starts at grp * row_stride, and elements past a row's
    // end but inside the span are masked below (keys 0).  The host keeps
    // (G - 1) * row_stride + cols below 2^29 floats.
    const long long row0 = (long long)blockIdx.x * RPB + __builtin_amdgcn_readfirstlane(threadIdx.x / 64) * G;
    const long long nlive = min((long long)G, max(0LL, a.rows - row0));
    // (1- and 2-byte rows: the range is rounded up to whole dwords, so the
    // dword holding a row's last elements is read whole; the rest of it is
    // masked below, and rows start 16-byte aligned, so it never crosses into
    // another page.)
    const char* wbase = reinterpret_cast<const char*>(a.in) + (nlive > 0 ? row0 * a.row_stride * EB : 0);
    const int nbytes = nlive > 0 ? (int)(((nlive - 1) * a.row_stride + cols) * EB + 3) & ~3 : 0;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wbase), (short)0, nbytes, kBufWord3);
    const int rbase = grp * (int)a.row_stride * EB;

    float4 x[E4];
#pragma unroll
    for (int j = 0; j < E4; ++j) {
        const int off = rbase + 16 * (j * L + sl);
        if constexpr (VEC) {
            const f32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kNT);
            x[j] = make_float4(v.x, v.y, v.z, v.w);
        } else {
            x[j] = make_float4(buf_ld_f32(rs, off), buf_ld_f32(rs, off + 4), buf_ld_f32(rs, off + 8),
                               buf_ld_f32(rs, off + 12));
        }
    }
    uint32_t key[E];
    constexpr uint32_t lm = LG ? 0u : 0xffffffffu;
    // Full float32 rows filter on the floats themselves: the bound T (a key)
    // becomes the float Tf it encodes, an element is a candidate when
    // !(x < Tf) (largest: NaN, whose key is above every other, passes) or
    // x <= Tf (smallest: NaN, below every other, fails), and keys are made
    // only for the listed candidates.  The lane maxima come from float max3,
    // which skips NaN: that can only lower the bound, which stays valid.
    const bool ffast = EB == 4 && a.ikind == 0 && cols == 4 * E4 * L;
    auto float_keys = [&]() {
#pragma unroll
        for (int j = 0; j < E4; ++j) {
            key[4 * j + 0] = live ? f2key_sel(x[j].x, lm) : 0u;
            key[4 * j + 1] = live ? f2key_sel(x[j].y, lm) : 0u;
            key[4 * j + 2] = live ? f2key_sel(x[j].z, lm) : 0u;
            key[4 * j + 3] = live ? f2key_sel(x[j].w, lm) : 0u;
        }
    };
    uint32_t mx = 0;  // the lane's largest key
    if (ffast) {
        float m = LG ? -__builtin_inff() : __builtin_inff();
#pragma unroll
        for (int j = 0; j < E4; ++j) {
            if constexpr (LG) {
                m = max3_f32(m, x[j].x, x[j].y);
                m = max3_f32(m, x[j].z, x[j].w);
            } else {
                m = min3_f32(m, x[j].x, x[j].y);
                m = min3_f32(m, x[j].z, x[j].w);
            }
        }
        mx = live ? f2key_sel(m, lm) : 0u;
    } else {
    if constexpr (EB < 4) {  // 1- and 2-byte integers (ikind 1 signed, 2 unsigned or bool)
        constexpr uint32_t em = EB == 1 ? 0xffu : 0xffffu;
        const uint32_t sm = a.ikind == 1 ? (em >> 1) + 1u : 0u;
#pragma unroll
        for (int j = 0; j < E4; ++j) {
            const uint32_t wv[4] = {__float_as_uint(x[j].x), __float_as_uint(x[j].y), __float_as_uint(x[j].z),
                                    __float_as_uint(x[j].w)};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
#pragma unroll
                for (int s = 0; s < EPW; ++s) {
                    const int q = (4 * j + c) * EPW + s;
                    const uint32_t kv = (((wv[c] >> (8 * EB * s)) & em) ^ sm ^ lm) & em;
                    key[q] = short_elem<L, EB>(q, sl) < cols ? kv : 0u;
                }
            }
        }
    } else if (a.ikind != 0) {  // 32-bit integers
        const uint32_t sm = a.ikind == 1 ? 0x80000000u : 0u;
#pragma unroll
        for (int j = 0; j < E4; ++j) {
            const int e = 4 * (j * L + sl);
            key[4 * j + 0] = (e + 0 < cols) ? i2key_sel(x[j].x, sm, lm) : 0u;
            key[4 * j + 1] = (e + 1 < cols) ? i2key_sel(x[j].y, sm, lm) : 0u;
            key[4 * j + 2] = (e + 2 < cols) ? i2key_sel(x[j].z, sm, lm) : 0u;
            key[4 * j + 3] = (e + 3 < cols) ? i2key_sel(x[j].w, sm, lm) : 0u;
        }
    } else if (cols == 4 * E4 * L) {  // every element of every lane is in the row
#pragma unroll
        for (int j = 0; j < E4; ++j) {
            key[4 * j + 0] = f2key_sel(x[j].x, lm);
            key[4 * j + 1] = f2key_sel(x[j].y, lm);
            key[4 * j + 2] = f2key_sel(x[j].z, lm);
            key[4 * j + 3] = f2key_sel(x[j].w, lm);
        }
    } else {
#pragma unroll
        for (int j = 0; j < E4; ++j) {
            const int e = 4 * (j * L + sl);
            key[4 * j + 0] = (e + 0 < cols) ? f2key_sel(x[j].x, lm) : 0u;
            key[4 * j + 1] = (e + 1 < cols) ? f2key_sel(x[j].y, lm) : 0u;
            key[4 * j + 2] = (e + 2 < cols) ? f2key_sel(x[j].z, lm) : 0u;
            key[4 * j + 3] = (e + 3 < cols) ? f2key_sel(x[j].w, lm) : 0u;
        }
    }
    if (!live) {
#pragma unroll
        for (int q = 0; q < E; ++q) key[q] = 0u;
    }
#pragma unroll
    for (int q = 0; q < E; ++q) mx = max(mx, key[q]);
    }
    // The bound: the k-th largest lane max (valid keys are >= 1); for k of
    // 57..128 (64-lane rows) the k-th largest of the lanes' two largest keys
    // (tighter near k = 64: MI355X [16384, 3000] k = 64 124 -> 90 us,
    // [16384, 2048] 50 -> 39; looser costs more than that below: k = 40..50
    // 3-12% slower).  One row per wave: a bit search with ballots; lane groups
    // of several rows: a bitonic sort of the group's lane maxima.
    uint32_t T, gmax = 0;
    if constexpr (L == 64) {
        if (k > 56) {
            if (ffast) float_keys();
            uint32_t mx2 = 0;  // the lane's second largest key
#pragma unroll
            for (int q = 0; q < E; ++q) mx2 = max(mx2, min(mx, key[q]));
            const uint32_t v2[2] = {mx, mx2};
            T = max(wave_rth_largest<2, 8 * EB>(v2, k), 1u);
        } else {
            const uint32_t v1[1] = {mx};
            T = max(wave_rth_largest<1, 8 * EB>(v1, min(k, L)), 1u);
        }
    } else {
        const uint32_t srt = group_sort_asc<L>(mx, sl);
        T = max(__shfl(srt, grp * L + (L - min(k, L)), 64), 1u);
        gmax = __shfl(srt, grp * L + L - 1, 64);
    }
    const bool bound_ok = k <= (L == 64 ? 2 * L : L);
    const bool fkeys = ffast && !(L == 64 && k > 56);  // filter on the floats
    const float Tf = __uint_as_float(key2bits(T, largest));
    auto xval = [&](int q) -> float {
        const float4& v = x[q >> 2];
        return (q & 3) == 0 ? v.x : (q & 3) == 1 ? v.y : (q & 3) == 2 ? v.z : v.w;
    };
    auto fcand = [&](int q) -> bool {
        const float f = xval(q);
        return LG ? !(f < Tf) : (f <= Tf);
    };
    int n = 0;
    if (fkeys) {
#pragma unroll
        for (int q = 0; q < E; ++q) n += fcand(q) ? 1 : 0;
    } else {
#pragma unroll
        for (int q = 0; q < E; ++q) n += (key[q] >= T) ? 1 : 0;
    }
    const int incl = group_scan<L>(n, sl);
    int c = bound_ok ? __shfl(incl, grp * L + L - 1, 64) : C + 1;  // candidates of this row
    // Fewer than k candidates: the row has keys of 0 (integers only; the
    // filter keeps keys >= 1), which the exact search below takes.
    if (c < k) c = C + 1;
    unsigned long long* list = cl[slot];
    if (c <= C) {
        int pos = incl - n;
        if (fkeys) {
            // the floats' bits in the keys' place, then the keys in place
#pragma unroll
            for (int q = 0; q < E; ++q) {
                if (fcand(q))
                    list[pos++] = comp_key(__float_as_uint(xval(q)), (uint32_t)short_elem<L, EB>(q, sl));
            }
            wave_sync_lds();
            for (int i = sl; i < c; i += L) {
                const unsigned long long e = list[i];
                list[i] = ((unsigned long long)f2key_sel(__uint_as_float((uint32_t)(e >> 32)), lm) << 32) |
                          (e & 0xffffffffull);
            }
        } else {
#pragma unroll
            for (int q = 0; q < E; ++q) {
                if (key[q] >= T) list[pos++] = comp_key(key[q], (uint32_t)short_elem<L, EB>(q, sl));
            }
        }
        if (c * c > 256 * L && c > 2 * k) {
            // Raise the bound with a 256-bin histogram of the candidates over
            // [T, row max] (the lower edge of the bin where the count from the
            // top reaches k), so the ranking below sees about k entries.  Only
            // when ranking all c candidates (c * c / L compares per lane) costs
            // more than the histogram (measured on MI355X: [16384, 1024] k = 32
            // 70 -> 38 us; [65536, 256] k = 8, about 30 candidates, is faster
            // without it).
            // The candidates move to registers and the row's list area holds the
            // 256-bin histogram meanwhile (C composites = 8L * 8 bytes >= 1 KiB),
            // which keeps the workgroup's LDS at the lists alone (occupancy).
            constexpr int PER = C / L;
            static_assert(C * sizeof(unsigned long long) >= 256 * sizeof(uint32_t), "histogram fits the list");
            uint32_t* hist = reinterpret_cast<uint32_t*>(list);
            wave_sync_lds();
            unsigned long long mine[PER];
#pragma unroll
            for (int r = 0; r < PER; ++r) mine[r] = (sl + r * L < c) ? list[sl + r * L] : 0ull;
            wave_sync_lds();  // every lane has its candidates before the area is cleared
#pragma unroll
            for (int b = 0; b < 256 / L; ++b) hist[sl * (256 / L) + b] = 0u;
            if (fkeys) {  // the row's largest key from its candidates (NaN included)
                uint32_t lmx = 0;
#pragma unroll
                for (int r = 0; r < PER; ++r) lmx = max(lmx, (uint32_t)(mine[r] >> 32));
                gmax = group_max<L>(lmx);
            } else if constexpr (L == 64) {
                gmax = wave_max_u32(mx);
            }
            const int shift = hist_shift(gmax, T);
            wave_sync_lds();
#pragma unroll
            for (int r = 0; r < PER; ++r)
                if (mine[r]) atomicAdd(&hist[((uint32_t)(mine[r] >> 32) - T) >> shift], 1u);
            wave_sync_lds();
            const uint32_t T1 = group_hist_threshold<L>(hist, k, T, shift, sl, grp);
            wave_sync_lds();  // every lane has read its bins before the survivors overwrite them
            int nk = 0;
#pragma unroll
            for (int r = 0; r < PER; ++r) nk += (mine[r] && (uint32_t)(mine[r] >> 32) >= T1) ? 1 : 0;
            const int kinc = group_scan<L>(nk, sl);
            c = __shfl(kinc, grp * L + L - 1, 64);
            int kpos = kinc - nk;
#pragma unroll
            for (int r = 0; r < PER; ++r)
                if (mine[r] && (uint32_t)(mine[r] >> 32) >= T1) list[kpos++] = mine[r];
        }
    } else {
        // exact k-th key by bit search over every key of the row (keys of
        // EB-byte elements are below 2^(8 EB))
        if (fkeys) float_keys();
        uint32_t pre = 0;
        for (int b = 8 * EB - 1; b >= 0; --b) {
            const uint32_t cand = pre | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int q = 0; q < E; ++q) cnt += (key[q] >= cand) ? 1 : 0;
            if (group_sum<L>(cnt) >= k) pre = cand;
        }
        int ng = 0;
#pragma unroll
        for (int q = 0; q < E; ++q) ng += (key[q] > pre) ? 1 : 0;
        const int gincl = group_scan<L>(ng, sl);
        const int cgt = __shfl(gincl, grp * L + L - 1, 64);  // < k
        int pos = gincl - ng;
#pragma unroll
        for (int q = 0; q < E; ++q) {
            if (key[q] > pre) list[pos++] = comp_key(key[q], (uint32_t)short_elem<L, EB>(q, sl));
        }
        // keys == pre in index order (vector j, lane, dword, element) until k are taken
        int taken = cgt;
        constexpr int KV = 4 * EPW;  // keys per vector
#pragma unroll
        for (int j = 0; j < E4; ++j) {
            int ne = 0;
#pragma unroll
            for (int q = 0; q < KV; ++q) ne += (key[KV * j + q] == pre) ? 1 : 0;
            const int einc = group_scan<L>(ne, sl);
            int at = taken + einc - ne;
#pragma unroll
            for (int q = 0; q < KV; ++q) {
                if (key[KV * j + q] == pre) {
                    if (at < k) list[at] = comp_key(pre, (uint32_t)short_elem<L, EB>(KV * j + q, sl));
                    ++at;
                }
            }
            taken += __shfl(einc, grp * L + L - 1, 64);
        }
        c = k;
    }
    wave_sync_lds();
    if (L == 64 && c > 36 && c <= 128) {
        // Few candidates per lane: a lane sort of 64 or 128 composites costs
        // fewer instructions than c compares per candidate.  Lane sl ends with
        // sorted positions sl*P .. sl*P+P-1.
        if (c <= 64) {
            unsigned long long x[1] = {sl < c ? list[sl] : 0ull};
            wave_sort_desc<1>(x);
            if (a.sample) {  // the sampler: the sorted k in the row's list, then the draw by this wave
                wave_sync_lds();
                if (sl < k) list[sl] = x[0];
                wave_sync_lds();
                if (live) sample_from_sel(a, row, p, list, k);
                return;
            }
            if (sl < k && live) write_ranked<EB>(a, row, k, p, largest, sl, x[0]);
        } else {
            unsigned long long x[2] = {2 * sl < c ? list[2 * sl] : 0ull, 2 * sl + 1 < c ? list[2 * sl + 1] : 0ull};
            wave_sort_desc<2>(x);
            if (a.sample) {
                wave_sync_lds();
                if (2 * sl < k) list[2 * sl] = x[0];
                if (2 * sl + 1 < k) list[2 * sl + 1] = x[1];
                wave_sync_lds();
                if (live) sample_from_sel(a, row, p, list, k);
                return;
            }
            if (2 * sl < k && live) write_ranked<EB>(a, row, k, p, largest, 2 * sl, x[0]);
            if (2 * sl + 1 < k && live) write_ranked<EB>(a, row, k, p, largest, 2 * sl + 1, x[1]);
        }
        return;
    }
    constexpr int PL = C / L;  // candidates per lane at most
    int rk[PL];
    unsigned long long cv[PL];
#pragma unroll
    for (int q = 0; q < PL; ++q) {
        const int i = sl + q * L;
        rk[q] = k;
        cv[q] = 0ull;
        if (i < c) {
            const unsigned long long ci = list[i];
            int r = 0;
            for (int j = 0; j < c; ++j) r += (list[j] > ci) ? 1 : 0;
            rk[q] = r;
            cv[q] = ci;
            if (r < k && live && !a.sample) write_ranked<EB>(a, row, k, p, largest, r, ci);
        }
    }
    if (a.sample) {  // L == 64 (one row per wave) when sampling
        wave_sync_lds();
#pragma unroll
        for (int q = 0; q < PL; ++q)
            if (rk[q] < k) list[rk[q]] = cv[q];
        wave_sync_lds();
        if (live) sample_from_sel(a, row, p, list, k);
    }
}

// ---------------------------------------------------------------------------
// Large k (k > 128, or k > 64 on rows the wave kernel does not take): one
// 1024-thread workgroup per row.  Exact radix select of the k-th key in four
// 8-bit passes over the row with LDS histograms (exact_select), the k
// selected composites gathered (every larger key, then the lowest-index equal
// keys), then a bitonic sort of the k survivors, padded to a power of two with
// zero composites (below every element), in LDS for k <= kRadixLds, else in
// the row's slice of the workspace.
// ---------------------------------------------------------------------------
constexpr int kRadixT = 256;    // threads per row (several rows per CU)
constexpr int kRadixLds = 4096;  // composites sorted in LDS (32 KiB)
constexpr int kRadixRegChunk = 8192;  // chunk of the global sort held in registers (1024 threads x 8)
constexpr int kRadixBins = 2048; // 11-bit digits: passes over key bits 31..21, 20..10, 9..0

__host__ __device__ inline int pow2_at_least(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}



// Composite (key, index) ordered by key, then by lowest index; never 0 for an
// element (0 pads the bitonic sort).
template <class K>
struct Comp {
    using C = typename std::conditional<(sizeof(K) > 4), unsigned __int128, unsigned long long>::type;
    __device__ static C make(K key, uint32_t idx) { return ((C)key << 32) | (C)(0xffffffffu - idx); }
    __device__ static uint32_t index(C c) { return 0xffffffffu - (uint32_t)(c & (C)0xffffffffu); }
};

// Descending bitonic sort of c[0..n) (n a power of two) by the NT threads.
template <int NT, class C>
__device__ void bitonic_desc(C* c, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < n / 2; t += NT) {
                const int i = ((t & ~(stride - 1)) << 1) | (t & (stride - 1));  // stride: a power of two
                const int j = i + stride;
                const C ci = c[i], cj = c[j];
                const bool desc = (i & size) == 0;  // this block's final direction
                if (desc ? (ci < cj) : (ci > cj)) {
                    c[i] = cj;
                    c[j] = ci;
                }
            }
            __syncthreads();
        }
    }
}

// The stages of one bitonic block size `size` with strides from `top` down to
// 1 on the B-composite chunk held in `lds` whose first element has global
// position g0 (the direction of a pair follows its global position, as in
// bitonic_desc).  Ends with a barrier.
template <int NT, class C, int B>
__device__ void bitonic_chunk_stages(C* lds, int g0, int size, int top) {
    for (int stride = top; stride > 0; stride >>= 1) {
        for (int t = threadIdx.x; t < B / 2; t += NT) {
            const int i = ((t & ~(stride - 1)) << 1) | (t & (stride - 1));
            const int j = i + stride;
            const C ci = lds[i], cj = lds[j];
            const bool desc = ((g0 + i) & size) == 0;
            if (desc ? (ci < cj) : (ci > cj)) {
                lds[i] = cj;
                lds[j] = ci;
            }
        }
        __syncthreads();
    }
}

// NST consecutive bitonic stages of block size `size`, strides dl << (NST-1)
// down to dl, in place in global memory: each thread holds the G = 2^NST
// elements base + m*dl (m < G) of a group in registers, so one read and one
// write of the composites serve NST stages.  Ends with a barrier.
template <int NT, class C, int NST>
__device__ void bitonic_global_stages(C* c, int n, int size, int dl) {
    constexpr int G = 1 << NST;
    const int sh = __builtin_ctz((unsigned)dl);
    for (int t = threadIdx.x; t < n / G; t += NT) {
        const int base = ((t >> sh) << (sh + NST)) | (t & (dl - 1));
        C v[G];
#pragma unroll
        for (int m = 0; m < G; ++m) v[m] = c[base + m * dl];
        const bool desc = (base & size) == 0;
#pragma unroll
        for (int s = G / 2; s >= 1; s >>= 1) {
#pragma unroll
            for (int m = 0; m < G; ++m) {
                if (m & s) continue;
                const C x = v[m], y = v[m + s];
                const bool sw = desc ? (x < y) : (x > y);
                v[m] = sw ? y : x;
                v[m + s] = sw ? x : y;
            }
        }
#pragma unroll
        for (int m = 0; m < G; ++m) c[base + m * dl] = v[m];
    }
    __syncthreads();
}

// The bitonic block sizes s_lo .. s_hi (powers of two) over an n-composite
// chunk held P per thread (thread t: positions t*P .. t*P+P-1, every thread of
// the workgroup active, n = NT*P) whose first element has global position g0:
// the direction of a pair follows its global position, strides start at
// min(s, n) / 2.  As reg_sort_desc: strides below P in registers, below 64*P
// by lane permutes, the rest through xb (LDS, NT*min(P, 4) composites) with
// barriers.
template <int NT, int P>
__device__ void reg_bitonic_range(unsigned long long (&x)[P], unsigned long long* xb, int n, int s_lo, int s_hi,
                                  int g0) {
    constexpr int Q = P < 4 ? P : 4;
    const int t = threadIdx.x;
    for (int s = s_lo; s <= s_hi; s <<= 1) {
        for (int d = min(s, n) >> 1; d >= P; d >>= 1) {
            const int m = d / P;  // partner thread t ^ m
            const bool desc = ((g0 + t * P) & s) == 0;
            const bool keep_max = ((t & m) == 0) == desc;
            switch (m) {
                case 1: sort_lane_stage<1, P>(x, keep_max); break;
                case 2: sort_lane_stage<2, P>(x, keep_max); break;
                case 4: sort_lane_stage<4, P>(x, keep_max); break;
                case 8: sort_lane_stage<8, P>(x, keep_max); break;
                case 16: sort_lane_stage<16, P>(x, keep_max); break;
                case 32: sort_lane_stage<32, P>(x, keep_max); break;
                default:
#pragma unroll
                    for (int p0 = 0; p0 < P; p0 += Q) {
#pragma unroll
                        for (int q = 0; q < Q; ++q) xb[q * NT + t] = x[p0 + q];
                        __syncthreads();
#pragma unroll
                        for (int q = 0; q < Q; ++q) {
                            const unsigned long long y = xb[q * NT + (t ^ m)];
                            x[p0 + q] = ((x[p0 + q] > y) == keep_max) ? x[p0 + q] : y;
                        }
                        __syncthreads();
                    }
            }
        }
#pragma unroll
        for (int dd = P / 2; dd >= 1; dd >>= 1) {
            if (dd < s) {
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    if ((p & dd) == 0) {
                        const bool desc = ((g0 + t * P + p) & s) == 0;
                        const unsigned long long u = x[p], v = x[p + dd];
                        const bool sw = (u > v) != desc;
                        x[p] = sw ? v : u;
                        x[p + dd] = sw ? u : v;
                    }
                }
            }
        }
    }
}

// bitonic_desc for n > B composites in global memory, with the B-composite
// LDS buffer `lds`: every stage of stride < B runs on B-element chunks staged
// in LDS (one load and one store per chunk for all of a block size's short
// strides; 64-bit composites held in registers, reg_bitonic_range); the
// strides >= B run in global memory, up to three per pass
// (bitonic_global_stages).  At n = 2^18: 9 global passes and 7 chunk passes
// with B = 4096, 5 and 5 with B = 16384, against 171 global stages.
template <int NT, class C, int B>
__device__ void bitonic_desc_blocked(C* c, int n, C* lds) {
    for (int size = 2; size <= n; size <<= 1) {
        if (size > B) {
            int cur = size / 2;
            while (cur >= B) {
                if ((cur >> 2) >= B) {
                    bitonic_global_stages<NT, C, 3>(c, n, size, cur >> 2);
                    cur >>= 3;
                } else if ((cur >> 1) >= B) {
                    bitonic_global_stages<NT, C, 2>(c, n, size, cur >> 1);
                    cur >>= 2;
                } else {
                    bitonic_global_stages<NT, C, 1>(c, n, size, cur);
                    cur >>= 1;
                }
            }
        }
        // the block sizes up to B all run in one visit per chunk
        if (size > B || size == 2) {
            if constexpr (std::is_same<C, unsigned long long>::value && B % NT == 0 && NT == 1024) {
                // 64-bit composites, 1024 threads: the chunk in registers, B / NT
                // per thread (the 256-thread kernel keeps the LDS stages: 16 per
                // thread would cost it occupancy in the select phase)
                constexpr int P = B / NT;
                const int t = threadIdx.x;
                for (int g0 = 0; g0 < n; g0 += B) {
                    unsigned long long x[P];
#pragma unroll
                    for (int p = 0; p < P; ++p) x[p] = c[g0 + t * P + p];
                    if (size > B) reg_bitonic_range<NT, P>(x, lds, B, size, size, g0);
                    else reg_bitonic_range<NT, P>(x, lds, B, 2, B, g0);
#pragma unroll
                    for (int p = 0; p < P; ++p) c[g0 + t * P + p] = x[p];
                }
                __syncthreads();
            } else {
                for (int g0 = 0; g0 < n; g0 += B) {
                    for (int e = threadIdx.x; e < B; e += NT) lds[e] = c[g0 + e];
                    __syncthreads();
                    if (size > B) {
                        bitonic_chunk_stages<NT, C, B>(lds, g0, size, B / 2);
                    } else {
                        for (int s = 2; s <= B; s <<= 1) bitonic_chunk_stages<NT, C, B>(lds, g0, s, s / 2);
                    }
                    for (int e = threadIdx.x; e < B; e += NT) c[g0 + e] = lds[e];
                    __syncthreads();
                }
            }
        }
    }
}

// Composites sorted in LDS: 32 KiB of them (4096 for 32-bit keys, 2048 for 64-bit).
template <class T>
constexpr int radix_lds_count() { return sizeof(T) > 4 ? 2048 : kRadixLds; }

template <class T>
struct RadixShared {
    typename Comp<typename SortKey<T>::K>::C cand[radix_lds_count<T>()];
    uint32_t hist[kRadixBins];
    int wtot[kMaxW];
    int digit, kk, cls, count, eq_taken;
};

// Inclusive suffix sum over the workgroup's threads (thread t gets the sum of
// v over threads t .. NT-1).  Ends with a barrier.
template <int NT>
__device__ int block_suffix_incl(int v, int* wtot) {
    constexpr int NW = NT / 64;
    const int lane = __lane_id();
    const int w = threadIdx.x / 64;
    const int pre = wave_incl_scan(v);
    const int wsum = __builtin_amdgcn_readlane(pre, 63);
    int suf = wsum - pre + v;  // lanes lane .. 63
    if (lane == 0) wtot[w] = wsum;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NW; ++i)
        if (i > w) suf += wtot[i];
    __syncthreads();
    return suf;
}

// Exact top-k selection of p[0..n) into cand[0..k) (unordered): the k-th key T
// by radix passes over the key bits from the top, 11 bits per pass (each pass
// counts the keys that match the digits found so far in a 2048-bin LDS
// histogram), then every key > T and the lowest-index keys == T.
// GB: the gather keeps several loads in flight per thread (more registers).
template <int NT, class T, bool GB = true>
__device__ void radix_select(RadixShared<T>& sh, typename Comp<typename SortKey<T>::K>::C* cand, const T* p, int n,
                             int k, int largest) {
    using K = typename SortKey<T>::K;
    using CP = Comp<K>;
    constexpr int BPT = kRadixBins / NT;  // histogram bins per thread in the digit search
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int w = tid / 64;
    K prefix = 0, pmask = 0;
    int kk = k;
    bool whole = false;  // the class sharing the found prefix is exactly the kk still wanted
    for (int hi = SortKey<T>::kBits; hi > 0 && !whole; hi -= 11) {
        const int shift = hi > 11 ? hi - 11 : 0;
        const K dmask = (K)((1u << (hi - shift)) - 1u);
        for (int i = tid; i < kRadixBins; i += NT) sh.hist[i] = 0u;
        __syncthreads();
        // eight loads in flight per thread before their histogram updates
        int e0 = tid;
        for (; e0 + 7 * NT < n; e0 += 8 * NT) {
            K key[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) key[u] = SortKey<T>::of(p[e0 + u * NT], largest);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if ((key[u] & pmask) == prefix) atomicAdd(&sh.hist[(uint32_t)((key[u] >> shift) & dmask)], 1u);
        }
        for (int e = e0; e < n; e += NT) {
            const K key = SortKey<T>::of(p[e], largest);
            if ((key & pmask) == prefix) atomicAdd(&sh.hist[(uint32_t)((key >> shift) & dmask)], 1u);
        }
        __syncthreads();
        uint32_t h[BPT];
        int own = 0;
#pragma unroll
        for (int b = 0; b < BPT; ++b) {
            h[b] = sh.hist[tid * BPT + b];
            own += (int)h[b];
        }
        const int suf = block_suffix_incl<NT>(own, sh.wtot);
        if (suf >= kk && suf - own < kk) {  // the thread whose bins hold the kk-th key from the top
            int cum = suf - own;
            int b = BPT - 1;
            for (; b > 0; --b) {
                if (cum + (int)h[b] >= kk) break;
                cum += (int)h[b];
            }
            sh.digit = tid * BPT + b;
            sh.kk = kk - cum;
            sh.cls = (int)h[b];
        }
        __syncthreads();
        prefix |= (K)sh.digit << shift;
        pmask |= dmask << shift;
        kk = sh.kk;
        whole = sh.cls == kk;
        __syncthreads();
    }
    if (whole) {
        // every key above the class and the whole class: exactly k, no ties to
        // order (most data: after two or three passes instead of all of them)
        if (tid == 0) sh.count = 0;
        __syncthreads();
        // GB: GU loads in flight per thread (8 in the 1024-thread kernel, which
        // runs one workgroup per CU anyway; 4 in the 256-thread one)
        constexpr int GU = NT == 1024 ? 8 : 4;
        int e0 = tid;
        for (; GB && e0 + (GU - 1) * NT < n; e0 += GU * NT) {
            K key[GU];
#pragma unroll
            for (int u = 0; u < GU; ++u) key[u] = SortKey<T>::of(p[e0 + u * NT], largest);
#pragma unroll
            for (int u = 0; u < GU; ++u)
                if ((key[u] & pmask) >= prefix)
                    cand[atomicAdd(&sh.count, 1)] = CP::make(key[u], (uint32_t)(e0 + u * NT));
        }
        for (int e = e0; e < n; e += NT) {
            const K key = SortKey<T>::of(p[e], largest);
            if ((key & pmask) >= prefix) cand[atomicAdd(&sh.count, 1)] = CP::make(key, (uint32_t)e);
        }
        __syncthreads();
        return;
    }
    const K Tk = prefix;  // the k-th key; take kk of the keys equal to it
    if (tid == 0) {
        sh.count = 0;
        sh.eq_taken = 0;
    }
    __syncthreads();
    for (int base = 0; base < n; base += NT) {
        const int e = base + tid;
        const K key = (e < n) ? SortKey<T>::of(p[e], largest) : (K)0;
        if (e < n && key > Tk) cand[atomicAdd(&sh.count, 1)] = CP::make(key, (uint32_t)e);
        const bool eq = (e < n) && key == Tk;
        const unsigned long long bal = __ballot(eq);
        if (lane == 0) sh.wtot[w] = __popcll(bal);
        __syncthreads();
        int before = sh.eq_taken + __popcll(bal & lanemask_lt());
        int total = 0;
        for (int i = 0; i < NT / 64; ++i) {
            if (i < w) before += sh.wtot[i];
            total += sh.wtot[i];
        }
        if (eq && before < kk) cand[atomicAdd(&sh.count, 1)] = CP::make(key, (uint32_t)e);
        __syncthreads();
        if (tid == 0) sh.eq_taken += total;
        __syncthreads();
        if (sh.eq_taken >= kk && base + NT < n) {
            // every equal key needed is taken: the rest only adds keys > T
            for (int e2 = base + NT + tid; e2 < n; e2 += NT) {
                const K k2 = SortKey<T>::of(p[e2], largest);
                if (k2 > Tk) cand[atomicAdd(&sh.count, 1)] = CP::make(k2, (uint32_t)e2);
            }
            break;
        }
    }
    __syncthreads();
}

// Values are the selected elements themselves (re-read at their index).
// GSORT: k's composites are sorted in the workspace (pow2(k) > the LDS count);
// only those launches carry the global sort's code and registers.  GB: see
// radix_select (off where two 1024-thread workgroups per CU must fit).
template <class T, int NT, bool GSORT, bool GB>
__global__ __launch_bounds__(NT) void k_topk_radix(TopkArgs a, void* gcand) {
    using C = typename Comp<typename SortKey<T>::K>::C;
    __shared__ RadixShared<T> sh;
    const long long row = blockIdx.x;
    if (a.flags && a.flags[row] == 0) return;  // finished by the wave kernel
    const T* p = reinterpret_cast<const T*>(a.in) + row * a.row_stride;
    const int k = a.k;
    const int n2 = pow2_at_least(k);
    C* cand = (n2 <= radix_lds_count<T>()) ? sh.cand : static_cast<C*>(gcand) + row * (long long)n2;
    radix_select<NT, T, GB>(sh, cand, p, a.cols, k, a.largest);
    for (int i = k + threadIdx.x; i < n2; i += NT) cand[i] = (C)0;
    __syncthreads();
    if constexpr (!GSORT) {
        bitonic_desc<NT, C>(cand, n2);
    } else {
        if (NT == 1024 && sizeof(C) == 8 && n2 > kRadixRegChunk)
            bitonic_desc_blocked<NT, C, kRadixRegChunk>(cand, n2, sh.cand);  // 8 composites per thread
        else
            bitonic_desc_blocked<NT, C, radix_lds_count<T>()>(cand, n2, sh.cand);
    }
    if constexpr (std::is_same<T, float>::value) {
        if (a.sample) {
            if (threadIdx.x < 64) sample_from_sel(a, row, p, cand, k);
            return;
        }
    }
    T* ov = reinterpret_cast<T*>(a.out_v);
    for (int i = threadIdx.x; i < k; i += NT) {
        const uint32_t idx = Comp<typename SortKey<T>::K>::index(cand[i]);
        ov[row * k + i] = p[idx];
        a.out_i[row * k + i] = (long long)idx;
    }
}

// ---------------------------------------------------------------------------
// Large k on rows of at most 32768 elements of <= 4 bytes (k_topk_rsel): one
// workgroup of NT threads per row keeps the row's EPT keys per thread in
// registers (element e = j*NT + t), read from HBM once.  The k-th key is
// radix-selected over the registers with a 2048-bin LDS histogram, 11 bits per
// pass, stopping as soon as the class of keys that share the found prefix
// holds exactly the number still wanted (after two passes on most data).  The
// k composites, padded with zeros to n = pow2(max(k, 64)), are then
// bitonic-sorted by n / P threads holding P each (reg_sort_desc): exchanges at
// a distance below P stay in registers, below 64*P in the wave (lane
// permutes), only the rest go through LDS with a barrier.
// ---------------------------------------------------------------------------
constexpr int kRselMaxCols = 32768;

__host__ __device__ constexpr int dtype_bytes(int32_t dtype) {
    return (dtype == TPR_INT64 || dtype == TPR_UINT64 || dtype == TPR_FLOAT64) ? 8
         : (dtype == TPR_INT32 || dtype == TPR_UINT32 || dtype == TPR_FLOAT32) ? 4
         : (dtype == TPR_INT16 || dtype == TPR_UINT16) ? 2 : 1;
}

template <int NT>
__device__ int block_prefix_excl(int v, int* wtot, int& total) {
    constexpr int NW = NT / 64;
    const int lane = __lane_id();
    const int w = threadIdx.x / 64;
    const int inc = wave_incl_scan(v);
    if (lane == 63) wtot[w] = inc;
    __syncthreads();
    int before = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int c = wtot[i];
        if (i < w) before += c;
        total += c;
    }
    __syncthreads();
    return before + inc - v;
}

// Descending bitonic sort of n composites (n / P threads, a multiple of 64,
// at most NT) held P per thread: thread t holds positions t*P .. t*P+P-1.
// Distances below P: compare-exchanges in registers; below 64*P: the partner
// lane's value by a lane permute; the rest through xb (LDS, NT*min(P, 4)
// composites) with a barrier, which every thread of the workgroup reaches.
template <int NT, int P>
__device__ void reg_sort_desc(unsigned long long (&x)[P], unsigned long long* xb, int n) {
    constexpr int Q = P < 4 ? P : 4;
    const int t = threadIdx.x;
    const bool active = t < n / P;  // whole waves
    for (int s = 2; s <= n; s <<= 1) {
        for (int d = s >> 1; d >= P; d >>= 1) {
            const int m = d / P;  // partner thread t ^ m
            const bool desc = ((t * P) & s) == 0;
            const bool keep_max = ((t & m) == 0) == desc;
            if (!active && m < 64) continue;
            switch (m) {
                case 1: sort_lane_stage<1, P>(x, keep_max); break;
                case 2: sort_lane_stage<2, P>(x, keep_max); break;
                case 4: sort_lane_stage<4, P>(x, keep_max); break;
                case 8: sort_lane_stage<8, P>(x, keep_max); break;
                case 16: sort_lane_stage<16, P>(x, keep_max); break;
                case 32: sort_lane_stage<32, P>(x, keep_max); break;
                default:
#pragma unroll
                    for (int p0 = 0; p0 < P; p0 += Q) {
                        if (active) {
#pragma unroll
                            for (int q = 0; q < Q; ++q) xb[q * NT + t] = x[p0 + q];
                        }
                        __syncthreads();
                        if (active) {
#pragma unroll
                            for (int q = 0; q < Q; ++q) {
                                const unsigned long long y = xb[q * NT + (t ^ m)];
                                x[p0 + q] = ((x[p0 + q] > y) == keep_max) ? x[p0 + q] : y;
                            }
                        }
                        __syncthreads();
                    }
            }
        }
        if (!active) continue;
#pragma unroll
        for (int dd = P / 2; dd >= 1; dd >>= 1) {
            if (dd < s) {
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    if ((p & dd) == 0) {
                        const bool desc = ((t * P + p) & s) == 0;
                        const unsigned long long u = x[p], v = x[p + dd];
                        const bool sw = (u > v) != desc;
                        x[p] = sw ? v : u;
                        x[p + dd] = sw ? u : v;
                    }
                }
            }
        }
    }
}

template <int NT, int P>
struct RselShared {
    static constexpr int kBuf = (NT * (P < 4 ? P : 4) > 1024) ? NT * (P < 4 ? P : 4) : 1024;
    union {
        uint32_t hist[kRadixBins];
        unsigned long long buf[kBuf];  // exchanges, staging of the list, the sampler's sorted list
    };
    int wtot[NT / 64];
    int digit, kk, cls;
};

// Element of the row held in register j of thread t: groups of four
// consecutive elements, group g = j / 4 of thread t at element 4 * (g * NT + t),
// so 4-byte elements load as one 128-bit vector per group.
template <int NT>
__device__ __forceinline__ int rsel_idx(int j, int t) {
    return ((j >> 2) * NT + t) * 4 + (j & 3);
}

template <class T, int NT, int EPT>
__device__ __forceinline__ void rsel_load(uint32_t (&key)[EPT], const void* base, int cols, int largest) {
    static_assert(EPT % 4 == 0, "groups of four");
    const T* p = static_cast<const T*>(base);
    const int t = (int)threadIdx.x;
    if constexpr (sizeof(T) == 4) {
        if ((reinterpret_cast<uintptr_t>(base) & 15u) == 0) {
            // past the row end the buffer range check returns zeros (masked below)
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                                                                 cols * 4, kBufWord3);
#pragma unroll
            for (int g = 0; g < EPT / 4; ++g) {
                const f32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (g * NT + t) * 16, 0, kNT);
                const float f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int e = (g * NT + t) * 4 + q;
                    key[4 * g + q] = e < cols ? (uint32_t)SortKey<T>::of(__builtin_bit_cast(T, f[q]), largest) : 0u;
                }
            }
            return;
        }
    }
    if constexpr (sizeof(T) < 4) {
        if ((reinterpret_cast<uintptr_t>(base) & (4 * sizeof(T) - 1)) == 0) {
            // a group of four 1- or 2-byte elements is one 32- or 64-bit load;
            // only the group that straddles the row end loads element-wise
            using W = typename std::conditional<sizeof(T) == 1, uint32_t, unsigned long long>::type;
            using U = typename std::make_unsigned<T>::type;
#pragma unroll
            for (int g = 0; g < EPT / 4; ++g) {
                const int e0 = (g * NT + t) * 4;
                if (e0 + 3 < cols) {
                    const W wv = *reinterpret_cast<const W*>(p + e0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const U u = (U)(wv >> (8 * sizeof(T) * q));
                        key[4 * g + q] = (uint32_t)SortKey<T>::of(__builtin_bit_cast(T, u), largest);
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) key[4 * g + q] = e0 + q < cols ? (uint32_t)SortKey<T>::of(p[e0 + q], largest) : 0u;
                }
            }
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = rsel_idx<NT>(j, t);
        key[j] = e < cols ? (uint32_t)SortKey<T>::of(p[e], largest) : 0u;
    }
}

// Raw bits of a selected element of <= 4 bytes, recovered from its sortable
// key (the inverse of SortKey::of); float32 reads the input only for +-0.0 and
// NaN, whose keys are canonical.
__device__ __forceinline__ uint32_t selected_bits(int dtype, uint32_t key, int largest, const void* row, uint32_t idx) {
    if (dtype == TPR_FLOAT32) return __float_as_uint(selected_value(static_cast<const float*>(row), key, idx, largest));
    const int bits = 8 * dtype_bytes(dtype);
    const uint32_t mask = bits == 32 ? 0xffffffffu : ((1u << bits) - 1u);
    const uint32_t k = (largest ? key : ~key) & mask;
    const bool sgn = dtype == TPR_INT8 || dtype == TPR_INT16 || dtype == TPR_INT32;
    return sgn ? (k ^ (1u << (bits - 1))) : k;
}

__device__ __forceinline__ void store_bits(void* out, long long i, int dtype, uint32_t v) {
    switch (dtype_bytes(dtype)) {
        case 4: static_cast<uint32_t*>(out)[i] = v; break;
        case 2: static_cast<uint16_t*>(out)[i] = (uint16_t)v; break;
        default: static_cast<uint8_t*>(out)[i] = (uint8_t)v; break;
    }
}

template <int NT, int EPT, int P>
__global__ __launch_bounds__(NT) void k_topk_rsel(TopkArgs a, int dtype, int sort_n) {
    using CP = Comp<uint32_t>;
    constexpr int BPT = kRadixBins / NT;
    __shared__ RselShared<NT, P> sh;
    const int tid = threadIdx.x;
    // nseg > 1: the row is cut into segments of seg_len elements, one
    // workgroup each, whose k winners (sorted composites with row indices) go
    // to the merge pass
    const long long row = blockIdx.x / a.nseg;
    const int seg = (int)(blockIdx.x % a.nseg);
    const int lo = seg * a.seg_len;
    const int cols = min(a.cols - lo, a.seg_len), k = a.k;
    const char* rowbase = reinterpret_cast<const char*>(a.in) + row * a.row_stride * dtype_bytes(dtype);
    const char* base = rowbase + (long long)lo * dtype_bytes(dtype);
    uint32_t key[EPT];
    switch (dtype) {
        case TPR_FLOAT32: rsel_load<float, NT, EPT>(key, base, cols, a.largest); break;
        case TPR_INT32: rsel_load<int, NT, EPT>(key, base, cols, a.largest); break;
        case TPR_UINT32: rsel_load<unsigned int, NT, EPT>(key, base, cols, a.largest); break;
        case TPR_INT16: rsel_load<short, NT, EPT>(key, base, cols, a.largest); break;
        case TPR_UINT16: rsel_load<unsigned short, NT, EPT>(key, base, cols, a.largest); break;
        case TPR_INT8: rsel_load<signed char, NT, EPT>(key, base, cols, a.largest); break;
        default: rsel_load<unsigned char, NT, EPT>(key, base, cols, a.largest); break;  // UINT8, BOOL
    }
    // ---- radix select: prefix / pmask name the class of the k-th key ----
    uint32_t prefix = 0, pmask = 0;
    int kk = k;
    bool whole = false;  // every key of the class is taken
    // keys of 1- and 2-byte elements are below 2^8 / 2^16: one / two passes
    for (int hi = 8 * dtype_bytes(dtype); hi > 0 && !whole; hi -= 11) {
        const int shift = hi > 11 ? hi - 11 : 0;
        const uint32_t dmask = (1u << (hi - shift)) - 1u;
#pragma unroll
        for (int b = 0; b < BPT; ++b) sh.hist[tid * BPT + b] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (rsel_idx<NT>(j, tid) < cols && (key[j] & pmask) == prefix) atomicAdd(&sh.hist[(key[j] >> shift) & dmask], 1u);
        __syncthreads();
        uint32_t h[BPT];
        int own = 0;
#pragma unroll
        for (int b = 0; b < BPT; ++b) {
            h[b] = sh.hist[tid * BPT + b];
            own += (int)h[b];
        }
        const int suf = block_suffix_incl<NT>(own, sh.wtot);
        if (suf >= kk && suf - own < kk) {
            int cum = suf - own;
            int b = BPT - 1;
            for (; b > 0; --b) {
                if (cum + (int)h[b] >= kk) break;
                cum += (int)h[b];
            }
            sh.digit = tid * BPT + b;
            sh.kk = kk - cum;
            sh.cls = (int)h[b];
        }
        __syncthreads();
        prefix |= (uint32_t)sh.digit << shift;
        pmask |= dmask << shift;
        kk = sh.kk;
        whole = sh.cls == kk;
        __syncthreads();
    }
    // ---- the k selected: every key above the class, and the class whole or
    // its kk lowest-index keys (exact ties) ----
    uint32_t take = 0;  // bit j: key[j] is selected
    int nt = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const bool v = rsel_idx<NT>(j, tid) < cols;
        const uint32_t hk = key[j] & pmask;
        const bool s = v && (hk > prefix || (whole && hk == prefix));
        take |= (uint32_t)s << j;
        nt += s;
    }
    if (!whole) {
        uint32_t eqm = 0;  // bit j: key[j] is in the class (equal to the k-th key)
#pragma unroll
        for (int j = 0; j < EPT; ++j) eqm |= (uint32_t)(rsel_idx<NT>(j, tid) < cols && key[j] == prefix) << j;
        // index order: group by group, in a group thread by thread, in a
        // thread its four elements in turn
        int run = 0;  // class members in groups before g
#pragma unroll 1
        for (int g = 0; g < EPT / 4; ++g) {
            const uint32_t m4 = (eqm >> (4 * g)) & 0xFu;
            int tot;
            int before = run + block_prefix_excl<NT>(__popc(m4), sh.wtot, tot);
            run += tot;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if ((m4 >> q) & 1u) {
                    if (before < kk) {
                        take |= 1u << (4 * g + q);
                        ++nt;
                    }
                    ++before;
                }
            }
        }
    }
    int tot;
    const int pos0 = block_prefix_excl<NT>(nt, sh.wtot, tot);
    // ---- stage the list into sort order (position r -> thread r / P), NT*Q
    // positions per round ----
    unsigned long long x[P];
#pragma unroll
    for (int p = 0; p < P; ++p) x[p] = 0ull;
    constexpr int Q = P < 4 ? P : 4;
    constexpr int RND = NT * Q;
    for (int r0 = 0; r0 < k; r0 += RND) {
        int pos = pos0;
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            if ((take >> j) & 1u) {
                if (pos >= r0 && pos < r0 + RND) sh.buf[pos - r0] = CP::make(key[j], (uint32_t)(lo + rsel_idx<NT>(j, tid)));
                ++pos;
            }
        }
        __syncthreads();
        const int first = tid * P;
        if (first >= r0 && first < r0 + RND) {
#pragma unroll
            for (int p = 0; p < P; ++p)
                if (first + p < k) x[p] = sh.buf[first + p - r0];
        }
        __syncthreads();
    }
    reg_sort_desc<NT, P>(x, sh.buf, sort_n);
    if (a.nseg > 1) {
        unsigned long long* dst = a.part + ((long long)row * a.nseg + seg) * k;
#pragma unroll
        for (int p = 0; p < P; ++p)
            if (tid * P + p < k) dst[tid * P + p] = x[p];
        return;
    }
    if (dtype == TPR_FLOAT32 && a.sample) {
        const int first = tid * P;
#pragma unroll
        for (int p = 0; p < P; ++p)
            if (first + p < k) sh.buf[first + p] = x[p];
        __syncthreads();
        if (tid < 64) sample_from_sel(a, row, reinterpret_cast<const float*>(base), sh.buf, k);
        return;
    }
    const int first = tid * P;
    long long* oi = a.out_i + row * k;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int r = first + p;
        if (r < k) {
            const uint32_t idx = CP::index(x[p]);
            oi[r] = (long long)idx;
            store_bits(a.out_v, row * k + r, dtype, selected_bits(dtype, (uint32_t)(x[p] >> 32), a.largest, base, idx));
        }
    }
}

// Candidate lists longer than this are cut to the k winners by a radix select
// before ranking (the O(m^2) ranking of 4096 candidates took ~0.9 ms).
constexpr int kMergeRankMax = 512;

struct MergeShared {
    unsigned long long cand[kMergeMax];  // also the sort's exchange buffer and rank_select's counts afterwards
    union {
        int rank[kMergeRankMax];
        uint32_t hist[kRadixBins];
    };
    unsigned long long surv[kKMax];  // the k winners before ranking
    unsigned long long sel[kKMax];
    int wtot[kMergeT / 64];
    int digit, kk, cls, count;
};

// Pass 2: exact top k of a row's nseg * k segment winners (float32 from the
// wave / workgroup kernels, any dtype of <= 4 bytes from k_topk_rsel).
__global__ __launch_bounds__(kMergeT) void k_topk_merge(TopkArgs a, int dtype) {
    __shared__ MergeShared sh;
    const long long row = blockIdx.x;
    const int k = a.k;
    const int m = a.nseg * k;
    const int tid = threadIdx.x;
    const unsigned long long* src = a.part + row * (long long)m;
    for (int i = tid; i < m; i += kMergeT) sh.cand[i] = src[i];
    __syncthreads();
    if (m <= kMergeRankMax) {
        rank_select<kMergeT>(sh.cand, sh.rank, sh.sel, m, k);
    } else {
        // The composites are distinct, so the k-th largest is found exactly by
        // radix passes over all 64 bits, 11 per pass (2048-bin LDS histogram of
        // the composites matching the digits found so far), stopping once the
        // class sharing the found prefix is exactly the number still wanted.
        constexpr int BPT = kRadixBins / kMergeT;
        unsigned long long prefix = 0, pmask = 0;
        int kk = k;
        bool whole = false;
        for (int hi = 64; hi > 0 && !whole; hi -= 11) {
            const int shift = hi > 11 ? hi - 11 : 0;
            const unsigned long long dmask = (1ull << (hi - shift)) - 1ull;
#pragma unroll
            for (int b = 0; b < BPT; ++b) sh.hist[tid * BPT + b] = 0u;
            __syncthreads();
            for (int i = tid; i < m; i += kMergeT) {
                const unsigned long long c = sh.cand[i];
                if ((c & pmask) == prefix) atomicAdd(&sh.hist[(uint32_t)((c >> shift) & dmask)], 1u);
            }
            __syncthreads();
            uint32_t h[BPT];
            int own = 0;
#pragma unroll
            for (int b = 0; b < BPT; ++b) {
                h[b] = sh.hist[tid * BPT + b];
                own += (int)h[b];
            }
            const int suf = block_suffix_incl<kMergeT>(own, sh.wtot);
            if (suf >= kk && suf - own < kk) {
                int cum = suf - own;
                int b = BPT - 1;
                for (; b > 0; --b) {
                    if (cum + (int)h[b] >= kk) break;
                    cum += (int)h[b];
                }
                sh.digit = tid * BPT + b;
                sh.kk = kk - cum;
                sh.cls = (int)h[b];
            }
            if (tid == 0) sh.count = 0;
            __syncthreads();
            prefix |= (unsigned long long)sh.digit << shift;
            pmask |= dmask << shift;
            kk = sh.kk;
            whole = sh.cls == kk;
            __syncthreads();
        }
        // every composite above the class plus the whole class: exactly k
        for (int i = tid; i < m; i += kMergeT) {
            const unsigned long long c = sh.cand[i];
            if ((c & pmask) >= prefix) {
                const int pos = atomicAdd(&sh.count, 1);
                if (pos < kKMax) sh.surv[pos] = c;  // exactly k by construction; the test keeps LDS writes in range
            }
        }
        __syncthreads();
        if (k <= 128) {
            rank_select<kMergeT>(sh.surv, reinterpret_cast<int*>(sh.cand), sh.sel, k, k);
        } else {
            // k of 129..1024: bitonic sort, 4 composites per thread, padded with
            // zeros (below every element) to a power of two
            const int n = pow2_at_least(k);
            unsigned long long x[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) x[q] = (tid * 4 + q < k) ? sh.surv[tid * 4 + q] : 0ull;
            reg_sort_desc<kMergeT, 4>(x, sh.cand, n);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (tid * 4 + q < k) sh.sel[tid * 4 + q] = x[q];
            __syncthreads();
        }
    }
    const float* p = a.in + row * a.row_stride;
    if (a.sample) {
        if (threadIdx.x < 64) sample_from_sel(a, row, p, sh.sel, k);
        return;
    }
    for (int i = threadIdx.x; i < k; i += kMergeT) {
        const uint32_t ci = comp_index(sh.sel[i]);
#ifdef TPR_DEBUG_KNOBS
        if (ci >= (uint32_t)a.cols) atomicAdd(&topk_merge_clamped, 1u);
#endif
        const uint32_t idx = min(ci, (uint32_t)(a.cols - 1));  // in range even for a bad workspace
        a.out_i[row * k + i] = (long long)idx;
        const char* rb = reinterpret_cast<const char*>(a.in) + row * a.row_stride * dtype_bytes(dtype);
        store_bits(a.out_v, row * k + i, dtype, selected_bits(dtype, (uint32_t)(sh.sel[i] >> 32), a.largest, rb, idx));
    }
}

struct TopkPlan {
    int nseg;
    int seg_len;
    bool wave;
    int nw;  // waves per wave-kernel workgroup (8 or 16)
    size_t ws;
};

// Grid: about 2 * CUs 512-thread workgroups (or CUs 1024-thread ones).  Many
// rows: one 512-thread workgroup per row.  Fewer rows than that: the wave
// kernel gives each row a 1024-thread workgroup and cuts rows into segments
// only when rows < CUs.  Every segment holds >= k elements (and, for the wave
// kernel, a full first slice per wave), and the merge list fits one merge
// workgroup.
// Many rows of 4096 .. 16383 elements: 4-wave (256-thread) workgroups of the
// wave kernel, so each wave streams two or more slices and a CU holds eight
// rows.  Measured on MI355X (us, 8-wave wave kernel / workgroup kernels ->
// 4 waves): [4096, 4096] k = 64 47.7 -> 29.2, [4096, 6000] k = 16 41.5 -> 26.0,
// k = 100 105 -> 50, [4096, 8192] k = 64 44.0 -> 37.0, [2048, 12288] k = 64
// 31.6 -> 26.6; [2048, 16384] even (32.7 / 32.0) and [512, 8192] slower (11.1 /
// 12.0), so rows >= 4 per CU and rows shorter than 16384.  Rows the
// lane-group kernel can hold (<= 4096) go there first (U(-1, 1) data:
// [2048, 4096] k = 64 14.0 against 17.7 us, [16384, 4096] k = 64 81 against
// 99).  topk_waves = 4 (debug knob) forces it on every row of >= 4096 elements.
bool wave4(long long rows, long long cols, long long k) {
    if (k > kWave4K || cols < 4 * kSlice) return false;
    if (knobs().topk_waves != 0) return knobs().topk_waves == 4;
    return cols < 2 * kWaveMinSeg && rows >= 4LL * device_info().cus;
}

__host__ inline bool short_exact(long long rows, long long cols, long long k) {
    if (k <= kShortMaxK || k > kShortK2) return false;
    if (knobs().topk_short > 0) return cols < kShortMaxCols;
    return cols <= 2048 && rows >= 8LL * device_info().cus;
}

TopkPlan plan_topk(long long rows, long long cols, long long k) {
    TopkPlan pl{1, (int)cols, false, 8, 0};
    const int cus = device_info().cus;
    const bool w4 = wave4(rows, cols, k);
    const bool wave_ok = k <= kWaveK && (cols >= kWaveMinSeg || w4);
    // 16 waves: rows <= 1 per CU from 16384 elements, 1..2 per CU from 32768
    // (at 16384 the 8-wave kernel wins there: [512, 16384] k = 64 13.6 against
    // 15.5 us)
    const int nw = w4 ? 4
                      : (wave_ok && cols >= 2 * kWaveMinSeg && (rows <= cus || (rows <= 2LL * cus && cols >= 4 * kWaveMinSeg)))
                            ? 16 : 8;
    const long long unit = wave_ok ? (long long)nw * kSlice : kCH;
    const long long units = (cols + unit - 1) / unit;
    const long long want = (nw == 16) ? cus : 2LL * cus;
    const long long merge_cap = std::max(1LL, (long long)kMergeMax / std::max(1LL, k));
    long long nseg = 1;
    if (rows < want) nseg = (want + rows - 1) / rows;
    nseg = std::min(nseg, std::max(1LL, units / 2));
    if (wave_ok) nseg = std::max(nseg, (cols + kWaveMaxSeg - 1) / kWaveMaxSeg);
    if (knobs().splits > 0) nseg = knobs().splits;
    nseg = std::max(1LL, std::min(nseg, merge_cap));
    const long long min_last = wave_ok ? std::max<long long>(k, unit) : k;
    for (; nseg > 1; --nseg) {
        const long long seg_len = (units + nseg - 1) / nseg * unit;
        const long long n = (cols + seg_len - 1) / seg_len;
        const long long last = cols - (n - 1) * seg_len;
        if (n > 1 && last >= min_last) {
            pl.nseg = (int)n;
            pl.seg_len = (int)seg_len;
            break;
        }
        if (n == 1) break;
    }
    // wave-kernel byte offsets are 32-bit: segments stay below 2^28 elements
    pl.wave = wave_ok && pl.seg_len <= kWaveMaxSeg;
    pl.nw = nw;
    if (knobs().topk_waves == 8 || knobs().topk_waves == 16) pl.nw = (int)knobs().topk_waves;
    pl.ws = pl.nseg > 1 ? (size_t)rows * pl.nseg * k * sizeof(unsigned long long) : 0;
    return pl;
}

int dtype_size(int32_t dtype) {
    switch (dtype) {
        case TPR_UINT8: case TPR_INT8: case TPR_BOOL: return 1;
        case TPR_INT16: case TPR_UINT16: return 2;
        case TPR_INT32: case TPR_UINT32: case TPR_FLOAT32: return 4;
        case TPR_INT64: case TPR_UINT64: case TPR_FLOAT64: return 8;
        default: return 0;
    }
}

// Large k takes the radix-select kernel (any k <= cols, any dtype); so does
// k > 128, k > 64 on rows shorter than the wave kernel's minimum segment
// (8192, or 4096 where wave4 picks 4-wave workgroups), and every input dtype
// but float32, int32 and uint32.
bool radix_route(long long rows, long long cols, long long k, int32_t dtype = TPR_FLOAT32) {
    if (k > kKMax || (dtype != TPR_FLOAT32 && dtype != TPR_INT32 && dtype != TPR_UINT32)) return true;
    if (knobs().topk_radix < 0 || knobs().topk_fallback) return false;
    if (knobs().topk_radix > 0) return true;
    return k > kWaveK || (k > kWave4K && cols < 2 * kWaveMinSeg) ||
           (k > kShortMaxK && cols < kWaveMinSeg && !wave4(rows, cols, k) && !short_exact(rows, cols, k));
}

// Rows the register-resident kernel takes (elements of <= 4 bytes, rows of
// <= 32768); topk_radix = 2 forces the streaming kernel for them.  4-byte
// rows longer than 16384 with k <= 1024 stream instead: there the register
// kernel runs 32 keys per thread, and the streaming kernel's passes (several
// loads in flight) and LDS sort of <= 1024 are faster.  MI355X, us, register
// / streaming: [1024, 24000] k = 300 139 / 102, k = 1000 156 / 142; [1024,
// 32768] k = 1000 165 / 159; [200, 32768] k = 700 44 / 36; but [1024, 16384]
// k = 1000 97 / 106 and [1024, 32768] k = 1500 185 / 226.
bool rsel_route(long long cols, long long k, int32_t dtype) {
    if (dtype_size(dtype) == 4 && cols > 16384 && k <= kKMax) return false;
    return dtype_size(dtype) <= 4 && cols <= kRselMaxCols && knobs().topk_radix != 2;
}

// Longer rows of elements of <= 4 bytes with k <= 1024 and at most kMergeMax
// segment winners, fewer than kSegMaxRows rows: segments of <= 32768 elements
// through k_topk_rsel, one workgroup each, then the merge pass.  Returns the
// segment count, 0 when the streaming kernel takes the row.  Few rows need
// the segments to fill the chip; from 64 rows on the streaming kernel (one
// workgroup per row, several loads in flight) is faster.  MI355X, us,
// segments against streaming: [16, 500000] k = 300 65 / 153; [64, 100000]
// k = 600 69 / 59, k = 1024 78 / 62; [256, 151936] k = 1000 229 / 105;
// [2048, 65536] k = 500 677 / 373.
constexpr long long kSegMaxRows = 64;
int rsel_segments(long long rows, long long cols, long long k, int32_t dtype) {
    if (dtype_size(dtype) > 4 || cols <= kRselMaxCols || k > kKMax || knobs().topk_radix == 2 || rows >= kSegMaxRows)
        return 0;
    const long long nseg = (cols + kRselMaxCols - 1) / kRselMaxCols;
    return nseg * k <= kMergeMax ? (int)nseg : 0;
}

// Workspace of the streaming radix kernel: composites sorted outside LDS (8
// bytes each for elements of at most 4 bytes, 16 for 8-byte elements).
size_t radix_ws(long long rows, long long cols, long long k, int32_t dtype = TPR_FLOAT32) {
    if (rsel_route(cols, k, dtype)) return 0;
    if (const int ns = rsel_segments(rows, cols, k, dtype)) return (size_t)rows * ns * k * sizeof(unsigned long long);
    const long long n2 = pow2_at_least((int)k);
    const bool wide = dtype_size(dtype) == 8;
    const long long lds = wide ? 2048 : kRadixLds;
    return n2 > lds ? (size_t)rows * (size_t)n2 * (wide ? 16 : 8) : 0;
}

// Which kernels serve a top-k call, and how rows are cut into segments.
enum TopkKind {
    TK_SHORT_SMALL = 1,  // k_topk_short on 1- / 2-byte elements
    TK_RSEL = 2,         // k_topk_rsel, one workgroup per row
    TK_RSEL_SEG = 3,     // k_topk_rsel per segment, then k_topk_merge
    TK_RADIX = 4,        // k_topk_radix (streaming)
    TK_SHORT = 5,        // k_topk_short on 4-byte elements
    TK_WAVE = 6,         // k_topk_wave (then k_topk_merge when nseg > 1)
    TK_BLOCK = 7,        // k_topk_block (then k_topk_merge when nseg > 1)
    TK_WAVE8 = 8,        // k_topk_wave on 8-byte rows, then k_topk_radix for the rows it flags
};
struct TopkRoute {
    int kind;
    int nseg;     // segments per row (1: no merge pass)
    int seg_len;  // elements per segment (the last one may be shorter)
    int nw;       // waves per k_topk_wave workgroup
    size_t ws;    // workspace bytes
};

// The planner of tpr_topk / tpr_sample, host only.  `aligned`: the input is
// 16-byte aligned and every row start stays so (rows == 1 or the row stride in
// bytes is a multiple of 16).  Segment contract of TK_RSEL_SEG, TK_WAVE and
// TK_BLOCK with nseg > 1: segment s covers [s * seg_len, min(cols, (s + 1) *
// seg_len)), every one of the nseg segments holds >= k elements (each writes
// exactly k composites for the merge), and nseg * k <= kMergeMax.
TopkRoute route_topk(long long rows, long long cols, long long k, int32_t dtype, long long row_stride, bool aligned) {
    const bool radix = radix_route(rows, cols, k, dtype);
    // (The lane-group kernel addresses up to 4 rows per wave with 32-bit offsets.)
    const bool short_ok = (k <= kShortMaxK || short_exact(rows, cols, k)) && cols <= kShortMaxCols &&
                          3 * row_stride + cols < (1LL << 29);
    const bool short_on = knobs().topk_short >= 0 && knobs().topk_fallback == 0 && knobs().splits <= 0;
    // 1- and 2-byte integer rows the lane-group kernel can hold, 16-byte
    // aligned: that kernel on integer keys (else the register radix select)
    const int eb = dtype_size(dtype);
    if (eb < 4 && short_ok && short_on && knobs().topk_radix <= 0 && aligned)
        return TopkRoute{TK_SHORT_SMALL, 1, (int)cols, 0, 0};
    // Longer 1- and 2-byte rows, 16-byte aligned, k <= 128: the wave kernel on
    // their integer keys wherever it takes a float32 row of the same shape
    if (eb < 4 && aligned && k <= kWaveSmallK && knobs().topk_radix <= 0 && !radix_route(rows, cols, k, TPR_FLOAT32) &&
        !(short_ok && short_on)) {
        const TopkPlan pl = plan_topk(rows, cols, k);
        if (pl.wave) return TopkRoute{TK_WAVE, pl.nseg, pl.seg_len, pl.nw, pl.ws};
    }
    // 8-byte rows (float64, int64, uint64), 16-byte aligned, k <= 128, where the
    // wave kernel takes a float32 row of the same shape in one segment: the
    // filter on the high halves of the keys, the ranking with the low halves;
    // rows it cannot finish (overflowing lists, keys of 0, too many candidates)
    // are flagged in the workspace and finished by the streaming radix select.
    if (eb == 8 && aligned && k <= kWaveSmallK && knobs().topk_radix <= 0 && !radix_route(rows, cols, k, TPR_FLOAT32)) {
        const TopkPlan pl = plan_topk(rows, cols, k);
        if (pl.wave && pl.nseg == 1) return TopkRoute{TK_WAVE8, 1, (int)cols, pl.nw, (size_t)rows * sizeof(int)};
    }
    if (radix && rsel_route(cols, k, dtype)) return TopkRoute{TK_RSEL, 1, (int)cols, 0, 0};
    if (const int ns = radix ? rsel_segments(rows, cols, k, dtype) : 0) {
        const int seg_len = (int)((cols + ns - 1) / ns + 3) & ~3;  // segment starts stay 16-byte aligned
        return TopkRoute{TK_RSEL_SEG, ns, seg_len, 0, radix_ws(rows, cols, k, dtype)};
    }
    if (radix) return TopkRoute{TK_RADIX, 1, (int)cols, 0, radix_ws(rows, cols, k, dtype)};
    // Every row the lane-group kernel can hold goes there: faster than the
    // workgroup kernel ([16384, 3000] k = 64: 124 against 181 us; [8192, 2500]
    // k = 40: 38 against 77 us) and, since its two-key bound, than the 4-wave
    // kernel on rows of 4096 ([16384, 4096] k = 64: 81 against 99 us).
    if (short_ok && short_on) return TopkRoute{TK_SHORT, 1, (int)cols, 0, 0};
    const TopkPlan pl = plan_topk(rows, cols, k);
    return TopkRoute{pl.wave ? TK_WAVE : TK_BLOCK, pl.nseg, pl.seg_len, pl.nw, pl.ws};
}

}  // namespace
}  // namespace tpr

extern "C" {

size_t tpr_topk_workspace_bytes(int32_t dtype, int64_t rows, int64_t cols, int64_t k) {
    if (rows <= 0 || cols <= 0 || k <= 0 || k > cols || cols > 0x7fffffffLL || tpr::dtype_size(dtype) == 0) return 0;
    // the plan can depend on the input's alignment (1- / 2-byte rows take the
    // wave kernel only when 16-byte aligned): enough for either
    return std::max(tpr::route_topk(rows, cols, k, dtype, cols, true).ws,
                    tpr::route_topk(rows, cols, k, dtype, cols, false).ws);
}

}  // extern "C"

namespace tpr {
namespace {
// Short rows: L = lanes per row (>= k, >= cols / 64, >= 16), E4 = float4 per lane.
template <int L, int E4>
void launch_short_le(const TopkArgs& a, bool vec, hipStream_t st) {
    constexpr int RPB = (kShortT / 64) * (64 / L);
    const dim3 grid((unsigned)((a.rows + RPB - 1) / RPB));
    if (a.largest) {
        if (vec) hipLaunchKernelGGL((k_topk_short<L, E4, true, true>), grid, dim3(kShortT), 0, st, a);
        else hipLaunchKernelGGL((k_topk_short<L, E4, false, true>), grid, dim3(kShortT), 0, st, a);
    } else {
        if (vec) hipLaunchKernelGGL((k_topk_short<L, E4, true, false>), grid, dim3(kShortT), 0, st, a);
        else hipLaunchKernelGGL((k_topk_short<L, E4, false, false>), grid, dim3(kShortT), 0, st, a);
    }
}

template <int L>
void launch_short_l(const TopkArgs& a, bool vec, hipStream_t st) {
    const int e4 = (a.cols + 4 * L - 1) / (4 * L);
    if (e4 <= 1) launch_short_le<L, 1>(a, vec, st);
    else if (e4 <= 2) launch_short_le<L, 2>(a, vec, st);
    else if (e4 <= 4) launch_short_le<L, 4>(a, vec, st);
    else if (e4 <= 8) launch_short_le<L, 8>(a, vec, st);
    else launch_short_le<L, 16>(a, vec, st);
}

// 1- and 2-byte integer rows (16-byte aligned): E4 vectors of 16 / EB
// elements per lane.
template <int L, int E4, int EB>
void launch_short_small_le(const TopkArgs& a, hipStream_t st) {
    constexpr int RPB = (kShortT / 64) * (64 / L);
    const dim3 grid((unsigned)((a.rows + RPB - 1) / RPB));
    if (a.largest) hipLaunchKernelGGL((k_topk_short<L, E4, true, true, EB>), grid, dim3(kShortT), 0, st, a);
    else hipLaunchKernelGGL((k_topk_short<L, E4, true, false, EB>), grid, dim3(kShortT), 0, st, a);
}

template <int L, int EB>
int launch_short_small_l(const TopkArgs& a, hipStream_t st) {
    constexpr int per = 16 / EB * L;  // elements of one vector round of the L lanes
    const int e4 = (a.cols + per - 1) / per;  // <= 4 * EB (cols <= 4096, L >= cols / 16 below 64 lanes)
    if (e4 <= 1) launch_short_small_le<L, 1, EB>(a, st);
    else if (e4 <= 2) launch_short_small_le<L, 2, EB>(a, st);
    else if (e4 <= 4) launch_short_small_le<L, 4, EB>(a, st);
    else if (EB == 2 && e4 <= 8) launch_short_small_le<L, EB == 2 ? 8 : 4, EB>(a, st);
    else return fail(TPR_ERR_INVALID_ARG, "tpr_topk: row too long for the lane-group kernel on 1- / 2-byte elements");
    return TPR_OK;
}

int launch_short_small(const TopkArgs& a, int eb, hipStream_t st) {
    int L = 16;  // as launch_short: L >= 2k, and L >= cols / 16 up to 64 lanes
    while (L < 64 && (L < 2 * a.k || L * 16 < a.cols)) L *= 2;
    int rc;
    if (eb == 1) {
        if (L == 16) rc = launch_short_small_l<16, 1>(a, st);
        else if (L == 32) rc = launch_short_small_l<32, 1>(a, st);
        else rc = launch_short_small_l<64, 1>(a, st);
    } else {
        if (L == 16) rc = launch_short_small_l<16, 2>(a, st);
        else if (L == 32) rc = launch_short_small_l<32, 2>(a, st);
        else rc = launch_short_small_l<64, 2>(a, st);
    }
    return rc != TPR_OK ? rc : check_launch("k_topk_short");
}

int launch_short(const TopkArgs& a, bool vec, hipStream_t st) {
    // L >= 2k where possible: the bound is then the k-th largest of at least
    // 2k lane maxima, well above their minimum, so fewer candidates reach the
    // ranking; and L >= cols / 16 where possible: at most 16 elements per lane
    // keep the registers (and the occupancy) low.  Measured on MI355X (us):
    // [16384, 1024] k = 32: L = 32 41.7, L = 64 18.8; k = 8: L = 16 24.7,
    // L = 64 15.3; [65536, 256] k = 8: L = 16 19.1, L = 32 21.9.
    int L = 16;
    while (L < 64 && (L < 2 * a.k || L * 16 < a.cols)) L *= 2;
    if (a.sample) L = 64;  // the draw runs on one wave per row
    if (L == 16) launch_short_l<16>(a, vec, st);
    else if (L == 32) launch_short_l<32>(a, vec, st);
    else launch_short_l<64>(a, vec, st);
    return check_launch("k_topk_short");
}

// Sort of n = pow2(max(k, 64)) composites, P = 4 per thread where n allows
// (fewer waves for small n, more composites per thread when n > 4 * NT).
// Measured on MI355X ([4096, 2048] k = 1000: P = 4 on 4 waves 73 us, P = 16
// on one wave 108 us; [4096, 2048] k = 200: P = 4 on one wave 43 us, P = 1 on
// 4 waves 51 us).
template <int NT, int EPT>
int launch_rsel_p(const TopkArgs& a, int32_t dtype, hipStream_t st) {
    const int n = std::max(64, pow2_at_least(a.k));
    int P = std::min(n / 64, std::max(4, n / NT));
    const long long pv = knobs().topk_variant;  // debug: composites per thread of the sort
    if (pv >= 1 && pv <= 32 && (pv & (pv - 1)) == 0 && n / pv >= 64 && n / pv <= NT) P = (int)pv;
    const dim3 g((unsigned)(a.rows * a.nseg)), b(NT);
    if (P == 1) hipLaunchKernelGGL((k_topk_rsel<NT, EPT, 1>), g, b, 0, st, a, (int)dtype, n);
    else if (P == 2) hipLaunchKernelGGL((k_topk_rsel<NT, EPT, 2>), g, b, 0, st, a, (int)dtype, n);
    else if (P == 4) hipLaunchKernelGGL((k_topk_rsel<NT, EPT, 4>), g, b, 0, st, a, (int)dtype, n);
    else if (P == 8) hipLaunchKernelGGL((k_topk_rsel<NT, EPT, 8>), g, b, 0, st, a, (int)dtype, n);
    else if (P == 16) hipLaunchKernelGGL((k_topk_rsel<NT, EPT, 16>), g, b, 0, st, a, (int)dtype, n);
    else if constexpr (NT == 1024 && EPT == 32) hipLaunchKernelGGL((k_topk_rsel<NT, EPT, 32>), g, b, 0, st, a, (int)dtype, n);
    else return fail(TPR_ERR_INVALID_ARG, "tpr_topk: sort size beyond the workgroup");  // n <= NT * EPT
    return check_launch("k_topk_rsel");
}

// Workgroup size and keys per thread by row length: NT * EPT >= cols, so
// pow2(k) / NT <= EPT.
int launch_rsel(const TopkArgs& a, int32_t dtype, hipStream_t st) {
    const int c = a.nseg > 1 ? a.seg_len : a.cols;  // elements per workgroup
    if (c <= 1024) return launch_rsel_p<256, 4>(a, dtype, st);
    if (c <= 2048) return launch_rsel_p<256, 8>(a, dtype, st);
    if (c <= 4096) return launch_rsel_p<256, 16>(a, dtype, st);
    if (c <= 8192) return launch_rsel_p<512, 16>(a, dtype, st);
    if (c <= 16384) return launch_rsel_p<1024, 16>(a, dtype, st);
    return launch_rsel_p<1024, 32>(a, dtype, st);
}

// tpr_topk, or (smp != nullptr) tpr_sample: the same selection with the draw
// in the final phase.
int topk_launch(const void* in, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride, int64_t k,
                int32_t largest, void* out_values, void* out_indices, void* workspace, size_t workspace_bytes,
                void* stream, const TopkArgs* smp) {
    if (dtype_size(dtype) == 0) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_topk: unknown dtype");
    if (smp && dtype != TPR_FLOAT32) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_sample: float32 logits only");
    if (rows < 0 || cols < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: negative shape");
    if (k < 0 || k > cols) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: selected index k out of range");
    if (rows == 0 || k == 0) return TPR_OK;
    if (cols > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: rows longer than 2^31-1");
    if (!in || (!smp && (!out_values || !out_indices))) return fail(TPR_ERR_INVALID_ARG, "tpr_topk: null pointer");
    if (rows > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: more than 2^31-1 rows");
    const bool aligned = ((reinterpret_cast<uintptr_t>(in) & 15u) == 0) &&
                         (rows == 1 || (row_stride * dtype_size(dtype)) % 16 == 0);
    const TopkRoute rt = route_topk(rows, cols, k, dtype, row_stride, aligned);
    if (rows * (long long)rt.nseg > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_topk: grid too large");
    if (rt.ws > 0 && (workspace == nullptr || workspace_bytes < rt.ws))
        return fail(TPR_ERR_WORKSPACE, "tpr_topk: workspace too small (need " + std::to_string(rt.ws) + " bytes)");
    TopkArgs a;
    a.in = static_cast<const float*>(in);
    a.rows = rows;
    a.cols = (int)cols;
    a.row_stride = row_stride;
    a.k = (int)k;
    a.largest = largest ? 1 : 0;
    a.ikind = (dtype == TPR_INT64 || dtype == TPR_INT32 || dtype == TPR_INT16 || dtype == TPR_INT8) ? 1
              : (dtype == TPR_UINT64 || dtype == TPR_UINT32 || dtype == TPR_UINT16 || dtype == TPR_UINT8 ||
                 dtype == TPR_BOOL) ? 2 : 0;
    a.force_fallback = knobs().topk_fallback ? 1 : 0;
    a.nseg = rt.nseg;
    a.seg_len = rt.seg_len;
    a.part = static_cast<unsigned long long*>(workspace);
    a.out_v = static_cast<float*>(out_values);
    a.out_i = static_cast<long long*>(out_indices);
    a.sample = smp ? 1 : 0;
    a.dyn = knobs().topk_dyn >= 0 ? 1 : 0;
    a.flags = nullptr;
    a.temperature = smp ? smp->temperature : 0.0f;
    a.top_p = smp ? smp->top_p : 1.0f;
    a.u = smp ? smp->u : nullptr;
    a.ids = smp ? smp->ids : nullptr;
    const bool vec = ((reinterpret_cast<uintptr_t>(in) & 15u) == 0) && (rows == 1 || row_stride % 4 == 0);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (rt.kind == TK_SHORT_SMALL) return launch_short_small(a, dtype_size(dtype), st);
    if (rt.kind == TK_RSEL) return launch_rsel(a, dtype, st);
    if (rt.kind == TK_RSEL_SEG) {
        const int rc = launch_rsel(a, dtype, st);
        if (rc != TPR_OK) return rc;
        hipLaunchKernelGGL(k_topk_merge, dim3((unsigned)rows), dim3(kMergeT), 0, st, a, (int)dtype);
        return check_launch("k_topk_merge");
    }
    auto launch_radix = [&]() {
        // few rows: 1024 threads per row (the passes over the row are latency bound)
        const int nt = rows < 2LL * device_info().cus ? 1024 : kRadixT;
#define TPR_RADIX(T)                                                                                  \
    {                                                                                                 \
        const bool gs = pow2_at_least((int)k) > radix_lds_count<T>();                                 \
        const dim3 g((unsigned)rows);                                                                 \
        if (nt == 1024) {                                                                             \
            if (gs) hipLaunchKernelGGL((k_topk_radix<T, 1024, true, true>), g, dim3(1024), 0, st, a, workspace); \
            else if (rows > device_info().cus)                                                        \
                hipLaunchKernelGGL((k_topk_radix<T, 1024, false, false>), g, dim3(1024), 0, st, a, workspace); \
            else hipLaunchKernelGGL((k_topk_radix<T, 1024, false, true>), g, dim3(1024), 0, st, a, workspace); \
        } else {                                                                                      \
            if (gs) hipLaunchKernelGGL((k_topk_radix<T, kRadixT, true, true>), g, dim3(kRadixT), 0, st, a, workspace); \
            else hipLaunchKernelGGL((k_topk_radix<T, kRadixT, false, true>), g, dim3(kRadixT), 0, st, a, workspace); \
        }                                                                                             \
    }
        switch (dtype) {
            case TPR_FLOAT32: TPR_RADIX(float) break;
            case TPR_FLOAT64: TPR_RADIX(double) break;
            case TPR_INT8: TPR_RADIX(signed char) break;
            case TPR_INT16: TPR_RADIX(short) break;
            case TPR_INT32: TPR_RADIX(int) break;
            case TPR_INT64: TPR_RADIX(long long) break;
            case TPR_UINT16: TPR_RADIX(unsigned short) break;
            case TPR_UINT32: TPR_RADIX(unsigned int) break;
            case TPR_UINT64: TPR_RADIX(unsigned long long) break;
            default: TPR_RADIX(unsigned char) break;  // UINT8, BOOL
        }
#undef TPR_RADIX
        return check_launch("k_topk_radix");
    };
    if (rt.kind == TK_RADIX) return launch_radix();
    if (rt.kind == TK_WAVE8) {
        a.flags = static_cast<int*>(workspace);
        const dim3 blk(rt.nw * 64);
        const dim3 grid((unsigned)rows);
        if (rt.nw == 16) hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 1, 16, kWB, 8>), grid, blk, 0, st, a);
        else if (rt.nw == 4) hipLaunchKernelGGL((k_topk_wave<true, 4, 8, 0, 4, kWB, 8>), grid, blk, 0, st, a);
        else hipLaunchKernelGGL((k_topk_wave<true, 4, 8, 0, 8, kWB, 8>), grid, blk, 0, st, a);
        const int rc = check_launch("k_topk_wave");
        if (rc != TPR_OK) return rc;
        return launch_radix();  // runs only the flagged rows
    }
    if (rt.kind == TK_SHORT) return launch_short(a, vec, st);
    const TopkPlan pl{rt.nseg, rt.seg_len, rt.kind == TK_WAVE, rt.nw, rt.ws};
    if (rt.kind == TK_WAVE && dtype_size(dtype) < 4) {
        // 1- / 2-byte rows (16-byte aligned, k <= 128): one or two 16-byte
        // vectors per lane hold a 1024-element slice
        const long long grid = rows * pl.nseg;
        const dim3 blk(pl.nw * 64);
#define TPR_WAVE_EB(EBV)                                                                                          \
        if (pl.nw == 16) hipLaunchKernelGGL((k_topk_wave<true, EBV, 4, 1, 16, kWB, EBV>), dim3(grid), blk, 0, st, a); \
        else if (pl.nw == 4) hipLaunchKernelGGL((k_topk_wave<true, EBV, 8, 0, 4, kWB, EBV>), dim3(grid), blk, 0, st, a); \
        else hipLaunchKernelGGL((k_topk_wave<true, EBV, 8, 0, 8, kWB, EBV>), dim3(grid), blk, 0, st, a);
        if (dtype_size(dtype) == 1) {
            TPR_WAVE_EB(1)
        } else {
            TPR_WAVE_EB(2)
        }
#undef TPR_WAVE_EB
        const int rc = check_launch("k_topk_wave");
        if (rc != TPR_OK || pl.nseg == 1) return rc;
        hipLaunchKernelGGL(k_topk_merge, dim3(rows), dim3(kMergeT), 0, st, a, (int)dtype);
        return check_launch("k_topk_merge");
    }
    const long long grid = rows * pl.nseg;
    if (pl.wave) {
        // 512-thread workgroups (many rows): 8 waves/SIMD without prefetch.
        // 1024-thread workgroups (few rows): one slice prefetched per wave.
        // (Measured on MI355X at [1024, 32768] k=64 and [256, 151936] k=50.)
        long long var = knobs().topk_variant;
        // 16 waves: one workgroup per CU (<= 1 row per CU) prefetches a slice
        // per wave; 1..2 rows per CU run two workgroups per CU, 8 waves/SIMD,
        // no prefetch (MI355X, us: [384, 65536] k = 100 33.5 -> 27.8,
        // [300, 100000] k = 50 38.8 -> 34.8, [512, 65536] k = 64 31.4 -> 28.1
        // against the 1-per-CU kernel or 8-wave workgroups)
        if (var == 0) var = pl.nw == 16 ? (rows > device_info().cus ? 5 : 2) : (pl.nseg == 1 ? 1 : 2);
        const dim3 blk(pl.nw * 64);
        if (k > 128) {
            // k of 129..256: 512-entry wave lists (twice the LDS: at most two
            // 8-wave workgroups per CU: 4 waves per SIMD, a one-slice prefetch)
            if (pl.nw == 16) {
                if (!vec) hipLaunchKernelGGL((k_topk_wave<false, 4, 4, 1, 16, 512>), dim3(grid), blk, 0, st, a);
                else hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 1, 16, 512>), dim3(grid), blk, 0, st, a);
            } else if (pl.nw == 4) {
                if (!vec) hipLaunchKernelGGL((k_topk_wave<false, 4, 4, 1, 4, 512>), dim3(grid), blk, 0, st, a);
                else hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 1, 4, 512>), dim3(grid), blk, 0, st, a);
            } else {
                if (!vec) hipLaunchKernelGGL((k_topk_wave<false, 4, 4, 1, 8, 512>), dim3(grid), blk, 0, st, a);
                else hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 1, 8, 512>), dim3(grid), blk, 0, st, a);
            }
        } else if (pl.nw == 16) {
            if (!vec) hipLaunchKernelGGL((k_topk_wave<false, 4, 4, 1, 16>), dim3(grid), blk, 0, st, a);
            else if (var == 1) hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 0, 16>), dim3(grid), blk, 0, st, a);
            else if (var == 3) hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 2, 16>), dim3(grid), blk, 0, st, a);
            else if (var == 5) hipLaunchKernelGGL((k_topk_wave<true, 4, 8, 0, 16>), dim3(grid), blk, 0, st, a);
            else hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 1, 16>), dim3(grid), blk, 0, st, a);
        } else if (pl.nw == 4) {
            if (!vec) hipLaunchKernelGGL((k_topk_wave<false, 4, 8, 0, 4>), dim3(grid), blk, 0, st, a);
            else if (var == 2) hipLaunchKernelGGL((k_topk_wave<true, 4, 6, 1, 4>), dim3(grid), blk, 0, st, a);
            else hipLaunchKernelGGL((k_topk_wave<true, 4, 8, 0, 4>), dim3(grid), blk, 0, st, a);
        } else {
            if (!vec) hipLaunchKernelGGL((k_topk_wave<false, 4, 6, 1, 8>), dim3(grid), blk, 0, st, a);
            else if (var == 1) hipLaunchKernelGGL((k_topk_wave<true, 4, 8, 0, 8>), dim3(grid), blk, 0, st, a);
            else if (var == 3) hipLaunchKernelGGL((k_topk_wave<true, 4, 4, 2, 8>), dim3(grid), blk, 0, st, a);
            else hipLaunchKernelGGL((k_topk_wave<true, 4, 6, 1, 8>), dim3(grid), blk, 0, st, a);
        }
    } else {
        if (vec) hipLaunchKernelGGL((k_topk_block<true>), dim3(grid), dim3(kT), 0, st, a);
        else hipLaunchKernelGGL((k_topk_block<false>), dim3(grid), dim3(kT), 0, st, a);
    }
    int rc = check_launch("k_topk_seg");
    if (rc != TPR_OK || pl.nseg == 1) return rc;
    hipLaunchKernelGGL(k_topk_merge, dim3(rows), dim3(kMergeT), 0, st, a, (int)dtype);
    return check_launch("k_topk_merge");
}
}  // namespace
}  // namespace tpr

extern "C" {

#ifdef TPR_DEBUG_KNOBS
// Test builds only: reads a device-side check counter and clears it.
int tpr_debug_get(const char* key, int64_t* value) {
    if (!key || !value) return tpr::fail(TPR_ERR_INVALID_ARG, "tpr_debug_get: null argument");
    if (std::strcmp(key, "topk_merge_clamped") != 0)
        return tpr::fail(TPR_ERR_INVALID_ARG, std::string("tpr_debug_get: unknown key ") + key);
    unsigned int v = 0;
    const unsigned int zero = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(topk_merge_clamped), sizeof(v)) != hipSuccess ||
        hipMemcpyToSymbol(HIP_SYMBOL(topk_merge_clamped), &zero, sizeof(zero)) != hipSuccess)
        return tpr::fail(TPR_ERR_HIP, "tpr_debug_get: device counter not readable");
    *value = (int64_t)v;
    return TPR_OK;
}
#endif

int tpr_topk_plan(int32_t dtype, int64_t rows, int64_t cols, int64_t k, int64_t row_stride, int32_t aligned,
                  int64_t* out) {
    if (!out) return tpr::fail(TPR_ERR_INVALID_ARG, "tpr_topk_plan: null output");
    if (tpr::dtype_size(dtype) == 0) return tpr::fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_topk_plan: unknown dtype");
    if (rows <= 0 || cols <= 0 || k <= 0 || k > cols || cols > 0x7fffffffLL || rows > 0x7fffffffLL)
        return tpr::fail(TPR_ERR_INVALID_ARG, "tpr_topk_plan: no kernel runs for this shape");
    const tpr::TopkRoute rt = tpr::route_topk(rows, cols, k, dtype, row_stride, aligned != 0);
    out[0] = rt.kind;
    out[1] = rt.nseg;
    out[2] = rt.seg_len;
    out[3] = rt.nw;
    out[4] = (int64_t)rt.ws;
    return TPR_OK;
}

int tpr_topk(const void* in, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride,
             int64_t k, int32_t largest, int32_t sorted, void* out_values, void* out_indices,
             void* workspace, size_t workspace_bytes, void* stream) {
    (void)sorted;
    return tpr::topk_launch(in, dtype, rows, cols, row_stride, k, largest, out_values, out_indices, workspace,
                            workspace_bytes, stream, nullptr);
}

size_t tpr_sample_workspace_bytes(int32_t dtype, int64_t rows, int64_t cols, int64_t k) {
    if (dtype == TPR_FLOAT32 && k > tpr::kKMax && k <= cols && rows > 0 && cols <= 0x7fffffffLL)
        return tpr::sample_sorted_layout(rows, cols, k).total;
    return tpr_topk_workspace_bytes(dtype, rows, cols, k);
}

int tpr_sample(const void* logits, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride, int64_t k,
               float temperature, float top_p, const float* uniforms, int64_t* out_ids, void* workspace,
               size_t workspace_bytes, void* stream) {
    using namespace tpr;
    if (dtype != TPR_FLOAT32) return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_sample: float32 logits only");
    if (rows < 0 || cols < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: negative shape");
    if (k < 1 || k > cols) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: k must be in [1, cols]");
    if (!(top_p > 0.0f) || top_p > 1.0f) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: top_p must be in (0, 1]");
    if (rows == 0) return TPR_OK;
    if (!logits || !uniforms || !out_ids) return fail(TPR_ERR_INVALID_ARG, "tpr_sample: null pointer");
    TopkArgs smp{};
    smp.temperature = temperature;
    smp.top_p = top_p;
    smp.u = uniforms;
    smp.ids = reinterpret_cast<long long*>(out_ids);
    if (k > kKMax) {
        // the sorted top k through tpr_topk into the workspace, then the draw
        // by one workgroup per row
        if (cols > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_sample: rows longer than 2^31-1");
        if (rows > 0x7fffffffLL) return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_sample: more than 2^31-1 rows");
        const SampleSortedLayout l = sample_sorted_layout(rows, cols, k);
        if (workspace == nullptr || workspace_bytes < l.total)
            return fail(TPR_ERR_WORKSPACE, "tpr_sample: workspace too small (need " + std::to_string(l.total) +
                                               " bytes)");
        char* ws = static_cast<char*>(workspace);
        float* vals = reinterpret_cast<float*>(ws + l.vals_off);
        long long* idx = reinterpret_cast<long long*>(ws + l.idx_off);
        const int rc = topk_launch(logits, dtype, rows, cols, row_stride, k, 1, vals, idx,
                                   l.topk_ws ? workspace : nullptr, l.topk_ws, stream, nullptr);
        if (rc != TPR_OK) return rc;
        hipLaunchKernelGGL((k_sample_sorted<kDrawNT>), dim3((unsigned)rows), dim3(kDrawNT), 0,
                           static_cast<hipStream_t>(stream), vals, idx, (int)k, temperature, top_p, uniforms, smp.ids);
        return check_launch("tpr_sample");
    }
    return topk_launch(logits, dtype, rows, cols, row_stride, k, 1, nullptr, nullptr, workspace, workspace_bytes,
                       stream, &smp);
}

}  // extern "C"
