// gfx950 reduction kernels (sum / mean / amax / amin / argmax / argmin / var /
// std) over arbitrary strided float32 views, and the host planner behind
// tpr_reduce().
//
// Semantics follow TensorPlay's CPU path
// (/root/reference/p10/src/backend/cpu/ReductionKernels.cpp):
//  * max/min keep the first occurrence under a strict compare, so NaN never
//    wins and ties go to the lowest index (:242, :294, :694, :732);
//  * sums accumulate in fp64 (the reference's full sum does, :30/:94; its dim
//    sum accumulates in fp32, :168, which is less accurate -- the result here is
//    closer to the exact sum than the reference's);
//  * var/std use a Welford/Chan merge of per-thread shifted sums instead of the
//    reference's five-pass mean/sub/mul/sum/div composite (:817-855).
//
// Layout classes after the host canonicalises the view (drop size-1 dims, merge
// adjacent dims that are contiguous with each other and share reduce status):
//   rows    [K, R]     R contiguous          -> k_rows   (128-bit loads along rows)
//   cols    [K1, R, K2] K2 contiguous         -> k_cols   (128-bit loads along K2)
//   general anything else                    -> k_general (index arithmetic)
// Any of them may split the reduced extent over S workgroups; the S partial
// states then go through k_finalize (no atomics; fixed combine order, so results
// are deterministic run to run).

#include <hip/hip_runtime.h>

#include <type_traits>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace tpr {
namespace {

constexpr long long kSentinel = 0x7fffffffffffffffLL;
constexpr int kBlock = 256;
// Ticket counters of split plans that finish in their own launch: one block
// of kTicketsPerStream counters for each of up to kTicketStreams streams.
constexpr int kTicketStreams = 64;
constexpr int kTicketsPerStream = 1024;

// ---------------------------------------------------------------------------
// Operator policies.  Acc = per-thread running state, State = mergeable state.
// ---------------------------------------------------------------------------
struct SumS { double s; };

struct SumOp {
    static constexpr bool kIndexed = false;
    using Acc = double;
    using State = SumS;
    using Wide = SumOp;
    __device__ static Acc init() { return 0.0; }
    template <class I>
    __device__ static void acc(Acc& a, float x, I, float) { a += (double)x; }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {0.0}; }
    __device__ static State comb(State a, State b) { return {a.s + b.s}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.s, m, kWave)}; }
};

// Product in fp64 (the reference multiplies in the output dtype, :424-427).
struct ProdOp {
    static constexpr bool kIndexed = false;
    using Acc = double;
    using State = SumS;
    using Wide = ProdOp;
    __device__ static Acc init() { return 1.0; }
    template <class I>
    __device__ static void acc(Acc& a, float x, I, float) { a *= (double)x; }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {1.0}; }
    __device__ static State comb(State a, State b) { return {a.s * b.s}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.s, m, kWave)}; }
};

// Sum of |x|^p in fp64 (norm_kernel's abs().pow(p).sum(), :858-872).  KIND 1:
// |x|, KIND 2: x*x (exact in fp64), KIND 0: powf(|x|, p) for any other p.
template <int KIND>
struct NormOp {
    static constexpr bool kIndexed = false;
    using Acc = double;
    using State = SumS;
    using Wide = NormOp;
    __device__ static Acc init() { return 0.0; }
    template <class I>
    __device__ static void acc(Acc& a, float x, I, float p) {
        if constexpr (KIND == 1) a += (double)fabsf(x);
        else if constexpr (KIND == 2) a = fma((double)x, (double)x, a);
        else a += (double)powf(fabsf(x), p);
    }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {0.0}; }
    __device__ static State comb(State a, State b) { return {a.s + b.s}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.s, m, kWave)}; }
};

// all / any: an element is true when x != 0 (NaN is true, -0.0 is false), as
// static_cast<bool> in all_kernel/any_kernel (:517-563).
struct BoolS { int b; };
template <bool ANY>
struct BoolOp {
    static constexpr bool kIndexed = false;
    using Acc = int;
    using State = BoolS;
    using Wide = BoolOp;
    __device__ static Acc init() { return ANY ? 0 : 1; }
    template <class I>
    __device__ static void acc(Acc& a, float x, I, float) {
        if constexpr (ANY) a |= (x != 0.0f) ? 1 : 0;
        else a &= (x != 0.0f) ? 1 : 0;
    }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {ANY ? 0 : 1}; }
    __device__ static State comb(State a, State b) { return {ANY ? (a.b | b.b) : (a.b & b.b)}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.b, m, kWave)}; }
};

struct ArgS { float v; long long i; };

// Strict compare in index order; lowest index wins equal values (-0.0 == +0.0).
// IdxT is the index type of the per-thread accumulator: int inside the row and
// column kernels (extent < 2^31, checked by the planner; 32-bit selects are
// cheaper per element), long long in the general kernel.  States always carry
// a 64-bit index.
// ABS compares |x| (norm with p = +-inf: max/min of |x|).
template <bool IS_MAX, class IdxT = int, bool ABS = false>
struct ArgOp {
    static constexpr bool kIndexed = true;
    static constexpr IdxT kNone = (IdxT)(sizeof(IdxT) == 4 ? 0x7fffffff : kSentinel);
    struct Acc { float v; IdxT i; };
    using State = ArgS;
    using Wide = ArgOp<IS_MAX, long long, ABS>;
    __device__ static Acc init() { return {IS_MAX ? -INFINITY : INFINITY, kNone}; }
    template <class I>
    __device__ static void acc(Acc& a, float x, I i, float) {
        if constexpr (ABS) x = fabsf(x);
        bool t = IS_MAX ? (x > a.v) : (x < a.v);
        a.v = t ? x : a.v;
        a.i = t ? (IdxT)i : a.i;
    }
    // state of an accumulator whose stored index is idx: element index = idx * mul + add
    __device__ static State state_scaled(Acc a, long long mul, long long add) {
        return {a.v, a.i == kNone ? kSentinel : (long long)a.i * mul + add};
    }
    __device__ static State state(Acc a) { return state_scaled(a, 1, 0); }
    __device__ static State identity() { return {IS_MAX ? -INFINITY : INFINITY, kSentinel}; }
    __device__ static State comb(State a, State b) {
        bool t = IS_MAX ? (b.v > a.v) : (b.v < a.v);
        t = t || (b.v == a.v && b.i < a.i);
        return t ? b : a;
    }
    __device__ static State shfl(State s, int m) {
        return {__shfl_xor(s.v, m, kWave), __shfl_xor(s.i, m, kWave)};
    }
};

struct WelS { double n, mean, m2; };
// Per-thread shifted sums: d = x - K with K the thread's first element, so the
// running sums stay small and M2 = S2 - S1^2/n loses nothing to cancellation.
struct WelAcc { float k; int n; double s1, s2; };

struct WelfordOp {
    static constexpr bool kIndexed = false;
    using Acc = WelAcc;
    using State = WelS;
    using Wide = WelfordOp;
    __device__ static Acc init() { return {0.0f, 0, 0.0, 0.0}; }
    template <class I>
    __device__ static void acc(Acc& a, float x, I, float) {
        a.k = (a.n == 0) ? x : a.k;
        double d = (double)x - (double)a.k;
        a.s1 += d;
        a.s2 = fma(d, d, a.s2);
        a.n += 1;
    }
    __device__ static State state(Acc a) {
        if (a.n == 0) return {0.0, 0.0, 0.0};
        double n = (double)a.n;
        double m = a.s1 / n;
        return {n, (double)a.k + m, fmax(0.0, a.s2 - a.s1 * m)};
    }
    __device__ static State identity() { return {0.0, 0.0, 0.0}; }
    // Chan et al. pairwise merge.
    __device__ static State comb(State a, State b) {
        if (a.n == 0.0) return b;
        if (b.n == 0.0) return a;
        const double n = a.n + b.n;
        const double d = b.mean - a.mean;
        // equal counts (every lane of a full row) need no divide: b.n / n == 1/2
        const double f = (a.n == b.n) ? 0.5 : b.n / n;
        return {n, a.mean + d * f, a.m2 + b.m2 + d * d * a.n * f};
    }
    __device__ static State shfl(State s, int m) {
        return {__shfl_xor(s.n, m, kWave), __shfl_xor(s.mean, m, kWave),
                __shfl_xor(s.m2, m, kWave)};
    }
};

// ---------------------------------------------------------------------------
// Finalisation: state -> output element.
// ---------------------------------------------------------------------------
struct Fin {
    int op;         // tpr_reduce_op
    int out_f64;    // SUM/MEAN write double
    double count;   // divisor count (reference semantics, duplicates included)
    double corr;    // VAR/STD correction
    float p;        // NORM exponent (passed to every op's acc; only NormOp reads it)
    int out_esize;  // bytes per output element (integer amax/amin write the input dtype)
    int out_umap;   // UInt64 amax/amin: undo the key's top-bit flip
    double inv_p;   // NORM: 1/p
};

__device__ __forceinline__ void fin_write(const SumS& s, const Fin& f, void* out, long long o) {
    double v = s.s;
    if (f.op == TPR_MEAN) v = v / f.count;
    if (f.op == TPR_NORM) v = (f.inv_p == 0.5) ? sqrt(v) : (f.inv_p == 1.0 ? v : pow(v, f.inv_p));
    if (f.out_f64) ((double*)out)[o] = v;
    else ((float*)out)[o] = (float)v;
}

__device__ __forceinline__ void fin_write(const ArgS& s, const Fin& f, void* out, long long o) {
    if (f.op == TPR_AMAX || f.op == TPR_AMIN || f.op == TPR_NORM) ((float*)out)[o] = s.v;
    else ((long long*)out)[o] = (s.i == kSentinel) ? 0 : s.i;
}

__device__ __forceinline__ void fin_write(const BoolS& s, const Fin&, void* out, long long o) {
    ((unsigned char*)out)[o] = (unsigned char)s.b;
}

__device__ __forceinline__ void fin_write(const WelS& s, const Fin& f, void* out, long long o) {
    // The reference centres on sum/count where count multiplies every listed dim
    // (duplicates included); with count == n this is the plain mean.  Expanding
    // sum((x - m')^2) = M2 + n (mean - m')^2 reproduces that centring exactly.
    double mp = s.mean * (s.n / f.count);
    double dm = s.mean - mp;
    double m2 = s.m2 + s.n * dm * dm;
    double div = fmax(0.0, f.count - f.corr);
    if (f.out_f64) {  // float64 input: var / std in double
        const double v = m2 / div;
        ((double*)out)[o] = (f.op == TPR_STD) ? sqrt(v) : v;
        return;
    }
    float var = (float)(m2 / div);
    ((float*)out)[o] = (f.op == TPR_STD) ? sqrtf(var) : var;
}

// ---------------------------------------------------------------------------
// Workgroup combine helpers.
// ---------------------------------------------------------------------------
template <class Op, int WIDTH>
__device__ __forceinline__ typename Op::State group_reduce_sub_wave(typename Op::State st) {
#pragma unroll
    for (int m = 1; m < WIDTH; m <<= 1) st = Op::comb(st, Op::shfl(st, m));
    return st;
}

template <class Op>
__device__ __forceinline__ typename Op::State block_reduce(typename Op::State st) {
    using State = typename Op::State;
    __shared__ State sh[kBlock / kWave];
    st = group_reduce_sub_wave<Op, kWave>(st);
    const int w = threadIdx.x / kWave;
    if (__lane_id() == 0) sh[w] = st;
    __syncthreads();
    State r = sh[0];
#pragma unroll
    for (int i = 1; i < kBlock / kWave; ++i) r = Op::comb(r, sh[i]);
    return r;  // valid in every thread
}

template <class Op, int BLK>
__device__ __forceinline__ typename Op::State block_reduce_n(typename Op::State st) {
    using State = typename Op::State;
    __shared__ State sh[BLK / kWave];
    st = group_reduce_sub_wave<Op, kWave>(st);
    if (__lane_id() == 0) sh[threadIdx.x / kWave] = st;
    __syncthreads();
    State r = sh[0];
#pragma unroll
    for (int i = 1; i < BLK / kWave; ++i) r = Op::comb(r, sh[i]);
    return r;  // valid in every thread
}

// ---------------------------------------------------------------------------
// Split plans finished inside the same launch.  Every workgroup of a split
// output stores its partial state, then draws a ticket from the output's
// counter; the workgroup that draws ticket S-1 combines the S partials in
// split order (as k_finalize_block does: thread t takes partials t, t+BLK, ...,
// then the fixed workgroup tree) and writes the output, then sets the counter
// back to 0 for the next launch.  The state words are written with
// device-scope atomic exchanges and read back with device-scope atomic ors of
// 0, and the ticket is a device-scope atomic add: read-modify-write atomics are
// performed at the device's point of coherence, so no L2 writeback or
// invalidate is needed (such fences cost microseconds per workgroup), and the
// wait for the exchanges to complete (vmcnt(0)) orders them before the ticket.
// ---------------------------------------------------------------------------
template <class State>
__device__ __forceinline__ void publish_state(State* dst, const State& v) {
    static_assert(sizeof(State) % 4 == 0, "states are whole 32-bit words");
    unsigned w[sizeof(State) / 4];
    __builtin_memcpy(w, &v, sizeof(State));
    unsigned* d = reinterpret_cast<unsigned*>(dst);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(State) / 4); ++i)
        __hip_atomic_exchange(d + i, w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class State>
__device__ __forceinline__ State fetch_state(State* src) {
    unsigned w[sizeof(State) / 4];
    unsigned* p = reinterpret_cast<unsigned*>(src);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(State) / 4); ++i)
        w[i] = __hip_atomic_fetch_or(p + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    State v;
    __builtin_memcpy(&v, w, sizeof(State));
    return v;
}

// st: the workgroup's partial state of output o (valid in thread 0); partial s
// of output o lives at part[s * stride + o].
template <class Op, int BLK, class Fn>
__device__ void split_finish(typename Op::State st, typename Op::State* part, unsigned* ticket, int S, int s,
                             long long stride, long long o, Fn&& write) {
    using State = typename Op::State;
    __shared__ int last;
    const int tid = threadIdx.x;
    if (tid == 0) {
        publish_state(part + (long long)s * stride + o, st);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
    }
    __syncthreads();
    if (!last) return;
    State r = Op::identity();
    for (int i = tid; i < S; i += BLK) r = Op::comb(r, fetch_state(part + (long long)i * stride + o));
    r = block_reduce_n<Op, BLK>(r);
    if (tid == 0) {
        write(r);
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Streaming 128-bit load; `nt` marks it nontemporal (read once, do not keep in cache).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4(const float4* p, int nt) {
    if (nt) {
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
        return make_float4(v.x, v.y, v.z, v.w);
    }
    return *p;
}

template <class Op, class I>
__device__ __forceinline__ void acc4(typename Op::Acc& a, float4 t, I e, float prm) {
    Op::acc(a, t.x, e, prm);
    Op::acc(a, t.y, e + 1, prm);
    Op::acc(a, t.z, e + 2, prm);
    Op::acc(a, t.w, e + 3, prm);
}

// A partial state of a chunk of a reduced run indexes from the chunk start;
// states that carry an index (arg ops) are moved to run coordinates.
template <class S>
__device__ __forceinline__ auto shift_index(S s, long long off, int) -> decltype(s.i, S()) {
    if (s.i != kSentinel) s.i += off;
    return s;
}
template <class S>
__device__ __forceinline__ S shift_index(S s, long long, long) { return s; }

// ---------------------------------------------------------------------------
// Row kernel: [rows, R] with R contiguous.  LANES threads per row segment.
// blockIdx.x = row_block * S + split.
// ---------------------------------------------------------------------------
struct RowArgs {
    const float* in;
    long long rows, R, row_stride;
    int S;
    int nt;
    void* out;
    void* part;
    Fin fin;
    long long idx_off;  // index of this launch's first reduced element (chunked runs)
    int partial;        // 1: write states to `part` (S > 1 or a chunk of a longer run)
    unsigned* tickets;  // S > 1, one row per workgroup: per-row counters of split_finish (else null)
};

template <class Op, int VEC, int LANES, int U>
__global__ __launch_bounds__(LANES > kBlock ? LANES : kBlock) void k_rows(RowArgs a) {
    using Acc = typename Op::Acc;
    using State = typename Op::State;
    constexpr int BLK = LANES > kBlock ? LANES : kBlock;  // one long row per 512/1024-thread block
    constexpr int GROUPS = (LANES >= BLK) ? 1 : BLK / LANES;
    // U = vectors in flight per lane
    constexpr int TILE = U * LANES;       // vectors per tile (contiguous in memory)
    const float prm = a.fin.p;            // op parameter (NORM exponent)
    const int tid = threadIdx.x;
    const int g = tid / LANES;
    const int l = tid % LANES;
    const long long rb = blockIdx.x / a.S;
    const int s = blockIdx.x % a.S;
    const long long row = rb * GROUPS + g;

    // The row is cut into tiles of U*LANES vectors; split s takes tiles s, s+S,
    // s+2S, ... so the S workgroups of a row sweep it front to back together.
    // Indexed ops (argmax/amax) keep one accumulator per float4 component with
    // a 32-bit vector index, so each element costs one compare and two selects.
    Acc acc = Op::init();
    Acc accq[Op::kIndexed ? 4 : 1];
#pragma unroll
    for (int q = 0; q < (Op::kIndexed ? 4 : 1); ++q) accq[q] = Op::init();
    if (row < a.rows) {
        const float* p = a.in + row * a.row_stride;
        const int step = a.S * TILE;
        if (VEC == 4) {
            const int nv = (int)(a.R >> 2);
            const float4* pv = reinterpret_cast<const float4*>(p);
            int t0 = s * TILE;
            for (; t0 + TILE <= nv; t0 += step) {
                float4 t[U];
#pragma unroll
                for (int u = 0; u < U; ++u) t[u] = ld4(pv + t0 + l + u * LANES, a.nt);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int v = t0 + l + u * LANES;
                    if constexpr (Op::kIndexed) {
                        Op::acc(accq[0], t[u].x, v, prm);
                        Op::acc(accq[1 % (Op::kIndexed ? 4 : 1)], t[u].y, v, prm);
                        Op::acc(accq[2 % (Op::kIndexed ? 4 : 1)], t[u].z, v, prm);
                        Op::acc(accq[3 % (Op::kIndexed ? 4 : 1)], t[u].w, v, prm);
                    } else {
                        acc4<Op>(acc, t[u], 4 * v, prm);
                    }
                }
            }
            if (t0 < nv) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int v = t0 + l + u * LANES;
                    if (v < nv) {
                        const float4 t = pv[v];
                        if constexpr (Op::kIndexed) {
                            Op::acc(accq[0], t.x, v, prm);
                            Op::acc(accq[1 % (Op::kIndexed ? 4 : 1)], t.y, v, prm);
                            Op::acc(accq[2 % (Op::kIndexed ? 4 : 1)], t.z, v, prm);
                            Op::acc(accq[3 % (Op::kIndexed ? 4 : 1)], t.w, v, prm);
                        } else {
                            acc4<Op>(acc, t, 4 * v, prm);
                        }
                    }
                }
            }
            for (int e = 4 * nv + s * LANES + l; e < a.R; e += a.S * LANES) Op::acc(acc, p[e], e, prm);
        } else {
            int t0 = s * TILE;
            for (; t0 + TILE <= a.R; t0 += step) {
                float x[U];
#pragma unroll
                for (int u = 0; u < U; ++u) x[u] = p[t0 + l + u * LANES];
#pragma unroll
                for (int u = 0; u < U; ++u) Op::acc(acc, x[u], t0 + l + u * LANES, prm);
            }
            if (t0 < a.R) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int e = t0 + l + u * LANES;
                    if (e < a.R) Op::acc(acc, p[e], e, prm);
                }
            }
        }
    }

    State st = Op::state(acc);
    if constexpr (Op::kIndexed) {
#pragma unroll
        for (int q = 0; q < 4; ++q) st = Op::comb(st, Op::state_scaled(accq[q % (Op::kIndexed ? 4 : 1)], 4, q));
    }
    constexpr int SUBW = LANES < kWave ? LANES : kWave;
    st = group_reduce_sub_wave<Op, SUBW>(st);
    if (LANES > kWave) {
        constexpr int WPG = LANES / kWave;  // waves per group
        __shared__ State sh[BLK / kWave];
        const int w = tid / kWave;
        if (__lane_id() == 0) sh[w] = st;
        __syncthreads();
        if (l == 0) {
            State r = sh[g * WPG];
#pragma unroll
            for (int i = 1; i < WPG; ++i) r = Op::comb(r, sh[g * WPG + i]);
            st = r;
        }
    }
    if constexpr (GROUPS == 1) {
        if (a.tickets) {
            split_finish<Op, BLK>(st, reinterpret_cast<State*>(a.part), a.tickets + row, a.S, s, a.rows, row,
                                  [&](const State& r) { fin_write(r, a.fin, a.out, row); });
            return;
        }
    }
    if (l == 0 && row < a.rows) {
        if (!a.partial) fin_write(st, a.fin, a.out, row);
        else reinterpret_cast<State*>(a.part)[(long long)s * a.rows + row] = shift_index(st, a.idx_off, 0);
    }
}

// ---------------------------------------------------------------------------
// Register-row kernel for ops whose identity is 0 (sum, mean, norm p = 1/2,
// any): [rows, R], R contiguous, R % 4 == 0, rows 16-byte aligned,
// R/4 <= 64*WPR*NV.  WPR waves share a row; every lane issues all of its NV
// 128-bit nontemporal loads before it adds anything, so a row is one burst of
// loads with no branch between them.  Loads go through a buffer resource whose
// range is the row (0 for a row past the end): vectors out of range read 0
// without touching memory, which these ops ignore.  RPB = BLK / (64*WPR) rows
// per workgroup.  Measured on MI355X (HIP events, 256 MiB inputs): sum over
// rows of 512-2048 floats 38.4 us against 40.1-40.6 us for k_rows; rows of
// 256 floats or ops with a heavier per-element step (Welford, argmax) were
// slower, so the planner uses it for the zero-identity ops only.
// ---------------------------------------------------------------------------
constexpr int kBufWord3 = 0x00020000;  // raw buffer resource, 32-bit data (gfx9 family)
constexpr int kAuxNT = 2;              // buffer-load cache policy: nontemporal

// fp64 sum over the 64 lanes of a wave with DPP lane moves (no LDS round
// trips): quad swaps, half-row and row mirrors leave every lane of a 16-lane
// row with the row's sum, then two row broadcasts carry the rows into lane 63.
// The result is valid in lane 63 only.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, ROW_MASK, 0xf, false);
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
__device__ __forceinline__ double wave_sum_f64_lane63(double v) {
    v += dpp_f64<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
    v += dpp_f64<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
    v += dpp_f64<0x141, 0xf>(v);  // row_half_mirror
    v += dpp_f64<0x140, 0xf>(v);  // row_mirror
    v += dpp_f64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

template <class Op, int NV, int WPR, int BLK>
__global__ __launch_bounds__(BLK) void k_rows_reg(RowArgs a) {
    using State = typename Op::State;
    constexpr int RPB = BLK / (kWave * WPR);
    static_assert(RPB >= 1 && RPB * kWave * WPR == BLK, "BLK must hold whole rows");
    const float prm = a.fin.p;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform: scalar buffer resource
    const int l = __lane_id();
    const int sub = w % WPR;
    const long long row = (long long)blockIdx.x * RPB + w / WPR;
    const bool live = row < a.rows;
    const float* p = a.in + (live ? row * a.row_stride : 0);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, live ? (int)(a.R * 4) : 0, kBufWord3);
    f32x4 t[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u)
        t[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, ((sub * NV + u) * kWave + l) * 16, 0, kAuxNT));
    // four independent accumulators (one per float4 component): the add chain
    // a lane runs after its loads arrive is NV long instead of 4 * NV, which
    // shortens the tail of the last waves (C1: 11.68 -> 11.52 us kernel time in
    // the trace for the same load pattern)
    typename Op::Acc q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = Op::init();
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        Op::acc(q[0], t[u].x, 0, prm);
        Op::acc(q[1], t[u].y, 0, prm);
        Op::acc(q[2], t[u].z, 0, prm);
        Op::acc(q[3], t[u].w, 0, prm);
    }
    State st = Op::comb(Op::comb(Op::state(q[0]), Op::state(q[1])), Op::comb(Op::state(q[2]), Op::state(q[3])));
    // the wave's total ends in lane 63 (sums: DPP moves) or every lane (the butterfly)
    constexpr bool kDpp = std::is_same<State, SumS>::value && std::is_same<typename Op::Acc, double>::value &&
                          !std::is_same<Op, ProdOp>::value;
    constexpr int kLead = kDpp ? kWave - 1 : 0;
    if constexpr (kDpp) st.s = wave_sum_f64_lane63(st.s);
    else st = group_reduce_sub_wave<Op, kWave>(st);
    if constexpr (WPR > 1) {
        __shared__ State sh[BLK / kWave];
        if (l == kLead) sh[w] = st;
        __syncthreads();
        if (sub == 0 && l == kLead) {
#pragma unroll
            for (int i = 1; i < WPR; ++i) st = Op::comb(st, sh[w + i]);
        }
    }
    if (sub == 0 && l == kLead && live) fin_write(st, a.fin, a.out, row);
}

// ---------------------------------------------------------------------------
// var / std over rows that fill WPR waves exactly (R == 4 * 64 * WPR * NV):
// every element is shifted by the row's first element K (one scalar load per
// wave), so the shifted sums S1 = sum(x - K), S2 = sum((x - K)^2) of all lanes
// add up directly -- no per-lane Welford state, no Chan merges, one divide per
// row: mean = K + S1/n, M2 = S2 - S1^2/n (fp64; K is an element of the row, the
// same kind of shift the per-thread Welford accumulator uses).  Four chains per
// lane (one per float4 component), all loads issued before the first add.
// ---------------------------------------------------------------------------
template <int NV, int WPR, int BLK>
__global__ __launch_bounds__(BLK) void k_rows_reg_var(RowArgs a) {
    constexpr int RPB = BLK / (kWave * WPR);
    static_assert(RPB >= 1 && RPB * kWave * WPR == BLK, "BLK must hold whole rows");
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform: scalar buffer resource
    const int l = __lane_id();
    const int sub = w % WPR;
    const long long row = (long long)blockIdx.x * RPB + w / WPR;
    const bool live = row < a.rows;
    const float* p = a.in + (live ? row * a.row_stride : 0);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, live ? (int)(a.R * 4) : 0, kBufWord3);
    f32x4 t[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u)
        t[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, ((sub * NV + u) * kWave + l) * 16, 0, kAuxNT));
    // K through the vector memory path (a buffer load of the row's first word,
    // the same cache line as lane 0's first vector load, which is in flight):
    // a scalar load would fetch that line a second time
    const double Kd = (double)__uint_as_float(
        __builtin_amdgcn_readfirstlane(__builtin_amdgcn_raw_buffer_load_b32(rs, 0, 0, 0)));
    double s1[4] = {0.0, 0.0, 0.0, 0.0}, s2[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const double d0 = (double)t[u].x - Kd, d1 = (double)t[u].y - Kd;
        const double d2 = (double)t[u].z - Kd, d3 = (double)t[u].w - Kd;
        s1[0] += d0; s2[0] = fma(d0, d0, s2[0]);
        s1[1] += d1; s2[1] = fma(d1, d1, s2[1]);
        s1[2] += d2; s2[2] = fma(d2, d2, s2[2]);
        s1[3] += d3; s2[3] = fma(d3, d3, s2[3]);
    }
    double S1 = (s1[0] + s1[1]) + (s1[2] + s1[3]);
    double S2 = (s2[0] + s2[1]) + (s2[2] + s2[3]);
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        S1 += __shfl_xor(S1, m, kWave);
        S2 += __shfl_xor(S2, m, kWave);
    }
    if constexpr (WPR > 1) {
        __shared__ double sh1[BLK / kWave], sh2[BLK / kWave];
        if (l == 0) {
            sh1[w] = S1;
            sh2[w] = S2;
        }
        __syncthreads();
        if (sub == 0 && l == 0) {
#pragma unroll
            for (int i = 1; i < WPR; ++i) {
                S1 += sh1[w + i];
                S2 += sh2[w + i];
            }
        }
    }
    if (sub == 0 && l == 0 && live) {
        const double n = (double)a.R;
        const double m = S1 / n;
        fin_write(WelS{n, Kd + m, fmax(0.0, S2 - S1 * m)}, a.fin, a.out, row);
    }
}

// ---------------------------------------------------------------------------
// Column kernel: [outer, R, inner], inner contiguous.  TX threads across the
// inner dim (VEC elements each), TY = 256/TX threads across R.
// blockIdx.x = (o * ncb + cb) * S + split.
// ---------------------------------------------------------------------------
struct ColArgs {
    const float* in;
    long long outer, os, R, rs, inner;
    int S;
    int nt;
    long long ncb;
    void* out;
    void* part;
    Fin fin;
    long long idx_off;  // as RowArgs
    int partial;
    unsigned* tickets;  // as RowArgs (rows only)
};

template <class Op, int VEC, int TX, int U, int BLK>
__global__ __launch_bounds__(BLK) void k_cols(ColArgs a) {
    using Acc = typename Op::Acc;
    using State = typename Op::State;
    constexpr int TY = BLK / TX;
    const float prm = a.fin.p;  // op parameter (NORM exponent)
    const int tid = threadIdx.x;
    const int tx = tid % TX;
    const int ty = tid / TX;
    const int s = blockIdx.x % a.S;
    const long long ob = blockIdx.x / a.S;
    const long long cb = ob % a.ncb;
    const long long o = ob / a.ncb;
    const long long col0 = (cb * TX + tx) * VEC;

    Acc acc[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[j] = Op::init();

    // rows of the reduced dim are interleaved over the TY thread rows and the S
    // splits (row r goes to split (r / TY) % S), so concurrently running
    // workgroups read neighbouring rows; U rows are in flight per thread
    if (col0 < a.inner) {
        const float* base = a.in + o * a.os + col0;
        const int R = (int)a.R;
        const int rstep = TY * a.S;
        const int r0 = s * TY + ty;
        if (VEC == 4 && col0 + 3 < a.inner) {
            int r = r0;
            for (; r + (U - 1) * rstep < R; r += U * rstep) {
                float4 t[U];
#pragma unroll
                for (int u = 0; u < U; ++u) t[u] = ld4(reinterpret_cast<const float4*>(base + (long long)(r + u * rstep) * a.rs), a.nt);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int ru = r + u * rstep;
                    Op::acc(acc[0], t[u].x, ru, prm);
                    Op::acc(acc[1 % VEC], t[u].y, ru, prm);
                    Op::acc(acc[2 % VEC], t[u].z, ru, prm);
                    Op::acc(acc[3 % VEC], t[u].w, ru, prm);
                }
            }
            for (; r < R; r += rstep) {
                float4 t = *reinterpret_cast<const float4*>(base + (long long)r * a.rs);
                Op::acc(acc[0], t.x, r, prm);
                Op::acc(acc[1 % VEC], t.y, r, prm);
                Op::acc(acc[2 % VEC], t.z, r, prm);
                Op::acc(acc[3 % VEC], t.w, r, prm);
            }
        } else {
            const int nj = (int)min((long long)VEC, a.inner - col0);
            for (int r = r0; r < R; r += rstep) {
                const float* q = base + (long long)r * a.rs;
#pragma unroll
                for (int j = 0; j < VEC; ++j)
                    if (j < nj) Op::acc(acc[j], q[j], r, prm);
            }
        }
    }

    State st[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) st[j] = Op::state(acc[j]);

    // combine the TY thread rows with a halving tree in LDS (fixed order)
    if constexpr (TY > 1) {
        __shared__ State sh[(TY > 1 ? TY / 2 : 1) * TX * VEC];
#pragma unroll
        for (int half = TY / 2; half >= 1; half /= 2) {
            if (ty >= half && ty < 2 * half) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) sh[((ty - half) * TX + tx) * VEC + j] = st[j];
            }
            __syncthreads();
            if (ty < half) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) st[j] = Op::comb(st[j], sh[(ty * TX + tx) * VEC + j]);
            }
            __syncthreads();
        }
    }
    if (ty == 0) {
        const long long nout = a.outer * a.inner;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const long long c = col0 + j;
            if (c < a.inner) {
                const long long oi = o * a.inner + c;
                if (!a.partial) fin_write(st[j], a.fin, a.out, oi);
                else reinterpret_cast<State*>(a.part)[(long long)s * nout + oi] = shift_index(st[j], a.idx_off, 0);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// General kernel: any strides.  One workgroup per (output, split); threads walk
// the reduced index space with div/mod.  Also serves empty reduced extents.
// ---------------------------------------------------------------------------
struct GenArgs {
    const float* in;
    int nk, nr;
    long long ksz[TPR_MAX_DIMS], kst[TPR_MAX_DIMS];
    long long rsz[TPR_MAX_DIMS], rst[TPR_MAX_DIMS];
    long long nout, count, seg;
    int S;
    void* out;
    void* part;
    Fin fin;
};

template <class Op>
__global__ __launch_bounds__(kBlock) void k_general(GenArgs a) {
    using Acc = typename Op::Acc;
    using State = typename Op::State;
    const float prm = a.fin.p;  // op parameter (NORM exponent)
    const long long o = blockIdx.x / a.S;
    const int s = blockIdx.x % a.S;
    long long base = 0;
    {
        long long rem = o;
        for (int d = a.nk - 1; d >= 0; --d) {
            base += (rem % a.ksz[d]) * a.kst[d];
            rem /= a.ksz[d];
        }
    }
    Acc acc = Op::init();
    const long long beg = (long long)s * a.seg;
    const long long end = min(a.count, beg + a.seg);
    for (long long j = beg + threadIdx.x; j < end; j += kBlock) {
        long long rem = j, off = 0;
        for (int d = a.nr - 1; d >= 0; --d) {
            off += (rem % a.rsz[d]) * a.rst[d];
            rem /= a.rsz[d];
        }
        Op::acc(acc, a.in[base + off], j, prm);
    }
    State st = block_reduce<Op>(Op::state(acc));
    if (threadIdx.x == 0) {
        if (a.S == 1) fin_write(st, a.fin, a.out, o);
        else reinterpret_cast<State*>(a.part)[(long long)s * a.nout + o] = st;
    }
}

// ---------------------------------------------------------------------------
// Finalize: combine S partial states per output in split order.
// ---------------------------------------------------------------------------
struct FinArgs {
    const void* part;
    long long nout;
    int S;
    void* out;
    Fin fin;
};

template <class Op>
__global__ __launch_bounds__(kBlock) void k_finalize_thread(FinArgs a) {
    using State = typename Op::State;
    const long long o = (long long)blockIdx.x * kBlock + threadIdx.x;
    if (o >= a.nout) return;
    const State* p = reinterpret_cast<const State*>(a.part);
    State st = p[o];
    for (int s = 1; s < a.S; ++s) st = Op::comb(st, p[(long long)s * a.nout + o]);
    fin_write(st, a.fin, a.out, o);
}

template <class Op>
__global__ __launch_bounds__(kBlock) void k_finalize_block(FinArgs a) {
    using State = typename Op::State;
    const long long o = blockIdx.x;
    const State* p = reinterpret_cast<const State*>(a.part);
    State st = Op::identity();
    for (int s = threadIdx.x; s < a.S; s += kBlock) st = Op::comb(st, p[(long long)s * a.nout + o]);
    st = block_reduce<Op>(st);
    if (threadIdx.x == 0) fin_write(st, a.fin, a.out, o);
}

// ---------------------------------------------------------------------------
// Host planner.
// ---------------------------------------------------------------------------
enum PlanKind { P_ROWS = 1, P_COLS = 2, P_GENERAL = 3 };

struct Plan {
    int kind = P_GENERAL;
    int vec = 1;
    int lanes = 64;  // rows
    int tx = 64;     // cols
    int unroll = 4;  // rows/cols: vectors in flight per thread
    int nt = 0;      // rows/cols: nontemporal input loads
    int colblock = 256;  // cols: threads per workgroup
    int reg_wpr = 0;     // rows: > 0 selects k_rows_reg with this many waves per row
    int var_nv = 0;      // rows, VAR/STD: > 0 selects k_rows_reg_var (float4 per lane; reg_wpr waves per row)
    long long S = 1;
    // A reduced run of 2^31 or more elements is cut into chunks of `chunk`
    // elements, one launch each (32-bit indices inside a launch); every launch
    // writes S partial states per output, finalized together (S * nchunk).
    long long nchunk = 1, chunk = 0, Rfull = 0;
    long long idx_off = 0;  // per launch: first reduced index of the chunk
    int partial = 0;        // per launch: write partial states
    size_t state_bytes = 8;
    size_t ws = 0;
    // geometry
    long long rows = 1, R = 1, row_stride = 0, seg = 1;       // rows
    long long outer = 1, os = 0, rs = 0, inner = 1, ncb = 1;  // cols
    int nk = 0, nr = 0;
    long long ksz[TPR_MAX_DIMS], kst[TPR_MAX_DIMS], rsz[TPR_MAX_DIMS], rst[TPR_MAX_DIMS];
    long long nout = 1, count = 1;
};

bool norm_is_inf(double p) { return std::isinf(p); }

size_t state_size(int op, double p) {
    switch (op) {
        case TPR_SUM: case TPR_MEAN: case TPR_PROD: return sizeof(SumS);
        case TPR_NORM: return norm_is_inf(p) ? sizeof(ArgS) : sizeof(SumS);
        case TPR_ALL: case TPR_ANY: return sizeof(BoolS);
        case TPR_AMAX: case TPR_AMIN: case TPR_ARGMAX: case TPR_ARGMIN: return sizeof(ArgS);
        default: return sizeof(WelS);
    }
}

long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }
long long pow2_ceil(long long v) {
    long long p = 1;
    while (p < v) p <<= 1;
    return p;
}

int esize_of(int dt);

int validate(const tpr_reduce_desc* d) {
    if (!d) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: null descriptor");
    if (d->ndim < 0 || d->ndim > TPR_MAX_DIMS)
        return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: ndim out of range [0, 8]");
    if (d->op < TPR_SUM || d->op > TPR_MEDIAN) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: bad op");
    for (int i = 0; i < d->ndim; ++i)
        if (d->sizes[i] < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: negative size");
    if (d->ndim < 32 && (d->reduce_mask >> d->ndim) != 0)
        return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: reduce_mask names a dim >= ndim");
    if (d->in_dtype == TPR_FLOAT64) {
        switch (d->op) {
            case TPR_SUM: case TPR_MEAN: case TPR_PROD:
                if (d->out_dtype != TPR_FLOAT32 && d->out_dtype != TPR_FLOAT64)
                    return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: sum/mean/prod output must be float32 or float64");
                return TPR_OK;
            case TPR_AMAX: case TPR_AMIN: case TPR_VAR: case TPR_STD: case TPR_NORM:
                if (d->out_dtype != TPR_FLOAT64)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: float64 amax/amin/var/std/norm write float64");
                return TPR_OK;
            case TPR_ARGMAX: case TPR_ARGMIN:
                if (d->out_dtype != TPR_INT64)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: argmax/argmin output must be int64");
                return TPR_OK;
            case TPR_ALL: case TPR_ANY:
                if (d->out_dtype != TPR_BOOL)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: all/any output must be bool");
                return TPR_OK;
            case TPR_MEDIAN: {
                if (d->out_dtype != d->in_dtype)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: median output dtype must equal input dtype");
                const uint32_t all = d->ndim >= 32 ? 0xffffffffu : ((1u << d->ndim) - 1u);
                if (d->ndim > 0 && d->reduce_mask != all)
                    return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce: median reduces all dims only");
                return TPR_OK;
            }
            default:
                return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce: op not implemented for float64");
        }
    }
    if (d->in_dtype != TPR_FLOAT32) {
        if (esize_of(d->in_dtype) == 0)
            return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: input dtype not implemented");
        switch (d->op) {
            case TPR_SUM: case TPR_PROD:
                if (d->out_dtype != TPR_INT64)
                    return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: integer sum/prod output must be int64");
                return TPR_OK;
            case TPR_MEAN:
                if (d->out_dtype != TPR_FLOAT32 && d->out_dtype != TPR_FLOAT64)
                    return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: mean output must be float32 or float64");
                return TPR_OK;
            case TPR_AMAX: case TPR_AMIN:
                if (d->out_dtype != d->in_dtype)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: amax/amin output dtype must equal input dtype");
                return TPR_OK;
            case TPR_ARGMAX: case TPR_ARGMIN:
                if (d->out_dtype != TPR_INT64)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: argmax/argmin output must be int64");
                return TPR_OK;
            case TPR_ALL: case TPR_ANY:
                if (d->out_dtype != TPR_BOOL)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: all/any output must be bool");
                return TPR_OK;
            case TPR_MEDIAN: {
                if (d->out_dtype != d->in_dtype)
                    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: median output dtype must equal input dtype");
                const uint32_t all = d->ndim >= 32 ? 0xffffffffu : ((1u << d->ndim) - 1u);
                if (d->ndim > 0 && d->reduce_mask != all)
                    return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce: median reduces all dims only");
                return TPR_OK;
            }
            default:
                return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: var/std/norm need a float32 or float64 input");
        }
    }
    switch (d->op) {
        case TPR_SUM: case TPR_MEAN: case TPR_PROD:
            if (d->out_dtype != TPR_FLOAT32 && d->out_dtype != TPR_FLOAT64)
                return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: sum/mean/prod output must be float32 or float64");
            break;
        case TPR_ALL: case TPR_ANY:
            if (d->out_dtype != TPR_BOOL)
                return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: all/any output must be bool");
            break;
        case TPR_MEDIAN: {
            if (d->out_dtype != TPR_FLOAT32)
                return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: median output must be float32");
            const uint32_t all = d->ndim >= 32 ? 0xffffffffu : ((1u << d->ndim) - 1u);
            if (d->ndim > 0 && d->reduce_mask != all)
                return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce: median reduces all dims only");
            break;
        }
        case TPR_AMAX: case TPR_AMIN:
            if (d->out_dtype != d->in_dtype)
                return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: amax/amin output dtype must equal input dtype");
            break;
        case TPR_ARGMAX: case TPR_ARGMIN:
            if (d->out_dtype != TPR_INT64)
                return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: argmax/argmin output must be int64");
            break;
        default:  // VAR, STD, NORM
            if (d->out_dtype != TPR_FLOAT32)
                return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: var/std/norm output must be float32");
    }
    return TPR_OK;
}

Plan make_plan(const tpr_reduce_desc* d, const void* in) {
    Plan p;
    p.state_bytes = state_size(d->op, d->p);
    const int nd = d->ndim;
    uint32_t mask = (nd == 0) ? 0u : d->reduce_mask;
    // counts (before dropping size-1 dims)
    p.nout = 1;
    p.count = 1;
    for (int i = 0; i < nd; ++i) {
        if (mask & (1u << i)) p.count *= d->sizes[i];
        else p.nout *= d->sizes[i];
    }
    // canonicalise: drop size-1 dims, merge contiguous neighbours of equal kind
    struct Dim { long long size, stride; bool red; };
    // at most TPR_MAX_DIMS entries each; fixed storage, so planning allocates nothing
    struct Dims {
        Dim d[TPR_MAX_DIMS];
        int n = 0;
        bool empty() const { return n == 0; }
        size_t size() const { return (size_t)n; }
        Dim& back() { return d[n - 1]; }
        const Dim& front() const { return d[0]; }
        Dim& operator[](size_t i) { return d[i]; }
        const Dim& operator[](size_t i) const { return d[i]; }
        void push_back(const Dim& x) { d[n++] = x; }
        const Dim* begin() const { return d; }
        const Dim* end() const { return d + n; }
    };
    Dims dims;
    for (int i = 0; i < nd; ++i) {
        if (d->sizes[i] == 1) continue;
        Dim x{d->sizes[i], d->strides[i], (mask & (1u << i)) != 0};
        if (!dims.empty() && dims.back().red == x.red && dims.back().stride == x.stride * x.size) {
            dims.back().size *= x.size;
            dims.back().stride = x.stride;
        } else {
            dims.push_back(x);
        }
    }
    Dims K, Rd;
    for (auto& x : dims) (x.red ? Rd : K).push_back(x);

    const auto& dev = device_info();
    const bool aligned16 = (reinterpret_cast<uintptr_t>(in) & 15u) == 0;
    const bool force_general = knobs().general != 0;
    const bool empty = (p.count == 0 || p.nout == 0);

    long long Rfull = 0;
    auto fill_general = [&]() {
        if (Rfull) {  // 64-bit index arithmetic: no chunks
            Rd[0].size = Rfull;
            Rfull = 0;
        }
        p.kind = P_GENERAL;
        p.nk = (int)K.size();
        p.nr = (int)Rd.size();
        for (int i = 0; i < p.nk; ++i) { p.ksz[i] = K[i].size; p.kst[i] = K[i].stride; }
        for (int i = 0; i < p.nr; ++i) { p.rsz[i] = Rd[i].size; p.rst[i] = Rd[i].stride; }
        p.S = 1;
        if (!empty) {
            long long blocks = p.nout;
            long long want = (long long)dev.cus * 8;
            if (blocks < want) p.S = std::min(ceil_div(want, blocks), std::max(1LL, p.count / (kBlock * 16)));
            if (knobs().splits > 0) p.S = knobs().splits;
            p.S = std::max(1LL, std::min(p.S, p.count));
        }
        p.seg = ceil_div(std::max(1LL, p.count), p.S);
        p.S = ceil_div(std::max(1LL, p.count), p.seg);
    };

    const long long kIntMax = 0x7fffffffLL;
    const long long kChunk = 1LL << 30;  // elements; a multiple of 16, so chunk starts keep 16-byte alignment
    if (!empty && !force_general && Rd.size() == 1 && Rd[0].size >= kIntMax) {
        Rfull = Rd[0].size;
        Rd[0].size = kChunk;  // plan one chunk; the general kernel takes the whole run back
    }
    const bool int_ok = Rd.empty() || (Rd.size() == 1 && Rd[0].size < kIntMax);
    if (empty || force_general || !int_ok) {
        fill_general();
    } else if (K.size() <= 1 && (Rd.empty() || (Rd.size() == 1 && Rd[0].stride == 1))) {
        // rows: [K?, R] with R contiguous (R may be absent: each output is one element)
        p.kind = P_ROWS;
        p.rows = K.empty() ? 1 : K[0].size;
        p.row_stride = K.empty() ? 0 : K[0].stride;
        p.R = Rd.empty() ? 1 : Rd[0].size;
        p.vec = (aligned16 && (p.rows == 1 || p.row_stride % 4 == 0) && p.R >= 4) ? 4 : 1;
        // lanes per row: >= ~32 elements per thread, and enough lanes that the
        // grid holds ~4096 threads per CU; rows are split over workgroups only
        // when even 256 lanes per row leave fewer than ~512 threads per CU
        const long long E = 32;
        long long lanes = std::max(pow2_ceil(ceil_div(p.R, E)),
                                   pow2_ceil(ceil_div((long long)dev.cus * 4096, p.rows)));
        lanes = std::min(256LL, std::max(16LL, std::min(lanes, pow2_ceil(ceil_div(p.R, 4)))));
        const long long target = (long long)dev.cus * 512;
        // few long rows: give one row a 512- or 1024-thread workgroup when that
        // avoids splitting rows over workgroups (a split costs a finalize
        // launch); rows that need a split anyway keep 256-thread workgroups
        if (p.rows * 1024 >= target)
            while (p.rows * lanes < 2 * target && lanes < 1024 && 16 * 2 * lanes <= p.R) lanes *= 2;
        if (knobs().lanes > 0) lanes = knobs().lanes;
        p.lanes = (int)lanes;
        // one row per 1024-thread workgroup: 2 vectors in flight per lane
        // (measured on MI355X, C5-shaped argmax/sum: 2% faster than 4 or 8)
        if (lanes == 1024) p.unroll = 2;
        // 32 lanes with exactly 8 vectors each (rows of 1024 floats): all eight
        // in flight at once (C2 var / std / argmax dim=-1 on MI355X: 41.7 /
        // 41.8 / 40.6 us against 42.2 / 42.2 / 41.3 us with two tiles of 4)
        if (lanes == 32 && p.vec == 4 && ceil_div(p.R, 4 * 32) == 8) p.unroll = 8;
        const long long tiles = std::max(1LL, ceil_div(p.R, 16 * lanes));  // 4 vectors x 4 floats per lane
        long long threads = p.rows * lanes;
        long long S = 1;
        if (threads < target) S = std::min(ceil_div(target, threads), tiles);
        if (knobs().splits > 0) S = knobs().splits;
        p.S = std::max(1LL, S);
        // Zero-identity ops over rows of 65-1024 float4, with enough rows to give
        // every CU at least 8 waves: one burst of two 128-bit loads per lane,
        // WPR waves per row (k_rows_reg).  The workspace stays zero, as for S == 1.
        const long long nv4 = p.R / 4;
        const bool zero_id = d->op == TPR_SUM || d->op == TPR_MEAN || d->op == TPR_ANY ||
                             (d->op == TPR_NORM && (d->p == 1.0 || d->p == 2.0));
        if (zero_id && p.vec == 4 && p.R % 4 == 0 && nv4 > kWave && nv4 <= 1024 && knobs().rowreg >= 0 &&
            knobs().splits <= 0 && knobs().lanes <= 0) {
            const long long wpr = std::max(1LL, pow2_ceil(ceil_div(nv4, 2 * kWave)));
            if (knobs().rowreg > 0 || p.rows * wpr >= (long long)dev.cus * 8) {
                p.reg_wpr = (int)wpr;
                p.S = 1;
            }
        }
        // var / std over rows of 1024, 2048 or 4096 floats (1, 2 or 4 waves of
        // four float4 per lane, exactly): the shifted two-sum kernel.  Measured
        // on MI355X: C2 var dim=-1 [65536, 1024] 39.9 us against 42.6 us,
        // [4096, 4096] 12.0 against 16.7 us, [16384, 2048] 21.6 against 23.3 us;
        // two float4 per lane (rows of 512) was slower than k_rows (48 us).
        if ((d->op == TPR_VAR || d->op == TPR_STD) && p.vec == 4 && p.R % 4 == 0 && nv4 % (4 * kWave) == 0 &&
            knobs().rowreg >= 0 && knobs().splits <= 0 && knobs().lanes <= 0) {
            const long long wv = nv4 / (4 * kWave);
            if ((wv == 1 || wv == 2 || wv == 4) && (knobs().rowreg > 0 || p.rows * wv >= (long long)dev.cus * 8)) {
                p.reg_wpr = (int)wv;
                p.var_nv = 4;
                p.S = 1;
            }
        }
    } else if (!K.empty() && K.back().stride == 1 && Rd.size() == 1 &&
               (K.size() == 1 ? true : (K.size() == 2)) &&
               (K.size() == 1 ? (dims.front().red) : (dims.size() == 3 && dims[1].red))) {
        // cols: [K1?, R, K2] with K2 contiguous
        p.kind = P_COLS;
        p.inner = K.back().size;
        p.outer = (K.size() == 2) ? K[0].size : 1;
        p.os = (K.size() == 2) ? K[0].stride : 0;
        p.R = Rd[0].size;
        p.rs = Rd[0].stride;
        p.vec = (aligned16 && p.rs % 4 == 0 && (p.outer == 1 || p.os % 4 == 0) && p.inner >= 4) ? 4 : 1;
        // plan on float4 columns whatever the alignment, so the workspace size
        // does not depend on the pointer
        const long long cols4 = ceil_div(p.inner, 4);
        const long long target = (long long)dev.cus * 512;
        if (p.outer * ceil_div(cols4, 256) * kBlock >= target || p.R < 16) p.tx = 256;
        else p.tx = 64;
        if (knobs().tx == 64 || knobs().tx == 128 || knobs().tx == 256) p.tx = (int)knobs().tx;
        p.unroll = (p.tx == 256) ? 2 : 4;  // measured: 2 rows in flight per thread at TX=256, 4 at TX=64
        // grow the workgroup (more thread rows over R) before splitting R over
        // workgroups: a split costs a finalize launch (~4-5 us on MI355X)
        const long long base_threads = p.outer * ceil_div(cols4, p.tx);
        while (p.colblock < 1024 && base_threads * p.colblock < target && p.R >= 8 * (2 * p.colblock / p.tx))
            p.colblock *= 2;
        if (knobs().colblock == 256 || knobs().colblock == 512 || knobs().colblock == 1024)
            p.colblock = (int)knobs().colblock;
        p.ncb = ceil_div(ceil_div(p.inner, p.vec), p.tx);
        const long long ty = p.colblock / p.tx;
        const long long threads = p.outer * ceil_div(cols4, p.tx) * p.colblock;
        long long S = 1;
        if (threads < target) S = std::min(ceil_div(target, threads), std::max(1LL, p.R / (ty * 8)));
        if (knobs().splits > 0) S = knobs().splits;
        p.S = std::max(1LL, std::min(S, ceil_div(p.R, ty)));
    } else {
        fill_general();
    }
    if (knobs().unroll == 1 || knobs().unroll == 2 || knobs().unroll == 4 || knobs().unroll == 8) p.unroll = (int)knobs().unroll;
    // Inputs are read exactly once: mark the loads nontemporal for large
    // reductions (measured on MI355X: +8..13% at 256 MiB and 1 GiB, +5% for a
    // [4096,4096] row sum at 64 MiB).
    p.nt = (p.count * p.nout >= (16LL << 20)) ? 1 : 0;  // >= 64 MiB of float32
    if (knobs().nt != 0) p.nt = knobs().nt > 0 ? 1 : 0;
    if (Rfull) {
        p.Rfull = Rfull;
        p.chunk = kChunk;
        p.nchunk = ceil_div(Rfull, kChunk);
    }
    p.ws = (p.S > 1 || p.nchunk > 1) ? (size_t)(p.S * p.nchunk) * (size_t)p.nout * p.state_bytes : 0;
    return p;
}

// Ops for which an element equal to 0 changes nothing (k_rows_reg reads 0 past a row's end).
template <class Op>
constexpr bool kZeroIdentity = std::is_same<Op, SumOp>::value || std::is_same<Op, NormOp<1>>::value ||
                               std::is_same<Op, NormOp<2>>::value || std::is_same<Op, BoolOp<true>>::value;

template <class Op>
int launch_rows_reg(const Plan& p, const float* in, void* out, Fin fin, hipStream_t st) {
    RowArgs a{in, p.rows, p.R, p.row_stride, 1, p.nt, out, nullptr, fin, 0, 0};
    switch (p.reg_wpr) {
        case 1: hipLaunchKernelGGL((k_rows_reg<Op, 2, 1, 256>), dim3(ceil_div(p.rows, 4)), dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((k_rows_reg<Op, 2, 2, 256>), dim3(ceil_div(p.rows, 2)), dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((k_rows_reg<Op, 2, 4, 256>), dim3(p.rows), dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL((k_rows_reg<Op, 2, 8, 512>), dim3(p.rows), dim3(512), 0, st, a); break;
        default: return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: register-row plan needs 1, 2, 4 or 8 waves per row");
    }
    return check_launch("k_rows_reg");
}

int launch_rows_reg_var(const Plan& p, const float* in, void* out, Fin fin, hipStream_t st) {
    RowArgs a{in, p.rows, p.R, p.row_stride, 1, p.nt, out, nullptr, fin};
    const int nv = p.var_nv;
    const int wpr = p.reg_wpr;
#define TPR_VAR_CASE(NV, WPR, BLK)                                                                             \
    if (nv == NV && wpr == WPR) {                                                                              \
        hipLaunchKernelGGL((k_rows_reg_var<NV, WPR, BLK>), dim3(ceil_div(p.rows, BLK / (kWave * WPR))), dim3(BLK), 0, st, a); \
        return check_launch("k_rows_reg_var");                                                                 \
    }
    TPR_VAR_CASE(4, 1, 256) TPR_VAR_CASE(4, 2, 256) TPR_VAR_CASE(4, 4, 256)
#undef TPR_VAR_CASE
    return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: no register-row var kernel for this row length");
}

template <class Op>
int launch_rows(const Plan& p, const float* in, void* out, void* ws, Fin fin, hipStream_t st,
                unsigned* tickets = nullptr) {
    if constexpr (std::is_same<Op, WelfordOp>::value) {
        if (p.var_nv > 0) return launch_rows_reg_var(p, in, out, fin, st);
    }
    if constexpr (kZeroIdentity<Op>) {
        if (p.reg_wpr > 0) return launch_rows_reg<Op>(p, in, out, fin, st);
    } else {
        if (p.reg_wpr > 0) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: register-row plan for an op without a zero identity");
    }
    RowArgs a{in, p.rows, p.R, p.row_stride, (int)p.S, p.nt, out, ws, fin, p.idx_off, p.partial || p.S > 1,
              tickets};
    const long long groups = (p.lanes >= kBlock) ? 1 : kBlock / p.lanes;
    const long long grid = ceil_div(p.rows, groups) * p.S;
#define TPR_ROWS_CASE(L)                                                                             \
    case L: {                                                                                        \
        constexpr int B = L > kBlock ? L : kBlock;                                                   \
        if (L == 32 && p.vec == 4 && p.unroll == 8) hipLaunchKernelGGL((k_rows<Op, 4, (L == 32 ? 32 : 16), 8>), dim3(grid), dim3(B), 0, st, a); \
        else if (p.vec == 4 && p.unroll == 1) hipLaunchKernelGGL((k_rows<Op, 4, L, 1>), dim3(grid), dim3(B), 0, st, a); \
        else if (p.vec == 4 && p.unroll == 2) hipLaunchKernelGGL((k_rows<Op, 4, L, 2>), dim3(grid), dim3(B), 0, st, a); \
        else if (p.vec == 4) hipLaunchKernelGGL((k_rows<Op, 4, L, 4>), dim3(grid), dim3(B), 0, st, a); \
        else hipLaunchKernelGGL((k_rows<Op, 1, L, 4>), dim3(grid), dim3(B), 0, st, a);             \
        break;                                                                                       \
    }
    switch (p.lanes) {
        TPR_ROWS_CASE(16)
        TPR_ROWS_CASE(32)
        TPR_ROWS_CASE(64)
        TPR_ROWS_CASE(128)
        TPR_ROWS_CASE(256)
        TPR_ROWS_CASE(512)
        TPR_ROWS_CASE(1024)
        default: return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: lanes must be 16/32/64/128/256/512/1024");
    }
#undef TPR_ROWS_CASE
    return check_launch("k_rows");
}

template <class Op>
int launch_cols(const Plan& p, const float* in, void* out, void* ws, Fin fin, hipStream_t st) {
    ColArgs a{in, p.outer, p.os, p.R, p.rs, p.inner, (int)p.S, p.nt, p.ncb, out, ws, fin, p.idx_off,
              p.partial || p.S > 1};
    const long long grid = p.outer * p.ncb * p.S;
#define TPR_COLS_LAUNCH(TXV, BLK)                                                                          \
    {                                                                                                     \
        if (p.vec != 4) hipLaunchKernelGGL((k_cols<Op, 1, TXV, 4, BLK>), dim3(grid), dim3(BLK), 0, st, a); \
        else if (p.unroll == 1) hipLaunchKernelGGL((k_cols<Op, 4, TXV, 1, BLK>), dim3(grid), dim3(BLK), 0, st, a); \
        else if (p.unroll == 2) hipLaunchKernelGGL((k_cols<Op, 4, TXV, 2, BLK>), dim3(grid), dim3(BLK), 0, st, a); \
        else hipLaunchKernelGGL((k_cols<Op, 4, TXV, 4, BLK>), dim3(grid), dim3(BLK), 0, st, a);            \
    }
#define TPR_COLS_CASE(TXV)                      \
    if (p.tx == TXV) {                          \
        if (p.colblock == 1024) TPR_COLS_LAUNCH(TXV, 1024)     \
        else if (p.colblock == 512) TPR_COLS_LAUNCH(TXV, 512)  \
        else TPR_COLS_LAUNCH(TXV, 256)                         \
    }
    TPR_COLS_CASE(256)
    else TPR_COLS_CASE(128)
    else TPR_COLS_CASE(64)
    else return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: tx must be 64, 128 or 256");
#undef TPR_COLS_LAUNCH
#undef TPR_COLS_CASE
    return check_launch("k_cols");
}

template <class Op>
int launch_general(const Plan& p, const float* in, void* out, void* ws, Fin fin, hipStream_t st) {
    GenArgs a;
    a.in = in;
    a.nk = p.nk;
    a.nr = p.nr;
    for (int i = 0; i < TPR_MAX_DIMS; ++i) {
        a.ksz[i] = i < p.nk ? p.ksz[i] : 1;
        a.kst[i] = i < p.nk ? p.kst[i] : 0;
        a.rsz[i] = i < p.nr ? p.rsz[i] : 1;
        a.rst[i] = i < p.nr ? p.rst[i] : 0;
    }
    a.nout = p.nout;
    a.count = p.count;
    a.seg = p.seg;
    a.S = (int)p.S;
    a.out = out;
    a.part = ws;
    a.fin = fin;
    hipLaunchKernelGGL((k_general<typename Op::Wide>), dim3(p.nout * p.S), dim3(kBlock), 0, st, a);
    return check_launch("k_general");
}

template <class Op>
int launch_finalize(const Plan& p, void* out, const void* ws, Fin fin, hipStream_t st) {
    FinArgs a{ws, p.nout, (int)p.S, out, fin};
    if (p.S >= 64 && p.nout <= 4096) {
        hipLaunchKernelGGL((k_finalize_block<Op>), dim3(p.nout), dim3(kBlock), 0, st, a);
    } else {
        hipLaunchKernelGGL((k_finalize_thread<Op>), dim3(ceil_div(p.nout, kBlock)), dim3(kBlock), 0, st, a);
    }
    return check_launch("k_finalize");
}

// Launches `launch(plan, in, ws)` once per chunk of a reduced run of 2^31 or
// more elements: the chunk's input, its R, its index offset and its slice of
// the partial states.  Then one finalize over the S * nchunk partials.
template <class Op, class Launch>
int run_chunks(const Plan& p, const void* in, size_t esize, void* out, void* ws, Fin fin, hipStream_t st,
               Launch&& launch) {
    const long long step = (p.kind == P_ROWS) ? 1 : p.rs;  // elements per reduced index
    for (long long c = 0; c < p.nchunk; ++c) {
        Plan pc = p;
        const long long r0 = c * p.chunk;
        pc.R = std::min(p.chunk, p.Rfull - r0);
        pc.idx_off = r0;
        pc.partial = 1;
        const char* inc = static_cast<const char*>(in) + r0 * step * (long long)esize;
        char* wsc = static_cast<char*>(ws) + (size_t)(c * p.S) * (size_t)p.nout * p.state_bytes;
        const int rc = launch(pc, static_cast<const void*>(inc), static_cast<void*>(wsc));
        if (rc != TPR_OK) return rc;
    }
    Plan pf = p;
    pf.S = p.S * p.nchunk;
    return launch_finalize<Op>(pf, out, ws, fin, st);
}

unsigned* stream_tickets(hipStream_t st);

// Counters for a split plan that finishes in its own launch (split_finish):
// row plans with S > 1 and one row per workgroup, on a stream that has a
// counter block.  Null: the plan takes the separate finalize launch.
unsigned* fused_split_tickets(const Plan& p, hipStream_t st) {
    if (p.kind != P_ROWS || p.S <= 1 || p.nchunk > 1 || p.partial || p.lanes < kBlock || p.reg_wpr > 0 ||
        p.var_nv > 0 || p.rows > kTicketsPerStream)
        return nullptr;
    return stream_tickets(st);
}

template <class Op>
int run(const Plan& p, const float* in, void* out, void* ws, Fin fin, hipStream_t st) {
    if (p.nchunk > 1)
        return run_chunks<Op>(p, in, sizeof(float), out, ws, fin, st, [&](const Plan& pc, const void* ic, void* wc) {
            const float* x = static_cast<const float*>(ic);
            return pc.kind == P_ROWS ? launch_rows<Op>(pc, x, out, wc, fin, st) : launch_cols<Op>(pc, x, out, wc, fin, st);
        });
    int rc = TPR_OK;
    unsigned* tk = fused_split_tickets(p, st);
    if (p.kind == P_ROWS) rc = launch_rows<Op>(p, in, out, ws, fin, st, tk);
    else if (p.kind == P_COLS) rc = launch_cols<Op>(p, in, out, ws, fin, st);
    else rc = launch_general<Op>(p, in, out, ws, fin, st);
    if (rc != TPR_OK) return rc;
    if (p.S > 1 && !tk) rc = launch_finalize<Op>(p, out, ws, fin, st);
    return rc;
}

// ---------------------------------------------------------------------------
// Integer and bool inputs (int8/int16/int32/int64/uint8/bool): sum/mean/prod,
// amax/amin/argmax/argmin and all/any.  Semantics of the reference's integer
// instantiations (ReductionKernels.cpp): mean converts to Float32 first
// (IntMeanOp), sum/prod accumulate in Int64
// (AccumulateType, :31-35; wrap-around, so the result does not depend on the
// order), max/min/argmax/argmin start from numeric_limits::lowest/max with the
// strict compare (:213-229), all/any test x != 0.  Results are bit-exact.
// The kernels read 16-byte vectors of 16/sizeof(T) elements; the planner is
// the float one, re-tuned for the element size (adapt_plan_int).
// ---------------------------------------------------------------------------
struct SumI { long long s; };
struct ArgSI { long long v; long long i; };

__device__ __forceinline__ long long wrap_add(long long a, long long b) {
    return (long long)((unsigned long long)a + (unsigned long long)b);
}
__device__ __forceinline__ long long wrap_mul(long long a, long long b) {
    return (long long)((unsigned long long)a * (unsigned long long)b);
}

template <class T, bool PROD>
struct IntSumOp {
    static constexpr bool kIndexed = false;
    using Acc = long long;
    using State = SumI;
    using Wide = IntSumOp;
    __device__ static Acc init() { return PROD ? 1 : 0; }
    template <class I>
    __device__ static void acc(Acc& a, T x, I, float) { a = PROD ? wrap_mul(a, (long long)x) : wrap_add(a, (long long)x); }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {PROD ? 1 : 0}; }
    __device__ static State comb(State a, State b) { return {PROD ? wrap_mul(a.s, b.s) : wrap_add(a.s, b.s)}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.s, m, kWave)}; }
};

// Mean of an integer input: the reference converts the input to Float32 first
// (mean_kernel / mean_dim_kernel pick Float32, sum_kernel's `.to(out_dtype)`,
// ReductionKernels.cpp:81-84,120-123), so the sum is a floating-point sum of
// the fp32-rounded values: no Int64 wrap-around.  Accumulated here in fp64.
template <class T>
struct IntMeanOp {
    static constexpr bool kIndexed = false;
    using Acc = double;
    using State = SumS;
    using Wide = IntMeanOp;
    __device__ static Acc init() { return 0.0; }
    template <class I>
    __device__ static void acc(Acc& a, T x, I, float) { a += (double)(float)x; }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {0.0}; }
    __device__ static State comb(State a, State b) { return {a.s + b.s}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.s, m, kWave)}; }
};

// Order-preserving signed 64-bit key of an integer element: the value itself,
// except for UInt64, whose top bit is flipped (so 2^63.. sort above 0..2^63-1);
// fin_write flips it back for amax / amin (Fin::out_umap).
template <class T>
__device__ __forceinline__ long long ikey(T x) {
    if constexpr (sizeof(T) == 8 && T(-1) > T(0)) return (long long)((unsigned long long)x ^ 0x8000000000000000ull);
    else return (long long)x;
}

// Keys of the dtype's lowest and highest values.
template <class T>
struct IntLimits {
    static constexpr bool U = T(-1) > T(0);
    static constexpr long long lo = U ? (sizeof(T) == 8 ? (-9223372036854775807LL - 1) : 0LL)
                                  : sizeof(T) == 1 ? -128LL
                                  : sizeof(T) == 2 ? -32768LL
                                  : sizeof(T) == 4 ? -2147483648LL : (-9223372036854775807LL - 1);
    static constexpr long long hi = U ? (sizeof(T) == 1 ? 255LL : sizeof(T) == 2 ? 65535LL
                                         : sizeof(T) == 4 ? 4294967295LL : 9223372036854775807LL)
                                  : sizeof(T) == 1 ? 127LL
                                  : sizeof(T) == 2 ? 32767LL
                                  : sizeof(T) == 4 ? 2147483647LL : 9223372036854775807LL;
};

// Strict compare in index order (first index wins), from lowest / highest.
template <class T, bool IS_MAX, class IdxT = int>
struct IntArgOp {
    static constexpr bool kIndexed = true;
    static constexpr IdxT kNone = (IdxT)(sizeof(IdxT) == 4 ? 0x7fffffff : kSentinel);
    struct Acc { long long v; IdxT i; };
    using State = ArgSI;
    using Wide = IntArgOp<T, IS_MAX, long long>;
    __device__ static Acc init() { return {IS_MAX ? IntLimits<T>::lo : IntLimits<T>::hi, kNone}; }
    template <class I>
    __device__ static void acc(Acc& a, T x, I i, float) {
        const long long v = ikey(x);
        const bool t = IS_MAX ? (v > a.v) : (v < a.v);
        a.v = t ? v : a.v;
        a.i = t ? (IdxT)i : a.i;
    }
    __device__ static State state(Acc a) { return {a.v, a.i == kNone ? kSentinel : (long long)a.i}; }
    __device__ static State identity() { return {IS_MAX ? IntLimits<T>::lo : IntLimits<T>::hi, kSentinel}; }
    __device__ static State comb(State a, State b) {
        bool t = IS_MAX ? (b.v > a.v) : (b.v < a.v);
        t = t || (b.v == a.v && b.i < a.i);
        return t ? b : a;
    }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.v, m, kWave), __shfl_xor(s.i, m, kWave)}; }
};

template <class T, bool ANY>
struct IntBoolOp {
    static constexpr bool kIndexed = false;
    using Acc = int;
    using State = BoolS;
    using Wide = IntBoolOp;
    __device__ static Acc init() { return ANY ? 0 : 1; }
    template <class I>
    __device__ static void acc(Acc& a, T x, I, float) {
        if constexpr (ANY) a |= (x != T(0)) ? 1 : 0;
        else a &= (x != T(0)) ? 1 : 0;
    }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {ANY ? 0 : 1}; }
    __device__ static State comb(State a, State b) { return {ANY ? (a.b | b.b) : (a.b & b.b)}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.b, m, kWave)}; }
};

__device__ __forceinline__ void fin_write(const SumI& s, const Fin&, void* out, long long o) {
    ((long long*)out)[o] = s.s;
}

__device__ __forceinline__ void fin_write(const ArgSI& s, const Fin& f, void* out, long long o) {
    if (f.op == TPR_ARGMAX || f.op == TPR_ARGMIN) {
        ((long long*)out)[o] = (s.i == kSentinel) ? 0 : s.i;
        return;
    }
    switch (f.out_esize) {  // amax / amin: the input dtype
        case 1: ((unsigned char*)out)[o] = (unsigned char)s.v; break;
        case 2: ((short*)out)[o] = (short)s.v; break;
        case 4: ((int*)out)[o] = (int)s.v; break;
        default: ((long long*)out)[o] = f.out_umap ? (long long)((unsigned long long)s.v ^ 0x8000000000000000ull) : s.v;
    }
}

struct ArgsI {
    const void* in;
    // rows
    long long rows, R, row_stride;
    // cols
    long long outer, os, rs, inner, ncb;
    int S;
    void* out;
    void* part;
    Fin fin;
    long long idx_off;  // as RowArgs
    int partial;
    unsigned* tickets;  // as RowArgs (rows only)
};

template <class T, int NV>
struct alignas(16) Vec16 {
    T v[NV];
};

// 16-byte nontemporal load of NV elements (the row kernel's read-once
// stream).  Measured on MI355X: float64 full reductions of 2^27 elements 171 ->
// 155 us against plain loads; the column kernel keeps plain loads (nontemporal
// ones were 2-6% slower there: int32 sum over dim 1 of [64, 1024, 1024] 44.9
// against 42.4 us).  A runtime choice between the two is not possible here: the
// compiler merges the two otherwise identical loads of the branches into one
// and drops the nontemporal mark.
template <class T, int NV>
__device__ __forceinline__ Vec16<T, NV> ld16_nt(const Vec16<T, NV>* p) {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    Vec16<T, NV> t;
    const i32x4 r = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
    __builtin_memcpy(&t, &r, 16);
    return t;
}

template <class Op, int LANES>
__device__ __forceinline__ typename Op::State combine_lanes(typename Op::State st, int tid) {
    using State = typename Op::State;
    constexpr int BLK = LANES > kBlock ? LANES : kBlock;
    constexpr int SUBW = LANES < kWave ? LANES : kWave;
    st = group_reduce_sub_wave<Op, SUBW>(st);
    if constexpr (LANES > kWave) {
        constexpr int WPG = LANES / kWave;
        __shared__ State sh[BLK / kWave];
        const int w = tid / kWave;
        const int g = tid / LANES;
        if (__lane_id() == 0) sh[w] = st;
        __syncthreads();
        if (tid % LANES == 0) {
            State r = sh[g * WPG];
#pragma unroll
            for (int i = 1; i < WPG; ++i) r = Op::comb(r, sh[g * WPG + i]);
            st = r;
        }
    }
    return st;
}

// Row kernel for integer inputs: [rows, R], R contiguous; NV elements per
// 16-byte vector (1 = scalar loads).  Split s takes vectors s*LANES + l + k*S*LANES.
template <class Op, class T, int NV, int LANES>
__global__ __launch_bounds__(LANES > kBlock ? LANES : kBlock) void k_rows_i(ArgsI a) {
    using Acc = typename Op::Acc;
    constexpr int BLK = LANES > kBlock ? LANES : kBlock;
    constexpr int GROUPS = (LANES >= BLK) ? 1 : BLK / LANES;
    const float prm = a.fin.p;
    const int tid = threadIdx.x;
    const int g = tid / LANES;
    const int l = tid % LANES;
    const long long rb = blockIdx.x / a.S;
    const int s = blockIdx.x % a.S;
    const long long row = rb * GROUPS + g;
    Acc acc = Op::init();
    if (row < a.rows) {
        const T* p = static_cast<const T*>(a.in) + row * a.row_stride;
        const int R = (int)a.R;
        int tail = 0;
        if constexpr (NV > 1) {
            const int nv = R / NV;
            const Vec16<T, NV>* pv = reinterpret_cast<const Vec16<T, NV>*>(p);
            const int step = a.S * LANES;
            int v = s * LANES + l;
            // four vectors in flight per lane; each lane still visits its
            // elements in increasing index order
            for (; v + 3 * step < nv; v += 4 * step) {
                Vec16<T, NV> t[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) t[u] = ld16_nt(pv + v + u * step);
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int j = 0; j < NV; ++j) Op::acc(acc, t[u].v[j], (v + u * step) * NV + j, prm);
            }
            for (; v < nv; v += step) {
                const Vec16<T, NV> t = ld16_nt(pv + v);
#pragma unroll
                for (int j = 0; j < NV; ++j) Op::acc(acc, t.v[j], v * NV + j, prm);
            }
            tail = nv * NV;
        }
        for (int e = tail + s * LANES + l; e < R; e += a.S * LANES) Op::acc(acc, p[e], e, prm);
    }
    using State = typename Op::State;
    State st = combine_lanes<Op, LANES>(Op::state(acc), tid);
    if constexpr (GROUPS == 1) {
        if (a.tickets) {
            split_finish<Op, BLK>(st, reinterpret_cast<State*>(a.part), a.tickets + row, a.S, s, a.rows, row,
                                  [&](const State& r) { fin_write(r, a.fin, a.out, row); });
            return;
        }
    }
    if (l == 0 && row < a.rows) {
        if (!a.partial) fin_write(st, a.fin, a.out, row);
        else reinterpret_cast<typename Op::State*>(a.part)[(long long)s * a.rows + row] = shift_index(st, a.idx_off, 0);
    }
}

// Column kernel for integer inputs: [outer, R, inner], inner contiguous; TX
// threads across inner (NV columns each), 256/TX thread rows across R.
template <class Op, class T, int NV, int TX>
__global__ __launch_bounds__(kBlock) void k_cols_i(ArgsI a) {
    using Acc = typename Op::Acc;
    using State = typename Op::State;
    constexpr int TY = kBlock / TX;
    const float prm = a.fin.p;
    const int tid = threadIdx.x;
    const int tx = tid % TX;
    const int ty = tid / TX;
    const int s = blockIdx.x % a.S;
    const long long ob = blockIdx.x / a.S;
    const long long cb = ob % a.ncb;
    const long long o = ob / a.ncb;
    const long long col0 = (cb * TX + tx) * NV;
    Acc acc[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) acc[j] = Op::init();
    if (col0 < a.inner) {
        const T* base = static_cast<const T*>(a.in) + o * a.os + col0;
        const int R = (int)a.R;
        const int rstep = TY * a.S;
        if (NV > 1 && col0 + NV <= a.inner) {
            int r = s * TY + ty;
            // four rows in flight per thread, visited in increasing row order
            for (; r + 3 * rstep < R; r += 4 * rstep) {
                Vec16<T, NV> t[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    t[u] = *reinterpret_cast<const Vec16<T, NV>*>(base + (long long)(r + u * rstep) * a.rs);
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int j = 0; j < NV; ++j) Op::acc(acc[j], t[u].v[j], r + u * rstep, prm);
            }
            for (; r < R; r += rstep) {
                const Vec16<T, NV> t = *reinterpret_cast<const Vec16<T, NV>*>(base + (long long)r * a.rs);
#pragma unroll
                for (int j = 0; j < NV; ++j) Op::acc(acc[j], t.v[j], r, prm);
            }
        } else {
            const int nj = (int)min((long long)NV, a.inner - col0);
            for (int r = s * TY + ty; r < R; r += rstep) {
                const T* q = base + (long long)r * a.rs;
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    if (j < nj) Op::acc(acc[j], q[j], r, prm);
            }
        }
    }
    State st[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) st[j] = Op::state(acc[j]);
    if constexpr (TY > 1) {
        __shared__ State sh[(TY > 1 ? TY / 2 : 1) * TX * NV];
#pragma unroll
        for (int half = TY / 2; half >= 1; half /= 2) {
            if (ty >= half && ty < 2 * half) {
#pragma unroll
                for (int j = 0; j < NV; ++j) sh[((ty - half) * TX + tx) * NV + j] = st[j];
            }
            __syncthreads();
            if (ty < half) {
#pragma unroll
                for (int j = 0; j < NV; ++j) st[j] = Op::comb(st[j], sh[(ty * TX + tx) * NV + j]);
            }
            __syncthreads();
        }
    }
    if (ty == 0) {
        const long long nout = a.outer * a.inner;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const long long c = col0 + j;
            if (c < a.inner) {
                const long long oi = o * a.inner + c;
                if (!a.partial) fin_write(st[j], a.fin, a.out, oi);
                else reinterpret_cast<State*>(a.part)[(long long)s * nout + oi] = shift_index(st[j], a.idx_off, 0);
            }
        }
    }
}

struct GenArgsI {
    const void* in;
    int nk, nr;
    long long ksz[TPR_MAX_DIMS], kst[TPR_MAX_DIMS];
    long long rsz[TPR_MAX_DIMS], rst[TPR_MAX_DIMS];
    long long nout, count, seg;
    int S;
    void* out;
    void* part;
    Fin fin;
};

template <class Op, class T>
__global__ __launch_bounds__(kBlock) void k_general_i(GenArgsI a) {
    using Acc = typename Op::Acc;
    using State = typename Op::State;
    const float prm = a.fin.p;
    const long long o = blockIdx.x / a.S;
    const int s = blockIdx.x % a.S;
    long long base = 0;
    {
        long long rem = o;
        for (int d = a.nk - 1; d >= 0; --d) {
            base += (rem % a.ksz[d]) * a.kst[d];
            rem /= a.ksz[d];
        }
    }
    const T* in = static_cast<const T*>(a.in);
    Acc acc = Op::init();
    const long long beg = (long long)s * a.seg;
    const long long end = min(a.count, beg + a.seg);
    for (long long j = beg + threadIdx.x; j < end; j += kBlock) {
        long long rem = j, off = 0;
        for (int d = a.nr - 1; d >= 0; --d) {
            off += (rem % a.rsz[d]) * a.rst[d];
            rem /= a.rsz[d];
        }
        Op::acc(acc, in[base + off], j, prm);
    }
    State st = block_reduce<Op>(Op::state(acc));
    if (threadIdx.x == 0) {
        if (a.S == 1) fin_write(st, a.fin, a.out, o);
        else reinterpret_cast<State*>(a.part)[(long long)s * a.nout + o] = st;
    }
}

// ---------------------------------------------------------------------------
// Float64 inputs: the reference computes in double for Float64 tensors
// (AccumulateType<double> = double, ReductionKernels.cpp:27-35; its CUDA path
// reduces Float64 through cuDNN with CUDNN_DATA_DOUBLE,
// ReductionKernels.cu:155-165).  The integer kernels above are generic in the
// element type, so Float64 reuses them (two doubles per 16-byte vector) with
// these double policies: sums / products / norms in double, max / min /
// argmax / argmin with the same strict compare (NaN ignored, first index
// wins), Welford in double, all / any as x != 0.
// ---------------------------------------------------------------------------
template <bool PROD>
struct F64SumOp {
    static constexpr bool kIndexed = false;
    using Acc = double;
    using State = SumS;
    using Wide = F64SumOp;
    __device__ static Acc init() { return PROD ? 1.0 : 0.0; }
    template <class I>
    __device__ static void acc(Acc& a, double x, I, float) { a = PROD ? a * x : a + x; }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {PROD ? 1.0 : 0.0}; }
    __device__ static State comb(State a, State b) { return {PROD ? a.s * b.s : a.s + b.s}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.s, m, kWave)}; }
};

template <int KIND>  // 1: |x|, 2: x*x, 0: pow(|x|, p)
struct F64NormOp {
    static constexpr bool kIndexed = false;
    using Acc = double;
    using State = SumS;
    using Wide = F64NormOp;
    __device__ static Acc init() { return 0.0; }
    template <class I>
    __device__ static void acc(Acc& a, double x, I, float p) {
        if constexpr (KIND == 1) a += fabs(x);
        else if constexpr (KIND == 2) a = fma(x, x, a);
        else a += pow(fabs(x), (double)p);
    }
    __device__ static State state(Acc a) { return {a}; }
    __device__ static State identity() { return {0.0}; }
    __device__ static State comb(State a, State b) { return {a.s + b.s}; }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.s, m, kWave)}; }
};

struct ArgSD { double v; long long i; };

template <bool IS_MAX, class IdxT = int, bool ABS = false>
struct F64ArgOp {
    static constexpr bool kIndexed = true;
    static constexpr IdxT kNone = (IdxT)(sizeof(IdxT) == 4 ? 0x7fffffff : kSentinel);
    struct Acc { double v; IdxT i; };
    using State = ArgSD;
    using Wide = F64ArgOp<IS_MAX, long long, ABS>;
    __device__ static Acc init() { return {IS_MAX ? -(double)INFINITY : (double)INFINITY, kNone}; }
    template <class I>
    __device__ static void acc(Acc& a, double x, I i, float) {
        if constexpr (ABS) x = fabs(x);
        const bool t = IS_MAX ? (x > a.v) : (x < a.v);
        a.v = t ? x : a.v;
        a.i = t ? (IdxT)i : a.i;
    }
    __device__ static State state(Acc a) { return {a.v, a.i == kNone ? kSentinel : (long long)a.i}; }
    __device__ static State identity() { return {IS_MAX ? -(double)INFINITY : (double)INFINITY, kSentinel}; }
    __device__ static State comb(State a, State b) {
        bool t = IS_MAX ? (b.v > a.v) : (b.v < a.v);
        t = t || (b.v == a.v && b.i < a.i);
        return t ? b : a;
    }
    __device__ static State shfl(State s, int m) { return {__shfl_xor(s.v, m, kWave), __shfl_xor(s.i, m, kWave)}; }
};

struct WelAccD { double k; long long n; double s1, s2; };

// Welford over double inputs: per-thread sums shifted by the thread's first
// element, merged with the same Chan combine as WelfordOp.
struct F64WelfordOp {
    using Acc = WelAccD;
    using State = WelS;
    using Wide = F64WelfordOp;
    __device__ static Acc init() { return {0.0, 0, 0.0, 0.0}; }
    template <class I>
    __device__ static void acc(Acc& a, double x, I, float) {
        a.k = (a.n == 0) ? x : a.k;
        const double d = x - a.k;
        a.s1 += d;
        a.s2 = fma(d, d, a.s2);
        a.n += 1;
    }
    __device__ static State state(Acc a) {
        if (a.n == 0) return {0.0, 0.0, 0.0};
        const double n = (double)a.n;
        const double m = a.s1 / n;
        return {n, a.k + m, fmax(0.0, a.s2 - a.s1 * m)};
    }
    __device__ static State identity() { return WelfordOp::identity(); }
    __device__ static State comb(State a, State b) { return WelfordOp::comb(a, b); }
    __device__ static State shfl(State s, int m) { return WelfordOp::shfl(s, m); }
};

__device__ __forceinline__ void fin_write(const ArgSD& s, const Fin& f, void* out, long long o) {
    if (f.op == TPR_AMAX || f.op == TPR_AMIN || f.op == TPR_NORM) ((double*)out)[o] = s.v;
    else ((long long*)out)[o] = (s.i == kSentinel) ? 0 : s.i;
}

int esize_of(int dt) {
    switch (dt) {
        case TPR_UINT8: case TPR_INT8: case TPR_BOOL: return 1;
        case TPR_INT16: case TPR_UINT16: return 2;
        case TPR_INT32: case TPR_UINT32: return 4;
        case TPR_INT64: case TPR_UINT64: case TPR_FLOAT64: return 8;
        default: return 0;
    }
}

size_t f64_state_size(int op, double p) {
    switch (op) {
        case TPR_SUM: case TPR_MEAN: case TPR_PROD: return sizeof(SumS);
        case TPR_NORM: return std::isinf(p) ? sizeof(ArgSD) : sizeof(SumS);
        case TPR_ALL: case TPR_ANY: return sizeof(BoolS);
        case TPR_AMAX: case TPR_AMIN: case TPR_ARGMAX: case TPR_ARGMIN: return sizeof(ArgSD);
        default: return sizeof(WelS);
    }
}

size_t int_state_size(int op) {
    switch (op) {
        case TPR_SUM: case TPR_PROD: return sizeof(SumI);
        case TPR_MEAN: return sizeof(SumS);
        case TPR_ALL: case TPR_ANY: return sizeof(BoolS);
        default: return sizeof(ArgSI);
    }
}

// Re-tunes a float plan for integer elements of `es` bytes (NV = 16/es per
// vector).  Rows: lanes rounded up to 16/64/256/1024.  Columns: 256-thread
// workgroups, TX 64/128/256, splits recomputed on NV-wide columns.  The
// workspace size depends on the descriptor only, never on the pointer.
void adapt_plan_int(Plan& p, const tpr_reduce_desc* d, const void* in, int es) {
    const int NV = 16 / es;
    const bool aligned16 = (reinterpret_cast<uintptr_t>(in) & 15u) == 0;
    const auto& dev = device_info();
    const long long target = (long long)dev.cus * 512;
    p.state_bytes = d->in_dtype == TPR_FLOAT64 ? f64_state_size(d->op, d->p) : int_state_size(d->op);
    p.reg_wpr = 0;  // the register-row kernels read float32 only
    p.var_nv = 0;
    if (p.kind == P_ROWS) {
        p.vec = (aligned16 && (p.rows == 1 || p.row_stride % NV == 0) && p.R >= NV) ? NV : 1;
        int L = 16;
        while (L < p.lanes && L < 1024) L *= 4;
        p.lanes = L;
        if (knobs().splits <= 0) {
            const long long threads = p.rows * p.lanes;
            const long long vecs = std::max(1LL, ceil_div(p.R, (long long)NV * p.lanes));
            p.S = threads < target ? std::max(1LL, std::min(ceil_div(target, threads), vecs)) : 1;
        }
    } else if (p.kind == P_COLS) {
        p.vec = (aligned16 && p.rs % NV == 0 && (p.outer == 1 || p.os % NV == 0) && p.inner >= NV) ? NV : 1;
        p.colblock = kBlock;
        const long long colsv = ceil_div(p.inner, NV);
        if (!(knobs().tx == 64 || knobs().tx == 128 || knobs().tx == 256))
            p.tx = (p.outer * ceil_div(colsv, 256) * kBlock >= target || p.R < 16) ? 256 : 64;
        p.ncb = ceil_div(ceil_div(p.inner, p.vec), p.tx);
        const long long ty = kBlock / p.tx;
        const long long threads = p.outer * ceil_div(colsv, p.tx) * kBlock;
        long long S = 1;
        if (threads < target) S = std::min(ceil_div(target, threads), std::max(1LL, p.R / (ty * 8)));
        if (knobs().splits > 0) S = knobs().splits;
        p.S = std::max(1LL, std::min(S, ceil_div(p.R, ty)));
    }
    p.ws = (p.S > 1 || p.nchunk > 1) ? (size_t)(p.S * p.nchunk) * (size_t)p.nout * p.state_bytes : 0;
}

template <class Op, class T>
int launch_int_layout(const Plan& p, const void* in, void* out, void* ws, Fin fin, hipStream_t st,
                      unsigned* tickets = nullptr) {
    constexpr int NV = 16 / (int)sizeof(T);
    if (p.kind == P_ROWS) {
        ArgsI a{};
        a.in = in; a.rows = p.rows; a.R = p.R; a.row_stride = p.row_stride;
        a.S = (int)p.S; a.out = out; a.part = ws; a.fin = fin;
        a.idx_off = p.idx_off; a.partial = p.partial || p.S > 1;
        a.tickets = tickets;
        const long long groups = (p.lanes >= kBlock) ? 1 : kBlock / p.lanes;
        const dim3 grid(ceil_div(p.rows, groups) * p.S);
        const dim3 blk(p.lanes > kBlock ? p.lanes : kBlock);
#define TPR_ROWS_I(L)                                                                               \
    case L:                                                                                         \
        if (p.vec > 1) hipLaunchKernelGGL((k_rows_i<Op, T, NV, L>), grid, blk, 0, st, a);          \
        else hipLaunchKernelGGL((k_rows_i<Op, T, 1, L>), grid, blk, 0, st, a);                     \
        break;
        switch (p.lanes) {
            TPR_ROWS_I(16)
            TPR_ROWS_I(64)
            TPR_ROWS_I(256)
            TPR_ROWS_I(1024)
            default: return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: lanes must be 16/64/256/1024 for integer inputs");
        }
#undef TPR_ROWS_I
    } else if (p.kind == P_COLS) {
        ArgsI a{};
        a.in = in; a.outer = p.outer; a.os = p.os; a.R = p.R; a.rs = p.rs; a.inner = p.inner; a.ncb = p.ncb;
        a.S = (int)p.S; a.out = out; a.part = ws; a.fin = fin;
        a.idx_off = p.idx_off; a.partial = p.partial || p.S > 1;
        const dim3 grid(p.outer * p.ncb * p.S);
#define TPR_COLS_I(TXV)                                                                             \
    if (p.tx == TXV) {                                                                              \
        if (p.vec > 1) hipLaunchKernelGGL((k_cols_i<Op, T, NV, TXV>), grid, dim3(kBlock), 0, st, a); \
        else hipLaunchKernelGGL((k_cols_i<Op, T, 1, TXV>), grid, dim3(kBlock), 0, st, a);          \
    }
        TPR_COLS_I(256)
        else TPR_COLS_I(128)
        else TPR_COLS_I(64)
        else return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: tx must be 64, 128 or 256");
#undef TPR_COLS_I
    } else {
        GenArgsI a{};
        a.in = in; a.nk = p.nk; a.nr = p.nr;
        for (int i = 0; i < TPR_MAX_DIMS; ++i) {
            a.ksz[i] = i < p.nk ? p.ksz[i] : 1;
            a.kst[i] = i < p.nk ? p.kst[i] : 0;
            a.rsz[i] = i < p.nr ? p.rsz[i] : 1;
            a.rst[i] = i < p.nr ? p.rst[i] : 0;
        }
        a.nout = p.nout; a.count = p.count; a.seg = p.seg; a.S = (int)p.S;
        a.out = out; a.part = ws; a.fin = fin;
        hipLaunchKernelGGL((k_general_i<typename Op::Wide, T>), dim3(p.nout * p.S), dim3(kBlock), 0, st, a);
    }
    return check_launch("k_reduce_int");
}

template <class Op, class T>
int run_int_op(const Plan& p, const void* in, void* out, void* ws, Fin fin, hipStream_t st) {
    if (p.nchunk > 1)
        return run_chunks<Op>(p, in, sizeof(T), out, ws, fin, st, [&](const Plan& pc, const void* ic, void* wc) {
            return launch_int_layout<Op, T>(pc, ic, out, wc, fin, st);
        });
    unsigned* tk = fused_split_tickets(p, st);
    int rc = launch_int_layout<Op, T>(p, in, out, ws, fin, st, tk);
    if (rc != TPR_OK) return rc;
    if (p.S > 1 && !tk) rc = launch_finalize<Op>(p, out, ws, fin, st);
    return rc;
}

template <class T>
int run_int_t(int op, const Plan& p, const void* in, void* out, void* ws, Fin fin, hipStream_t st) {
    switch (op) {
        case TPR_SUM: return run_int_op<IntSumOp<T, false>, T>(p, in, out, ws, fin, st);
        case TPR_MEAN: return run_int_op<IntMeanOp<T>, T>(p, in, out, ws, fin, st);
        case TPR_PROD: return run_int_op<IntSumOp<T, true>, T>(p, in, out, ws, fin, st);
        case TPR_AMAX: case TPR_ARGMAX: return run_int_op<IntArgOp<T, true>, T>(p, in, out, ws, fin, st);
        case TPR_AMIN: case TPR_ARGMIN: return run_int_op<IntArgOp<T, false>, T>(p, in, out, ws, fin, st);
        case TPR_ALL: return run_int_op<IntBoolOp<T, false>, T>(p, in, out, ws, fin, st);
        case TPR_ANY: return run_int_op<IntBoolOp<T, true>, T>(p, in, out, ws, fin, st);
        default: return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_reduce: op not implemented for integer inputs");
    }
}

int run_f64(const tpr_reduce_desc* d, const Plan& p, const void* in, void* out, void* ws, Fin fin, hipStream_t st) {
    using T = double;
    switch (d->op) {
        case TPR_SUM: case TPR_MEAN: return run_int_op<F64SumOp<false>, T>(p, in, out, ws, fin, st);
        case TPR_PROD: return run_int_op<F64SumOp<true>, T>(p, in, out, ws, fin, st);
        case TPR_AMAX: case TPR_ARGMAX: return run_int_op<F64ArgOp<true>, T>(p, in, out, ws, fin, st);
        case TPR_AMIN: case TPR_ARGMIN: return run_int_op<F64ArgOp<false>, T>(p, in, out, ws, fin, st);
        case TPR_ALL: return run_int_op<IntBoolOp<T, false>, T>(p, in, out, ws, fin, st);
        case TPR_ANY: return run_int_op<IntBoolOp<T, true>, T>(p, in, out, ws, fin, st);
        case TPR_NORM:
            if (std::isinf(d->p)) {
                if (d->p > 0) return run_int_op<F64ArgOp<true, int, true>, T>(p, in, out, ws, fin, st);
                return run_int_op<F64ArgOp<false, int, true>, T>(p, in, out, ws, fin, st);
            }
            if (d->p == 1.0) return run_int_op<F64NormOp<1>, T>(p, in, out, ws, fin, st);
            if (d->p == 2.0) return run_int_op<F64NormOp<2>, T>(p, in, out, ws, fin, st);
            return run_int_op<F64NormOp<0>, T>(p, in, out, ws, fin, st);
        case TPR_VAR: case TPR_STD: return run_int_op<F64WelfordOp, T>(p, in, out, ws, fin, st);
        default: return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce: op not implemented for float64 inputs");
    }
}

int run_int(const tpr_reduce_desc* d, const Plan& p, const void* in, void* out, void* ws, Fin fin, hipStream_t st) {
    switch (d->in_dtype) {
        case TPR_UINT8: case TPR_BOOL: return run_int_t<unsigned char>(d->op, p, in, out, ws, fin, st);
        case TPR_INT8: return run_int_t<signed char>(d->op, p, in, out, ws, fin, st);
        case TPR_INT16: return run_int_t<short>(d->op, p, in, out, ws, fin, st);
        case TPR_INT32: return run_int_t<int>(d->op, p, in, out, ws, fin, st);
        case TPR_UINT16: return run_int_t<unsigned short>(d->op, p, in, out, ws, fin, st);
        case TPR_UINT32: return run_int_t<unsigned int>(d->op, p, in, out, ws, fin, st);
        case TPR_UINT64: return run_int_t<unsigned long long>(d->op, p, in, out, ws, fin, st);
        default: return run_int_t<long long>(d->op, p, in, out, ws, fin, st);
    }
}


// ---------------------------------------------------------------------------
// Median (median_kernel, ReductionKernels.cpp:874-901: the (n-1)/2-th smallest
// element).  Exact radix select over ascending sortable keys in three passes of
// 11/11/10 bits.  Each pass streams the input once: workgroups build LDS
// histograms of the keys that match the prefix found so far and store them as
// partials (no atomics in global memory, nothing to clear beforehand); one
// workgroup then sums the partials and picks the digit.
// ---------------------------------------------------------------------------
constexpr int kMedBins = 2048;
constexpr int kMedSelT = 1024;

struct MedState {
    uint32_t prefix;
    uint32_t pmask;
    long long kk;  // rank still to skip inside the current prefix
};

struct MedArgs {
    const float* in;
    long long n;
    int G;            // histogram workgroups
    int vec;          // 16-byte aligned input
    uint32_t* hist;   // [G][kMedBins]
    MedState* st;
    float* out;
};

// Ascending sortable key: -0.0 -> +0.0, every NaN -> one canonical NaN above +inf.
__device__ __forceinline__ uint32_t asc_key(float f) {
    uint32_t u = __float_as_uint(f);
    u = ((u & 0x7fffffffu) > 0x7f800000u) ? 0x7fc00000u : u;
    u = (u == 0x80000000u) ? 0u : u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int PASS>
__global__ __launch_bounds__(kBlock) void k_med_hist(MedArgs a) {
    constexpr int shift = PASS == 0 ? 21 : (PASS == 1 ? 10 : 0);
    constexpr uint32_t dmask = PASS == 2 ? 1023u : 2047u;
    __shared__ uint32_t h[kMedBins];
    for (int i = threadIdx.x; i < kMedBins; i += kBlock) h[i] = 0;
    uint32_t prefix = 0, pmask = 0;
    if (PASS > 0) {
        prefix = a.st->prefix;
        pmask = a.st->pmask;
    }
    __syncthreads();
    auto add = [&](float x) {
        const uint32_t k = asc_key(x);
        if ((k & pmask) == prefix) atomicAdd(&h[(k >> shift) & dmask], 1u);
    };
    const long long tid = (long long)blockIdx.x * kBlock + threadIdx.x;
    const long long nthr = (long long)a.G * kBlock;
    long long tail = 0;
    if (a.vec) {
        const long long nv = a.n >> 2;
        const float4* v = reinterpret_cast<const float4*>(a.in);
        for (long long i = tid; i < nv; i += nthr) {
            const float4 t = v[i];
            add(t.x);
            add(t.y);
            add(t.z);
            add(t.w);
        }
        tail = nv << 2;
    }
    for (long long i = tail + tid; i < a.n; i += nthr) add(a.in[i]);
    __syncthreads();
    uint32_t* dst = a.hist + (long long)blockIdx.x * kMedBins;
    for (int i = threadIdx.x; i < kMedBins; i += kBlock) dst[i] = h[i];
}

template <int PASS>
__global__ __launch_bounds__(kMedSelT) void k_med_select(MedArgs a) {
    constexpr int shift = PASS == 0 ? 21 : (PASS == 1 ? 10 : 0);
    constexpr uint32_t dmask = PASS == 2 ? 1023u : 2047u;
    __shared__ long long wsum[kMedSelT / kWave];
    __shared__ MedState next;
    const int t = threadIdx.x;
    // thread t owns bins 2t and 2t+1
    long long c0 = 0, c1 = 0;
    for (int g = 0; g < a.G; ++g) {
        const uint32_t* hg = a.hist + (long long)g * kMedBins;
        c0 += hg[2 * t];
        c1 += hg[2 * t + 1];
    }
    MedState cur;
    if (PASS == 0) cur = {0u, 0u, (a.n - 1) / 2};
    else cur = *a.st;
    // exclusive prefix sum of (c0 + c1) over threads, in bin order
    const long long own = c0 + c1;
    long long inc = own;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const long long y = __shfl_up(inc, d, kWave);
        if (__lane_id() >= d) inc += y;
    }
    const int w = t / kWave;
    if (__lane_id() == kWave - 1) wsum[w] = inc;
    __syncthreads();
    long long before = 0;
    for (int i = 0; i < w; ++i) before += wsum[i];
    const long long excl = before + inc - own;
    const long long kk = cur.kk;
    if (kk >= excl && kk < excl + own) {
        const bool first = kk < excl + c0;
        const uint32_t digit = 2u * t + (first ? 0u : 1u);
        next.prefix = cur.prefix | (digit << shift);
        next.pmask = cur.pmask | (dmask << shift);
        next.kk = kk - excl - (first ? 0 : c0);
    }
    __syncthreads();
    if (t == 0) {
        if (PASS < 2) {
            *a.st = next;
        } else {
            const uint32_t key = next.prefix;
            const uint32_t bits = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
            a.out[0] = __uint_as_float(bits);
        }
    }
}

__global__ void k_med_fill(float* out, float v) { out[0] = v; }

// Median of the other dtypes (float64, every integer width, bool; the
// reference's median_kernel instantiates every scalar type): the same radix
// select on an ascending key of the element's width, 11 bits per pass from the
// top; the last pass writes the element back in its own dtype.
struct MedStateG {
    unsigned long long prefix;
    unsigned long long pmask;
    long long kk;
};

template <class T>
struct MedKey {
    static constexpr int kBits = (int)sizeof(T) * 8;
    static constexpr int kPasses = (kBits + 10) / 11;
    __device__ static unsigned long long key(T x) {
        if constexpr (std::is_same<T, double>::value) {
            unsigned long long u = (unsigned long long)__double_as_longlong(x);
            if ((u & 0x7fffffffffffffffull) > 0x7ff0000000000000ull) u = 0x7ff8000000000000ull;  // one NaN
            if (u == 0x8000000000000000ull) u = 0;                                            // -0 -> +0
            return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
        } else if constexpr (T(-1) < T(0)) {  // signed: flip the sign bit
            return (unsigned long long)(typename std::make_unsigned<T>::type)x ^ (1ull << (kBits - 1));
        } else {
            return (unsigned long long)x;
        }
    }
    __device__ static T value(unsigned long long k) {
        if constexpr (std::is_same<T, double>::value) {
            const unsigned long long u = (k & 0x8000000000000000ull) ? (k & 0x7fffffffffffffffull) : ~k;
            return __longlong_as_double((long long)u);
        } else if constexpr (T(-1) < T(0)) {
            return (T)(typename std::make_unsigned<T>::type)(k ^ (1ull << (kBits - 1)));
        } else {
            return (T)k;
        }
    }
};

template <class T, int PASS>
struct MedPass {
    static constexpr int hi = MedKey<T>::kBits - 11 * PASS;
    static constexpr int w = hi < 11 ? hi : 11;
    static constexpr int shift = hi - w;
    static constexpr unsigned long long dmask = (1ull << w) - 1ull;
};

struct MedArgsG {
    const void* in;
    long long n;
    int G;
    uint32_t* hist;  // [G][kMedBins]
    MedStateG* st;
    void* out;
};

template <class T, int PASS>
__global__ __launch_bounds__(kBlock) void k_medg_hist(MedArgsG a) {
    using P = MedPass<T, PASS>;
    __shared__ uint32_t h[kMedBins];
    for (int i = threadIdx.x; i < kMedBins; i += kBlock) h[i] = 0;
    unsigned long long prefix = 0, pmask = 0;
    if (PASS > 0) {
        prefix = a.st->prefix;
        pmask = a.st->pmask;
    }
    __syncthreads();
    const T* in = static_cast<const T*>(a.in);
    const long long nthr = (long long)a.G * kBlock;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < a.n; i += nthr) {
        const unsigned long long k = MedKey<T>::key(in[i]);
        if ((k & pmask) == prefix) atomicAdd(&h[(k >> P::shift) & P::dmask], 1u);
    }
    __syncthreads();
    uint32_t* dst = a.hist + (long long)blockIdx.x * kMedBins;
    for (int i = threadIdx.x; i < kMedBins; i += kBlock) dst[i] = h[i];
}

template <class T, int PASS>
__global__ __launch_bounds__(kMedSelT) void k_medg_select(MedArgsG a) {
    using P = MedPass<T, PASS>;
    __shared__ long long wsum[kMedSelT / kWave];
    __shared__ MedStateG next;
    const int t = threadIdx.x;
    long long c0 = 0, c1 = 0;  // thread t owns bins 2t and 2t+1
    for (int g = 0; g < a.G; ++g) {
        const uint32_t* hg = a.hist + (long long)g * kMedBins;
        c0 += hg[2 * t];
        c1 += hg[2 * t + 1];
    }
    MedStateG cur;
    if (PASS == 0) cur = {0ull, 0ull, (a.n - 1) / 2};
    else cur = *a.st;
    const long long own = c0 + c1;
    long long inc = own;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const long long y = __shfl_up(inc, d, kWave);
        if (__lane_id() >= d) inc += y;
    }
    const int w = t / kWave;
    if (__lane_id() == kWave - 1) wsum[w] = inc;
    __syncthreads();
    long long before = 0;
    for (int i = 0; i < w; ++i) before += wsum[i];
    const long long excl = before + inc - own;
    const long long kk = cur.kk;
    if (kk >= excl && kk < excl + own) {
        const bool first = kk < excl + c0;
        const unsigned long long digit = 2ull * t + (first ? 0ull : 1ull);
        next.prefix = cur.prefix | (digit << P::shift);
        next.pmask = cur.pmask | (P::dmask << P::shift);
        next.kk = kk - excl - (first ? 0 : c0);
    }
    __syncthreads();
    if (t == 0) {
        if (PASS + 1 < MedKey<T>::kPasses) *a.st = next;
        else static_cast<T*>(a.out)[0] = MedKey<T>::value(next.prefix);
    }
}

template <class T, int PASS>
void launch_medg(const MedArgsG& a, hipStream_t st) {
    if constexpr (PASS < MedKey<T>::kPasses) {
        hipLaunchKernelGGL((k_medg_hist<T, PASS>), dim3(a.G), dim3(kBlock), 0, st, a);
        hipLaunchKernelGGL((k_medg_select<T, PASS>), dim3(1), dim3(kMedSelT), 0, st, a);
        launch_medg<T, PASS + 1>(a, st);
    }
}

size_t median_ws_bytes(long long n, int* G) {
    const long long g = std::max(1LL, std::min((long long)device_info().cus * 2, (n + 4095) / 4096));
    if (G) *G = (int)g;
    return 256 + (size_t)g * kMedBins * sizeof(uint32_t);
}

template <class T>
int run_median_g(const Plan& p, const void* in, void* out, void* ws, hipStream_t st) {
    MedArgsG a;
    a.in = in;
    a.n = p.count;
    median_ws_bytes(p.count, &a.G);
    a.st = static_cast<MedStateG*>(ws);
    a.hist = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + 256);
    a.out = out;
    launch_medg<T, 0>(a, st);
    return check_launch("k_medg");
}

int run_median(const tpr_reduce_desc* d, const Plan& p, const void* vin, void* out, void* ws, size_t ws_bytes,
               hipStream_t st) {
    const float* in = static_cast<const float*>(vin);
    if (d->in_dtype != TPR_FLOAT32) {
        if (p.count == 0) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: median of an empty non-float32 input");
        if (!(p.kind == P_ROWS && p.rows == 1))
            return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce: median needs a contiguous view (make it dense first)");
        if (ws == nullptr || ws_bytes < median_ws_bytes(p.count, nullptr))
            return fail(TPR_ERR_WORKSPACE, "tpr_reduce: workspace too small for median");
        switch (d->in_dtype) {
            case TPR_FLOAT64: return run_median_g<double>(p, vin, out, ws, st);
            case TPR_INT8: return run_median_g<signed char>(p, vin, out, ws, st);
            case TPR_INT16: return run_median_g<short>(p, vin, out, ws, st);
            case TPR_INT32: return run_median_g<int>(p, vin, out, ws, st);
            case TPR_INT64: return run_median_g<long long>(p, vin, out, ws, st);
            case TPR_UINT16: return run_median_g<unsigned short>(p, vin, out, ws, st);
            case TPR_UINT32: return run_median_g<unsigned int>(p, vin, out, ws, st);
            case TPR_UINT64: return run_median_g<unsigned long long>(p, vin, out, ws, st);
            default: return run_median_g<unsigned char>(p, vin, out, ws, st);  // UINT8, BOOL (0 / 1)
        }
    }
    if (p.count == 0) {
        hipLaunchKernelGGL(k_med_fill, dim3(1), dim3(1), 0, st, static_cast<float*>(out), __builtin_nanf(""));
        return check_launch("k_med_fill");
    }
    if (!(p.kind == P_ROWS && p.rows == 1))
        return fail(TPR_ERR_NOT_IMPLEMENTED, "tpr_reduce: median needs a contiguous view (make it dense first)");
    int G = 1;
    const size_t need = median_ws_bytes(p.count, &G);
    if (ws == nullptr || ws_bytes < need)
        return fail(TPR_ERR_WORKSPACE, "tpr_reduce: workspace too small (need " + std::to_string(need) + " bytes)");
    MedArgs a;
    a.in = in;
    a.n = p.count;
    a.G = G;
    a.vec = (reinterpret_cast<uintptr_t>(in) & 15u) == 0;
    a.st = static_cast<MedState*>(ws);
    a.hist = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + 256);
    a.out = static_cast<float*>(out);
    hipLaunchKernelGGL(k_med_hist<0>, dim3(G), dim3(kBlock), 0, st, a);
    hipLaunchKernelGGL(k_med_select<0>, dim3(1), dim3(kMedSelT), 0, st, a);
    hipLaunchKernelGGL(k_med_hist<1>, dim3(G), dim3(kBlock), 0, st, a);
    hipLaunchKernelGGL(k_med_select<1>, dim3(1), dim3(kMedSelT), 0, st, a);
    hipLaunchKernelGGL(k_med_hist<2>, dim3(G), dim3(kBlock), 0, st, a);
    hipLaunchKernelGGL(k_med_select<2>, dim3(1), dim3(kMedSelT), 0, st, a);
    return check_launch("k_med");
}

}  // namespace
}  // namespace tpr

extern "C" {

size_t tpr_reduce_workspace_bytes(const tpr_reduce_desc* desc) {
    if (tpr::validate(desc) != TPR_OK) return 0;
    // alignment does not change the workspace size; plan with an aligned pointer
    tpr::Plan p = tpr::make_plan(desc, nullptr);
    if (desc->op == TPR_MEDIAN) return p.count > 0 ? tpr::median_ws_bytes(p.count, nullptr) : 0;
    if (desc->in_dtype != TPR_FLOAT32) tpr::adapt_plan_int(p, desc, nullptr, tpr::esize_of(desc->in_dtype));
    return p.ws;
}

int tpr_reduce(const tpr_reduce_desc* desc, const void* in, void* out, void* workspace,
               size_t workspace_bytes, void* stream) {
    using namespace tpr;
    int rc = validate(desc);
    if (rc != TPR_OK) return rc;
    Plan p = make_plan(desc, in);
    if (p.nout == 0) return TPR_OK;
    if (!out) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: null output");
    if (!in && p.count > 0) return fail(TPR_ERR_INVALID_ARG, "tpr_reduce: null input");
    if (desc->op == TPR_MEDIAN)
        return run_median(desc, p, in, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
    const bool int_in = desc->in_dtype != TPR_FLOAT32;
    if (int_in) adapt_plan_int(p, desc, in, esize_of(desc->in_dtype));
    if (p.ws > 0 && (workspace == nullptr || workspace_bytes < p.ws))
        return fail(TPR_ERR_WORKSPACE, "tpr_reduce: workspace too small (need " +
                                           std::to_string(p.ws) + " bytes)");
    Fin fin;
    fin.op = desc->op;
    fin.out_f64 = desc->out_dtype == TPR_FLOAT64;
    fin.count = (double)(desc->count_override > 0 ? desc->count_override : p.count);
    fin.corr = (double)desc->correction;
    fin.p = (float)desc->p;
    fin.inv_p = 1.0 / desc->p;
    fin.out_esize = int_in ? esize_of(desc->in_dtype) : 4;
    fin.out_umap = desc->in_dtype == TPR_UINT64 ? 1 : 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (desc->in_dtype == TPR_FLOAT64) return run_f64(desc, p, in, out, workspace, fin, st);
    if (int_in) return run_int(desc, p, in, out, workspace, fin, st);
    const float* x = static_cast<const float*>(in);
    switch (desc->op) {
        case TPR_SUM: case TPR_MEAN: return run<SumOp>(p, x, out, workspace, fin, st);
        case TPR_PROD: return run<ProdOp>(p, x, out, workspace, fin, st);
        case TPR_AMAX: case TPR_ARGMAX: return run<ArgOp<true>>(p, x, out, workspace, fin, st);
        case TPR_AMIN: case TPR_ARGMIN: return run<ArgOp<false>>(p, x, out, workspace, fin, st);
        case TPR_ALL: return run<BoolOp<false>>(p, x, out, workspace, fin, st);
        case TPR_ANY: return run<BoolOp<true>>(p, x, out, workspace, fin, st);
        case TPR_NORM:
            if (norm_is_inf(desc->p)) {
                if (desc->p > 0) return run<ArgOp<true, int, true>>(p, x, out, workspace, fin, st);
                return run<ArgOp<false, int, true>>(p, x, out, workspace, fin, st);
            }
            if (desc->p == 1.0) return run<NormOp<1>>(p, x, out, workspace, fin, st);
            if (desc->p == 2.0) return run<NormOp<2>>(p, x, out, workspace, fin, st);
            return run<NormOp<0>>(p, x, out, workspace, fin, st);
        default: return run<WelfordOp>(p, x, out, workspace, fin, st);
    }
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Ticket counters of split plans finished in one launch (split_finish).  Zero
// when the library loads; every launch that draws tickets leaves its counters
// at 0 again.  Each stream gets its own block of counters, so launches that can
// run at the same time never share a counter: launches on one stream run one
// after another.  Streams beyond kTicketStreams, the per-thread default stream
// (one handle for many streams) and streams under graph capture (a captured
// launch may replay on another stream) take the separate finalize launch.
// ---------------------------------------------------------------------------
static __device__ unsigned int split_tickets[tpr::kTicketStreams * tpr::kTicketsPerStream];

namespace tpr {
namespace {
unsigned* stream_tickets(hipStream_t st) {
    if (knobs().split_fin < 0) return nullptr;
    if (st == hipStreamPerThread) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
        (void)hipGetLastError();  // not an error of this call: take the finalize launch
        return nullptr;
    }
    if (cs != hipStreamCaptureStatusNone) return nullptr;
    static constexpr int kMaxDev = 64;
    struct DevTickets {
        unsigned* base = nullptr;
        int n = 0;
        hipStream_t streams[kTicketStreams];
    };
    static std::mutex mu;
    static DevTickets devs[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> g(mu);
    DevTickets& d = devs[dev];
    if (!d.base) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(split_tickets)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        d.base = static_cast<unsigned*>(ptr);
    }
    for (int i = 0; i < d.n; ++i)
        if (d.streams[i] == st) return d.base + (size_t)i * kTicketsPerStream;
    if (d.n == kTicketStreams) return nullptr;
    d.streams[d.n] = st;
    return d.base + (size_t)(d.n++) * kTicketsPerStream;
}
}  // namespace
}  // namespace tpr

// ---------------------------------------------------------------------------
// Workspace-free entry point.  The partial states of split plans (and the
// median's histograms) live in a fixed per-device array instead of a caller
// workspace, so tpr_reduce_noalloc needs no device allocation anywhere.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[TPR_REDUCE_SCRATCH_BYTES];

namespace {

// Device address of `scratch` on the current device.  The host-side name of a
// __device__ array is only a stand-in for the runtime's symbol table, never a
// device address, so the address is looked up once per device with that
// device current and kept.
int scratch_address(void** ptr) {
    static constexpr int kMaxDev = 64;
    static std::mutex mu;
    static void* addr[kMaxDev] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return tpr::fail(TPR_ERR_HIP, std::string("tpr_reduce_noalloc: hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDev) return tpr::fail(TPR_ERR_INVALID_ARG, "tpr_reduce_noalloc: device index out of range");
    std::lock_guard<std::mutex> g(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return tpr::fail(TPR_ERR_HIP, std::string("tpr_reduce_noalloc: hipGetSymbolAddress(scratch): ") +
                                              hipGetErrorString(e));
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return TPR_OK;
}

}  // namespace

extern "C" int tpr_reduce_noalloc(const tpr_reduce_desc* desc, const void* in, void* out, void* stream) {
    const size_t need = tpr_reduce_workspace_bytes(desc);  // 0 for an invalid descriptor: tpr_reduce reports it
    if (need > (size_t)TPR_REDUCE_SCRATCH_BYTES)
        return tpr::fail(TPR_ERR_WORKSPACE, "tpr_reduce_noalloc: this reduction needs " + std::to_string(need) +
                                                " bytes of scratch, more than the fixed " +
                                                std::to_string((size_t)TPR_REDUCE_SCRATCH_BYTES) +
                                                "; use tpr_reduce with a workspace");
    void* ws = nullptr;
    if (need > 0) {
        const int rc = scratch_address(&ws);
        if (rc != TPR_OK) return rc;
    }
    return tpr_reduce(desc, in, out, ws, need, stream);
}
