// Strided, casting copy: dst[i...] = static_cast<DstT>(src[i...]) for every
// index of `sizes`, both sides at arbitrary element strides (a stride-0 source
// dim broadcasts).  Counterpart of TensorPlay's copy_ kernels:
//   CUDA copy_cast_kernel_impl / copy_kernel
//     (/root/reference/p10/src/backend/cuda/CopyKernels.cu:42-157): one thread
//     per element, index -> offset by div/mod on both sides;
//   CPU copy_recursive / copy_kernel
//     (/root/reference/p10/src/backend/cpu/CopyKernels.cpp:27-55,110-127):
//     the same static_cast per element, row-major over sizes.
// The result does not depend on the visiting order (each destination element
// is written once from one source element), so the host planner reorders and
// merges dims freely and picks one of four HBM-bound kernels:
//   k_copy_contig  both sides one dense run: one 16-byte vector per thread
//                  over a grid covering the run (faster than several per
//                  thread on MI355X: 89 vs 92 us for a 256 MiB clone, 136 vs
//                  156 us for a float32 -> float64 cast), casts in registers;
//   k_copy_rows    the innermost dim dense on both sides: the same per row,
//                  the row's base offsets from a div/mod over the outer dims
//                  once per workgroup;
//   k_copy_tile    the dst-fastest dim and the src-fastest dim differ (a
//                  transpose / permute): 64x64 tiles staged through LDS so that
//                  reads run along the source's unit-stride dim and writes
//                  along the destination's;
//   k_copy_elem    anything else: one element per thread, div/mod per element,
//                  elements in destination order so writes coalesce.
// Casts follow C++ static_cast as the reference does: to Bool is x != 0
// (NaN -> true); float -> integer truncates toward zero (out-of-range values
// are undefined behaviour in the reference; the GPU result saturates).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <vector>
#include <type_traits>

#include "common.h"

namespace tpr {
namespace {

constexpr int kCopyBlock = 256;
constexpr int kTile = 64;

template <class D, class S>
__device__ __forceinline__ D cvt(S x) {
    return static_cast<D>(x);
}

// ---- dense run ----------------------------------------------------------------
// V source elements per 16-byte vector; each thread moves U vectors.
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <class D, class S>
struct VecT {
    static constexpr int V = 16 / (int)sizeof(S);
    struct alignas(16) In { S v[V]; };
    static constexpr int kOutBytes = V * (int)sizeof(D);
    static constexpr int kOutAlign = kOutBytes >= 16 ? 16 : kOutBytes;
    struct alignas(kOutAlign) Out { D v[V]; };
};

// One 16-byte source vector (V elements) per step: load, convert in
// registers, store.  NT (nontemporal loads and stores) is a template
// parameter: a runtime choice compiles to plain accesses only, because the
// compiler merges the two branches' otherwise identical loads and stores and
// drops the nontemporal mark.
template <class D, class S, bool NT>
__device__ __forceinline__ typename VecT<D, S>::In vload(const typename VecT<D, S>::In* p) {
    using VT = VecT<D, S>;
    if constexpr (!NT) return *p;
    typename VT::In t;
    const f32x4v bits = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(p));
    __builtin_memcpy(&t, &bits, 16);
    return t;
}

template <class D, class S, bool NT>
__device__ __forceinline__ void vstore(typename VecT<D, S>::Out* p, const typename VecT<D, S>::Out& o) {
    using VT = VecT<D, S>;
    if constexpr (NT && VT::kOutBytes % 16 == 0) {
        f32x4v* dst = reinterpret_cast<f32x4v*>(p);
#pragma unroll
        for (int k = 0; k < VT::kOutBytes / 16; ++k) {
            f32x4v bits;
            __builtin_memcpy(&bits, reinterpret_cast<const char*>(&o) + 16 * k, 16);
            __builtin_nontemporal_store(bits, dst + k);
        }
    } else {
        *p = o;
    }
}

// A workgroup moves one chunk of kCopyBlock * U vectors: U loads in flight per
// thread, each wave's accesses contiguous.  `n` elements start at dst/src.
template <class D, class S, int U, bool NT>
__device__ __forceinline__ void copy_chunk(D* __restrict__ dst, const S* __restrict__ src, long long n) {
    using VT = VecT<D, S>;
    constexpr int V = VT::V;
    const long long nv = n / V;
    const auto* sv = reinterpret_cast<const typename VT::In*>(src);
    auto* dv = reinterpret_cast<typename VT::Out*>(dst);
    typename VT::In t[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long v = u * kCopyBlock + threadIdx.x;
        if (v < nv) t[u] = vload<D, S, NT>(sv + v);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long v = u * kCopyBlock + threadIdx.x;
        if (v < nv) {
            typename VT::Out o;
#pragma unroll
            for (int j = 0; j < V; ++j) o.v[j] = cvt<D>(t[u].v[j]);
            vstore<D, S, NT>(dv + v, o);
        }
    }
    for (long long e = nv * V + threadIdx.x; e < n; e += kCopyBlock) dst[e] = cvt<D>(src[e]);
}

constexpr int kChunkVecs = 1;  // vectors per thread per workgroup chunk

struct ContigArgs {
    void* dst;
    const void* src;
    long long n;
};

template <class D, class S, bool NT>
__global__ __launch_bounds__(kCopyBlock) void k_copy_contig(ContigArgs a) {
    constexpr long long CH = (long long)kCopyBlock * kChunkVecs * VecT<D, S>::V;
    const long long e0 = (long long)blockIdx.x * CH;
    copy_chunk<D, S, kChunkVecs, NT>(static_cast<D*>(a.dst) + e0, static_cast<const S*>(a.src) + e0,
                                     min(CH, a.n - e0));
}

// ---- rows ------------------------------------------------------------------------
struct RowsArgs {
    void* dst;
    const void* src;
    int nouter;                              // outer dims (innermost last)
    long long osz[TPR_MAX_DIMS];
    long long ods[TPR_MAX_DIMS], oss[TPR_MAX_DIMS];
    long long L;                             // row length (dense on both sides)
    long long nchunk;                        // workgroups per row
    long long chunk;                         // elements per workgroup
};

__device__ __forceinline__ void outer_offsets(const RowsArgs& a, unsigned row, long long& doff, long long& soff) {
    doff = 0;
    soff = 0;
    for (int d = a.nouter - 1; d >= 0; --d) {
        const unsigned m = a.osz[d] > 0xffffffffLL ? 0xffffffffu : (unsigned)a.osz[d];
        const unsigned q = row / m, r = row - q * m;  // 32-bit: row < 2^32
        doff += (long long)r * a.ods[d];
        soff += (long long)r * a.oss[d];
        row = q;
    }
}

template <class D, class S, bool VEC>
__global__ __launch_bounds__(kCopyBlock) void k_copy_rows(RowsArgs a) {
    const unsigned nch = a.nchunk > 0xffffffffLL ? 0xffffffffu : (unsigned)a.nchunk;
    const unsigned row = blockIdx.x / nch;
    const long long c = blockIdx.x - row * nch;
    long long doff, soff;
    outer_offsets(a, row, doff, soff);
    D* dst = static_cast<D*>(a.dst) + doff;
    const S* src = static_cast<const S*>(a.src) + soff;
    const long long e0 = c * a.chunk;
    const long long n = min(a.chunk, a.L - e0);
    if constexpr (VEC) {
        // chunk is a multiple of the vector width, so every chunk starts aligned
        copy_chunk<D, S, kChunkVecs, false>(dst + e0, src + e0, n);
    } else {
        for (long long e = threadIdx.x; e < n; e += kCopyBlock) dst[e0 + e] = cvt<D>(src[e0 + e]);
    }
}

// ---- tiles (transpose / permute) -------------------------------------------------
// I = the destination's fastest dim, J = the source's unit-stride dim.  Tile
// [64 (J) x 64 (I)]; reads: a wave covers 64 consecutive j (source-contiguous);
// writes: a wave covers 64 consecutive i (destination-contiguous).
struct TileArgs {
    void* dst;
    const void* src;
    long long nI, nJ;
    long long dsI, dsJ, ssI;                 // ssJ == 1
    long long tilesI, tilesJ;
    int nb;                                  // batch dims (innermost last)
    long long bsz[TPR_MAX_DIMS];
    long long bds[TPR_MAX_DIMS], bss[TPR_MAX_DIMS];
};

// 32-bit division of a workgroup index (< 2^32) by m: a divisor of 2^32 or
// more leaves the index whole.  A 64-bit division is a long software sequence.
__device__ __forceinline__ unsigned div32(unsigned& b, long long m) {
    const unsigned d = m > 0xffffffffLL ? 0xffffffffu : (unsigned)m;
    const unsigned q = b / d, r = b - q * d;
    b = q;
    return r;
}

// The tile (ti, tj) and batch offsets of this workgroup.
__device__ __forceinline__ void tile_origin(const TileArgs& a, long long& ti, long long& tj, long long& doff,
                                            long long& soff) {
    unsigned b = blockIdx.x;
    ti = div32(b, a.tilesI);
    tj = div32(b, a.tilesJ);
    doff = 0;
    soff = 0;
    for (int d = a.nb - 1; d >= 0; --d) {
        const long long r = div32(b, a.bsz[d]);
        doff += r * a.bds[d];
        soff += r * a.bss[d];
    }
}

template <class D, class S>
__global__ __launch_bounds__(kCopyBlock) void k_copy_tile(TileArgs a) {
    // +1 element of padding per row: column walks hit distinct banks for 4-byte D
    __shared__ D tile[kTile][kTile + 1];
    long long ti, tj, doff, soff;
    tile_origin(a, ti, tj, doff, soff);
    D* dst = static_cast<D*>(a.dst) + doff;
    const S* src = static_cast<const S*>(a.src) + soff;
    const long long i0 = ti * kTile, j0 = tj * kTile;
    const int lane = threadIdx.x % kTile;
    const int r0 = threadIdx.x / kTile;  // 0..3
    constexpr int kRowsPerPass = kCopyBlock / kTile;
    // read: lane walks j, rows walk i
    const long long j = j0 + lane;
    for (int il = r0; il < kTile; il += kRowsPerPass) {
        const long long i = i0 + il;
        if (i < a.nI && j < a.nJ) tile[il][lane] = cvt<D>(src[j + i * a.ssI]);
    }
    __syncthreads();
    // write: lane walks i, rows walk j
    const long long i = i0 + lane;
    for (int jl = r0; jl < kTile; jl += kRowsPerPass) {
        const long long jj = j0 + jl;
        if (i < a.nI && jj < a.nJ) dst[i * a.dsI + jj * a.dsJ] = tile[lane][jl];
    }
}

// Vector tiles: [TJ (source-contiguous) x TI (destination-contiguous)], 16-byte
// loads along J and 16-byte stores along I (measured on MI355X for a
// [64,1024,1024] fp32 transpose: 5.6 TB/s read+write against 4.4 TB/s for
// the scalar 64x64 tile).  Needs dsI == 1 and 16-byte aligned rows on both
// sides; edge tiles take guarded element-wise loads and stores.
template <class D, class S, int TI, int TJ, bool NT>
__global__ __launch_bounds__(kCopyBlock) void k_copy_tile_v(TileArgs a) {
    using VT = VecT<D, S>;
    constexpr int VL = 16 / (int)sizeof(S);
    constexpr int VS = 16 / (int)sizeof(D);
    struct alignas(16) OutV { D v[VS]; };
    __shared__ D tile[TJ][TI + 1];
    long long ti, tj, doff, soff;
    tile_origin(a, ti, tj, doff, soff);
    const long long i0 = ti * TI, j0 = tj * TJ;
    D* dst = static_cast<D*>(a.dst) + doff + i0 + j0 * a.dsJ;
    const S* src = static_cast<const S*>(a.src) + soff + j0 + i0 * a.ssI;
    const int tid = threadIdx.x;
    const bool full = i0 + TI <= a.nI && j0 + TJ <= a.nJ;
    if (full) {
        constexpr int LPR = TJ / VL;            // threads per source row
        constexpr int RPP = kCopyBlock / LPR;   // source rows per pass
        static_assert(TI % RPP == 0, "source passes must tile TI");
        const int c = tid % LPR;
#pragma unroll
        for (int pass = 0; pass < TI / RPP; ++pass) {
            const int il = tid / LPR + pass * RPP;
            const typename VT::In v = vload<D, S, NT>(reinterpret_cast<const typename VT::In*>(src + il * a.ssI + c * VL));
#pragma unroll
            for (int k = 0; k < VL; ++k) tile[c * VL + k][il] = cvt<D>(v.v[k]);
        }
    } else {
        const int ni = (int)min((long long)TI, a.nI - i0), nj = (int)min((long long)TJ, a.nJ - j0);
        for (int x = tid; x < TI * TJ; x += kCopyBlock) {
            const int jl = x % TJ, il = x / TJ;
            if (il < ni && jl < nj) tile[jl][il] = cvt<D>(src[il * a.ssI + jl]);
        }
    }
    __syncthreads();
    if (full) {
        constexpr int WPR = TI / VS;            // threads per destination row
        constexpr int WPP = kCopyBlock / WPR;   // destination rows per pass
        static_assert(TJ % WPP == 0, "destination passes must tile TJ");
        const int w = tid % WPR;
#pragma unroll
        for (int pass = 0; pass < TJ / WPP; ++pass) {
            const int jl = tid / WPR + pass * WPP;
            OutV o;
#pragma unroll
            for (int k = 0; k < VS; ++k) o.v[k] = tile[jl][w * VS + k];
            if constexpr (NT) {
                f32x4v bits;
                __builtin_memcpy(&bits, &o, 16);
                __builtin_nontemporal_store(bits, reinterpret_cast<f32x4v*>(dst + jl * a.dsJ + w * VS));
            } else {
                *reinterpret_cast<OutV*>(dst + jl * a.dsJ + w * VS) = o;
            }
        }
    } else {
        const int ni = (int)min((long long)TI, a.nI - i0), nj = (int)min((long long)TJ, a.nJ - j0);
        for (int x = tid; x < TI * TJ; x += kCopyBlock) {
            const int il = x % TI, jl = x / TI;
            if (il < ni && jl < nj) dst[il + jl * a.dsJ] = tile[jl][il];
        }
    }
}

// ---- general ---------------------------------------------------------------------
struct ElemArgs {
    void* dst;
    const void* src;
    int nd;
    long long sz[TPR_MAX_DIMS];
    long long ds[TPR_MAX_DIMS], ss[TPR_MAX_DIMS];
    long long n;
};

template <class D, class S>
__global__ __launch_bounds__(kCopyBlock) void k_copy_elem(ElemArgs a) {
    D* dst = static_cast<D*>(a.dst);
    const S* src = static_cast<const S*>(a.src);
    const long long step = (long long)gridDim.x * kCopyBlock;
    for (long long e = (long long)blockIdx.x * kCopyBlock + threadIdx.x; e < a.n; e += step) {
        long long rem = e, doff = 0, soff = 0;
        for (int d = a.nd - 1; d >= 0; --d) {
            const long long q = rem / a.sz[d];
            const long long r = rem - q * a.sz[d];
            doff += r * a.ds[d];
            soff += r * a.ss[d];
            rem = q;
        }
        dst[doff] = cvt<D>(src[soff]);
    }
}

// ---- host planner --------------------------------------------------------------
struct CDim {
    long long size, ds, ss;
};

int esize(int dt) {
    switch (dt) {
        case TPR_UINT8: case TPR_INT8: case TPR_BOOL: return 1;
        case TPR_INT16: case TPR_UINT16: return 2;
        case TPR_INT32: case TPR_UINT32: case TPR_FLOAT32: return 4;
        case TPR_INT64: case TPR_UINT64: case TPR_FLOAT64: return 8;
        default: return 0;
    }
}

enum CopyKind { C_CONTIG, C_ROWS, C_TILE, C_ELEM };

struct CopyPlan {
    int kind = C_ELEM;
    std::vector<CDim> dims;  // reordered + merged, dst-slowest first
    long long n = 0;
    int J = -1;              // C_TILE: index of the source's unit-stride dim
    bool vec = false;        // C_CONTIG / C_ROWS: 16-byte vector path
};

bool aligned(const void* p, long long a) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)a) == 0; }

CopyPlan plan_copy(const tpr_copy_desc* d, void* dst, const void* src) {
    CopyPlan p;
    p.n = 1;
    for (int i = 0; i < d->ndim; ++i) p.n *= d->sizes[i];
    for (int i = 0; i < d->ndim; ++i)
        if (d->sizes[i] != 1) p.dims.push_back({d->sizes[i], d->dst_strides[i], d->src_strides[i]});
    if (p.dims.empty()) p.dims.push_back({1, 1, 1});
    // destination-fastest dim last; ties keep the source's order
    std::stable_sort(p.dims.begin(), p.dims.end(), [](const CDim& x, const CDim& y) {
        const long long ax = std::llabs(x.ds), ay = std::llabs(y.ds);
        if (ax != ay) return ax > ay;
        return std::llabs(x.ss) > std::llabs(y.ss);
    });
    // merge a dim into the next inner one when it continues it on both sides
    const std::vector<CDim> m = p.dims;
    std::vector<CDim> out;
    for (int i = (int)m.size() - 1; i >= 0; --i) {
        if (!out.empty()) {
            CDim& in = out.back();  // the inner neighbour (already merged)
            if (m[i].ds == in.ds * in.size && m[i].ss == in.ss * in.size) {
                in.size *= m[i].size;
                continue;
            }
        }
        out.push_back(m[i]);
    }
    std::reverse(out.begin(), out.end());
    p.dims = out;
    const int nd = (int)p.dims.size();
    const CDim& last = p.dims.back();
    const int sde = esize(d->src_dtype), dde = esize(d->dst_dtype);
    const long long V = 16 / sde;
    const long long oalign = std::min(16LL, V * dde);
    if (nd == 1 && last.ds == 1 && last.ss == 1) {
        p.kind = C_CONTIG;
        p.vec = aligned(src, 16) && aligned(dst, oalign);
        return p;
    }
    const long long kMaxGrid = 0x7fffffffLL;
    if (last.ds == 1 && last.ss == 1 && last.size >= 256 && (p.n / last.size) * ((last.size + 4095) / 4096) < kMaxGrid) {
        p.kind = C_ROWS;
        bool v = aligned(src, 16) && aligned(dst, oalign);
        for (int i = 0; i + 1 < nd; ++i)
            v = v && ((p.dims[i].ss * sde) % 16 == 0) && ((p.dims[i].ds * dde) % oalign == 0);
        p.vec = v;
        return p;
    }
    for (int i = 0; i + 1 < nd; ++i)
        if (p.dims[i].ss == 1 && p.dims[i].size >= 16 && last.size >= 16 &&
            p.n / (p.dims[i].size * last.size) * ((p.dims[i].size + kTile - 1) / kTile) *
                    ((last.size + kTile - 1) / kTile) < kMaxGrid) {
            p.kind = C_TILE;
            p.J = i;
            // vector tiles: 16-byte rows on both sides
            const long long VL = 16 / sde, VS = 16 / dde;
            bool v = last.ds == 1 && aligned(src, 16) && aligned(dst, 16) && last.ss % VL == 0 &&
                     p.dims[i].ds % VS == 0;
            for (int k = 0; k + 1 < nd; ++k)
                if (k != i) v = v && p.dims[k].ss % VL == 0 && p.dims[k].ds % VS == 0;
            p.vec = v;
            return p;
        }
    p.kind = C_ELEM;
    return p;
}

template <class D, class S>
int launch_copy(const CopyPlan& p, void* dst, const void* src, hipStream_t st) {
    const auto& dev = device_info();
    const int nd = (int)p.dims.size();
    if (p.kind == C_CONTIG) {
        const long long bytes = p.n * (long long)(sizeof(D) + sizeof(S));
        ContigArgs a{dst, src, p.n};
        if (p.vec) {
            const long long per_block = (long long)kCopyBlock * kChunkVecs * VecT<D, S>::V;
            const long long blocks = (p.n + per_block - 1) / per_block;
            // Nontemporal loads (and, for same-size copies, stores) from 64 MiB
            // when the destination element is not wider than the source.
            // Measured on MI355X at [64, 1024, 1024] float32 sources: clone 88.6 ->
            // 83.0 us, to int32 88.2 -> 83.0, to int8 59.6 -> 57.5; float64 ->
            // float32 135 -> 133.5; widening casts keep plain accesses (to float64
            // 136.5 against 140 with nontemporal loads, 195 with nontemporal
            // stores too); a 16 MiB clone (cache resident) is faster plain (6.1
            // against 6.7 us).  The nt debug knob < 0 turns them off.
            if constexpr (sizeof(D) <= sizeof(S)) {
                if (bytes >= (64LL << 20) && knobs().nt >= 0) {
                    hipLaunchKernelGGL((k_copy_contig<D, S, true>), dim3((unsigned)blocks), dim3(kCopyBlock), 0, st, a);
                    return check_launch("k_copy_contig");
                }
            }
            hipLaunchKernelGGL((k_copy_contig<D, S, false>), dim3((unsigned)blocks), dim3(kCopyBlock), 0, st, a);
        } else {
            ElemArgs e{};
            e.dst = dst; e.src = src; e.nd = 1; e.sz[0] = p.n; e.ds[0] = 1; e.ss[0] = 1; e.n = p.n;
            const long long blocks = std::max(1LL, std::min((p.n + kCopyBlock - 1) / kCopyBlock, (long long)dev.cus * 64));
            hipLaunchKernelGGL((k_copy_elem<D, S>), dim3(blocks), dim3(kCopyBlock), 0, st, e);
        }
        return check_launch("k_copy_contig");
    }
    if (p.kind == C_ROWS) {
        RowsArgs a{};
        a.dst = dst; a.src = src; a.nouter = nd - 1;
        long long rows = 1;
        for (int i = 0; i < nd - 1; ++i) {
            a.osz[i] = p.dims[i].size; a.ods[i] = p.dims[i].ds; a.oss[i] = p.dims[i].ss;
            rows *= p.dims[i].size;
        }
        a.L = p.dims.back().size;
        const long long V = 16 / (long long)sizeof(S);
        a.chunk = (long long)kCopyBlock * V * kChunkVecs;
        a.nchunk = (a.L + a.chunk - 1) / a.chunk;
        const dim3 grid((unsigned)(rows * a.nchunk));
        if (p.vec) hipLaunchKernelGGL((k_copy_rows<D, S, true>), grid, dim3(kCopyBlock), 0, st, a);
        else hipLaunchKernelGGL((k_copy_rows<D, S, false>), grid, dim3(kCopyBlock), 0, st, a);
        return check_launch("k_copy_rows");
    }
    if (p.kind == C_TILE) {
        TileArgs a{};
        a.dst = dst; a.src = src;
        const CDim& I = p.dims.back();
        const CDim& J = p.dims[p.J];
        a.nI = I.size; a.nJ = J.size; a.dsI = I.ds; a.dsJ = J.ds; a.ssI = I.ss;
        // vector tiles: 64 (I) x 128 (J) for 1/2-byte types, 64 x 64 for 8-byte destinations (LDS <= 33 KB)
        constexpr int TI = 64, TJ = sizeof(D) == 8 ? 64 : 128;
        // 4-byte elements: 128 (I) x 64 (J) when the destination rows are that
        // long (512-byte store runs), else 64 x 64.  Measured on MI355X at
        // [64, 1024, 1024] fp32: transpose(1, 2) 91 us (64 x 128: 98 us),
        // permute(1, 2, 0) (I = 64) 101 us (64 x 128: 105 us).
        const int tv = (sizeof(D) == 4 && sizeof(S) == 4) ? (a.nI >= 128 ? 1 : 2) : 0;
        const long long TIr = tv == 1 ? 128 : TI;
        const long long TJr = tv != 0 ? 64 : TJ;
        const long long ti = p.vec ? TIr : kTile, tj = p.vec ? TJr : kTile;
        a.tilesI = (a.nI + ti - 1) / ti;
        a.tilesJ = (a.nJ + tj - 1) / tj;
        long long batch = 1;
        for (int i = 0; i < nd - 1; ++i) {
            if (i == p.J) continue;
            a.bsz[a.nb] = p.dims[i].size; a.bds[a.nb] = p.dims[i].ds; a.bss[a.nb] = p.dims[i].ss;
            ++a.nb;
            batch *= p.dims[i].size;
        }
        const dim3 grid((unsigned)(a.tilesI * a.tilesJ * batch));
        // Nontemporal loads and stores for large same-type transposes (measured on
        // MI355X at [64, 1024, 1024] fp32: permute(1, 2, 0) 101 -> 92 us,
        // transpose(1, 2) 91 -> 87 us).
        const bool nt = std::is_same<D, S>::value && p.n * (long long)(sizeof(D) + sizeof(S)) >= (64LL << 20);
        if (!p.vec) {
            hipLaunchKernelGGL((k_copy_tile<D, S>), grid, dim3(kCopyBlock), 0, st, a);
        } else if constexpr (sizeof(D) == 4 && sizeof(S) == 4) {
            if (tv == 1 && nt) hipLaunchKernelGGL((k_copy_tile_v<D, S, 128, 64, std::is_same<D, S>::value>), grid, dim3(kCopyBlock), 0, st, a);
            else if (tv == 1) hipLaunchKernelGGL((k_copy_tile_v<D, S, 128, 64, false>), grid, dim3(kCopyBlock), 0, st, a);
            else if (nt) hipLaunchKernelGGL((k_copy_tile_v<D, S, 64, 64, std::is_same<D, S>::value>), grid, dim3(kCopyBlock), 0, st, a);
            else hipLaunchKernelGGL((k_copy_tile_v<D, S, 64, 64, false>), grid, dim3(kCopyBlock), 0, st, a);
        } else {
            if (nt) hipLaunchKernelGGL((k_copy_tile_v<D, S, TI, TJ, std::is_same<D, S>::value>), grid, dim3(kCopyBlock), 0, st, a);
            else hipLaunchKernelGGL((k_copy_tile_v<D, S, TI, TJ, false>), grid, dim3(kCopyBlock), 0, st, a);
        }
        return check_launch("k_copy_tile");
    }
    ElemArgs e{};
    e.dst = dst; e.src = src; e.nd = nd; e.n = p.n;
    for (int i = 0; i < nd; ++i) { e.sz[i] = p.dims[i].size; e.ds[i] = p.dims[i].ds; e.ss[i] = p.dims[i].ss; }
    const long long blocks = std::max(1LL, std::min((p.n + kCopyBlock - 1) / kCopyBlock, (long long)dev.cus * 64));
    hipLaunchKernelGGL((k_copy_elem<D, S>), dim3(blocks), dim3(kCopyBlock), 0, st, e);
    return check_launch("k_copy_elem");
}

template <class D>
int dispatch_src(int sdt, const CopyPlan& p, void* dst, const void* src, hipStream_t st) {
    switch (sdt) {
        case TPR_UINT8: return launch_copy<D, uint8_t>(p, dst, src, st);
        case TPR_INT8: return launch_copy<D, int8_t>(p, dst, src, st);
        case TPR_INT16: return launch_copy<D, int16_t>(p, dst, src, st);
        case TPR_INT32: return launch_copy<D, int32_t>(p, dst, src, st);
        case TPR_INT64: return launch_copy<D, int64_t>(p, dst, src, st);
        case TPR_UINT16: return launch_copy<D, uint16_t>(p, dst, src, st);
        case TPR_UINT32: return launch_copy<D, uint32_t>(p, dst, src, st);
        case TPR_UINT64: return launch_copy<D, uint64_t>(p, dst, src, st);
        case TPR_FLOAT32: return launch_copy<D, float>(p, dst, src, st);
        case TPR_FLOAT64: return launch_copy<D, double>(p, dst, src, st);
        case TPR_BOOL: return launch_copy<D, bool>(p, dst, src, st);
        default: return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_copy: unknown source dtype");
    }
}

// Same dtype: only the element size matters.
int dispatch_same(int es, const CopyPlan& p, void* dst, const void* src, hipStream_t st) {
    switch (es) {
        case 1: return launch_copy<uint8_t, uint8_t>(p, dst, src, st);
        case 2: return launch_copy<uint16_t, uint16_t>(p, dst, src, st);
        case 4: return launch_copy<uint32_t, uint32_t>(p, dst, src, st);
        default: return launch_copy<uint64_t, uint64_t>(p, dst, src, st);
    }
}

}  // namespace

int copy_plan_kind_for_test(const tpr_copy_desc* d, void* dst, const void* src) {
    const CopyPlan p = plan_copy(d, dst, src);
    return p.kind | (p.vec ? 4 : 0);
}

}  // namespace tpr

extern "C" int tpr_copy(const tpr_copy_desc* desc, void* dst, const void* src, void* stream) {
    using namespace tpr;
    if (!desc) return fail(TPR_ERR_INVALID_ARG, "tpr_copy: null descriptor");
    if (desc->ndim < 0 || desc->ndim > TPR_MAX_DIMS) return fail(TPR_ERR_INVALID_ARG, "tpr_copy: ndim out of range");
    if (esize(desc->dst_dtype) == 0 || esize(desc->src_dtype) == 0)
        return fail(TPR_ERR_UNSUPPORTED_DTYPE, "tpr_copy: unknown dtype");
    long long n = 1;
    for (int i = 0; i < desc->ndim; ++i) {
        if (desc->sizes[i] < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_copy: negative size");
        n *= desc->sizes[i];
    }
    if (n == 0) return TPR_OK;
    if (!dst || !src) return fail(TPR_ERR_INVALID_ARG, "tpr_copy: null pointer");
    const CopyPlan p = plan_copy(desc, dst, src);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (desc->dst_dtype == desc->src_dtype) return dispatch_same(esize(desc->dst_dtype), p, dst, src, st);
    switch (desc->dst_dtype) {
        case TPR_UINT8: return dispatch_src<uint8_t>(desc->src_dtype, p, dst, src, st);
        case TPR_INT8: return dispatch_src<int8_t>(desc->src_dtype, p, dst, src, st);
        case TPR_INT16: return dispatch_src<int16_t>(desc->src_dtype, p, dst, src, st);
        case TPR_INT32: return dispatch_src<int32_t>(desc->src_dtype, p, dst, src, st);
        case TPR_INT64: return dispatch_src<int64_t>(desc->src_dtype, p, dst, src, st);
        case TPR_UINT16: return dispatch_src<uint16_t>(desc->src_dtype, p, dst, src, st);
        case TPR_UINT32: return dispatch_src<uint32_t>(desc->src_dtype, p, dst, src, st);
        case TPR_UINT64: return dispatch_src<uint64_t>(desc->src_dtype, p, dst, src, st);
        case TPR_FLOAT32: return dispatch_src<float>(desc->src_dtype, p, dst, src, st);
        case TPR_FLOAT64: return dispatch_src<double>(desc->src_dtype, p, dst, src, st);
        default: return dispatch_src<bool>(desc->src_dtype, p, dst, src, st);
    }
}

extern "C" int tpr_copy_plan(const tpr_copy_desc* desc, const void* dst, const void* src) {
    using namespace tpr;
    if (!desc || desc->ndim < 0 || desc->ndim > TPR_MAX_DIMS) return -1;
    if (esize(desc->dst_dtype) == 0 || esize(desc->src_dtype) == 0) return -1;
    return copy_plan_kind_for_test(desc, const_cast<void*>(dst), src);
}

extern "C" int tpr_copy_strided(const void* in, int32_t elem_size, int32_t ndim, const int64_t* sizes,
                                const int64_t* in_strides, void* out, void* stream) {
    using namespace tpr;
    if (ndim < 0 || ndim > TPR_MAX_DIMS) return fail(TPR_ERR_INVALID_ARG, "tpr_copy_strided: ndim out of range");
    tpr_copy_desc d{};
    d.ndim = ndim;
    switch (elem_size) {
        case 1: d.dst_dtype = d.src_dtype = TPR_UINT8; break;
        case 2: d.dst_dtype = d.src_dtype = TPR_UINT16; break;
        case 4: d.dst_dtype = d.src_dtype = TPR_UINT32; break;
        case 8: d.dst_dtype = d.src_dtype = TPR_UINT64; break;
        default: return fail(TPR_ERR_INVALID_ARG, "tpr_copy_strided: elem_size must be 1, 2, 4 or 8");
    }
    long long st = 1;
    for (int i = ndim - 1; i >= 0; --i) {
        if (sizes[i] < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_copy_strided: negative size");
        d.sizes[i] = sizes[i];
        d.src_strides[i] = in_strides[i];
        d.dst_strides[i] = st;
        st *= sizes[i];
    }
    return tpr_copy(&d, out, in, stream);
}
