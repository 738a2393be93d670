/*
 * TEST INFRASTRUCTURE ONLY -- see tp_cpu_reduce.h.  Never part of the product.
 *
 * CPU restatement of TensorPlay's CPU reduction kernels (float32 only):
 *   /root/reference/p10/src/backend/cpu/ReductionKernels.cpp
 *   /root/reference/p10/src/backend/cpu/ArithmeticKernels.cpp:1502-1532 (div by Scalar)
 * Each function follows the reference's accumulation type and visiting order so
 * that its result has the reference path's rounding.  Compile with
 * -ffp-contract=off so that a*b+c is never fused (the reference rounds each op).
 *
 * Parity pins (tests/test_oracle.py): the reference tests' known answers
 * (tests/golden/reference_known_answers.json), numpy closed forms
 * (np.add.accumulate is a strictly sequential sum), torch.var/std at the
 * reference's own rtol (test/test_statistical.py:10-17), and brute force.
 */
#include "tp_cpu_reduce.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>

#define MAXD 16

/* Row-major logical walk over all dims; calls back with (input offset, output offset).
 * Output offsets use contiguous strides over the kept dims, as the reference's
 * inp_dim_to_out_stride table does (ReductionKernels.cpp:135-152). */
typedef struct {
    int ndim;
    const int64_t* sizes;
    const int64_t* strides;
    int64_t ostride[MAXD];
} walk_t;

static void walk_init(walk_t* w, int ndim, const int64_t* sizes, const int64_t* strides,
                      uint32_t reduce_mask) {
    w->ndim = ndim; w->sizes = sizes; w->strides = strides;
    int64_t acc = 1;
    for (int d = ndim - 1; d >= 0; --d) {
        if (reduce_mask & (1u << d)) { w->ostride[d] = 0; }
        else { w->ostride[d] = acc; acc *= sizes[d]; }
    }
}

static int64_t numel_of(int ndim, const int64_t* sizes) {
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) n *= sizes[d];
    return n;
}

static int64_t kept_numel(int ndim, const int64_t* sizes, uint32_t mask) {
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) if (!(mask & (1u << d))) n *= sizes[d];
    return n;
}

/* Logical (row-major) element i -> memory offset. */
static int64_t logical_offset(int ndim, const int64_t* sizes, const int64_t* strides, int64_t i) {
    int64_t off = 0;
    for (int d = ndim - 1; d >= 0; --d) {
        int64_t s = sizes[d];
        off += (i % s) * strides[d];
        i /= s;
    }
    return off;
}

/* Iterative odometer walk (same order as the reference's recursive lambda). */
#define WALK_BEGIN(w)                                                         \
    {                                                                         \
        int64_t _idx[MAXD] = {0};                                             \
        int64_t _in = 0, _out = 0;                                            \
        int64_t _total = numel_of((w)->ndim, (w)->sizes);                     \
        for (int64_t _t = 0; _t < _total; ++_t) {                             \
            int64_t in_off = _in, out_off = _out;
#define WALK_END(w)                                                           \
            for (int _d = (w)->ndim - 1; _d >= 0; --_d) {                     \
                _idx[_d]++;                                                   \
                _in += (w)->strides[_d];                                      \
                _out += (w)->ostride[_d];                                     \
                if (_idx[_d] < (w)->sizes[_d]) break;                         \
                _in -= (w)->strides[_d] * (w)->sizes[_d];                     \
                _out -= (w)->ostride[_d] * (w)->sizes[_d];                    \
                _idx[_d] = 0;                                                 \
            }                                                                 \
        }                                                                     \
    }

/* ReductionKernels.cpp:72-106: acc_t = double for float; sequential; fill_ rounds. */
float or_sum_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides) {
    int64_t n = numel_of(ndim, sizes);
    double acc = 0.0;
    for (int64_t i = 0; i < n; ++i) acc += (double)x[logical_offset(ndim, sizes, strides, i)];
    return (float)acc;
}

/* ReductionKernels.cpp:108-189: out zero-initialised, out[o] += x (fp32) in walk order. */
void or_sum_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                uint32_t reduce_mask, float* out) {
    walk_t w; walk_init(&w, ndim, sizes, strides, reduce_mask);
    int64_t no = kept_numel(ndim, sizes, reduce_mask);
    for (int64_t i = 0; i < no; ++i) out[i] = 0.0f;
    WALK_BEGIN(&w)
        out[out_off] = out[out_off] + x[in_off];
    WALK_END(&w)
}

/* div_scalar_kernel (ArithmeticKernels.cpp:1502-1532): (float)(a / (double)Scalar),
 * Scalar built from (float)count (ReductionKernels.cpp:195,210). */
static float div_by_count(float a, int64_t count) {
    double c = (double)(float)count;
    return (float)((double)a / c);
}

float or_mean_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides) {
    float s = or_sum_all(x, ndim, sizes, strides);
    return div_by_count(s, numel_of(ndim, sizes));
}

/* count multiplies the size of every listed dim, duplicates included
 * (ReductionKernels.cpp:203-208). */
static int64_t list_count(int ndim, const int64_t* sizes, const int64_t* dims, int nd) {
    int64_t c = 1;
    for (int i = 0; i < nd; ++i) {
        int64_t d = dims[i];
        if (d < 0) d += ndim;
        c *= sizes[d];
    }
    return c;
}

void or_mean_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 uint32_t reduce_mask, const int64_t* dims_list, int n_dims_list, float* out) {
    or_sum_dim(x, ndim, sizes, strides, reduce_mask, out);
    int64_t count = list_count(ndim, sizes, dims_list, n_dims_list);
    int64_t no = kept_numel(ndim, sizes, reduce_mask);
    for (int64_t i = 0; i < no; ++i) out[i] = div_by_count(out[i], count);
}

/* ReductionKernels.cpp:231-254 / 317-340: init -inf/+inf, strict compare
 * (NaN never replaces), empty -> RuntimeError. */
int or_minmax_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                  int is_max, float* out) {
    int64_t n = numel_of(ndim, sizes);
    if (n == 0) return -1;
    float best = is_max ? -INFINITY : INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        float v = x[logical_offset(ndim, sizes, strides, i)];
        if (is_max ? (v > best) : (v < best)) best = v;
    }
    *out = best;
    return 0;
}

/* ReductionKernels.cpp:256-315 / 342-401. */
void or_minmax_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                   uint32_t reduce_mask, int is_max, float* out) {
    walk_t w; walk_init(&w, ndim, sizes, strides, reduce_mask);
    int64_t no = kept_numel(ndim, sizes, reduce_mask);
    for (int64_t i = 0; i < no; ++i) out[i] = is_max ? -INFINITY : INFINITY;
    WALK_BEGIN(&w)
        float v = x[in_off];
        if (is_max ? (v > out[out_off]) : (v < out[out_off])) out[out_off] = v;
    WALK_END(&w)
}

/* ReductionKernels.cpp:683-708: flat, strict compare, first index wins, 0 if none. */
int64_t or_argminmax_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                         int is_max) {
    int64_t n = numel_of(ndim, sizes), bi = 0;
    float best = is_max ? -INFINITY : INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        float v = x[logical_offset(ndim, sizes, strides, i)];
        if (is_max ? (v > best) : (v < best)) { best = v; bi = i; }
    }
    return bi;
}

/* ReductionKernels.cpp:710-745.  quirk=1: rows enumerate the transpose(d,-1)
 * prefix dims in row-major order and are written linearly (the CPU layout);
 * quirk=0: rows enumerate the kept dims in their original order. */
void or_argminmax_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                      int dim, int is_max, int quirk, int64_t* out) {
    int order[MAXD]; int np = 0;
    if (quirk) {
        for (int p = 0; p < ndim - 1; ++p) order[np++] = (p == dim) ? ndim - 1 : p;
    } else {
        for (int p = 0; p < ndim; ++p) if (p != dim) order[np++] = p;
    }
    int64_t rows = 1;
    for (int p = 0; p < np; ++p) rows *= sizes[order[p]];
    int64_t len = sizes[dim], st = strides[dim];
    for (int64_t r = 0; r < rows; ++r) {
        int64_t rem = r, base = 0;
        for (int p = np - 1; p >= 0; --p) {
            int64_t s = sizes[order[p]];
            base += (rem % s) * strides[order[p]];
            rem /= s;
        }
        float best = is_max ? -INFINITY : INFINITY;
        int64_t bi = 0;
        for (int64_t j = 0; j < len; ++j) {
            float v = x[base + j * st];
            if (is_max ? (v > best) : (v < best)) { best = v; bi = j; }
        }
        out[r] = bi;
    }
}

/* ReductionKernels.cpp:817-827 (+ std :849-851).  mean (fp32) -> diff (fp32) ->
 * diff*diff (fp32) -> sum (double acc, rounded to float) -> / max(0, n-corr). */
float or_var_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 int64_t correction, int take_sqrt) {
    int64_t n = numel_of(ndim, sizes);
    if (n == 0) return NAN;
    float m = or_mean_all(x, ndim, sizes, strides);
    double acc = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        float d = x[logical_offset(ndim, sizes, strides, i)] - m;
        float sq = d * d;
        acc += (double)sq;
    }
    float sum_sq = (float)acc;
    double div = (double)(n - correction);
    if (div < 0.0) div = 0.0;
    float v = (float)((double)sum_sq / div);
    return take_sqrt ? sqrtf(v) : v;
}

/* ReductionKernels.cpp:829-847 (+ std :853-855). */
void or_var_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                uint32_t reduce_mask, const int64_t* dims_list, int n_dims_list,
                int64_t correction, int take_sqrt, float* out) {
    int64_t no = kept_numel(ndim, sizes, reduce_mask);
    int64_t n = numel_of(ndim, sizes);
    if (n == 0) { for (int64_t i = 0; i < no; ++i) out[i] = NAN; return; }
    float* mean = (float*)malloc(sizeof(float) * (size_t)(no ? no : 1));
    or_mean_dim(x, ndim, sizes, strides, reduce_mask, dims_list, n_dims_list, mean);
    walk_t w; walk_init(&w, ndim, sizes, strides, reduce_mask);
    for (int64_t i = 0; i < no; ++i) out[i] = 0.0f;
    WALK_BEGIN(&w)
        float d = x[in_off] - mean[out_off];
        float sq = d * d;
        out[out_off] = out[out_off] + sq;
    WALK_END(&w)
    free(mean);
    int64_t cnt = list_count(ndim, sizes, dims_list, n_dims_list);
    double div = (double)(cnt - correction);
    if (div < 0.0) div = 0.0;
    for (int64_t i = 0; i < no; ++i) {
        float v = (float)((double)out[i] / div);
        out[i] = take_sqrt ? sqrtf(v) : v;
    }
}

/* ---- topk (this build's definition; no reference counterpart) ---- */
static inline uint32_t f2key(float f, int largest) {
    uint32_t u; memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) u = 0x7fc00000u;   /* NaN: largest */
    if (u == 0x80000000u) u = 0u;                            /* -0 == +0     */
    uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return largest ? k : ~k;
}

/* composite: higher key first, then lower index first */
static inline uint64_t comp_key(uint32_t key, int64_t idx) {
    return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

static void heap_sift_down(uint64_t* h, int64_t n, int64_t i) {
    for (;;) {
        int64_t l = 2 * i + 1, r = l + 1, m = i;
        if (l < n && h[l] < h[m]) m = l;
        if (r < n && h[r] < h[m]) m = r;
        if (m == i) return;
        uint64_t t = h[i]; h[i] = h[m]; h[m] = t; i = m;
    }
}

static int cmp_desc_u64(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x < y) - (x > y);
}

static void topk_rows(const float* x, int64_t r0, int64_t r1, int64_t cols, int64_t row_stride,
                      int64_t k, int largest, float* out_vals, int64_t* out_idx) {
    if (k <= 0) return;
    uint64_t* h = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)k);
    for (int64_t r = r0; r < r1; ++r) {
        const float* p = x + r * row_stride;
        int64_t n = 0;
        for (int64_t j = 0; j < cols; ++j) {
            uint64_t c = comp_key(f2key(p[j], largest), j);
            if (n < k) {                        /* build min-heap of the best k */
                h[n++] = c;
                if (n == k) for (int64_t i = k / 2 - 1; i >= 0; --i) heap_sift_down(h, k, i);
            } else if (c > h[0]) {
                h[0] = c; heap_sift_down(h, k, 0);
            }
        }
        qsort(h, (size_t)n, sizeof(uint64_t), cmp_desc_u64);
        for (int64_t i = 0; i < k; ++i) {
            int64_t j = (int64_t)(0xffffffffu - (uint32_t)(h[i] & 0xffffffffu));
            out_idx[r * k + i] = j;
            out_vals[r * k + i] = p[j];
        }
    }
    free(h);
}

void or_topk(const float* x, int64_t rows, int64_t cols, int64_t row_stride, int64_t k,
             int largest, float* out_vals, int64_t* out_idx) {
    topk_rows(x, 0, rows, cols, row_stride, k, largest, out_vals, out_idx);
}

typedef struct {
    const float* x; int64_t r0, r1, cols, row_stride, k; int largest;
    float* ov; int64_t* oi;
} topk_job;

static void* topk_thread(void* a) {
    topk_job* j = (topk_job*)a;
    topk_rows(j->x, j->r0, j->r1, j->cols, j->row_stride, j->k, j->largest, j->ov, j->oi);
    return NULL;
}

void or_topk_mt(const float* x, int64_t rows, int64_t cols, int64_t row_stride, int64_t k,
                int largest, float* out_vals, int64_t* out_idx, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    pthread_t th[256]; topk_job jobs[256];
    int64_t per = (rows + n_threads - 1) / n_threads;
    int used = 0;
    for (int t = 0; t < n_threads; ++t) {
        int64_t r0 = t * per, r1 = r0 + per;
        if (r1 > rows) r1 = rows;
        if (r0 >= r1) break;
        jobs[t] = (topk_job){x, r0, r1, cols, row_stride, k, largest, out_vals, out_idx};
        pthread_create(&th[t], NULL, topk_thread, &jobs[t]);
        used++;
    }
    for (int t = 0; t < used; ++t) pthread_join(th[t], NULL);
}

/* ---- prod / all / any / norm / median (ReductionKernels.cpp:406-677, :858-901) ---- */

/* prod_kernel (:406-439): out dtype float32 for float input, `ctype prod_val = 1`
 * multiplied sequentially in float over the contiguous copy. */
float or_prod_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides) {
    int64_t n = numel_of(ndim, sizes);
    float acc = 1.0f;
    for (int64_t i = 0; i < n; ++i) acc = acc * x[logical_offset(ndim, sizes, strides, i)];
    return acc;
}

/* prod_dim_kernel (:441-514): out = ones, out[o] *= x (float) in walk order. */
void or_prod_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 uint32_t reduce_mask, float* out) {
    walk_t w; walk_init(&w, ndim, sizes, strides, reduce_mask);
    int64_t no = kept_numel(ndim, sizes, reduce_mask);
    for (int64_t i = 0; i < no; ++i) out[i] = 1.0f;
    WALK_BEGIN(&w)
        out[out_off] = out[out_off] * x[in_off];
    WALK_END(&w)
}

/* all_kernel / any_kernel (:517-563): static_cast<bool>(x), i.e. x != 0 (NaN is
 * true); empty all = true, empty any = false. */
int or_allany_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides, int is_any) {
    int64_t n = numel_of(ndim, sizes);
    for (int64_t i = 0; i < n; ++i) {
        int b = x[logical_offset(ndim, sizes, strides, i)] != 0.0f;
        if (is_any && b) return 1;
        if (!is_any && !b) return 0;
    }
    return is_any ? 0 : 1;
}

/* all_dim_kernel / any_dim_kernel (:565-677): out initialised to 1 / 0. */
void or_allany_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                   uint32_t reduce_mask, int is_any, uint8_t* out) {
    walk_t w; walk_init(&w, ndim, sizes, strides, reduce_mask);
    int64_t no = kept_numel(ndim, sizes, reduce_mask);
    for (int64_t i = 0; i < no; ++i) out[i] = is_any ? 0 : 1;
    WALK_BEGIN(&w)
        int b = x[in_off] != 0.0f;
        if (is_any && b) out[out_off] = 1;
        if (!is_any && !b) out[out_off] = 0;
    WALK_END(&w)
}

/* abs().pow(Scalar(p)) (PointwiseKernels.cpp:392-395): std::pow(float, double)
 * in double, stored as float. */
static float abs_pow(float v, double p) { return (float)pow((double)fabsf(v), p); }

/* norm_kernel (:858-864).  p = +-inf: abs().max() / abs().min() (max_kernel's
 * strict compare; returns -1 for an empty tensor, which raises there).
 * Otherwise abs().pow(p).sum() (double accumulation, :94) then .pow(1/p) on the
 * float result. */
int or_norm_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides, double p,
                float* out) {
    int64_t n = numel_of(ndim, sizes);
    if (isinf(p)) {
        if (n == 0) return -1;
        int is_max = p > 0;
        float best = is_max ? -INFINITY : INFINITY;
        for (int64_t i = 0; i < n; ++i) {
            float v = fabsf(x[logical_offset(ndim, sizes, strides, i)]);
            if (is_max ? (v > best) : (v < best)) best = v;
        }
        *out = best;
        return 0;
    }
    double acc = 0.0;
    for (int64_t i = 0; i < n; ++i) acc += (double)abs_pow(x[logical_offset(ndim, sizes, strides, i)], p);
    *out = (float)pow((double)(float)acc, 1.0 / p);
    return 0;
}

/* norm_dim_kernel (:866-872): abs().pow(p).sum(dim) (fp32 accumulation in walk
 * order, :157-178) then .pow(1/p); p = +-inf: abs().max(dim) / min(dim). */
void or_norm_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 uint32_t reduce_mask, double p, float* out) {
    walk_t w; walk_init(&w, ndim, sizes, strides, reduce_mask);
    int64_t no = kept_numel(ndim, sizes, reduce_mask);
    if (isinf(p)) {
        int is_max = p > 0;
        for (int64_t i = 0; i < no; ++i) out[i] = is_max ? -INFINITY : INFINITY;
        WALK_BEGIN(&w)
            float v = fabsf(x[in_off]);
            if (is_max ? (v > out[out_off]) : (v < out[out_off])) out[out_off] = v;
        WALK_END(&w)
        return;
    }
    for (int64_t i = 0; i < no; ++i) out[i] = 0.0f;
    WALK_BEGIN(&w)
        out[out_off] = out[out_off] + abs_pow(x[in_off], p);
    WALK_END(&w)
    for (int64_t i = 0; i < no; ++i) out[i] = (float)pow((double)out[i], 1.0 / p);
}

/* median_kernel (:874-901): the (n-1)/2-th smallest element of the flattened
 * tensor; NaN for an empty one.  std::nth_element leaves the order of NaN and of
 * -0.0 vs +0.0 unspecified; this restatement fixes it as the build's median does:
 * ascending sortable keys, -0.0 == +0.0 (returned as +0.0), NaN above +inf. */
static inline uint32_t asc_key(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) u = 0x7fc00000u;
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
static int cmp_u32(const void* a, const void* b) {
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return (x > y) - (x < y);
}
float or_median(const float* x, int ndim, const int64_t* sizes, const int64_t* strides) {
    int64_t n = numel_of(ndim, sizes);
    if (n == 0) return NAN;
    uint32_t* k = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
    for (int64_t i = 0; i < n; ++i) k[i] = asc_key(x[logical_offset(ndim, sizes, strides, i)]);
    qsort(k, (size_t)n, sizeof(uint32_t), cmp_u32);
    uint32_t key = k[(n - 1) / 2];
    free(k);
    uint32_t bits = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
    float v;
    memcpy(&v, &bits, 4);
    return v;
}

