/*
 * TEST INFRASTRUCTURE ONLY.  CPU restatement of TensorPlay's P10 CPU reduction
 * path (p10/src/backend/cpu/ReductionKernels.cpp) plus this build's topk
 * definition.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load this library, and only as the checker / the timed CPU baseline.
 * The product path (libtpr_rocm.so, tensorplay_amd._C) never links it.
 *
 * All tensors are float32; shapes/strides are in elements (int64).
 */
#ifndef TP_CPU_REDUCE_H
#define TP_CPU_REDUCE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* a1: sum_kernel (ReductionKernels.cpp:72-106): double accumulation in memory
 * order of the contiguous copy, then one rounding to float. */
float or_sum_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides);
/* a2: sum_dim_kernel (ReductionKernels.cpp:108-189): fp32 accumulation in the
 * output buffer, visiting input elements in row-major logical order.
 * reduce_mask bit d set = dim d reduced.  out is contiguous over kept dims. */
void or_sum_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                uint32_t reduce_mask, float* out);
/* a3: mean_kernel / mean_dim_kernel (ReductionKernels.cpp:191-211) followed by
 * div_scalar_kernel (ArithmeticKernels.cpp:1502-1532). */
float or_mean_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides);
void or_mean_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 uint32_t reduce_mask, const int64_t* dims_list, int n_dims_list, float* out);
/* a4: max_kernel/min_kernel (:231-254, :317-340); max_dim/min_dim (:256-315, :342-401).
 * is_max = 1 for max.  Returns 0 on success, -1 for an empty full reduction. */
int or_minmax_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                  int is_max, float* out);
void or_minmax_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                   uint32_t reduce_mask, int is_max, float* out);
/* a5: argmax_kernel/argmin_kernel (:682-812).  dim < 0 after wrapping means flat.
 * quirk = 1 reproduces the CPU path's transpose(d,-1) row layout (:714-735);
 * quirk = 0 gives the permute (CUDA path, ReductionKernels.cu:67-75) layout. */
int64_t or_argminmax_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                         int is_max);
void or_argminmax_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                      int dim, int is_max, int quirk, int64_t* out);
/* a6: var_kernel/var_dim_kernel/std_* (:817-855). */
float or_var_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 int64_t correction, int take_sqrt);
void or_var_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                uint32_t reduce_mask, const int64_t* dims_list, int n_dims_list,
                int64_t correction, int take_sqrt, float* out);
/* prod_kernel / prod_dim_kernel (:406-514): float multiplies, sequential. */
float or_prod_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides);
void or_prod_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 uint32_t reduce_mask, float* out);
/* all/any (:517-677): x != 0 is true (NaN true).  out is one byte per output. */
int or_allany_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides, int is_any);
void or_allany_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                   uint32_t reduce_mask, int is_any, uint8_t* out);
/* norm_kernel / norm_dim_kernel (:858-872).  or_norm_all returns -1 for p = +-inf
 * on an empty tensor (the reference raises there). */
int or_norm_all(const float* x, int ndim, const int64_t* sizes, const int64_t* strides, double p,
                float* out);
void or_norm_dim(const float* x, int ndim, const int64_t* sizes, const int64_t* strides,
                 uint32_t reduce_mask, double p, float* out);
/* median_kernel (:874-901): lower median; NaN for an empty tensor. */
float or_median(const float* x, int ndim, const int64_t* sizes, const int64_t* strides);
/* a11: topk (absent from the reference; this build's definition).  Rows of a
 * [rows, cols] view with row_stride.  Order: key descending, index ascending,
 * where key canonicalises -0.0 to +0.0 and treats NaN as the largest value.
 * largest = 0 reverses the key order (NaN then the smallest).  Values are the
 * input elements at the selected indices (original bits). */
void or_topk(const float* x, int64_t rows, int64_t cols, int64_t row_stride, int64_t k,
             int largest, float* out_vals, int64_t* out_idx);
/* Same selection, rows split over n_threads pthreads (CPU baseline at all cores). */
void or_topk_mt(const float* x, int64_t rows, int64_t cols, int64_t row_stride, int64_t k,
                int largest, float* out_vals, int64_t* out_idx, int n_threads);

/* copy_ (cpu/CopyKernels.cpp:27-55, :73-127): dst[idx] = (dst type) src[idx]
 * over sizes, strides in elements per side, dtypes numbered as P10's
 * ScalarType (UInt8 0 .. Bool 10).  Returns 0, or -1 for an unknown dtype. */
int or_copy(void* dst, int dst_dtype, const int64_t* dst_strides, const void* src, int src_dtype,
            const int64_t* src_strides, int ndim, const int64_t* sizes);

/* Softmax family and nll_loss (tp_cpu_softmax.c): dense [outer, n, inner]
 * float32; see that file for the reference lines each follows. */
void or_softmax(const float* x, int64_t outer, int64_t n, int64_t inner, int32_t log_mode, float* y);
void or_softmax_bwd(const float* g, const float* y, int64_t outer, int64_t n, int64_t inner, int32_t log_mode,
                    float* gx);
int32_t or_nll_loss(const float* x, int64_t N, int64_t C, const int64_t* t, const float* w, int64_t reduction,
                    int64_t ignore_index, float* out, float* total_weight);
void or_nll_loss_backward(const float* g, const int64_t* t, const float* w, int64_t reduction,
                          int64_t ignore_index, int32_t has_tw, float tw_in, int64_t N, int64_t C, float* gi);

#ifdef __cplusplus
}
#endif
#endif
