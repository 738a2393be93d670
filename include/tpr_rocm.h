/*
 * tpr_rocm.h -- C-ABI launch layer of the MI355X (gfx950) reduction + top-k
 * backend.  Plain pointers, sizes and int status codes; no C++ or torch types;
 * no exceptions cross this boundary.  Every call is asynchronous on the given
 * HIP stream (passed as void*, NULL = the default stream) and never allocates
 * user-visible memory: outputs and the workspace are owned by the caller.
 *
 * It replaces the CUDA backend's reduction registrations in TensorPlay
 * (/root/reference/p10/src/backend/cuda/ReductionKernels.cu:385-418), which are
 * reached through the P10 dispatcher
 * (/root/reference/p10/include/Dispatcher.h:46-59, DispatchStub::call).
 * The host adapters in tensorplay_amd/csrc/core/ROCmReductionKernels.cpp
 * register under DispatchKey::ROCm with the dispatcher's exact argument types
 * (tools/codegen/gen.py:38-53, STUB_TYPE_MAP) and call into this layer.
 */
#ifndef TPR_ROCM_H
#define TPR_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TPR_MAX_DIMS 8

/* Status codes.  tpr_last_error() holds a message for the calling thread. */
enum tpr_status {
    TPR_OK = 0,
    TPR_ERR_INVALID_ARG = 1,       /* bad shape, dim, k, pointer, descriptor   */
    TPR_ERR_UNSUPPORTED_DTYPE = 2, /* dtype not implemented on this backend    */
    TPR_ERR_HIP = 3,               /* a HIP runtime call or launch failed      */
    TPR_ERR_WORKSPACE = 4,         /* workspace smaller than *_workspace_bytes */
    TPR_ERR_NOT_IMPLEMENTED = 5
};

/* Element types.  Numbering follows P10's ScalarType
 * (/root/reference/p10/include/DType.h:63-79) so adapters pass it through. */
enum tpr_dtype {
    TPR_UINT8 = 0, TPR_INT8 = 1, TPR_INT16 = 2, TPR_INT32 = 3, TPR_INT64 = 4,
    TPR_UINT16 = 5, TPR_UINT32 = 6, TPR_UINT64 = 7,
    TPR_FLOAT32 = 8, TPR_FLOAT64 = 9, TPR_BOOL = 10
};

/* Reduction operators.  Each maps to the reference kernels named beside it
 * (/root/reference/p10/src/backend/cpu/ReductionKernels.cpp). */
enum tpr_reduce_op {
    TPR_SUM = 0,    /* sum_kernel :72-106, sum_dim_kernel :108-189            */
    TPR_MEAN = 1,   /* mean_kernel :191-196, mean_dim_kernel :198-211         */
    TPR_AMAX = 2,   /* max_kernel :231-254, max_dim_kernel :256-315            */
    TPR_AMIN = 3,   /* min_kernel :317-340, min_dim_kernel :342-401            */
    TPR_ARGMAX = 4, /* argmax_kernel :682-746                                  */
    TPR_ARGMIN = 5, /* argmin_kernel :748-812                                  */
    TPR_VAR = 6,    /* var_kernel :817-827, var_dim_kernel :829-847            */
    TPR_STD = 7,    /* std_kernel :849-851, std_dim_kernel :853-855            */
    TPR_PROD = 8,   /* prod_kernel :406-439, prod_dim_kernel :441-514          */
    TPR_NORM = 9,   /* norm_kernel :858-864, norm_dim_kernel :866-872 (p = desc.p) */
    TPR_ALL = 10,   /* all_kernel :517-539, all_dim_kernel :565-620            */
    TPR_ANY = 11,   /* any_kernel :541-563, any_dim_kernel :622-677            */
    TPR_MEDIAN = 12 /* median_kernel :874-901 (full reductions only)           */
};

/* One reduction over an arbitrary strided view.
 *  - sizes/strides are in elements; strides may be any value (including 0).
 *  - reduce_mask bit d set => dim d is reduced.  reduce_mask == all dims (or
 *    ndim == 0) is a full reduction to one value.
 *  - The output is written densely (row-major over the kept dims, in their
 *    original order); keepdim only changes the shape the caller reports.
 *  - out_dtype: SUM/MEAN/PROD: FLOAT32 or FLOAT64.  AMAX/AMIN: the input
 *    dtype.  ARGMAX/ARGMIN: INT64 (index along the reduced dims, row-major;
 *    first index wins ties; NaN never wins, as the reference's strict
 *    compare).  VAR/STD/NORM: FLOAT32 (FLOAT64 for a FLOAT64 input: every op
 *    takes FLOAT64 inputs and computes in double).  MEDIAN: the input dtype.
 *    Integer and BOOL inputs (every signed and unsigned width) take SUM/PROD
 *    (INT64 output, wrap-around), MEAN (of the values converted to float32),
 *    AMAX/AMIN, ARGMAX/ARGMIN (unsigned order for UINT*), ALL/ANY and MEDIAN.
 *    ALL/ANY: BOOL (one byte, 0/1; an element counts as true when it is != 0,
 *    so NaN is true).
 *  - NORM: (sum |x|^p)^(1/p); p = +inf / -inf: max / min of |x| (NaN ignored,
 *    as AMAX/AMIN); p = 0 gives the reference's n^(1/0).
 *  - MEDIAN: lower median ((n-1)/2-th smallest) of all elements, output in the
 *    input dtype (every dtype); -0.0 == +0.0 (a zero median is returned as
 *    +0.0); NaN ranks above every number.  Only full reductions of a
 *    contiguous view (TPR_ERR_NOT_IMPLEMENTED otherwise); an empty input is
 *    NaN for FLOAT32 and TPR_ERR_INVALID_ARG for the other dtypes.
 *  - count_override > 0 replaces the element count used by MEAN/VAR/STD (the
 *    reference multiplies the size of every listed dim, duplicates included,
 *    ReductionKernels.cpp:203-208 and :840-845); 0 = product of reduced sizes.
 *  - correction: VAR/STD divisor is max(0, count - correction).
 * An empty reduced extent writes: SUM 0, MEAN NaN, AMAX -inf, AMIN +inf,
 * ARGMAX/ARGMIN 0, VAR/STD NaN, PROD 1, ALL 1, ANY 0, NORM 0^(1/p) (-inf / +inf
 * for p = +inf / -inf), MEDIAN NaN (the reference's full max/min raise instead;
 * the adapters check that before calling). */
typedef struct tpr_reduce_desc {
    int32_t op;          /* enum tpr_reduce_op */
    int32_t in_dtype;    /* enum tpr_dtype     */
    int32_t out_dtype;   /* enum tpr_dtype     */
    int32_t ndim;        /* 0..TPR_MAX_DIMS    */
    int64_t sizes[TPR_MAX_DIMS];
    int64_t strides[TPR_MAX_DIMS];
    uint32_t reduce_mask;
    int32_t reserved0;
    int64_t correction;
    int64_t count_override;
    double p;            /* NORM exponent (ignored by the other ops) */
} tpr_reduce_desc;

/* Bytes of device workspace tpr_reduce needs for this descriptor (0 is
 * common).  Deterministic in the descriptor. */
size_t tpr_reduce_workspace_bytes(const tpr_reduce_desc* desc);

/* Launch the reduction.  `in` points at element [0,...,0] of the view.
 * Replaces: DispatchStub<...>::call("sum" | "sum.dim_IntList" | "mean" |
 * "mean.dim" | "max" | "max.dim" | "min" | "min.dim" | "argmax" | "argmin" |
 * "var" | "var.dim" | "std" | "std.dim", DispatchKey::CUDA, ...)
 * (/root/reference/p10/src/backend/cuda/ReductionKernels.cu:385-418).
 * Reductions split over several workgroups per output (few long rows, the
 * full tensor) finish in the same launch: the last workgroup of an output
 * combines the partial states held in the workspace, counted by per-stream
 * ticket counters inside the library (zero at load, left at zero by every
 * launch).  Under graph capture, on the per-thread default stream and beyond
 * 64 streams per device they take a second, finalize launch instead; results
 * are identical either way. */
int tpr_reduce(const tpr_reduce_desc* desc, const void* in, void* out,
               void* workspace, size_t workspace_bytes, void* stream);

/* Size of the fixed per-device scratch array behind tpr_reduce_noalloc. */
#define TPR_REDUCE_SCRATCH_BYTES (8u << 20)

/* tpr_reduce without a workspace argument and without any device allocation:
 * split partial states (and the median's histograms) go to a fixed
 * TPR_REDUCE_SCRATCH_BYTES array that each device holds from the library's
 * load until the process ends.  Results equal tpr_reduce's.
 *  - No counterpart in the reference: for callers that cannot allocate device
 *    memory (code under HIP graph capture, tight serving loops, harnesses that
 *    forbid hipMalloc).
 *  - A descriptor whose tpr_reduce_workspace_bytes exceeds
 *    TPR_REDUCE_SCRATCH_BYTES fails with TPR_ERR_WORKSPACE.
 *  - Every call on one device shares that device's array: calls that overlap
 *    on one device (several streams or host threads) race and give wrong
 *    results; serialise them.  Nothing in the array needs clearing between
 *    calls (every partial is written before it is read). */
int tpr_reduce_noalloc(const tpr_reduce_desc* desc, const void* in, void* out, void* stream);

/* Gradient of a SUM / MEAN / VAR / STD reduction with respect to its input:
 * the formulas of /root/reference/config/derivatives.yaml:82-86 (sum, mean)
 * and :182-186 (var, std), which TensorPlay's autograd composes from expand /
 * div.Scalar / mul / sub / mean, fused into one pass here:
 *   SUM:  gx = g;   MEAN: gx = g / count;
 *   VAR:  gx = (g * 2) * (x - mean) / (count - correction);
 *   STD:  gx = g * (x - mean) / (result * (count - correction)),
 * evaluated in float32 in that order (the divisions by count as the
 * reference's div.Scalar, in double).  `desc` is the forward descriptor (op,
 * in_dtype = out_dtype = FLOAT32, x's sizes / strides, reduce_mask,
 * correction, count_override as for tpr_reduce).  grad_out and result (STD
 * only) are dense over the kept dims, as tpr_reduce writes them; `in` (x) is
 * read by VAR / STD only; grad_in is written dense row-major over sizes.  VAR
 * and STD recompute the mean with tpr_reduce into the workspace; MEAN divides
 * grad_out by the count there, once per output. */
size_t tpr_reduce_backward_workspace_bytes(const tpr_reduce_desc* desc);
int tpr_reduce_backward(const tpr_reduce_desc* desc, const void* grad_out, const void* in, const void* result,
                        void* grad_in, void* workspace, size_t workspace_bytes, void* stream);

/* Top-k along the last dim of a [rows, cols] view whose rows start
 * row_stride elements apart (elements within a row are contiguous).
 * Outputs are dense [rows, k]: values in the input dtype, indices int64.
 * Order: value descending for largest=1 (ascending for largest=0), equal
 * values by lowest index; -0.0 == +0.0; NaN ranks above every number.
 * sorted=0 is accepted and returns the same (sorted) order.
 * k must satisfy 0 <= k <= cols.  No reference counterpart: TensorPlay has no
 * topk; this adds the schema row
 *   topk(Tensor self, int64_t k, int64_t dim=-1, bool largest=true,
 *        bool sorted=true) -> (Tensor values, Tensor indices)
 * next to the reduction rows of config/native_functions.yaml:695-809. */
size_t tpr_topk_workspace_bytes(int32_t dtype, int64_t rows, int64_t cols, int64_t k);
int tpr_topk(const void* in, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride,
             int64_t k, int32_t largest, int32_t sorted, void* out_values, void* out_indices,
             void* workspace, size_t workspace_bytes, void* stream);

/* The plan tpr_topk would run for this call, host only, launches nothing (a
 * test hook with no reference counterpart): out[0] = kernel family (1 lane-group
 * kernel on 1- / 2-byte elements, 2 register radix select, 3 register radix
 * select per segment + merge, 4 streaming radix select, 5 lane-group kernel,
 * 6 wave kernel, 7 workgroup kernel; 6 and 7 add the merge when out[1] > 1; 8 wave kernel on
 * 8-byte rows, then the streaming radix select for the rows it flags),
 * out[1] = segments per row, out[2] = segment length (segment s covers
 * [s * out[2], min(cols, (s + 1) * out[2]))), out[3] = waves per wave-kernel
 * workgroup, out[4] = workspace bytes.  `aligned`: the input and every row
 * start are 16-byte aligned.  Every segment of a split row holds >= k
 * elements: each writes exactly k composites that the merge ranks. */
int tpr_topk_plan(int32_t dtype, int64_t rows, int64_t cols, int64_t k, int64_t row_stride, int32_t aligned,
                  int64_t* out);

/* Top-k / top-p (nucleus) sampling of one token id per row of float32 logits
 * (a consumer of tpr_topk; TensorPlay has no sampler, so the definition is
 * this build's): for the k largest logits of a row, sorted v_0 >= ... >=
 * v_{k-1} (ties to the lowest index, as tpr_topk),
 *   p_j = exp(v_j / T - v_0 / T),  c_j = p_0 + ... + p_j,
 *   m   = the first j with c_j >= top_p * c_{k-1},
 *   out = the column index of the first j <= m with c_j > u * c_m,
 * with u = uniforms[row] in [0, 1) (device float32 [rows], drawn by the
 * caller).  temperature <= 0 selects v_0 (greedy).  top_p in (0, 1], 1 <= k <=
 * cols (k = cols: top-p alone).  out_ids: device int64 [rows].  Workspace:
 * tpr_sample_workspace_bytes: for k <= 1024 tpr_topk's (the draw runs in
 * top-k's last phase, nothing else is written); for k > 1024 tpr_topk's, then
 * the sorted values (float32 [rows][k]) and indices (int64 [rows][k]) that
 * tpr_topk writes there and a second kernel draws from. */
size_t tpr_sample_workspace_bytes(int32_t dtype, int64_t rows, int64_t cols, int64_t k);
int tpr_sample(const void* logits, int32_t dtype, int64_t rows, int64_t cols, int64_t row_stride, int64_t k,
               float temperature, float top_p, const float* uniforms, int64_t* out_ids, void* workspace,
               size_t workspace_bytes, void* stream);

/* Strided, casting copy: dst[idx] = static_cast<dst_dtype>(src[idx]) for
 * every index of sizes[0..ndim).  Strides are in elements, per side; a
 * stride-0 source dim broadcasts.  Replaces DispatchStub::call("copy_",
 * DispatchKey::CUDA, self, src) -> copy_kernel / copy_cast_kernel_impl
 * (/root/reference/p10/src/backend/cuda/CopyKernels.cu:42-157) for a
 * device-resident source; casts follow the CPU path's static_cast
 * (/root/reference/p10/src/backend/cpu/CopyKernels.cpp:27-55).  Overlapping
 * destination elements are undefined, as in the reference. */
typedef struct tpr_copy_desc {
    int32_t ndim;
    int32_t dst_dtype;   /* tpr_dtype */
    int32_t src_dtype;   /* tpr_dtype */
    int32_t reserved0;
    int64_t sizes[TPR_MAX_DIMS];
    int64_t dst_strides[TPR_MAX_DIMS];
    int64_t src_strides[TPR_MAX_DIMS];
} tpr_copy_desc;

int tpr_copy(const tpr_copy_desc* desc, void* dst, const void* src, void* stream);

/* Kernel the planner picks for this copy: bits 0-1 = 0 dense run, 1 rows,
 * 2 LDS tiles, 3 per element; bit 2 set = the 16-byte vector variant;
 * -1 = bad descriptor.  Host only, launches nothing; a test hook with no
 * reference counterpart. */
int tpr_copy_plan(const tpr_copy_desc* desc, const void* dst, const void* src);

/* Strided -> dense copy (row-major over sizes); tpr_copy with a dense
 * destination and equal dtypes.  Counterpart of the CUDA
 * backend's copy_cast_kernel_impl / copy_kernel
 * (/root/reference/p10/src/backend/cuda/CopyKernels.cu:42-157) for the layout
 * normalisation the reduction path needs (Tensor::contiguous, topk on a
 * non-last dim).  elem_size in {1,2,4,8}. */
int tpr_copy_strided(const void* in, int32_t elem_size, int32_t ndim, const int64_t* sizes,
                     const int64_t* in_strides, void* out, void* stream);

/* Softmax family along one dim of a logical [outer, n, inner] view (the
 * softmax dim is n).  Modes:
 *   TPR_SOFTMAX_FWD      out = exp(x - max) / sum(exp(x - max))
 *   TPR_LOG_SOFTMAX_FWD  out = (x - max) - log(sum(exp(x - max)))
 *     replacing softmax_kernel / log_softmax_kernel
 *     (/root/reference/p10/src/backend/cpu/PointwiseKernels.cpp:519-545) and
 *     softmax_kernel_cudnn / log_softmax_kernel_cudnn
 *     (/root/reference/p10/src/backend/cuda/ActivationKernels.cu:136-181);
 *     max ignores NaN, a NaN in a slice makes the slice NaN, and a slice with
 *     no value above -inf is NaN, as the reference composite;
 *   TPR_SOFTMAX_BWD      out = (g - sum(g * y)) * y
 *   TPR_LOG_SOFTMAX_BWD  out = g - exp(y) * sum(g)
 *     the autograd formulas of /root/reference/config/derivatives.yaml:91-95,
 *     with a = g (dL/dy) and b = y (the forward output).
 * a: x (forward) or g (backward), strides a_strides (elements, per logical
 * dim); b: y (backward only, strides b_strides; NULL forward).  out is written
 * dense row-major [outer, n, inner], in the input dtype: FLOAT32, or FLOAT64
 * (computed in double; the reference composite keeps the input dtype).  Workspace:
 * tpr_softmax_workspace_bytes(desc) bytes (0 for most shapes; rows longer than
 * the register-resident kernels hold, when there are few of them, use
 * per-chunk partial statistics).  Some shapes (long rows, gradients, strided
 * dims of 513..1024) split a slice over several workgroups that exchange
 * partial statistics through a fixed per-device array of the library (2 MiB
 * of device memory, not the workspace), tagged per call: calls on different
 * streams may run at the same time; a partner that is not seen within about
 * 40 us is recomputed, so the result never depends on scheduling. */
enum tpr_softmax_mode {
    TPR_SOFTMAX_FWD = 0,
    TPR_LOG_SOFTMAX_FWD = 1,
    TPR_SOFTMAX_BWD = 2,
    TPR_LOG_SOFTMAX_BWD = 3
};

typedef struct tpr_softmax_desc {
    int32_t mode;  /* enum tpr_softmax_mode */
    int32_t dtype; /* TPR_FLOAT32 or TPR_FLOAT64 (a, b and out alike) */
    int64_t outer, n, inner;
    int64_t a_strides[3];
    int64_t b_strides[3];
} tpr_softmax_desc;

size_t tpr_softmax_workspace_bytes(const tpr_softmax_desc* desc);
int tpr_softmax(const tpr_softmax_desc* desc, const void* a, const void* b, void* out, void* workspace,
                size_t workspace_bytes, void* stream);

/* nll_loss forward (/root/reference/p10/src/backend/cpu/LossKernels.cpp:12-55;
 * CUDA nll_loss_cuda, /root/reference/p10/src/backend/cuda/LossKernels.cu:66-113).
 * input: float32 [n, c] with strides (s0, s1); target: int64 [n], stride ts;
 * weight: float32 [c] dense or NULL.  reduction 0 = none (out: float32 [n],
 * dense), 1 = mean, 2 = sum (out: one float32).  total_weight (one float32)
 * receives the sum of weight[target] over samples whose target is not
 * ignore_index, for every reduction.  A target outside [0, c) that is not
 * ignore_index contributes nothing and sets *status (one device int32) to 1;
 * otherwise *status is 0 (the reference CPU path raises "Target out of
 * bounds"; the adapter reads the flag and raises the same).  Loss and weight
 * sums accumulate in fp64; mean divides by the float32-rounded total weight
 * when it is > 0, as the reference.  Workspace: tpr_nll_loss_workspace_bytes. */
size_t tpr_nll_loss_workspace_bytes(int64_t n);
int tpr_nll_loss(const void* input, int32_t dtype, int64_t n, int64_t c, int64_t s0, int64_t s1,
                 const int64_t* target, int64_t ts, const void* weight, int64_t reduction,
                 int64_t ignore_index, void* out, void* total_weight, int32_t* status,
                 void* workspace, size_t workspace_bytes, void* stream);

/* nll_loss_backward (/root/reference/p10/src/backend/cpu/LossKernels.cpp:57-101;
 * CUDA /root/reference/p10/src/backend/cuda/LossKernels.cu:115-170): writes the
 * dense float32 [n, c] grad_input in one pass: 0 everywhere except
 * grad_input[i, target[i]] = -weight[target[i]] * g_i for samples whose target
 * is in [0, c) and not ignore_index.  g_i = grad_output[i * gs] (reduction 0)
 * or grad_output[0]; reduction 1 divides it by *total_weight (device float32)
 * when that is > 0. */
int tpr_nll_loss_backward(const void* grad_output, int64_t gs, const int64_t* target, int64_t ts,
                          const void* weight, const void* total_weight, int64_t n, int64_t c,
                          int64_t reduction, int64_t ignore_index, void* grad_input, void* stream);

/* Thread-local message for the last non-OK status on this thread. */
const char* tpr_last_error(void);

/* ABI version (major << 16 | minor); 1.4 accepts UINT16/32/64 reduction inputs. */
int32_t tpr_abi_version(void);

/* Tuning / test hook, exported by the test build libtpr_rocm_dev.so only (built
 * with -DTPR_DEBUG_KNOBS); the shipped libtpr_rocm.so does not export it and
 * plans every launch from its arguments and the device alone.  Forces plan
 * choices.  Keys: "splits" (row/full/column
 * split count, 0 = automatic), "lanes" (threads per row in the row kernel, 16..1024,
 * 0 = automatic), "general" (1 = always use the generic strided kernel),
 * "topk_fallback" (1 = always take top-k's exact multi-pass path), "tx" (64, 128
 * or 256: threads across the contiguous dim in the column kernel, 0 = automatic),
 * "unroll" (1, 2 or 4 vectors in flight per thread in the row/column and gradient-row kernels,
 * 0 = automatic), "colblock" (256, 512 or 1024 threads per column-kernel
 * workgroup, 0 = automatic),
 * "smx_two_pass" (1 = softmax rows always take the two-pass kernel),
 * "smx_split" (1 / -1 = long softmax rows always / never split over chunk
 * workgroups, 0 = automatic), "smx_lanes" (512 = softmax rows of 16385..32768
 * floats on 512-thread workgroups, 0 = automatic), "smx_res" (-1 = never hold long
 * softmax rows or strided-dim slices on chip: two-pass kernels, 0 = automatic),
 * "topk_variant" (wave kernel prefetch depth: 1 = none, 2 = one slice, 3 = two
 * slices; also, as a power of two 1..32, the register radix select's sort
 * composites per thread where the sort size allows; 0 = automatic),
 * "topk_waves" (4, 8 or 16 waves per wave-kernel workgroup, 0 = automatic),
 * "split_fin" (-1 = split reductions always take the separate finalize launch),
 * "smx_pieces" (-1 = softmax gradients never take the row-piece kernels, nor
 * does the forward), "smx_fwd_pieces" (1 = the forward row-piece kernel for
 * every row it can hold, -1 = never, 0 = automatic),
 * "smx_spin" (-1 = row pieces never wait for each other's partial statistics:
 * every piece recomputes them from memory),
 * "topk_short" (1 = the lane-group kernel for every row it can hold, -1 =
 * never), "topk_radix" (1 = the radix-select kernels for every k, 2 = the
 * streaming one, -1 = never where another kernel can), "topk_dyn" (-1 = static
 * slice order in the 16-wave kernel), "rowreg" (-1 = no register-row sum
 * kernel), "nt" (1 / -1 = nontemporal accesses always / never where a kernel
 * chooses them, 0 = automatic).
 * Process-wide in the test build; not synchronised with concurrent launches.  Returns
 * TPR_ERR_INVALID_ARG for an unknown key.  No reference counterpart. */
int tpr_debug_set(const char* key, int64_t value);

/* Test build only, like tpr_debug_set: reads a device-side check counter into
 * *value and clears it (synchronous copies on the default stream).  Key
 * "topk_merge_clamped": outputs of the split-row top-k merge whose row index
 * lay past the row (a segment that broke the contract of writing k
 * composites); the merge clamps such an index into the row in every build,
 * and counts it here.  No reference counterpart. */
int tpr_debug_get(const char* key, int64_t* value);

#ifdef __cplusplus
}
#endif
#endif /* TPR_ROCM_H */
