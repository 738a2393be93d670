// ROCm backend for the P10 reduction schemas: host adapters registered under
// DispatchKey::ROCm.  Each adapter takes exactly the argument types
// DispatchStub passes (TensorPlay's STUB_TYPE_MAP, tools/codegen/gen.py:38-53 --
// int64_t[] arrives as const std::vector<int64_t>&), reproduces the reference
// kernel's shape / dtype / error rules
// (/root/reference/p10/src/backend/cpu/ReductionKernels.cpp), allocates the
// output with the caching allocator and launches through the C-ABI
// (include/tpr_rocm.h).  The CUDA registrations these replace are
// /root/reference/p10/src/backend/cuda/ReductionKernels.cu:385-418.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>

#include "Allocator.h"
#include "Dispatcher.h"
#include "Exception.h"
#include "Tensor.h"
#include "tpr_rocm.h"

namespace tensorplay {
namespace rocm {
namespace {

[[noreturn]] void throw_status(int rc, const char* op) {
    std::string msg = std::string(op) + ": " + tpr_last_error();
    switch (rc) {
        case TPR_ERR_UNSUPPORTED_DTYPE:
        case TPR_ERR_NOT_IMPLEMENTED: TP_THROW(NotImplementedError, msg);
        case TPR_ERR_INVALID_ARG: TP_THROW(RuntimeError, msg);
        default: TP_THROW(RuntimeError, msg);
    }
}

int64_t wrap(int64_t d, int64_t nd) {
    const int64_t w = d < 0 ? d + nd : d;
    if (w < 0 || w >= nd) TP_THROW(RuntimeError, "Dimension out of range");
    return w;
}

uint32_t mask_of(const Tensor& self, const std::vector<int64_t>& dims) {
    uint32_t m = 0;
    for (int64_t d : dims) m |= 1u << wrap(d, self.dim());
    return m;
}

// count of the listed dims, duplicates included (ReductionKernels.cpp:203-208)
int64_t listed_count(const Tensor& self, const std::vector<int64_t>& dims) {
    int64_t c = 1;
    for (int64_t d : dims) c *= self.size(wrap(d, self.dim()));
    return c;
}

void require_float32_input(const Tensor& self, const char* op) {
    if (self.dtype() != DType::Float32)
        TP_THROW(NotImplementedError, std::string(op) + " not implemented for dtype " + toString(self.dtype()) +
                                          " on ROCm (float32 only)");
    if (self.dim() > TPR_MAX_DIMS) TP_THROW(NotImplementedError, std::string(op) + ": more than 8 dims on ROCm");
}

// var/std/norm: Float32 or Float64 (computed in double for Float64, as the
// reference's AccumulateType<double>).
void require_float_input(const Tensor& self, const char* op) {
    if (self.dtype() != DType::Float32 && self.dtype() != DType::Float64)
        TP_THROW(NotImplementedError, std::string(op) + " not implemented for dtype " + toString(self.dtype()) +
                                          " on ROCm (float32 / float64)");
    if (self.dim() > TPR_MAX_DIMS) TP_THROW(NotImplementedError, std::string(op) + ": more than 8 dims on ROCm");
}

// sum/mean/prod, max/min, argmax/argmin and all/any also take Float64, the
// every integer dtype and Bool (the reference instantiates them for every
// scalar type).
void require_reducible_input(const Tensor& self, const char* op) {
    switch (self.dtype()) {
        case DType::Float32: case DType::Float64: case DType::UInt8: case DType::Int8: case DType::Int16:
        case DType::Int32: case DType::Int64: case DType::UInt16: case DType::UInt32: case DType::UInt64:
        case DType::Bool: break;
        default:
            TP_THROW(NotImplementedError, std::string(op) + " not implemented for dtype " + toString(self.dtype()) +
                                              " on ROCm");
    }
    if (self.dim() > TPR_MAX_DIMS) TP_THROW(NotImplementedError, std::string(op) + ": more than 8 dims on ROCm");
}

Tensor launch(const Tensor& self, int op, uint32_t mask, DType out_dtype, const std::vector<int64_t>& out_shape,
              int64_t correction, int64_t count_override, const char* name, double p = 2.0) {
    Tensor out = Tensor::empty(out_shape, out_dtype, self.device());
    tpr_reduce_desc d;
    std::memset(&d, 0, sizeof(d));
    d.op = op;
    d.in_dtype = (int32_t)self.dtype();
    d.out_dtype = (int32_t)out_dtype;
    d.ndim = (int32_t)self.dim();
    for (int i = 0; i < d.ndim; ++i) {
        d.sizes[i] = self.shape()[i];
        d.strides[i] = self.strides()[i];
    }
    d.reduce_mask = mask;
    d.correction = correction;
    d.count_override = count_override;
    d.p = p;
    const size_t wsb = tpr_reduce_workspace_bytes(&d);
    std::shared_ptr<void> ws;
    if (wsb) ws = allocate(wsb, self.device());
    DeviceGuard guard(self.device());
    const int rc = tpr_reduce(&d, self.data_ptr(), out.data_ptr(), ws.get(), wsb, currentStream(self.device().index));
    if (rc != TPR_OK) throw_status(rc, name);
    return out;  // `ws` returns to the cache; reuse is ordered on the same stream
}

uint32_t all_dims(const Tensor& self) { return self.dim() == 0 ? 0u : ((1u << self.dim()) - 1u); }

DType sum_out_dtype(const Tensor& self, DType dtype) {
    if (dtype != DType::Undefined) return dtype;
    return isIntegralType(self.dtype(), true) ? DType::Int64 : self.dtype();
}

DType mean_out_dtype(const Tensor& self, DType dtype) {
    if (dtype != DType::Undefined) return dtype;
    return isFloatingType(self.dtype()) ? self.dtype() : DType::Float32;
}

}  // namespace

// sum_kernel (ReductionKernels.cpp:72-106)
Tensor sum_kernel(const Tensor& self, DType dtype) {
    require_reducible_input(self, "sum");
    return launch(self, TPR_SUM, all_dims(self), sum_out_dtype(self, dtype), {}, 0, 0, "sum");
}

// sum_dim_kernel (ReductionKernels.cpp:108-189); empty dims -> full sum
Tensor sum_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, bool keepdim, DType dtype) {
    if (dims.empty()) return sum_kernel(self, dtype);
    require_reducible_input(self, "sum");
    const auto shape = reductionShape(self.shape(), dims, keepdim);
    return launch(self, TPR_SUM, mask_of(self, dims), sum_out_dtype(self, dtype), shape, 0, 0, "sum");
}

// mean_kernel (ReductionKernels.cpp:191-196)
Tensor mean_kernel(const Tensor& self, DType dtype) {
    require_reducible_input(self, "mean");
    return launch(self, TPR_MEAN, all_dims(self), mean_out_dtype(self, dtype), {}, 0, 0, "mean");
}

// mean_dim_kernel (ReductionKernels.cpp:198-211)
Tensor mean_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, bool keepdim, DType dtype) {
    if (dims.empty()) return mean_kernel(self, dtype);
    require_reducible_input(self, "mean");
    const auto shape = reductionShape(self.shape(), dims, keepdim);
    return launch(self, TPR_MEAN, mask_of(self, dims), mean_out_dtype(self, dtype), shape, 0,
                  listed_count(self, dims), "mean");
}

// max_kernel / min_kernel (ReductionKernels.cpp:231-254, :317-340): empty -> RuntimeError
Tensor max_kernel(const Tensor& self) {
    require_reducible_input(self, "max");
    if (self.numel() == 0) TP_THROW(RuntimeError, "max(): Expected reduction dim to be non-empty");
    return launch(self, TPR_AMAX, all_dims(self), self.dtype(), {}, 0, 0, "max");
}
Tensor min_kernel(const Tensor& self) {
    require_reducible_input(self, "min");
    if (self.numel() == 0) TP_THROW(RuntimeError, "min(): Expected reduction dim to be non-empty");
    return launch(self, TPR_AMIN, all_dims(self), self.dtype(), {}, 0, 0, "min");
}

// max_dim_kernel / min_dim_kernel (ReductionKernels.cpp:256-315, :342-401)
Tensor max_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, bool keepdim) {
    if (dims.empty()) return max_kernel(self);
    require_reducible_input(self, "max");
    return launch(self, TPR_AMAX, mask_of(self, dims), self.dtype(), reductionShape(self.shape(), dims, keepdim), 0,
                  0, "max");
}
Tensor min_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, bool keepdim) {
    if (dims.empty()) return min_kernel(self);
    require_reducible_input(self, "min");
    return launch(self, TPR_AMIN, mask_of(self, dims), self.dtype(), reductionShape(self.shape(), dims, keepdim), 0,
                  0, "min");
}

// argmax_kernel / argmin_kernel (ReductionKernels.cpp:682-812).  dim == None:
// flat index, 0-dim Int64 result (keepdim ignored, as the reference).  With a
// dim the result follows the permute layout of the CUDA path
// (ReductionKernels.cu:67-75): out[i0..] = index along `dim` for the kept
// dims in their original order.
static Tensor arg_kernel(const Tensor& self, std::optional<int64_t> dim, bool keepdim, bool is_max) {
    const char* name = is_max ? "argmax" : "argmin";
    require_reducible_input(self, name);
    const int op = is_max ? TPR_ARGMAX : TPR_ARGMIN;
    if (!dim.has_value()) return launch(self, op, all_dims(self), DType::Int64, {}, 0, 0, name);
    int64_t d = *dim;
    if (d < 0) d += self.dim();
    if (d < 0 || d >= self.dim()) TP_THROW(IndexError, "Dimension out of range");
    if (self.size(d) == 0) TP_THROW(RuntimeError, std::string(name) + "(): Expected reduction dim to be non-empty");
    return launch(self, op, 1u << d, DType::Int64, reductionShape(self.shape(), {d}, keepdim), 0, 0, name);
}
Tensor argmax_kernel(const Tensor& self, std::optional<int64_t> dim, bool keepdim) {
    return arg_kernel(self, dim, keepdim, true);
}
Tensor argmin_kernel(const Tensor& self, std::optional<int64_t> dim, bool keepdim) {
    return arg_kernel(self, dim, keepdim, false);
}

// var_kernel / std_kernel (ReductionKernels.cpp:817-827, :849-851)
static Tensor var_full(const Tensor& self, int64_t correction, bool take_sqrt) {
    const char* name = take_sqrt ? "std" : "var";
    require_float_input(self, name);
    return launch(self, take_sqrt ? TPR_STD : TPR_VAR, all_dims(self), self.dtype(), {}, correction, 0, name);
}
// var_dim_kernel / std_dim_kernel (ReductionKernels.cpp:829-847, :853-855)
static Tensor var_dims(const Tensor& self, const std::vector<int64_t>& dims, int64_t correction, bool keepdim,
                       bool take_sqrt) {
    const char* name = take_sqrt ? "std" : "var";
    require_float_input(self, name);
    // An empty dim list is the full-tensor variance here.  (The reference's
    // var_dim_kernel with {} centres on the un-divided full sum and divides by
    // max(0, 1 - correction); that result is not meaningful and is not copied.)
    if (dims.empty()) return var_full(self, correction, take_sqrt);
    const auto shape = reductionShape(self.shape(), dims, keepdim);
    return launch(self, take_sqrt ? TPR_STD : TPR_VAR, mask_of(self, dims), self.dtype(), shape, correction,
                  listed_count(self, dims), name);
}
Tensor var_kernel(const Tensor& self, int64_t correction) { return var_full(self, correction, false); }
Tensor std_kernel(const Tensor& self, int64_t correction) { return var_full(self, correction, true); }
Tensor var_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, int64_t correction, bool keepdim) {
    return var_dims(self, dims, correction, keepdim, false);
}
Tensor std_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, int64_t correction, bool keepdim) {
    return var_dims(self, dims, correction, keepdim, true);
}

// prod_kernel / prod_dim_kernel (ReductionKernels.cpp:406-514).  Output dtype as
// sum (integral -> Int64); float inputs multiply in fp64 here (the reference
// multiplies in the output dtype).  Empty dims -> full product.
Tensor prod_kernel(const Tensor& self, DType dtype) {
    require_reducible_input(self, "prod");
    return launch(self, TPR_PROD, all_dims(self), sum_out_dtype(self, dtype), {}, 0, 0, "prod");
}
Tensor prod_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, bool keepdim, DType dtype) {
    if (dims.empty()) return prod_kernel(self, dtype);
    require_reducible_input(self, "prod");
    const auto shape = reductionShape(self.shape(), dims, keepdim);
    return launch(self, TPR_PROD, mask_of(self, dims), sum_out_dtype(self, dtype), shape, 0, 0, "prod");
}

// all_kernel / any_kernel / all_dim_kernel / any_dim_kernel
// (ReductionKernels.cpp:517-677): Bool output, x != 0 is true (NaN is true).
static Tensor bool_reduce(const Tensor& self, const std::vector<int64_t>* dims, bool keepdim, bool is_any) {
    const char* name = is_any ? "any" : "all";
    require_reducible_input(self, name);
    const int op = is_any ? TPR_ANY : TPR_ALL;
    if (!dims || dims->empty()) return launch(self, op, all_dims(self), DType::Bool, {}, 0, 0, name);
    return launch(self, op, mask_of(self, *dims), DType::Bool, reductionShape(self.shape(), *dims, keepdim), 0, 0,
                  name);
}
Tensor all_kernel(const Tensor& self) { return bool_reduce(self, nullptr, false, false); }
Tensor any_kernel(const Tensor& self) { return bool_reduce(self, nullptr, false, true); }
Tensor all_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, bool keepdim) {
    return bool_reduce(self, &dims, keepdim, false);
}
Tensor any_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, bool keepdim) {
    return bool_reduce(self, &dims, keepdim, true);
}

// norm_kernel / norm_dim_kernel (ReductionKernels.cpp:858-872): (sum |x|^p)^(1/p);
// p = +-inf: max / min of |x| (an empty full reduction raises, as max()/min()).
// Every p is served on ROCm (the CUDA path serves p = 2 only,
// ReductionKernels.cu:295-321).
Tensor norm_kernel(const Tensor& self, double p) {
    require_float_input(self, "norm");
    if (std::isinf(p) && self.numel() == 0)
        TP_THROW(RuntimeError, std::string(p > 0 ? "max" : "min") + "(): Expected reduction dim to be non-empty");
    return launch(self, TPR_NORM, all_dims(self), self.dtype(), {}, 0, 0, "norm", p);
}
Tensor norm_dim_kernel(const Tensor& self, const std::vector<int64_t>& dims, double p, bool keepdim) {
    require_float_input(self, "norm");
    if (dims.empty()) return norm_kernel(self, p);
    const auto shape = reductionShape(self.shape(), dims, keepdim);
    return launch(self, TPR_NORM, mask_of(self, dims), self.dtype(), shape, 0, 0, "norm", p);
}

// median_kernel (ReductionKernels.cpp:874-901): lower median of all elements
// (every dtype the reference instantiates), a 0-dim tensor of the input dtype; an empty input gives a one-element NaN
// tensor (shape [1]), as the reference's Tensor::tensor({NaN}).
Tensor median_kernel(const Tensor& self) {
    require_reducible_input(self, "median");
    if (self.numel() == 0) {  // Float32 NaN whatever the input dtype, as the reference
        const Tensor flat = Tensor::empty({0}, DType::Float32, self.device());
        return launch(flat, TPR_MEDIAN, 1u, DType::Float32, {}, 0, 0, "median").reshape({1});
    }
    const Tensor x = self.contiguous();
    return launch(x, TPR_MEDIAN, all_dims(x), x.dtype(), {}, 0, 0, "median");
}

// topk(Tensor self, int64_t k, int64_t dim=-1, bool largest=true, bool sorted=true)
//   -> (Tensor values, Tensor indices)
// New schema (TensorPlay has no topk).  The selected dim is moved last and made
// contiguous when it is not already; the results are returned with `dim` in its
// original position, dense.
std::tuple<Tensor, Tensor> topk_kernel(const Tensor& self, int64_t k, int64_t dim, bool largest, bool sorted) {
    // every dtype: values keep the input dtype (tpr_topk orders by the dtype's
    // sortable key: floats with -0.0 == +0.0 and NaN largest, integers by value)
    if (self.dim() > TPR_MAX_DIMS) TP_THROW(NotImplementedError, "topk: more than 8 dims on ROCm");
    const int64_t nd = self.dim();
    const int64_t d = (nd == 0) ? 0 : wrap(dim, nd);
    const int64_t n = (nd == 0) ? 1 : self.size(d);
    if (k < 0 || k > n || (nd == 0 && k != 1)) TP_THROW(RuntimeError, "selected index k out of range");
    // move dim last
    Tensor x = self;
    if (nd > 0 && d != nd - 1) {
        std::vector<int64_t> perm;
        for (int64_t i = 0; i < nd; ++i)
            if (i != d) perm.push_back(i);
        perm.push_back(d);
        x = self.permute(perm);
    }
    std::vector<int64_t> lead(x.shape().begin(), x.shape().end() - (nd > 0 ? 1 : 0));
    int64_t rows = 1;
    for (auto s : lead) rows *= s;
    // rows must be evenly strided with a unit inner stride: [rows, n]
    bool ok = nd == 0 || (x.stride(-1) == 1 || n <= 1);
    int64_t row_stride = n;
    if (ok && !lead.empty()) {
        // the leading dims must collapse to a single row stride
        int64_t expect = -1, acc = 1;
        bool first = true;
        for (int64_t i = (int64_t)lead.size() - 1; i >= 0; --i) {
            if (lead[i] == 1) continue;
            const int64_t st = x.strides()[i];
            if (first) {
                expect = st;
                first = false;
            } else if (st != expect * acc) {
                ok = false;
            }
            acc *= lead[i];
        }
        row_stride = first ? n : expect;
    }
    if (!ok) {
        x = x.contiguous();
        row_stride = n;
    }
    std::vector<int64_t> oshape = lead;
    oshape.push_back(k);
    Tensor vals = Tensor::empty(oshape, self.dtype(), self.device());
    Tensor idx = Tensor::empty(oshape, DType::Int64, self.device());
    const int32_t tdt = (int32_t)self.dtype();  // P10 ScalarType numbering == tpr_dtype
    const size_t wsb = tpr_topk_workspace_bytes(tdt, rows, n, k);
    std::shared_ptr<void> ws;
    if (wsb) ws = allocate(wsb, self.device());
    DeviceGuard guard(self.device());
    const int rc = tpr_topk(x.data_ptr(), tdt, rows, n, row_stride, k, largest ? 1 : 0, sorted ? 1 : 0,
                            vals.data_ptr(), idx.data_ptr(), ws.get(), wsb, currentStream(self.device().index));
    if (rc != TPR_OK) throw_status(rc, "topk");
    if (nd > 0 && d != nd - 1) {
        // results are [..., k] in the permuted order: put k back at position d
        std::vector<int64_t> inv(nd);
        for (int64_t i = 0; i < nd - 1; ++i) inv[i < d ? i : i + 1] = i;
        inv[d] = nd - 1;
        vals = vals.permute(inv).contiguous();
        idx = idx.permute(inv).contiguous();
    }
    if (nd == 0) {
        vals = vals.reshape({});
        idx = idx.reshape({});
    }
    return {vals, idx};
}

// topk_topp_sample(Tensor self, Tensor uniforms, int64_t k=50, double temperature=1.0,
//                  double top_p=1.0) -> Tensor
// New schema (TensorPlay has no sampler): one token id (Int64) per row of the
// last dim of float32 logits, drawn from the top-k / top-p nucleus with the
// caller's uniforms (one per row, in [0, 1)); definition in include/tpr_rocm.h.
Tensor topk_topp_sample_kernel(const Tensor& self, const Tensor& uniforms, int64_t k, double temperature,
                               double top_p) {
    require_float32_input(self, "topk_topp_sample");
    if (self.dim() == 0) TP_THROW(RuntimeError, "topk_topp_sample: logits need at least one dim");
    if (uniforms.dtype() != DType::Float32) TP_THROW(NotImplementedError, "topk_topp_sample: uniforms must be float32");
    const int64_t n = self.size(-1);
    std::vector<int64_t> lead(self.shape().begin(), self.shape().end() - 1);
    int64_t rows = 1;
    for (auto s : lead) rows *= s;
    if (uniforms.numel() != rows) TP_THROW(RuntimeError, "topk_topp_sample: one uniform per row expected");
    const Tensor x = self.contiguous();
    const Tensor u = uniforms.contiguous();
    Tensor out = Tensor::empty(lead, DType::Int64, self.device());
    const size_t wsb = tpr_sample_workspace_bytes(TPR_FLOAT32, rows, n, k);
    std::shared_ptr<void> ws;
    if (wsb) ws = allocate(wsb, self.device());
    DeviceGuard guard(self.device());
    const int rc = tpr_sample(x.data_ptr(), TPR_FLOAT32, rows, n, n, k, (float)temperature, (float)top_p,
                              static_cast<const float*>(u.data_ptr()), static_cast<int64_t*>(out.data_ptr()), ws.get(),
                              wsb, currentStream(self.device().index));
    if (rc != TPR_OK) throw_status(rc, "topk_topp_sample");
    return out;
}

// Gradients of sum / mean / var / std (config/derivatives.yaml:82-86,
// :182-186) as single fused ops.  `dim` empty = the full reduction (the only
// form derivatives.yaml lists); a dim list gives the same formulas per output.
// grad: float32 with one element per output (either keepdim shape).
static Tensor reduce_backward(int op, const char* name, const Tensor& grad, const Tensor& self, const Tensor* result,
                              const std::vector<int64_t>& dims, int64_t correction) {
    require_float32_input(self, name);
    if (grad.dtype() != DType::Float32 || (result && result->dtype() != DType::Float32))
        TP_THROW(NotImplementedError, std::string(name) + ": float32 only on ROCm");
    const uint32_t mask = dims.empty() ? all_dims(self) : mask_of(self, dims);
    int64_t nout = 1;
    for (int64_t i = 0; i < self.dim(); ++i)
        if (!((mask >> i) & 1u)) nout *= self.size(i);
    if (grad.numel() != nout || (result && result->numel() != nout))
        TP_THROW(RuntimeError, std::string(name) + ": grad has the wrong number of elements");
    if (!(grad.device() == self.device())) TP_THROW(RuntimeError, std::string(name) + ": tensors on different devices");
    const Tensor g = grad.contiguous();
    const Tensor r = result ? result->contiguous() : Tensor();
    Tensor out = Tensor::empty(self.shape(), DType::Float32, self.device());
    tpr_reduce_desc d;
    std::memset(&d, 0, sizeof(d));
    d.op = op;
    d.in_dtype = TPR_FLOAT32;
    d.out_dtype = TPR_FLOAT32;
    d.ndim = (int32_t)self.dim();
    for (int i = 0; i < d.ndim; ++i) {
        d.sizes[i] = self.shape()[i];
        d.strides[i] = self.strides()[i];
    }
    d.reduce_mask = mask;
    d.correction = correction;
    d.count_override = dims.empty() ? 0 : listed_count(self, dims);
    const size_t wsb = tpr_reduce_backward_workspace_bytes(&d);
    std::shared_ptr<void> ws;
    if (wsb) ws = allocate(wsb, self.device());
    DeviceGuard guard(self.device());
    const int rc = tpr_reduce_backward(&d, g.data_ptr(), self.data_ptr(), result ? r.data_ptr() : nullptr,
                                       out.data_ptr(), ws.get(), wsb, currentStream(self.device().index));
    if (rc != TPR_OK) throw_status(rc, name);
    return out;
}
Tensor sum_backward_kernel(const Tensor& grad, const Tensor& self, const std::vector<int64_t>& dims, bool) {
    return reduce_backward(TPR_SUM, "sum_backward", grad, self, nullptr, dims, 0);
}
Tensor mean_backward_kernel(const Tensor& grad, const Tensor& self, const std::vector<int64_t>& dims, bool) {
    return reduce_backward(TPR_MEAN, "mean_backward", grad, self, nullptr, dims, 0);
}
Tensor var_backward_kernel(const Tensor& grad, const Tensor& self, const std::vector<int64_t>& dims, int64_t correction,
                           bool) {
    return reduce_backward(TPR_VAR, "var_backward", grad, self, nullptr, dims, correction);
}
Tensor std_backward_kernel(const Tensor& grad, const Tensor& self, const Tensor& result,
                           const std::vector<int64_t>& dims, int64_t correction, bool) {
    return reduce_backward(TPR_STD, "std_backward", grad, self, &result, dims, correction);
}

}  // namespace rocm

TENSORPLAY_LIBRARY_IMPL(ROCm, ReductionKernels) {
    using V = const std::vector<int64_t>&;
    m.impl<Tensor(const Tensor&, DType)>("sum", rocm::sum_kernel);
    m.impl<Tensor(const Tensor&, V, bool, DType)>("sum.dim_IntList", rocm::sum_dim_kernel);
    m.impl<Tensor(const Tensor&, DType)>("mean", rocm::mean_kernel);
    m.impl<Tensor(const Tensor&, V, bool, DType)>("mean.dim", rocm::mean_dim_kernel);
    m.impl<Tensor(const Tensor&)>("max", rocm::max_kernel);
    m.impl<Tensor(const Tensor&, V, bool)>("max.dim", rocm::max_dim_kernel);
    m.impl<Tensor(const Tensor&)>("min", rocm::min_kernel);
    m.impl<Tensor(const Tensor&, V, bool)>("min.dim", rocm::min_dim_kernel);
    m.impl<Tensor(const Tensor&, std::optional<int64_t>, bool)>("argmax", rocm::argmax_kernel);
    m.impl<Tensor(const Tensor&, std::optional<int64_t>, bool)>("argmin", rocm::argmin_kernel);
    m.impl<Tensor(const Tensor&, int64_t)>("var", rocm::var_kernel);
    m.impl<Tensor(const Tensor&, V, int64_t, bool)>("var.dim", rocm::var_dim_kernel);
    m.impl<Tensor(const Tensor&, int64_t)>("std", rocm::std_kernel);
    m.impl<Tensor(const Tensor&, V, int64_t, bool)>("std.dim", rocm::std_dim_kernel);
    m.impl<Tensor(const Tensor&, DType)>("prod", rocm::prod_kernel);
    m.impl<Tensor(const Tensor&, V, bool, DType)>("prod.dim_IntList", rocm::prod_dim_kernel);
    m.impl<Tensor(const Tensor&)>("all", rocm::all_kernel);
    m.impl<Tensor(const Tensor&, V, bool)>("all.dim", rocm::all_dim_kernel);
    m.impl<Tensor(const Tensor&)>("any", rocm::any_kernel);
    m.impl<Tensor(const Tensor&, V, bool)>("any.dim", rocm::any_dim_kernel);
    m.impl<Tensor(const Tensor&)>("median", rocm::median_kernel);
    m.impl<Tensor(const Tensor&, double)>("norm", rocm::norm_kernel);
    m.impl<Tensor(const Tensor&, V, double, bool)>("norm.dim", rocm::norm_dim_kernel);
    m.impl<std::tuple<Tensor, Tensor>(const Tensor&, int64_t, int64_t, bool, bool)>("topk", rocm::topk_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, int64_t, double, double)>("topk_topp_sample", rocm::topk_topp_sample_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, V, bool)>("sum_backward", rocm::sum_backward_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, V, bool)>("mean_backward", rocm::mean_backward_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, V, int64_t, bool)>("var_backward", rocm::var_backward_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, const Tensor&, V, int64_t, bool)>("std_backward", rocm::std_backward_kernel);
}

}  // namespace tensorplay
