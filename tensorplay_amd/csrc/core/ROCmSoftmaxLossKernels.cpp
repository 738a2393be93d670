// ROCm backend for the softmax / log_softmax and nll_loss schemas, the
// consumers of the reduction primitives: host adapters registered under
// DispatchKey::ROCm with the STUB_TYPE_MAP argument types
// (/root/reference/tools/codegen/gen.py:38-53).  They reproduce the reference
// kernels' dtype / shape / error rules
// (/root/reference/p10/src/backend/cpu/PointwiseKernels.cpp:519-545,
//  /root/reference/p10/src/backend/cpu/LossKernels.cpp:12-101) and launch
// through the C-ABI (include/tpr_rocm.h).  The CUDA registrations these
// replace are ActivationKernels.cu:234-235 (cuDNN softmax) and
// LossKernels.cu (nll_loss_cuda / nll_loss_backward_cuda).
#include <cstring>
#include <optional>
#include <tuple>

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
    if (rc == TPR_ERR_UNSUPPORTED_DTYPE || rc == TPR_ERR_NOT_IMPLEMENTED) TP_THROW(NotImplementedError, msg);
    TP_THROW(RuntimeError, msg);
}

// Collapse dims [b, e) of x into one (size, stride); false if they are not
// evenly strided.
bool collapse(const Tensor& x, int64_t b, int64_t e, int64_t& size, int64_t& stride) {
    size = 1;
    stride = 1;
    bool first = true;
    for (int64_t i = e - 1; i >= b; --i) {
        const int64_t s = x.shape()[i];
        if (s == 1) continue;
        if (first) {
            stride = x.strides()[i];
            first = false;
        } else if (x.strides()[i] != stride * size) {
            return false;
        }
        size *= s;
    }
    for (int64_t i = b; i < e; ++i) if (x.shape()[i] == 0) size = 0;
    return true;
}

// [outer, n, inner] view of x around dim d (x made contiguous when the outer
// or inner dims do not collapse).
Tensor view3(const Tensor& x0, int64_t d, int64_t (&ext)[3], int64_t (&str)[3]) {
    Tensor x = x0;
    const int64_t nd = x.dim();
    for (int attempt = 0; attempt < 2; ++attempt) {
        int64_t so, si;
        const bool ok_o = collapse(x, 0, d, ext[0], so);
        const bool ok_i = collapse(x, d + 1, nd, ext[2], si);
        if (ok_o && ok_i) {
            ext[1] = nd == 0 ? 1 : x.shape()[d];
            str[0] = so;
            str[1] = nd == 0 ? 1 : x.strides()[d];
            str[2] = si;
            if (ext[0] == 1) str[0] = ext[1] * ext[2];
            if (ext[2] == 1) str[2] = 1;
            return x;
        }
        x = x.contiguous();
    }
    TP_THROW(RuntimeError, "softmax: could not form a strided view");
}

int64_t wrap_dim(int64_t dim, int64_t nd) {
    const int64_t n = nd == 0 ? 1 : nd;
    const int64_t w = dim < 0 ? dim + n : dim;
    if (w < 0 || w >= n) TP_THROW(IndexError, "Dimension out of range");
    return w;
}

Tensor run_softmax(const Tensor& a, const Tensor* b, int64_t d, int mode, const char* name) {
    int64_t ext[3], sa[3], sb[3] = {0, 0, 0};
    const Tensor av = view3(a, d, ext, sa);
    Tensor bv;
    if (b) {
        int64_t e2[3];
        bv = view3(*b, d, e2, sb);
    }
    Tensor out = Tensor::empty(a.shape(), a.dtype(), a.device());
    tpr_softmax_desc desc;
    std::memset(&desc, 0, sizeof(desc));
    desc.mode = mode;
    desc.dtype = a.dtype() == DType::Float64 ? TPR_FLOAT64 : TPR_FLOAT32;
    desc.outer = ext[0];
    desc.n = ext[1];
    desc.inner = ext[2];
    for (int i = 0; i < 3; ++i) {
        desc.a_strides[i] = sa[i];
        desc.b_strides[i] = sb[i];
    }
    const size_t wsb = tpr_softmax_workspace_bytes(&desc);
    std::shared_ptr<void> ws;
    if (wsb) ws = allocate(wsb, a.device());
    DeviceGuard guard(a.device());
    const int rc = tpr_softmax(&desc, av.data_ptr(), b ? bv.data_ptr() : nullptr, out.data_ptr(), ws.get(), wsb,
                               currentStream(a.device().index));
    if (rc != TPR_OK) throw_status(rc, name);
    return out;
}

// softmax_kernel / log_softmax_kernel (PointwiseKernels.cpp:519-545): the
// compute dtype is `dtype` if given, else the input's; integral types compute
// in Float32; the input is cast first.
Tensor softmax_common(const Tensor& self, int64_t dim, DType dtype, bool log) {
    const char* name = log ? "log_softmax" : "softmax";
    DType out = dtype == DType::Undefined ? self.dtype() : dtype;
    if (isIntegralType(out, false)) out = DType::Float32;
    if (out != DType::Float32 && out != DType::Float64)
        TP_THROW(NotImplementedError, std::string(name) + " not implemented for dtype " + toString(out) +
                                          " on ROCm (float32 / float64)");
    if (self.dim() > TPR_MAX_DIMS) TP_THROW(NotImplementedError, std::string(name) + ": more than 8 dims on ROCm");
    const int64_t d = wrap_dim(dim, self.dim());
    const Tensor x = self.dtype() == out ? self : self.to(out);
    return run_softmax(x, nullptr, d, log ? TPR_LOG_SOFTMAX_FWD : TPR_SOFTMAX_FWD, name);
}

}  // namespace

Tensor softmax_kernel(const Tensor& self, int64_t dim, DType dtype) { return softmax_common(self, dim, dtype, false); }
Tensor log_softmax_kernel(const Tensor& self, int64_t dim, DType dtype) {
    return softmax_common(self, dim, dtype, true);
}

// _softmax_backward_data / _log_softmax_backward_data: the gradient formulas
// of config/derivatives.yaml:91-95 as one fused kernel (TensorPlay composes
// them from sum / mul / sub / exp in its autograd; PyTorch names these ops
// this way).  grad_output and output: float32 or float64 (the same), same shape.
static Tensor softmax_bwd_common(const Tensor& grad, const Tensor& output, int64_t dim, bool log) {
    const char* name = log ? "_log_softmax_backward_data" : "_softmax_backward_data";
    if ((grad.dtype() != DType::Float32 && grad.dtype() != DType::Float64) || output.dtype() != grad.dtype())
        TP_THROW(NotImplementedError, std::string(name) + ": float32 or float64 (both alike) on ROCm");
    if (grad.shape() != output.shape()) TP_THROW(RuntimeError, std::string(name) + ": grad/output shape mismatch");
    if (!(grad.device() == output.device())) TP_THROW(RuntimeError, std::string(name) + ": tensors on different devices");
    if (grad.dim() > TPR_MAX_DIMS) TP_THROW(NotImplementedError, std::string(name) + ": more than 8 dims on ROCm");
    const int64_t d = wrap_dim(dim, grad.dim());
    return run_softmax(grad, &output, d, log ? TPR_LOG_SOFTMAX_BWD : TPR_SOFTMAX_BWD, name);
}
Tensor softmax_backward_data_kernel(const Tensor& grad, const Tensor& output, int64_t dim, DType) {
    return softmax_bwd_common(grad, output, dim, false);
}
Tensor log_softmax_backward_data_kernel(const Tensor& grad, const Tensor& output, int64_t dim, DType) {
    return softmax_bwd_common(grad, output, dim, true);
}

// nll_loss_kernel (LossKernels.cpp:12-55): input float32 [N, C], target Int64
// [N]; returns (output, total_weight) with output [N] (reduction 0) or a 0-dim
// tensor, and total_weight a one-element tensor of shape [1].  A target outside
// [0, C) that is not ignore_index raises RuntimeError("Target out of bounds"),
// as the CPU path (this reads a device flag back, so it synchronises).
std::tuple<Tensor, Tensor> nll_loss_kernel(const Tensor& input, const Tensor& target, std::optional<Tensor> weight,
                                           int64_t reduction, int64_t ignore_index) {
    if (input.dtype() != DType::Float32) TP_THROW(NotImplementedError, "nll_loss only supports Float32");
    if (target.dtype() != DType::Int64) TP_THROW(NotImplementedError, "nll_loss target must be Int64");
    if (reduction < 0 || reduction > 2) TP_THROW(ValueError, "Invalid reduction mode");
    if (input.dim() != 2) TP_THROW(RuntimeError, "nll_loss: input must be 2-D [N, C] on ROCm");
    const int64_t n = input.size(0), c = input.size(1);
    if (target.dim() != 1 || target.size(0) != n) TP_THROW(RuntimeError, "nll_loss: target must be [N]");
    Tensor w;
    if (weight.has_value() && weight->defined()) {
        if (weight->dtype() != DType::Float32 || weight->numel() != c)
            TP_THROW(RuntimeError, "nll_loss: weight must be float32 with C elements");
        w = weight->contiguous();
    }
    Tensor out = reduction == 0 ? Tensor::empty({n}, DType::Float32, input.device())
                                : Tensor::empty({}, DType::Float32, input.device());
    Tensor tw = Tensor::empty({1}, DType::Float32, input.device());
    Tensor status = Tensor::empty({1}, DType::Int32, input.device());
    const size_t wsb = tpr_nll_loss_workspace_bytes(n);
    std::shared_ptr<void> ws = allocate(wsb, input.device());
    DeviceGuard guard(input.device());
    const int rc = tpr_nll_loss(input.data_ptr(), TPR_FLOAT32, n, c, input.stride(0), input.stride(1),
                                static_cast<const int64_t*>(target.data_ptr()), target.stride(0),
                                w.defined() ? w.data_ptr() : nullptr, reduction, ignore_index, out.data_ptr(),
                                tw.data_ptr(), static_cast<int32_t*>(status.data_ptr()), ws.get(), wsb,
                                currentStream(input.device().index));
    if (rc != TPR_OK) throw_status(rc, "nll_loss");
    if (status.item_int() != 0) TP_THROW(RuntimeError, "Target out of bounds");
    return {out, tw};
}

// nll_loss_backward_kernel (LossKernels.cpp:57-101): dense float32 [N, C]
// gradient.  Reduction 1 divides by total_weight when it is defined, else by
// the total weight recomputed from target / weight (as the reference).
Tensor nll_loss_backward_kernel(const Tensor& grad_output, const Tensor& input, const Tensor& target,
                                std::optional<Tensor> weight, int64_t reduction, int64_t ignore_index,
                                const Tensor& total_weight) {
    if (input.dtype() != DType::Float32 || grad_output.dtype() != DType::Float32)
        TP_THROW(NotImplementedError, "nll_loss_backward only supports Float32");
    if (target.dtype() != DType::Int64) TP_THROW(NotImplementedError, "nll_loss target must be Int64");
    if (reduction < 0 || reduction > 2) TP_THROW(ValueError, "Invalid reduction mode");
    if (input.dim() != 2) TP_THROW(RuntimeError, "nll_loss_backward: input must be 2-D [N, C] on ROCm");
    const int64_t n = input.size(0), c = input.size(1);
    if (target.dim() != 1 || target.size(0) != n) TP_THROW(RuntimeError, "nll_loss_backward: target must be [N]");
    if (reduction == 0 ? grad_output.numel() != n : grad_output.numel() != 1)
        TP_THROW(RuntimeError, "nll_loss_backward: grad_output has the wrong number of elements");
    Tensor w;
    if (weight.has_value() && weight->defined()) {
        if (weight->dtype() != DType::Float32 || weight->numel() != c)
            TP_THROW(RuntimeError, "nll_loss_backward: weight must be float32 with C elements");
        w = weight->contiguous();
    }
    Tensor tw;
    if (total_weight.defined()) {
        if (total_weight.dtype() != DType::Float32 || total_weight.numel() != 1)
            TP_THROW(RuntimeError, "nll_loss_backward: total_weight must be one float32");
        tw = total_weight.contiguous();
    } else if (reduction == 1) {
        tw = std::get<1>(nll_loss_kernel(input, target, w.defined() ? std::optional<Tensor>(w) : std::nullopt, 2,
                                         ignore_index));
    }
    const Tensor g = grad_output.reshape({grad_output.numel()});
    Tensor gi = Tensor::empty({n, c}, DType::Float32, input.device());
    DeviceGuard guard(input.device());
    const int rc = tpr_nll_loss_backward(g.data_ptr(), g.numel() ? g.stride(0) : 1,
                                         static_cast<const int64_t*>(target.data_ptr()), target.stride(0),
                                         w.defined() ? w.data_ptr() : nullptr, tw.defined() ? tw.data_ptr() : nullptr,
                                         n, c, reduction, ignore_index, gi.data_ptr(),
                                         currentStream(input.device().index));
    if (rc != TPR_OK) throw_status(rc, "nll_loss_backward");
    return gi;
}

}  // namespace rocm

TENSORPLAY_LIBRARY_IMPL(ROCm, SoftmaxLossKernels) {
    // clang-format off
    m.impl<Tensor(const Tensor&, int64_t, DType)>("softmax", rocm::softmax_kernel);
    m.impl<Tensor(const Tensor&, int64_t, DType)>("log_softmax", rocm::log_softmax_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, int64_t, DType)>("_softmax_backward_data", rocm::softmax_backward_data_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, int64_t, DType)>("_log_softmax_backward_data", rocm::log_softmax_backward_data_kernel);
    m.impl<std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&, std::optional<Tensor>, int64_t, int64_t)>("nll_loss", rocm::nll_loss_kernel);
    m.impl<Tensor(const Tensor&, const Tensor&, const Tensor&, std::optional<Tensor>, int64_t, int64_t, const Tensor&)>("nll_loss_backward", rocm::nll_loss_backward_kernel);
    // clang-format on
}

}  // namespace tensorplay
