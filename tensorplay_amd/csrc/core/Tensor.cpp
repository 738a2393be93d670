#include "Tensor.h"

#include <hip/hip_runtime_api.h>

#include <cstring>
#include <numeric>

#include "Allocator.h"
#include "Dispatcher.h"
#include "Exception.h"
#include "tpr_rocm.h"

namespace tensorplay {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) TP_THROW(RuntimeError, std::string(what) + ": " + hipGetErrorString(e));
}

int64_t wrap_dim(int64_t d, int64_t ndim, bool index_error) {
    int64_t w = d < 0 ? d + ndim : d;
    if (w < 0 || w >= ndim) {
        if (index_error) TP_THROW(IndexError, "Dimension out of range");
        TP_THROW(RuntimeError, "Dimension out of range");
    }
    return w;
}

}  // namespace

std::vector<int64_t> Tensor::contiguousStrides(const std::vector<int64_t>& shape) {
    std::vector<int64_t> st(shape.size());
    int64_t acc = 1;
    for (int i = (int)shape.size() - 1; i >= 0; --i) {
        st[i] = acc;
        acc *= std::max<int64_t>(shape[i], 1);
    }
    return st;
}

Tensor Tensor::empty(const std::vector<int64_t>& shape, DType dtype, const Device& device) {
    if (elementSize(dtype) == 0) TP_THROW(TypeError, "empty: unsupported dtype");
    for (auto s : shape)
        if (s < 0) TP_THROW(RuntimeError, "negative dimension in shape");
    int64_t n = 1;
    for (auto s : shape) n *= s;
    auto st = std::make_shared<StorageImpl>();
    st->nbytes = (size_t)n * elementSize(dtype);
    st->device = device;
    if (device.is_rocm() && device.index >= rocmDeviceCount())
        TP_THROW(RuntimeError, "ROCm device " + std::to_string(device.index) + " is not available");
    st->data = allocate(st->nbytes, device);
    auto impl = std::make_shared<TensorImpl>();
    impl->storage = st;
    impl->sizes = shape;
    impl->strides = contiguousStrides(shape);
    impl->dtype = dtype;
    return Tensor(impl);
}

Tensor Tensor::fromHost(const void* src, const std::vector<int64_t>& shape, DType dtype, const Device& device) {
    Tensor t = empty(shape, dtype, device);
    const size_t nb = (size_t)t.numel() * elementSize(dtype);
    if (nb == 0) return t;
    if (device.is_cpu()) {
        std::memcpy(t.data_ptr(), src, nb);
    } else {
        DeviceGuard g(device);
        hip_check(hipMemcpy(t.data_ptr(), src, nb, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    return t;
}

Tensor Tensor::fromExternal(void* ptr, const std::vector<int64_t>& shape, const std::vector<int64_t>& strides,
                            DType dtype, const Device& device, std::shared_ptr<void> owner) {
    if (shape.size() != strides.size()) TP_THROW(ValueError, "shape/strides rank mismatch");
    auto st = std::make_shared<StorageImpl>();
    st->device = device;
    st->data = std::shared_ptr<void>(owner, ptr);  // aliasing: keeps `owner` alive
    st->nbytes = 0;
    auto impl = std::make_shared<TensorImpl>();
    impl->storage = st;
    impl->sizes = shape;
    impl->strides = strides;
    impl->dtype = dtype;
    return Tensor(impl);
}

int64_t Tensor::size(int64_t d) const { return impl_->sizes[wrap_dim(d, dim(), true)]; }
int64_t Tensor::stride(int64_t d) const { return impl_->strides[wrap_dim(d, dim(), true)]; }

int64_t Tensor::numel() const {
    int64_t n = 1;
    for (auto s : impl_->sizes) n *= s;
    return n;
}

bool Tensor::is_contiguous() const {
    int64_t expect = 1;
    for (int i = (int)impl_->sizes.size() - 1; i >= 0; --i) {
        if (impl_->sizes[i] == 1) continue;
        if (impl_->strides[i] != expect) return false;
        expect *= impl_->sizes[i];
    }
    return true;
}

void* Tensor::data_ptr() const {
    return static_cast<char*>(impl_->storage->data.get()) + impl_->offset * (int64_t)element_size();
}

Tensor Tensor::as_strided(const std::vector<int64_t>& sizes, const std::vector<int64_t>& strides, int64_t offset) const {
    auto impl = std::make_shared<TensorImpl>(*impl_);
    impl->sizes = sizes;
    impl->strides = strides;
    impl->offset = offset;
    return Tensor(impl);
}

// ViewKernels.cpp:12-24 semantics (IndexError on a bad dim).
Tensor Tensor::transpose(int64_t d0, int64_t d1) const {
    const int64_t a = wrap_dim(d0, dim(), true), b = wrap_dim(d1, dim(), true);
    auto sz = impl_->sizes;
    auto st = impl_->strides;
    std::swap(sz[a], sz[b]);
    std::swap(st[a], st[b]);
    return as_strided(sz, st, impl_->offset);
}

Tensor Tensor::permute(const std::vector<int64_t>& dims) const {
    const int64_t nd = dim();
    if ((int64_t)dims.size() != nd) TP_THROW(RuntimeError, "permute: number of dimensions mismatch");
    std::vector<int64_t> sz(nd), st(nd);
    std::vector<bool> seen(nd, false);
    for (int64_t i = 0; i < nd; ++i) {
        const int64_t d = wrap_dim(dims[i], nd, true);
        if (seen[d]) TP_THROW(RuntimeError, "permute: duplicate dimension");
        seen[d] = true;
        sz[i] = impl_->sizes[d];
        st[i] = impl_->strides[d];
    }
    return as_strided(sz, st, impl_->offset);
}

Tensor Tensor::reshape(const std::vector<int64_t>& shape) const {
    int64_t n = 1, infer = -1;
    std::vector<int64_t> s = shape;
    for (size_t i = 0; i < s.size(); ++i) {
        if (s[i] == -1) {
            if (infer >= 0) TP_THROW(RuntimeError, "reshape: only one dimension can be inferred");
            infer = (int64_t)i;
        } else {
            n *= s[i];
        }
    }
    if (infer >= 0) s[infer] = n ? numel() / n : 0;
    int64_t m = 1;
    for (auto v : s) m *= v;
    if (m != numel()) TP_THROW(RuntimeError, "reshape: shape is invalid for input size");
    Tensor c = contiguous();
    return c.as_strided(s, contiguousStrides(s), c.impl_->offset);
}

// Tensor.cpp:473-513 of the reference: clone = empty + copy_, contiguous =
// clone when not contiguous, to(dtype) = empty of the new dtype + copy_.
Tensor Tensor::contiguous() const {
    if (is_contiguous()) return *this;
    return clone();
}

Tensor Tensor::clone() const {
    Tensor out = empty(impl_->sizes, impl_->dtype, device());
    out.copy_(*this);
    return out;
}

Tensor Tensor::to(DType dtype) const {
    if (dtype == impl_->dtype) return *this;
    Tensor out = empty(impl_->sizes, dtype, device());
    out.copy_(*this);
    return out;
}

Tensor& Tensor::copy_(const Tensor& src) {
    return DispatchStub<Tensor&, Tensor&, const Tensor&>::call("copy_", computeDispatchKey(device()), *this, src);
}

Tensor Tensor::to(const Device& target) const {
    if (target == device()) return *this;
    Tensor src = contiguous();
    Tensor out = empty(impl_->sizes, impl_->dtype, target);
    const size_t nb = (size_t)numel() * element_size();
    if (nb == 0) return out;
    if (device().is_cpu()) {  // H2D
        DeviceGuard g(target);
        hip_check(hipMemcpy(out.data_ptr(), src.data_ptr(), nb, hipMemcpyHostToDevice), "hipMemcpy H2D");
    } else if (target.is_cpu()) {  // D2H (waits for the producing stream)
        DeviceGuard g(device());
        hip_check(hipStreamSynchronize((hipStream_t)currentStream(device().index)), "hipStreamSynchronize");
        hip_check(hipMemcpy(out.data_ptr(), src.data_ptr(), nb, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    } else {  // device to device
        DeviceGuard g(device());
        hip_check(hipStreamSynchronize((hipStream_t)currentStream(device().index)), "hipStreamSynchronize");
        hip_check(hipMemcpyPeer(out.data_ptr(), target.index, src.data_ptr(), device().index, nb), "hipMemcpyPeer");
    }
    return out;
}

void Tensor::copyToHost(void* dst) const {
    Tensor h = cpu().contiguous();
    const size_t nb = (size_t)numel() * element_size();
    if (nb) std::memcpy(dst, h.data_ptr(), nb);
}

double Tensor::item() const {
    if (numel() != 1) TP_THROW(RuntimeError, "item(): a Tensor with " + std::to_string(numel()) +
                                                 " elements cannot be converted to Scalar");
    Tensor h = cpu();
    const void* p = h.data_ptr();
    switch (dtype()) {
        case DType::Float32: return *static_cast<const float*>(p);
        case DType::Float64: return *static_cast<const double*>(p);
        case DType::Int64: return (double)*static_cast<const int64_t*>(p);
        case DType::Int32: return *static_cast<const int32_t*>(p);
        case DType::Int16: return *static_cast<const int16_t*>(p);
        case DType::Int8: return *static_cast<const int8_t*>(p);
        case DType::UInt8: return *static_cast<const uint8_t*>(p);
        case DType::Bool: return *static_cast<const bool*>(p) ? 1.0 : 0.0;
        default: TP_THROW(TypeError, "item(): unsupported dtype");
    }
}

int64_t Tensor::item_int() const {
    if (dtype() == DType::Int64) {
        if (numel() != 1) TP_THROW(RuntimeError, "item(): tensor must have exactly one element");
        int64_t v = 0;
        cpu().copyToHost(&v);
        return v;
    }
    return (int64_t)item();
}

std::vector<int64_t> reductionShape(const std::vector<int64_t>& shape, const std::vector<int64_t>& dims, bool keepdim) {
    std::vector<bool> red(shape.size(), false);
    for (int64_t d : dims) red[wrap_dim(d, (int64_t)shape.size(), false)] = true;
    std::vector<int64_t> out;
    for (size_t i = 0; i < shape.size(); ++i) {
        if (red[i]) {
            if (keepdim) out.push_back(1);
        } else {
            out.push_back(shape[i]);
        }
    }
    return out;
}

// ---- dispatching methods (STUB_TYPE_MAP argument types) ----
#define TP_KEY computeDispatchKey(device())

Tensor Tensor::sum(DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, DType>::call("sum", TP_KEY, *this, dtype);
}
Tensor Tensor::sum(const std::vector<int64_t>& dim, bool keepdim, DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, bool, DType>::call(
        "sum.dim_IntList", TP_KEY, *this, dim, keepdim, dtype);
}
Tensor Tensor::mean(DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, DType>::call("mean", TP_KEY, *this, dtype);
}
Tensor Tensor::mean(const std::vector<int64_t>& dim, bool keepdim, DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, bool, DType>::call(
        "mean.dim", TP_KEY, *this, dim, keepdim, dtype);
}
Tensor Tensor::max() const { return DispatchStub<Tensor, const Tensor&>::call("max", TP_KEY, *this); }
Tensor Tensor::max(const std::vector<int64_t>& dim, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, bool>::call("max.dim", TP_KEY, *this,
                                                                                       dim, keepdim);
}
Tensor Tensor::min() const { return DispatchStub<Tensor, const Tensor&>::call("min", TP_KEY, *this); }
Tensor Tensor::min(const std::vector<int64_t>& dim, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, bool>::call("min.dim", TP_KEY, *this,
                                                                                       dim, keepdim);
}
Tensor Tensor::argmax(std::optional<int64_t> dim, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, std::optional<int64_t>, bool>::call("argmax", TP_KEY, *this, dim,
                                                                                  keepdim);
}
Tensor Tensor::argmin(std::optional<int64_t> dim, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, std::optional<int64_t>, bool>::call("argmin", TP_KEY, *this, dim,
                                                                                  keepdim);
}
Tensor Tensor::var(int64_t correction) const {
    return DispatchStub<Tensor, const Tensor&, int64_t>::call("var", TP_KEY, *this, correction);
}
Tensor Tensor::var(const std::vector<int64_t>& dim, int64_t correction, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, int64_t, bool>::call(
        "var.dim", TP_KEY, *this, dim, correction, keepdim);
}
Tensor Tensor::std(int64_t correction) const {
    return DispatchStub<Tensor, const Tensor&, int64_t>::call("std", TP_KEY, *this, correction);
}
Tensor Tensor::std(const std::vector<int64_t>& dim, int64_t correction, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, int64_t, bool>::call(
        "std.dim", TP_KEY, *this, dim, correction, keepdim);
}
Tensor Tensor::prod(DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, DType>::call("prod", TP_KEY, *this, dtype);
}
Tensor Tensor::prod(const std::vector<int64_t>& dim, bool keepdim, DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, bool, DType>::call(
        "prod.dim_IntList", TP_KEY, *this, dim, keepdim, dtype);
}
Tensor Tensor::all() const { return DispatchStub<Tensor, const Tensor&>::call("all", TP_KEY, *this); }
Tensor Tensor::all(const std::vector<int64_t>& dim, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, bool>::call("all.dim", TP_KEY, *this, dim,
                                                                                       keepdim);
}
Tensor Tensor::any() const { return DispatchStub<Tensor, const Tensor&>::call("any", TP_KEY, *this); }
Tensor Tensor::any(const std::vector<int64_t>& dim, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, bool>::call("any.dim", TP_KEY, *this, dim,
                                                                                       keepdim);
}
Tensor Tensor::median() const { return DispatchStub<Tensor, const Tensor&>::call("median", TP_KEY, *this); }
Tensor Tensor::norm(double p) const {
    return DispatchStub<Tensor, const Tensor&, double>::call("norm", TP_KEY, *this, p);
}
Tensor Tensor::norm(const std::vector<int64_t>& dim, double p, bool keepdim) const {
    return DispatchStub<Tensor, const Tensor&, const std::vector<int64_t>&, double, bool>::call(
        "norm.dim", TP_KEY, *this, dim, p, keepdim);
}
std::tuple<Tensor, Tensor> Tensor::topk(int64_t k, int64_t dim, bool largest, bool sorted) const {
    return DispatchStub<std::tuple<Tensor, Tensor>, const Tensor&, int64_t, int64_t, bool, bool>::call(
        "topk", TP_KEY, *this, k, dim, largest, sorted);
}
Tensor Tensor::softmax(int64_t dim, DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, int64_t, DType>::call("softmax", TP_KEY, *this, dim, dtype);
}
Tensor Tensor::log_softmax(int64_t dim, DType dtype) const {
    return DispatchStub<Tensor, const Tensor&, int64_t, DType>::call("log_softmax", TP_KEY, *this, dim, dtype);
}
#undef TP_KEY

std::tuple<Tensor, Tensor> nll_loss(const Tensor& self, const Tensor& target, const std::optional<Tensor>& weight,
                                    int64_t reduction, int64_t ignore_index) {
    return DispatchStub<std::tuple<Tensor, Tensor>, const Tensor&, const Tensor&, std::optional<Tensor>, int64_t,
                        int64_t>::call("nll_loss", computeDispatchKey(self.device()), self, target, weight, reduction,
                                       ignore_index);
}
Tensor nll_loss_backward(const Tensor& grad_output, const Tensor& self, const Tensor& target,
                         const std::optional<Tensor>& weight, int64_t reduction, int64_t ignore_index,
                         const Tensor& total_weight) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, const Tensor&, std::optional<Tensor>, int64_t, int64_t,
                        const Tensor&>::call("nll_loss_backward", computeDispatchKey(grad_output.device()),
                                             grad_output, self, target, weight, reduction, ignore_index,
                                             total_weight);
}
Tensor _softmax_backward_data(const Tensor& grad_output, const Tensor& output, int64_t dim, DType input_dtype) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, int64_t, DType>::call(
        "_softmax_backward_data", computeDispatchKey(grad_output.device()), grad_output, output, dim, input_dtype);
}
Tensor _log_softmax_backward_data(const Tensor& grad_output, const Tensor& output, int64_t dim, DType input_dtype) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, int64_t, DType>::call(
        "_log_softmax_backward_data", computeDispatchKey(grad_output.device()), grad_output, output, dim,
        input_dtype);
}

Tensor topk_topp_sample(const Tensor& self, const Tensor& uniforms, int64_t k, double temperature, double top_p) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, int64_t, double, double>::call(
        "topk_topp_sample", computeDispatchKey(self.device()), self, uniforms, k, temperature, top_p);
}
using IntList = const std::vector<int64_t>&;
Tensor sum_backward(const Tensor& grad, const Tensor& self, IntList dim, bool keepdim) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, IntList, bool>::call(
        "sum_backward", computeDispatchKey(self.device()), grad, self, dim, keepdim);
}
Tensor mean_backward(const Tensor& grad, const Tensor& self, IntList dim, bool keepdim) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, IntList, bool>::call(
        "mean_backward", computeDispatchKey(self.device()), grad, self, dim, keepdim);
}
Tensor var_backward(const Tensor& grad, const Tensor& self, IntList dim, int64_t correction, bool keepdim) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, IntList, int64_t, bool>::call(
        "var_backward", computeDispatchKey(self.device()), grad, self, dim, correction, keepdim);
}
Tensor std_backward(const Tensor& grad, const Tensor& self, const Tensor& result, IntList dim, int64_t correction,
                    bool keepdim) {
    return DispatchStub<Tensor, const Tensor&, const Tensor&, const Tensor&, IntList, int64_t, bool>::call(
        "std_backward", computeDispatchKey(self.device()), grad, self, result, dim, correction, keepdim);
}

void Tensor::record_stream(void* stream) const {
    if (device().is_rocm()) recordStream(impl_->storage->data.get(), device().index, stream);
}

}  // namespace tensorplay
