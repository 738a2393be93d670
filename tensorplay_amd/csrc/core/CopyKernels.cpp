// copy_ registrations of the host core.
//
// ROCm key: the counterpart of the CUDA copy_kernel
// (/root/reference/p10/src/backend/cuda/CopyKernels.cu:55-157).  Same contract:
// numel must match; a host source is staged to the device first; every
// layout / dtype combination goes through one tpr_copy launch (the reference
// takes cudaMemcpy for dense same-dtype pairs and one thread per element
// otherwise; tpr_copy picks a dense-run, rows, LDS-tile or per-element kernel).
//
// CPU key: plumbing for this package's host tensors only (TensorPlay's CPU
// backend keeps its own copy_kernel, cpu/CopyKernels.cpp:73-127).  A device
// source is cast and densified on the device, then copied down once; host to
// host copies move bytes of equal dtypes and do not cast.
#include <hip/hip_runtime_api.h>

#include <cstring>

#include "Allocator.h"
#include "Dispatcher.h"
#include "Exception.h"
#include "Tensor.h"
#include "tpr_rocm.h"

namespace tensorplay {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) TP_THROW(RuntimeError, std::string(what) + ": " + hipGetErrorString(e));
}

void check_numel(const Tensor& self, const Tensor& src) {
    if (self.numel() != src.numel()) TP_THROW(RuntimeError, "Sizes do not match for copy");
}

// Strided host-to-host move of equal-size elements (row-major over sizes).
void host_strided_copy(char* dst, const std::vector<int64_t>& dst_strides, const char* src,
                       const std::vector<int64_t>& src_strides, const std::vector<int64_t>& sizes, size_t esz) {
    int64_t n = 1;
    for (auto s : sizes) n *= s;
    if (n == 0) return;
    const int nd = (int)sizes.size();
    std::vector<int64_t> idx(nd, 0);
    int64_t doff = 0, soff = 0;
    for (int64_t i = 0; i < n; ++i) {
        std::memcpy(dst + doff * (int64_t)esz, src + soff * (int64_t)esz, esz);
        for (int d = nd - 1; d >= 0; --d) {
            idx[d]++;
            doff += dst_strides[d];
            soff += src_strides[d];
            if (idx[d] < sizes[d]) break;
            doff -= dst_strides[d] * sizes[d];
            soff -= src_strides[d] * sizes[d];
            idx[d] = 0;
        }
    }
}

}  // namespace

namespace rocm {

Tensor& copy_kernel(Tensor& self, const Tensor& src) {
    check_numel(self, src);
    if (!self.device().is_rocm()) TP_THROW(RuntimeError, "copy_kernel dispatched to ROCm but dst is not a ROCm tensor");
    if (self.numel() == 0) return self;
    if (self.dim() > TPR_MAX_DIMS || src.dim() > TPR_MAX_DIMS)
        TP_THROW(RuntimeError, "Tensor dimension exceeds MAX_DIMS (8) for ROCm copy");
    Tensor s = src;
    if (s.device().is_cpu()) {
        // stage a dense host copy on the destination device (CopyKernels.cu:85-101)
        Tensor hc = s.contiguous();
        Tensor d = Tensor::empty(s.shape(), s.dtype(), self.device());
        DeviceGuard g(self.device());
        hip_check(hipMemcpy(d.data_ptr(), hc.data_ptr(), (size_t)hc.numel() * hc.element_size(),
                            hipMemcpyHostToDevice),
                  "hipMemcpy H2D");
        s = d;
    } else if (s.device() != self.device()) {
        s = s.to(self.device());
    }
    // equal numel, different shapes: the source is read in its row-major order
    // (what the reference's dense memcpy does); densify it first if needed
    const bool same_shape = s.shape() == self.shape();
    if (!same_shape && !s.is_contiguous()) s = s.contiguous();
    tpr_copy_desc d;
    std::memset(&d, 0, sizeof(d));
    d.ndim = (int32_t)self.dim();
    d.dst_dtype = (int32_t)self.dtype();
    d.src_dtype = (int32_t)s.dtype();
    const std::vector<int64_t> dense = Tensor::contiguousStrides(self.shape());
    for (int i = 0; i < d.ndim; ++i) {
        d.sizes[i] = self.shape()[i];
        d.dst_strides[i] = self.strides()[i];
        d.src_strides[i] = same_shape ? s.strides()[i] : dense[i];
    }
    DeviceGuard g(self.device());
    const int rc = tpr_copy(&d, self.data_ptr(), s.data_ptr(), currentStream(self.device().index));
    if (rc == TPR_ERR_UNSUPPORTED_DTYPE) TP_THROW(NotImplementedError, tpr_last_error());
    if (rc != TPR_OK) TP_THROW(RuntimeError, tpr_last_error());
    return self;
}

}  // namespace rocm

namespace host {

Tensor& copy_kernel(Tensor& self, const Tensor& src) {
    check_numel(self, src);
    if (self.numel() == 0) return self;
    Tensor s = src;
    if (s.device().is_rocm()) {
        // cast + densify on the device in the destination's dtype and shape, then one D2H copy
        Tensor d = Tensor::empty(self.shape(), self.dtype(), s.device());
        rocm::copy_kernel(d, s);
        Tensor h = Tensor::empty(self.shape(), self.dtype(), self.device());
        DeviceGuard g(s.device());
        hip_check(hipStreamSynchronize((hipStream_t)currentStream(s.device().index)), "hipStreamSynchronize");
        hip_check(hipMemcpy(h.data_ptr(), d.data_ptr(), (size_t)d.numel() * d.element_size(), hipMemcpyDeviceToHost),
                  "hipMemcpy D2H");
        s = h;
    }
    if (s.dtype() != self.dtype())
        TP_THROW(NotImplementedError, "copy_: dtype casts between host tensors are TensorPlay's CPU backend");
    const bool same_shape = s.shape() == self.shape();
    if (!same_shape && !s.is_contiguous()) s = s.contiguous();
    host_strided_copy(static_cast<char*>(self.data_ptr()), self.strides(), static_cast<const char*>(s.data_ptr()),
                      same_shape ? s.strides() : Tensor::contiguousStrides(self.shape()), self.shape(),
                      self.element_size());
    return self;
}

}  // namespace host

TENSORPLAY_LIBRARY_IMPL(ROCm, ROCmCopyKernels) {
    m.impl<Tensor&(Tensor&, const Tensor&)>("copy_", rocm::copy_kernel);
}

TENSORPLAY_LIBRARY_IMPL(CPU, HostCopyKernels) {
    m.impl<Tensor&(Tensor&, const Tensor&)>("copy_", host::copy_kernel);
}

}  // namespace tensorplay
