// Tensor of the host core: shared storage + sizes/strides/offset (in
// elements) + dtype + device, with the reduction methods of TensorPlay's
// generated Tensor API (/root/reference/tools/codegen/gen.py:408-543): every
// method computes the DispatchKey from the device and calls the kernel
// registered under the full schema name, with the STUB_TYPE_MAP argument types.
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <tuple>
#include <vector>

#include "DType.h"
#include "Device.h"

namespace tensorplay {

struct StorageImpl {
    std::shared_ptr<void> data;
    size_t nbytes = 0;
    Device device;
};

struct TensorImpl {
    std::shared_ptr<StorageImpl> storage;
    std::vector<int64_t> sizes;
    std::vector<int64_t> strides;  // elements
    int64_t offset = 0;            // elements
    DType dtype = DType::Float32;
};

class Tensor {
public:
    Tensor() = default;
    explicit Tensor(std::shared_ptr<TensorImpl> impl) : impl_(std::move(impl)) {}

    // ---- factories ----
    static Tensor empty(const std::vector<int64_t>& shape, DType dtype, const Device& device);
    // Copies a dense row-major host buffer into a new tensor on `device`.
    static Tensor fromHost(const void* src, const std::vector<int64_t>& shape, DType dtype, const Device& device);
    // Wraps memory owned elsewhere (kept alive by `owner`); no copy.
    static Tensor fromExternal(void* ptr, const std::vector<int64_t>& shape, const std::vector<int64_t>& strides,
                               DType dtype, const Device& device, std::shared_ptr<void> owner);
    static std::vector<int64_t> contiguousStrides(const std::vector<int64_t>& shape);

    // ---- metadata ----
    bool defined() const { return (bool)impl_; }
    const std::vector<int64_t>& shape() const { return impl_->sizes; }
    const std::vector<int64_t>& strides() const { return impl_->strides; }
    int64_t size(int64_t d) const;
    int64_t stride(int64_t d) const;
    int64_t dim() const { return (int64_t)impl_->sizes.size(); }
    int64_t numel() const;
    int64_t storage_offset() const { return impl_->offset; }
    DType dtype() const { return impl_->dtype; }
    Device device() const { return impl_->storage->device; }
    // Marks this tensor's device memory as used on `stream` (a hipStream_t)
    // besides the stream it was allocated on: freeing it then waits for the
    // work queued on `stream` before the memory is reused.
    void record_stream(void* stream) const;
    size_t element_size() const { return elementSize(impl_->dtype); }
    bool is_contiguous() const;
    void* data_ptr() const;  // address of element [0, ..., 0]

    // ---- views and copies ----
    Tensor as_strided(const std::vector<int64_t>& sizes, const std::vector<int64_t>& strides, int64_t offset) const;
    Tensor transpose(int64_t d0, int64_t d1) const;
    Tensor permute(const std::vector<int64_t>& dims) const;
    Tensor reshape(const std::vector<int64_t>& shape) const;  // view when contiguous, else copy first
    Tensor contiguous() const;
    Tensor clone() const;
    Tensor to(const Device& device) const;
    Tensor to(DType dtype) const;                  // cast (copy_ into a new tensor)
    Tensor& copy_(const Tensor& src);              // copy_ (dispatched on this tensor's device)
    Tensor cpu() const { return to(Device(DeviceType::CPU)); }
    // Copies the (logically ordered) elements into a dense host buffer.
    void copyToHost(void* dst) const;
    double item() const;  // single-element tensor -> double (int64 values are exact below 2^53)
    int64_t item_int() const;

    // ---- reductions (schema names in config/native_functions.yaml:695-809) ----
    Tensor sum(DType dtype = DType::Undefined) const;                                              // sum
    Tensor sum(const std::vector<int64_t>& dim, bool keepdim = false, DType dtype = DType::Undefined) const;  // sum.dim_IntList
    Tensor mean(DType dtype = DType::Undefined) const;                                             // mean
    Tensor mean(const std::vector<int64_t>& dim, bool keepdim = false, DType dtype = DType::Undefined) const; // mean.dim
    Tensor max() const;                                                                            // max
    Tensor max(const std::vector<int64_t>& dim, bool keepdim = false) const;                       // max.dim
    Tensor min() const;                                                                            // min
    Tensor min(const std::vector<int64_t>& dim, bool keepdim = false) const;                       // min.dim
    Tensor argmax(std::optional<int64_t> dim = std::nullopt, bool keepdim = false) const;          // argmax
    Tensor argmin(std::optional<int64_t> dim = std::nullopt, bool keepdim = false) const;          // argmin
    Tensor var(int64_t correction = 1) const;                                                      // var
    Tensor var(const std::vector<int64_t>& dim, int64_t correction = 1, bool keepdim = false) const;  // var.dim
    Tensor std(int64_t correction = 1) const;                                                      // std
    Tensor std(const std::vector<int64_t>& dim, int64_t correction = 1, bool keepdim = false) const;  // std.dim
    Tensor prod(DType dtype = DType::Undefined) const;                                             // prod
    Tensor prod(const std::vector<int64_t>& dim, bool keepdim = false, DType dtype = DType::Undefined) const;  // prod.dim_IntList
    Tensor all() const;                                                                            // all
    Tensor all(const std::vector<int64_t>& dim, bool keepdim = false) const;                       // all.dim
    Tensor any() const;                                                                            // any
    Tensor any(const std::vector<int64_t>& dim, bool keepdim = false) const;                       // any.dim
    Tensor median() const;                                                                         // median
    Tensor norm(double p = 2.0) const;                                                             // norm
    Tensor norm(const std::vector<int64_t>& dim, double p = 2.0, bool keepdim = false) const;      // norm.dim
    Tensor softmax(int64_t dim, DType dtype = DType::Undefined) const;                            // softmax
    Tensor log_softmax(int64_t dim, DType dtype = DType::Undefined) const;                        // log_softmax
    // topk (schema added by this backend; TensorPlay has none)
    std::tuple<Tensor, Tensor> topk(int64_t k, int64_t dim = -1, bool largest = true, bool sorted = true) const;

private:
    std::shared_ptr<TensorImpl> impl_;
};

// Function-only schemas (config/native_functions.yaml:904-914), dispatched on
// the device of the first tensor argument.
std::tuple<Tensor, Tensor> nll_loss(const Tensor& self, const Tensor& target, const std::optional<Tensor>& weight,
                                    int64_t reduction = 1, int64_t ignore_index = -100);
Tensor nll_loss_backward(const Tensor& grad_output, const Tensor& self, const Tensor& target,
                         const std::optional<Tensor>& weight, int64_t reduction, int64_t ignore_index,
                         const Tensor& total_weight);
// Softmax gradients as single ops (added by this backend; TensorPlay's autograd
// composes config/derivatives.yaml:91-95 from sum / mul / sub / exp).
Tensor _softmax_backward_data(const Tensor& grad_output, const Tensor& output, int64_t dim,
                              DType input_dtype = DType::Float32);
Tensor _log_softmax_backward_data(const Tensor& grad_output, const Tensor& output, int64_t dim,
                                  DType input_dtype = DType::Float32);

// Top-k / top-p sampling of one Int64 id per row of the last dim (added by this
// backend; TensorPlay has no sampler).
Tensor topk_topp_sample(const Tensor& self, const Tensor& uniforms, int64_t k = 50, double temperature = 1.0,
                        double top_p = 1.0);
// Gradients of sum / mean / var / std (config/derivatives.yaml:82-86, :182-186)
// as single ops (added by this backend); dim empty = the full reduction.
Tensor sum_backward(const Tensor& grad, const Tensor& self, const std::vector<int64_t>& dim, bool keepdim);
Tensor mean_backward(const Tensor& grad, const Tensor& self, const std::vector<int64_t>& dim, bool keepdim);
Tensor var_backward(const Tensor& grad, const Tensor& self, const std::vector<int64_t>& dim, int64_t correction,
                    bool keepdim);
Tensor std_backward(const Tensor& grad, const Tensor& self, const Tensor& result, const std::vector<int64_t>& dim,
                    int64_t correction, bool keepdim);

// Output shape of a reduction over `dims` (ReductionKernels.cpp:48-70 semantics:
// negative dims wrap, out-of-range dims raise RuntimeError).
std::vector<int64_t> reductionShape(const std::vector<int64_t>& shape, const std::vector<int64_t>& dims, bool keepdim);

}  // namespace tensorplay
