// Strided -> dense copy (any element size of 1/2/4/8 bytes, up to 8 dims).
// Counterpart of TensorPlay's CUDA copy_cast_kernel_impl / copy_kernel
// (/root/reference/p10/src/backend/cuda/CopyKernels.cu:42-157) for the layout
// normalisation this backend needs.  One thread per output element, grid-stride;
// the output side is written fully coalesced.
#include <hip/hip_runtime.h>

#include "common.h"

namespace tpr {
namespace {

struct CopyArgs {
    const char* in;
    char* out;
    int ndim;
    long long sizes[TPR_MAX_DIMS];
    long long strides[TPR_MAX_DIMS];
    long long n;
};

template <typename T>
__global__ __launch_bounds__(256) void k_copy_strided(CopyArgs a) {
    const T* in = reinterpret_cast<const T*>(a.in);
    T* out = reinterpret_cast<T*>(a.out);
    const long long step = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += step) {
        long long rem = i, off = 0;
        for (int d = a.ndim - 1; d >= 0; --d) {
            off += (rem % a.sizes[d]) * a.strides[d];
            rem /= a.sizes[d];
        }
        out[i] = in[off];
    }
}

}  // namespace
}  // namespace tpr

extern "C" int tpr_copy_strided(const void* in, int32_t elem_size, int32_t ndim, const int64_t* sizes,
                                const int64_t* in_strides, void* out, void* stream) {
    using namespace tpr;
    if (ndim < 0 || ndim > TPR_MAX_DIMS) return fail(TPR_ERR_INVALID_ARG, "tpr_copy_strided: ndim out of range");
    CopyArgs a;
    a.in = static_cast<const char*>(in);
    a.out = static_cast<char*>(out);
    a.ndim = ndim;
    a.n = 1;
    for (int d = 0; d < ndim; ++d) {
        if (sizes[d] < 0) return fail(TPR_ERR_INVALID_ARG, "tpr_copy_strided: negative size");
        a.sizes[d] = sizes[d];
        a.strides[d] = in_strides[d];
        a.n *= sizes[d];
    }
    if (a.n == 0) return TPR_OK;
    if (!in || !out) return fail(TPR_ERR_INVALID_ARG, "tpr_copy_strided: null pointer");
    const long long blocks = std::min<long long>((a.n + 255) / 256, (long long)device_info().cus * 16);
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (elem_size) {
        case 1: hipLaunchKernelGGL(k_copy_strided<uint8_t>, dim3(blocks), dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(k_copy_strided<uint16_t>, dim3(blocks), dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(k_copy_strided<uint32_t>, dim3(blocks), dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL(k_copy_strided<uint64_t>, dim3(blocks), dim3(256), 0, st, a); break;
        default: return fail(TPR_ERR_INVALID_ARG, "tpr_copy_strided: elem_size must be 1, 2, 4 or 8");
    }
    return check_launch("k_copy_strided");
}
