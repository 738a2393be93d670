"""tensorplay_amd: MI355X (gfx950) backend for TensorPlay's P10 reduction + top-k path.

The Python surface mirrors the parts of TensorPlay this path touches:
``Tensor`` methods sum/mean/max/min/argmax/argmin/var/std (the overload set of
/root/reference/src/bindings/python/Tensor.cpp:1099-1224) plus ``topk``, and the
module functions of /root/reference/tensorplay/functional.py:401-432, plus
softmax / log_softmax / nll_loss (functional.py:313-317, 496-500) and their
gradients.  Tensors
live on ``"cpu"`` or ``"rocm[:N]"``; reductions run on ROCm devices only (the
CPU key has no kernels here -- that path stays TensorPlay's own).

The native library must be built (``python tensorplay_amd/build.py``); there is
no fallback.
"""
try:
    # One HIP runtime per process: torch ships its own libamdhip64 (same soname)
    # and its libraries load it by file name, so if this package's runtime were
    # loaded first the process would hold two.  Loading torch first makes both
    # resolve to torch's copy.
    import torch as _torch  # noqa: F401
except ImportError:
    pass
from . import _C  # noqa: E402

__version__ = "0.1.0"

Tensor = _C.TensorBase
DType = _C.DType
Device = _C.Device

uint8 = DType.uint8
int8 = DType.int8
int16 = DType.int16
int32 = DType.int32
int64 = DType.int64
uint16 = DType.uint16
uint32 = DType.uint32
uint64 = DType.uint64
float32 = DType.float32
float64 = DType.float64
bool_ = DType.bool
undefined = DType.undefined


def device(spec):
    return Device(spec)


def tensor(data, dtype=None, device="cpu"):
    """Copy array-like `data` into a new tensor on `device` ("cpu" / "rocm[:N]")."""
    import numpy as np
    arr = np.asarray(data)
    if dtype is None and arr.dtype == np.float64 and not isinstance(data, np.ndarray):
        arr = arr.astype(np.float32)  # Python floats default to float32, as TensorPlay's tensor()
    return _C.tensor(arr, dtype, str(device))


def from_numpy(arr, device="cpu"):
    return _C.tensor(arr, None, str(device))


def empty(shape, dtype=float32, device="cpu"):
    return _C.empty(list(shape), dtype, str(device))


def from_torch(t):
    """Zero-copy view of a torch tensor that lives on an AMD GPU (keeps `t` alive)."""
    import torch
    if not t.is_cuda:
        return _C.tensor(t.detach().numpy(), None, "cpu")
    dt = {torch.float32: float32, torch.float64: float64, torch.int64: int64, torch.int32: int32,
          torch.int16: int16, torch.int8: int8, torch.uint8: uint8, torch.bool: bool_}[t.dtype]
    return _C._from_device_ptr(t.data_ptr(), list(t.shape), list(t.stride()), dt, t.device.index or 0, t)


# ---- functional forms (tensorplay/functional.py:401-432 + topk) ----
def sum(input, dim=None, keepdim=False, dtype=None):
    return input.sum(dtype=dtype) if dim is None else input.sum(dim, keepdim, dtype=dtype)


def mean(input, dim=None, keepdim=False, dtype=None):
    return input.mean(dtype=dtype) if dim is None else input.mean(dim, keepdim, dtype=dtype)


def max(input, dim=None, keepdim=False):
    return input.max() if dim is None else input.max(dim, keepdim)


def min(input, dim=None, keepdim=False):
    return input.min() if dim is None else input.min(dim, keepdim)


def amax(input, dim=None, keepdim=False):
    return max(input, dim, keepdim)


def amin(input, dim=None, keepdim=False):
    return min(input, dim, keepdim)


def argmax(input, dim=None, keepdim=False):
    return input.argmax(dim, keepdim)


def argmin(input, dim=None, keepdim=False):
    return input.argmin(dim, keepdim)


def var(input, dim=None, correction=1, keepdim=False):
    return input.var(correction) if dim is None else input.var(dim, correction, keepdim)


def std(input, dim=None, correction=1, keepdim=False):
    return input.std(correction) if dim is None else input.std(dim, correction, keepdim)


def prod(input, dim=None, keepdim=False, dtype=None):
    return input.prod(dtype=dtype) if dim is None else input.prod(dim, keepdim, dtype=dtype)


def all(input, dim=None, keepdim=False):
    return input.all() if dim is None else input.all(dim, keepdim)


def any(input, dim=None, keepdim=False):
    return input.any() if dim is None else input.any(dim, keepdim)


def median(input):
    return input.median()


def norm(input, p=2.0, dim=None, keepdim=False):
    return input.norm(p) if dim is None else input.norm(dim, p, keepdim)


def topk(input, k, dim=-1, largest=True, sorted=True):
    return input.topk(k, dim, largest, sorted)


def softmax(input, dim, dtype=None):
    return input.softmax(dim, dtype)


def log_softmax(input, dim, dtype=None):
    return input.log_softmax(dim, dtype)


def nll_loss(input, target, weight=None, reduction=1, ignore_index=-100):
    """(output, total_weight), as tensorplay/functional.py:496-497."""
    return _C.nll_loss(input, target, weight, reduction, ignore_index)


def nll_loss_backward(grad_output, input, target, weight=None, reduction=1, ignore_index=-100,
                      total_weight=None):
    return _C.nll_loss_backward(grad_output, input, target, weight, reduction, ignore_index, total_weight)


def _softmax_backward_data(grad_output, output, dim):
    return _C._softmax_backward_data(grad_output, output, dim)


def _log_softmax_backward_data(grad_output, output, dim):
    return _C._log_softmax_backward_data(grad_output, output, dim)


def topk_topp_sample(input, uniforms, k=50, temperature=1.0, top_p=1.0):
    """One token id per row of the last dim: top-k, then the top-p nucleus, drawn with `uniforms`."""
    return _C.topk_topp_sample(input, uniforms, k, temperature, top_p)


def sum_backward(grad, input, dim=(), keepdim=False):
    return _C.sum_backward(grad, input, list(dim), keepdim)


def mean_backward(grad, input, dim=(), keepdim=False):
    return _C.mean_backward(grad, input, list(dim), keepdim)


def var_backward(grad, input, dim=(), correction=1, keepdim=False):
    return _C.var_backward(grad, input, list(dim), correction, keepdim)


def std_backward(grad, input, result, dim=(), correction=1, keepdim=False):
    return _C.std_backward(grad, input, result, list(dim), correction, keepdim)


_REDUCTION = {"none": 0, "mean": 1, "sum": 2}


def cross_entropy(input, target, weight=None, ignore_index=-100, reduction="mean"):
    """nll_loss(log_softmax(input, 1), target, ...), the composition of
    tensorplay/nn/functional.py:442-444 (forward only; its gradient is
    _log_softmax_backward_data(nll_loss_backward(...), log_probs, 1))."""
    out, _ = nll_loss(log_softmax(input, 1), target, weight, _REDUCTION[reduction], ignore_index)
    return out


class rocm:
    """ROCm runtime helpers (the counterpart of tensorplay.cuda for this backend)."""

    is_available = staticmethod(_C._rocm.is_available)
    device_count = staticmethod(_C._rocm.device_count)
    synchronize = staticmethod(_C._rocm.synchronize)
    set_stream = staticmethod(_C._rocm.set_stream)
    current_stream = staticmethod(_C._rocm.current_stream)
    empty_cache = staticmethod(_C._rocm.empty_cache)
    memory_stats = staticmethod(_C._rocm.memory_stats)
