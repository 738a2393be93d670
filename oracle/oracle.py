"""ctypes + numpy front-end of the C restatement in tp_cpu_reduce.c.

TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
baseline.  Arrays are float32 numpy arrays (any strides); dims follow the
reference's wrapping rules (ReductionKernels.cpp:48-70).

Parity status of each function (see tests/test_oracle.py):
  sum_all, sum_dim, mean_all, mean_dim  pinned: reference known answers + np.add.accumulate closed forms
  minmax_all, minmax_dim                pinned: known answers + np.max/np.min + brute force on +-0/NaN
  argminmax_all, argminmax_dim          pinned: known answers (test_reduction.py:35-52) + np.argmax
  var_all, var_dim (+std)               pinned: known answers (test_cuda_reductions.py:78-91) + torch.var/std
                                        at the reference's own rtol (test_statistical.py:10-17)
  topk                                  pinned: np.argsort(kind="stable") on canonical keys + torch.topk values
  copy                                  pinned: numpy astype on the same views (C casts), brute force on tiny shapes
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libtp_cpu_reduce.so")
_lib = None

_i64p = ctypes.POINTER(ctypes.c_int64)
_f32p = ctypes.POINTER(ctypes.c_float)


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i32, u32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_int64
        L.or_sum_all.argtypes = [vp, i32, _i64p, _i64p]; L.or_sum_all.restype = ctypes.c_float
        L.or_sum_dim.argtypes = [vp, i32, _i64p, _i64p, u32, vp]
        L.or_mean_all.argtypes = [vp, i32, _i64p, _i64p]; L.or_mean_all.restype = ctypes.c_float
        L.or_mean_dim.argtypes = [vp, i32, _i64p, _i64p, u32, _i64p, i32, vp]
        L.or_minmax_all.argtypes = [vp, i32, _i64p, _i64p, i32, _f32p]; L.or_minmax_all.restype = i32
        L.or_minmax_dim.argtypes = [vp, i32, _i64p, _i64p, u32, i32, vp]
        L.or_argminmax_all.argtypes = [vp, i32, _i64p, _i64p, i32]; L.or_argminmax_all.restype = i64
        L.or_argminmax_dim.argtypes = [vp, i32, _i64p, _i64p, i32, i32, i32, vp]
        L.or_var_all.argtypes = [vp, i32, _i64p, _i64p, i64, i32]; L.or_var_all.restype = ctypes.c_float
        L.or_var_dim.argtypes = [vp, i32, _i64p, _i64p, u32, _i64p, i32, i64, i32, vp]
        L.or_prod_all.argtypes = [vp, i32, _i64p, _i64p]; L.or_prod_all.restype = ctypes.c_float
        L.or_prod_dim.argtypes = [vp, i32, _i64p, _i64p, u32, vp]
        L.or_allany_all.argtypes = [vp, i32, _i64p, _i64p, i32]; L.or_allany_all.restype = i32
        L.or_allany_dim.argtypes = [vp, i32, _i64p, _i64p, u32, i32, vp]
        L.or_norm_all.argtypes = [vp, i32, _i64p, _i64p, ctypes.c_double, _f32p]; L.or_norm_all.restype = i32
        L.or_norm_dim.argtypes = [vp, i32, _i64p, _i64p, u32, ctypes.c_double, vp]
        L.or_median.argtypes = [vp, i32, _i64p, _i64p]; L.or_median.restype = ctypes.c_float
        L.or_copy.argtypes = [vp, i32, _i64p, vp, i32, _i64p, i32, _i64p]; L.or_copy.restype = i32
        L.or_topk.argtypes = [vp, i64, i64, i64, i64, i32, vp, vp]
        L.or_topk_mt.argtypes = [vp, i64, i64, i64, i64, i32, vp, vp, i32]
        _lib = L
    return _lib


def _geom(x):
    assert x.dtype == np.float32
    sizes = (ctypes.c_int64 * max(1, x.ndim))(*x.shape)
    strides = (ctypes.c_int64 * max(1, x.ndim))(*[s // 4 for s in x.strides])
    return ctypes.c_void_p(x.ctypes.data), x.ndim, sizes, strides


def _wrap_dims(ndim, dims):
    out = []
    for d in dims:
        dd = d + ndim if d < 0 else d
        if dd < 0 or dd >= ndim:
            raise RuntimeError("Dimension out of range")
        out.append(dd)
    return out


def _reduced_shape(shape, dims, keepdim):
    red = set(dims)
    s = []
    for i, n in enumerate(shape):
        if i in red:
            if keepdim:
                s.append(1)
        else:
            s.append(n)
    return tuple(s)


def _mask(dims):
    m = 0
    for d in dims:
        m |= 1 << d
    return m


def sum(x, dims=None, keepdim=False):
    L = lib()
    p, nd, sz, st = _geom(x)
    if not dims:
        return np.float32(L.or_sum_all(p, nd, sz, st))
    dd = _wrap_dims(nd, dims)
    out = np.empty(_reduced_shape(x.shape, dd, keepdim), np.float32)
    L.or_sum_dim(p, nd, sz, st, _mask(dd), ctypes.c_void_p(out.ctypes.data))
    return out


def mean(x, dims=None, keepdim=False):
    L = lib()
    p, nd, sz, st = _geom(x)
    if not dims:
        return np.float32(L.or_mean_all(p, nd, sz, st))
    dd = _wrap_dims(nd, dims)
    lst = (ctypes.c_int64 * len(dims))(*dims)
    out = np.empty(_reduced_shape(x.shape, dd, keepdim), np.float32)
    L.or_mean_dim(p, nd, sz, st, _mask(dd), lst, len(dims), ctypes.c_void_p(out.ctypes.data))
    return out


def amax(x, dims=None, keepdim=False, is_max=True):
    L = lib()
    p, nd, sz, st = _geom(x)
    if not dims:
        v = ctypes.c_float()
        if L.or_minmax_all(p, nd, sz, st, int(is_max), ctypes.byref(v)) != 0:
            raise RuntimeError("max(): Expected reduction dim to be non-empty")
        return np.float32(v.value)
    dd = _wrap_dims(nd, dims)
    out = np.empty(_reduced_shape(x.shape, dd, keepdim), np.float32)
    L.or_minmax_dim(p, nd, sz, st, _mask(dd), int(is_max), ctypes.c_void_p(out.ctypes.data))
    return out


def amin(x, dims=None, keepdim=False):
    return amax(x, dims, keepdim, is_max=False)


def argmax(x, dim=None, keepdim=False, is_max=True, quirk=False):
    L = lib()
    p, nd, sz, st = _geom(x)
    if dim is None:
        return np.int64(L.or_argminmax_all(p, nd, sz, st, int(is_max)))
    d = _wrap_dims(nd, [dim])[0]
    out = np.empty(_reduced_shape(x.shape, [d], keepdim), np.int64)
    L.or_argminmax_dim(p, nd, sz, st, d, int(is_max), int(quirk), ctypes.c_void_p(out.ctypes.data))
    return out


def argmin(x, dim=None, keepdim=False, quirk=False):
    return argmax(x, dim, keepdim, is_max=False, quirk=quirk)


def var(x, dims=None, correction=1, keepdim=False, take_sqrt=False):
    L = lib()
    p, nd, sz, st = _geom(x)
    if dims is None:
        return np.float32(L.or_var_all(p, nd, sz, st, correction, int(take_sqrt)))
    dd = _wrap_dims(nd, dims)
    lst = (ctypes.c_int64 * max(1, len(dims)))(*dims)
    out = np.empty(_reduced_shape(x.shape, dd, keepdim), np.float32)
    L.or_var_dim(p, nd, sz, st, _mask(dd), lst, len(dims), correction, int(take_sqrt),
                 ctypes.c_void_p(out.ctypes.data))
    return out


def std(x, dims=None, correction=1, keepdim=False):
    return var(x, dims, correction, keepdim, take_sqrt=True)


def prod(x, dims=None, keepdim=False):
    L = lib()
    p, nd, sz, st = _geom(x)
    if not dims:
        return np.float32(L.or_prod_all(p, nd, sz, st))
    dd = _wrap_dims(nd, dims)
    out = np.empty(_reduced_shape(x.shape, dd, keepdim), np.float32)
    L.or_prod_dim(p, nd, sz, st, _mask(dd), ctypes.c_void_p(out.ctypes.data))
    return out


def all_(x, dims=None, keepdim=False, is_any=False):
    L = lib()
    p, nd, sz, st = _geom(x)
    if not dims:
        return np.bool_(L.or_allany_all(p, nd, sz, st, int(is_any)))
    dd = _wrap_dims(nd, dims)
    out = np.empty(_reduced_shape(x.shape, dd, keepdim), np.uint8)
    L.or_allany_dim(p, nd, sz, st, _mask(dd), int(is_any), ctypes.c_void_p(out.ctypes.data))
    return out.astype(np.bool_)


def any_(x, dims=None, keepdim=False):
    return all_(x, dims, keepdim, is_any=True)


def norm(x, p=2.0, dims=None, keepdim=False):
    L = lib()
    ptr, nd, sz, st = _geom(x)
    if not dims:
        v = ctypes.c_float()
        if L.or_norm_all(ptr, nd, sz, st, float(p), ctypes.byref(v)) != 0:
            raise RuntimeError("max(): Expected reduction dim to be non-empty")
        return np.float32(v.value)
    dd = _wrap_dims(nd, dims)
    out = np.empty(_reduced_shape(x.shape, dd, keepdim), np.float32)
    L.or_norm_dim(ptr, nd, sz, st, _mask(dd), float(p), ctypes.c_void_p(out.ctypes.data))
    return out


def median(x):
    L = lib()
    p, nd, sz, st = _geom(x)
    return np.float32(L.or_median(p, nd, sz, st))


def topk(x2d, k, largest=True, threads=1):
    """Top-k along the last dim of a 2-D float32 array (rows may be strided)."""
    L = lib()
    assert x2d.ndim == 2 and x2d.strides[1] == 4
    rows, cols = x2d.shape
    vals = np.empty((rows, k), np.float32)
    idx = np.empty((rows, k), np.int64)
    args = (ctypes.c_void_p(x2d.ctypes.data), rows, cols, x2d.strides[0] // 4, k, int(largest),
            ctypes.c_void_p(vals.ctypes.data), ctypes.c_void_p(idx.ctypes.data))
    if threads == 1:
        L.or_topk(*args)
    else:
        L.or_topk_mt(*args, threads)
    return vals, idx


# P10 ScalarType numbering of numpy dtypes
DTYPE_CODES = {np.dtype(np.uint8): 0, np.dtype(np.int8): 1, np.dtype(np.int16): 2, np.dtype(np.int32): 3,
               np.dtype(np.int64): 4, np.dtype(np.uint16): 5, np.dtype(np.uint32): 6, np.dtype(np.uint64): 7,
               np.dtype(np.float32): 8, np.dtype(np.float64): 9, np.dtype(np.bool_): 10}


def copy(dst, src):
    """copy_ of `src` into `dst` (numpy arrays of one shape, any strides,
    including stride-0 broadcast views of src).  Writes dst in place."""
    L = lib()
    assert dst.shape == src.shape
    nd = dst.ndim
    sz = (ctypes.c_int64 * max(nd, 1))(*dst.shape)
    ds = (ctypes.c_int64 * max(nd, 1))(*[s // dst.itemsize for s in dst.strides])
    ss = (ctypes.c_int64 * max(nd, 1))(*[s // src.itemsize for s in src.strides])
    rc = L.or_copy(ctypes.c_void_p(dst.ctypes.data), DTYPE_CODES[dst.dtype], ds,
                   ctypes.c_void_p(src.ctypes.data), DTYPE_CODES[src.dtype], ss, nd, sz)
    assert rc == 0
    return dst
