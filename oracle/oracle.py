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
  softmax, log_softmax                  pinned: known answer (test_pointwise.py:154-172) + torch fp64 softmax /
                                        log_softmax within fp32 rounding; NaN / inf rows by brute force
  softmax_bwd (both modes)              pinned: torch.autograd fp64 gradients of softmax / log_softmax
  nll_loss, nll_loss_backward           pinned: torch.nn.functional.nll_loss (+ autograd) in fp64 with weights,
                                        ignore_index and every reduction; closed form -x[i, t_i]
  reduce_backward (sum/mean/var/std)    pinned: torch.autograd fp64 gradients of sum / mean / var / std,
                                        full and along dims, corrections 0 / 1 / 2
  sample (top-k / top-p)                pinned: inverse-CDF over the full softmax when k = cols and top_p = 1;
                                        argmax when k = 1 or T <= 0; brute-force frequencies over a grid of u
  reduce_f64 (float64 inputs)           pinned: math.fsum / numpy fp64 reductions, argmax first occurrence,
                                        torch.var / torch.std / torch.norm in fp64
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
        L.or_softmax.argtypes = [vp, i64, i64, i64, i32, vp]
        L.or_softmax_bwd.argtypes = [vp, vp, i64, i64, i64, i32, vp]
        L.or_nll_loss.argtypes = [vp, i64, i64, vp, vp, i64, i64, vp, vp]; L.or_nll_loss.restype = i32
        L.or_nll_loss_backward.argtypes = [vp, vp, vp, i64, i64, i32, ctypes.c_float, i64, i64, vp]
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


def sort_keys(x):
    """Ascending sortable unsigned keys of any numpy dtype, the order tpr_topk
    uses: floats by value with -0.0 == +0.0 and every NaN above +inf, signed
    integers by value (sign bit flipped), unsigned integers and bool as they
    are.  uint64 for 8-byte dtypes, uint32 otherwise."""
    x = np.asarray(x)
    if x.dtype == np.bool_:
        return x.astype(np.uint32)
    if x.dtype.kind == "f":
        bits, ut, sign, qnan = ((np.uint64, np.uint64, np.uint64(1 << 63), np.uint64(0x7ff8000000000000))
                                if x.dtype.itemsize == 8 else
                                (np.uint32, np.uint32, np.uint32(1 << 31), np.uint32(0x7fc00000)))
        u = x.view(bits).copy()
        u[np.isnan(x)] = qnan
        neg = (u & sign) != 0
        out = np.where(neg, (~u) + ut(1), u | sign)  # -0.0 and +0.0 both map to `sign`
        return out.astype(ut)
    ut = np.uint64 if x.dtype.itemsize == 8 else np.uint32
    if x.dtype.kind == "i":
        w = x.dtype.itemsize * 8
        u = x.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[x.dtype.itemsize])
        return (u ^ np.array(1 << (w - 1), u.dtype)).astype(ut)
    return x.astype(ut)


def topk_any(x2d, k, largest=True):
    """Top-k of a 2-D array of any dtype in this build's order (tpr_topk):
    key descending (ascending for largest=False), equal keys by lowest index;
    values are the selected elements.  numpy stable sort on sort_keys."""
    x2d = np.asarray(x2d)
    key = sort_keys(x2d)
    order = np.argsort(~key if largest else key, axis=1, kind="stable")[:, :k]
    return np.take_along_axis(x2d, order, axis=1), order.astype(np.int64)


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


def _dim3(x, dim):
    """Dense float32 copy of x viewed as [outer, n, inner] around `dim`."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nd = x.ndim
    d = (dim + max(nd, 1)) % max(nd, 1) if nd else 0
    shp = x.shape if nd else (1,)
    outer = int(np.prod(shp[:d])) if d else 1
    inner = int(np.prod(shp[d + 1:])) if d + 1 < len(shp) else 1
    return x, outer, (shp[d] if nd else 1), inner


def softmax(x, dim, log=False):
    """softmax / log_softmax along `dim` (PointwiseKernels.cpp:519-545)."""
    x, outer, n, inner = _dim3(x, dim)
    y = np.empty_like(x)
    lib().or_softmax(ctypes.c_void_p(x.ctypes.data), outer, n, inner, int(log), ctypes.c_void_p(y.ctypes.data))
    return y


def log_softmax(x, dim):
    return softmax(x, dim, log=True)


def softmax_backward(grad, y, dim, log=False):
    """Gradient of softmax (log=False) or log_softmax (log=True) given its output y
    (config/derivatives.yaml:91-95)."""
    g, outer, n, inner = _dim3(grad, dim)
    y = np.ascontiguousarray(y, dtype=np.float32)
    gx = np.empty_like(g)
    lib().or_softmax_bwd(ctypes.c_void_p(g.ctypes.data), ctypes.c_void_p(y.ctypes.data), outer, n, inner,
                         int(log), ctypes.c_void_p(gx.ctypes.data))
    return gx


def nll_loss(x, target, weight=None, reduction=1, ignore_index=-100):
    """(output, total_weight) of nll_loss_kernel (LossKernels.cpp:12-55); raises
    RuntimeError("Target out of bounds") as the reference."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    t = np.ascontiguousarray(target, dtype=np.int64)
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    N, C = x.shape
    out = np.zeros(N if reduction == 0 else 1, dtype=np.float32)
    tw = np.zeros(1, dtype=np.float32)
    rc = lib().or_nll_loss(ctypes.c_void_p(x.ctypes.data), N, C, ctypes.c_void_p(t.ctypes.data),
                           None if w is None else ctypes.c_void_p(w.ctypes.data), reduction, ignore_index,
                           ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(tw.ctypes.data))
    if rc:
        raise RuntimeError("Target out of bounds")
    return (out if reduction == 0 else out.reshape(())), tw


def nll_loss_backward(grad, target, C, weight=None, reduction=1, ignore_index=-100, total_weight=None):
    """grad_input [N, C] of nll_loss_backward_kernel (LossKernels.cpp:57-101)."""
    g = np.ascontiguousarray(np.asarray(grad, dtype=np.float32).reshape(-1))
    t = np.ascontiguousarray(target, dtype=np.int64)
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    N = t.shape[0]
    gi = np.empty((N, C), dtype=np.float32)
    has_tw = total_weight is not None
    tw = float(np.asarray(total_weight, dtype=np.float32).reshape(-1)[0]) if has_tw else 0.0
    lib().or_nll_loss_backward(ctypes.c_void_p(g.ctypes.data), ctypes.c_void_p(t.ctypes.data),
                               None if w is None else ctypes.c_void_p(w.ctypes.data), reduction, ignore_index,
                               int(has_tw), tw, N, C, ctypes.c_void_p(gi.ctypes.data))
    return gi


def reduce_backward(grad, x, op, dims=None, correction=1, result=None):
    """Gradient of sum / mean / var / std w.r.t. x given the output gradient,
    restating config/derivatives.yaml:82-86, :182-186 as TensorPlay's autograd
    evaluates them, op by op in float32:
      sum:  grad.expand(self.shape())
      mean: grad.expand(self.shape()) / self.numel()          div.Scalar: (float)(a / (double)n)
      var:  grad * 2 * (self - self.mean()) / (self.numel() - correction)
      std:  grad * (self - self.mean()) / (result * (self.numel() - correction))
    (mul.Scalar by an integer Scalar multiplies in float, ArithmeticKernels.cpp:1469-1491;
    div.Scalar divides in double, :1502-1532).  dims None / empty = the full
    reduction; with dims the same formulas apply per output (count = the product
    of the listed dims' sizes, duplicates included)."""
    x = np.asarray(x, dtype=np.float32)
    nd = x.ndim
    full = not dims
    rd = list(range(nd)) if full else _wrap_dims(nd, dims)
    count = int(np.prod([x.shape[d] for d in rd])) if rd else 1
    kshape = [1 if i in rd else x.shape[i] for i in range(nd)]
    g = np.asarray(grad, dtype=np.float32).reshape(kshape)
    if op == "sum":
        return np.ascontiguousarray(np.broadcast_to(g, x.shape))
    if op == "mean":
        return np.ascontiguousarray(np.broadcast_to((g.astype(np.float64) / count).astype(np.float32), x.shape))
    m = np.asarray(mean(x, None if full else rd, keepdim=True), np.float32).reshape(kshape)
    if op == "var":
        t = (g * np.float32(2)) * (x - m)
        return (t.astype(np.float64) / float(count - correction)).astype(np.float32)
    if op == "std":
        r = np.asarray(result, dtype=np.float32).reshape(kshape)
        t = g * (x - m)
        with np.errstate(divide="ignore", invalid="ignore"):
            return t / (r * np.float32(count - correction))
    raise ValueError(op)


def sample(x2d, u, k, temperature=1.0, top_p=1.0, details=False):
    """Top-k / top-p sampling (this build's definition; TensorPlay has none):
    the k largest logits per row (topk order: descending, ties to the lowest
    index), p_j = exp(v_j/T - v_0/T), c_j = cumulative sums, nucleus 0..m with m
    the first j where c_j >= top_p * c_{k-1}, then the first j <= m with
    c_j > u * c_m.  T <= 0 is greedy.  Computed in float64.
    Returns (ids, margin): margin is the smallest relative distance of the two
    decision thresholds (top_p cut, u draw) to a cumulative sum -- where it is
    below the float32 rounding of the GPU's sums, either neighbour is a valid
    draw.  details=True also returns, per row, the nucleus end m, the drawn
    position j (both in top-k order) and the cut's own relative margin."""
    x2d = np.asarray(x2d, np.float32)
    rows = x2d.shape[0]
    vals, idx = topk(x2d, k)
    if not temperature > 0:
        if details:
            z = np.zeros(rows, np.int64)
            return idx[:, 0].copy(), np.full(rows, np.inf), z, z.copy(), np.full(rows, np.inf)
        return idx[:, 0].copy(), np.full(rows, np.inf)
    ids = np.empty(rows, np.int64)
    margin = np.empty(rows)
    ms = np.empty(rows, np.int64)
    js = np.empty(rows, np.int64)
    cut_margin = np.empty(rows)
    for r in range(rows):
        z = vals[r].astype(np.float64) / temperature
        p = np.exp(z - z[0])
        c = np.cumsum(p)
        cut = top_p * c[-1]
        hit = np.nonzero(c >= cut)[0]
        m = int(hit[0]) if hit.size else k - 1
        thr = float(u[r]) * c[m]
        hit = np.nonzero(c[: m + 1] > thr)[0]
        j = int(hit[0]) if hit.size else m
        ids[r] = idx[r, j]
        cut_margin[r] = np.min(np.abs(c - cut)) / c[-1]
        margin[r] = min(cut_margin[r], np.min(np.abs(c[: m + 1] - thr)) / c[m])
        ms[r], js[r] = m, j
    if details:
        return ids, margin, ms, js, cut_margin
    return ids, margin


def reduce_f64(x, op, dims=None, correction=1, p=2.0):
    """Float64 reductions as TensorPlay's CPU path computes them for Float64
    tensors (ReductionKernels.cpp, AccumulateType<double> = double): sums and
    products accumulate sequentially in double in memory order; max / min /
    argmax / argmin use the strict compare from -inf / +inf (NaN ignored, first
    index wins); var / std are the two-pass mean / (x - mean)^2 / sum /
    (n - correction) composite in double; norm is (sum |x|^p)^(1/p).  Numpy,
    sequential where the reference is (np.add.accumulate / np.multiply.accumulate)."""
    x = np.asarray(x, dtype=np.float64)
    nd = x.ndim
    ax = tuple(range(nd)) if not dims else tuple(_wrap_dims(nd, dims))
    kept = [i for i in range(nd) if i not in ax]
    y = np.moveaxis(x, kept + list(ax), list(range(nd))).reshape([x.shape[i] for i in kept] + [-1])
    if op == "sum":
        return np.add.accumulate(y, axis=-1)[..., -1] if y.shape[-1] else np.zeros(y.shape[:-1])
    if op == "mean":
        return reduce_f64(x, "sum", dims) / y.shape[-1]
    if op == "prod":
        return np.multiply.accumulate(y, axis=-1)[..., -1] if y.shape[-1] else np.ones(y.shape[:-1])
    if op in ("amax", "amin", "argmax", "argmin"):
        is_max = op in ("amax", "argmax")
        z = np.where(np.isnan(y), -np.inf if is_max else np.inf, y)
        i = np.argmax(z, axis=-1) if is_max else np.argmin(z, axis=-1)
        v = np.take_along_axis(z, i[..., None], -1)[..., 0]
        return v if op in ("amax", "amin") else i.astype(np.int64)
    if op in ("var", "std"):
        n = y.shape[-1]
        m = np.add.accumulate(y, axis=-1)[..., -1:] / n
        d = (y - m) ** 2
        v = np.add.accumulate(d, axis=-1)[..., -1] / max(0, n - correction)
        return np.sqrt(v) if op == "std" else v
    if op == "norm":
        if np.isinf(p):
            a = np.abs(y)
            return a.max(axis=-1) if p > 0 else a.min(axis=-1)
        with np.errstate(divide="ignore"):
            return np.add.accumulate(np.abs(y) ** p, axis=-1)[..., -1] ** (1.0 / p)
    raise ValueError(op)
