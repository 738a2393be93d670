"""ctypes binding of the C-ABI launch layer (include/tpr_rocm.h).

This is the same stub a TensorPlay maintainer would add on the reference side
to reach the backend from Python; the C++ host core (tensorplay_amd._C) calls
the same entry points directly.  Device memory and streams come from PyTorch
(plumbing only): tensors are passed as raw device pointers + element strides.

The library must have been built (python tensorplay_amd/build.py); loading
fails loudly otherwise -- there is no CPU fallback.  With TPR_ROCM_DEV=1 in the
environment (the test suite sets it) this loads the test build
libtpr_rocm_dev.so instead, the same kernels plus the plan-override hook
tpr_debug_set; the shipped libtpr_rocm.so has no such hook.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libtpr_rocm.so")
DEV_LIB_PATH = os.path.join(PKG, "libtpr_rocm_dev.so")

MAX_DIMS = 8

# enum tpr_status
OK, ERR_INVALID_ARG, ERR_UNSUPPORTED_DTYPE, ERR_HIP, ERR_WORKSPACE, ERR_NOT_IMPLEMENTED = range(6)
# enum tpr_dtype (P10 ScalarType numbering)
UINT8, INT8, INT16, INT32, INT64, UINT16, UINT32, UINT64, FLOAT32, FLOAT64, BOOL = range(11)
# enum tpr_reduce_op
SUM, MEAN, AMAX, AMIN, ARGMAX, ARGMIN, VAR, STD, PROD, NORM, ALL, ANY, MEDIAN = range(13)
OP_NAMES = {"sum": SUM, "mean": MEAN, "amax": AMAX, "amin": AMIN, "argmax": ARGMAX,
            "argmin": ARGMIN, "var": VAR, "std": STD, "prod": PROD, "norm": NORM, "all": ALL,
            "any": ANY, "median": MEDIAN}

EXPORTED = ["tpr_reduce_workspace_bytes", "tpr_reduce", "tpr_topk_workspace_bytes", "tpr_topk",
            "tpr_copy", "tpr_copy_plan", "tpr_copy_strided", "tpr_last_error", "tpr_abi_version",
            "tpr_debug_set", "tpr_softmax", "tpr_softmax_workspace_bytes", "tpr_nll_loss_workspace_bytes", "tpr_nll_loss",
            "tpr_nll_loss_backward", "tpr_reduce_backward_workspace_bytes", "tpr_reduce_backward",
            "tpr_sample_workspace_bytes", "tpr_sample", "tpr_reduce_noalloc", "tpr_topk_plan", "tpr_debug_get"]
TEST_BUILD_ONLY = {"tpr_debug_set", "tpr_debug_get"}  # exported by libtpr_rocm_dev.so alone
REDUCE_SCRATCH_BYTES = 8 << 20  # TPR_REDUCE_SCRATCH_BYTES
# enum tpr_softmax_mode
SOFTMAX_FWD, LOG_SOFTMAX_FWD, SOFTMAX_BWD, LOG_SOFTMAX_BWD = range(4)
# tpr_copy_plan kinds (bits 0-1) and the vector-variant flag (bit 2)
COPY_CONTIG, COPY_ROWS, COPY_TILE, COPY_ELEM = range(4)
COPY_VEC = 4


class TprError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"tpr status {status}: {msg}")
        self.status = status


class CopyDesc(ctypes.Structure):
    _fields_ = [
        ("ndim", ctypes.c_int32),
        ("dst_dtype", ctypes.c_int32),
        ("src_dtype", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("sizes", ctypes.c_int64 * MAX_DIMS),
        ("dst_strides", ctypes.c_int64 * MAX_DIMS),
        ("src_strides", ctypes.c_int64 * MAX_DIMS),
    ]


class ReduceDesc(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_int32),
        ("in_dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("sizes", ctypes.c_int64 * MAX_DIMS),
        ("strides", ctypes.c_int64 * MAX_DIMS),
        ("reduce_mask", ctypes.c_uint32),
        ("reserved0", ctypes.c_int32),
        ("correction", ctypes.c_int64),
        ("count_override", ctypes.c_int64),
        ("p", ctypes.c_double),
    ]


class SoftmaxDesc(ctypes.Structure):
    _fields_ = [
        ("mode", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("outer", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("inner", ctypes.c_int64),
        ("a_strides", ctypes.c_int64 * 3),
        ("b_strides", ctypes.c_int64 * 3),
    ]


_lib = None


def lib_path():
    """The library lib() loads: the test build when TPR_ROCM_DEV=1."""
    return DEV_LIB_PATH if os.environ.get("TPR_ROCM_DEV") == "1" else LIB_PATH


def lib():
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise ImportError(f"{path} is not built; run `python tensorplay_amd/build.py`")
        L = ctypes.CDLL(path)
        vp, sz, i32, i64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_int64
        dp = ctypes.POINTER(ReduceDesc)
        i64p = ctypes.POINTER(ctypes.c_int64)
        L.tpr_reduce_workspace_bytes.argtypes = [dp]
        L.tpr_reduce_workspace_bytes.restype = sz
        L.tpr_reduce.argtypes = [dp, vp, vp, vp, sz, vp]
        L.tpr_reduce.restype = ctypes.c_int
        L.tpr_reduce_noalloc.argtypes = [dp, vp, vp, vp]
        L.tpr_reduce_noalloc.restype = ctypes.c_int
        L.tpr_topk_workspace_bytes.argtypes = [i32, i64, i64, i64]
        L.tpr_topk_workspace_bytes.restype = sz
        L.tpr_topk.argtypes = [vp, i32, i64, i64, i64, i64, i32, i32, vp, vp, vp, sz, vp]
        L.tpr_topk.restype = ctypes.c_int
        L.tpr_topk_plan.argtypes = [i32, i64, i64, i64, i64, i32, i64p]
        L.tpr_topk_plan.restype = ctypes.c_int
        cdp = ctypes.POINTER(CopyDesc)
        L.tpr_copy.argtypes = [cdp, vp, vp, vp]
        L.tpr_copy.restype = ctypes.c_int
        L.tpr_copy_plan.argtypes = [cdp, vp, vp]
        L.tpr_copy_plan.restype = ctypes.c_int
        L.tpr_copy_strided.argtypes = [vp, i32, i32, i64p, i64p, vp, vp]
        L.tpr_copy_strided.restype = ctypes.c_int
        L.tpr_last_error.argtypes = []
        L.tpr_last_error.restype = ctypes.c_char_p
        L.tpr_abi_version.argtypes = []
        L.tpr_abi_version.restype = i32
        if hasattr(L, "tpr_debug_set"):  # test build only
            L.tpr_debug_set.argtypes = [ctypes.c_char_p, i64]
            L.tpr_debug_set.restype = ctypes.c_int
            L.tpr_debug_get.argtypes = [ctypes.c_char_p, ctypes.POINTER(i64)]
            L.tpr_debug_get.restype = ctypes.c_int
        L.tpr_softmax.argtypes = [ctypes.POINTER(SoftmaxDesc), vp, vp, vp, vp, sz, vp]
        L.tpr_reduce_backward_workspace_bytes.argtypes = [dp]
        L.tpr_reduce_backward_workspace_bytes.restype = sz
        L.tpr_reduce_backward.argtypes = [dp, vp, vp, vp, vp, vp, sz, vp]
        L.tpr_reduce_backward.restype = ctypes.c_int
        L.tpr_sample_workspace_bytes.argtypes = [i32, i64, i64, i64]
        L.tpr_sample_workspace_bytes.restype = sz
        L.tpr_sample.argtypes = [vp, i32, i64, i64, i64, i64, ctypes.c_float, ctypes.c_float, vp, vp, vp, sz, vp]
        L.tpr_sample.restype = ctypes.c_int
        L.tpr_softmax_workspace_bytes.argtypes = [ctypes.POINTER(SoftmaxDesc)]
        L.tpr_softmax_workspace_bytes.restype = sz
        L.tpr_softmax.restype = ctypes.c_int
        L.tpr_nll_loss_workspace_bytes.argtypes = [i64]
        L.tpr_nll_loss_workspace_bytes.restype = sz
        L.tpr_nll_loss.argtypes = [vp, i32, i64, i64, i64, i64, vp, i64, vp, i64, i64, vp, vp, vp, vp, sz, vp]
        L.tpr_nll_loss.restype = ctypes.c_int
        L.tpr_nll_loss_backward.argtypes = [vp, i64, vp, i64, vp, vp, i64, i64, i64, i64, vp, vp]
        L.tpr_nll_loss_backward.restype = ctypes.c_int
        _lib = L
    return _lib


def _check(rc):
    if rc != OK:
        raise TprError(rc, lib().tpr_last_error().decode())


def debug_set(key, value):
    L = lib()
    if not hasattr(L, "tpr_debug_set"):
        raise RuntimeError("plan overrides need the test build: set TPR_ROCM_DEV=1 before the library loads")
    _check(L.tpr_debug_set(key.encode(), int(value)))


def debug_get(key):
    """A device-side check counter of the test build, read and cleared
    (tpr_debug_get): "topk_merge_clamped"."""
    L = lib()
    if not hasattr(L, "tpr_debug_get"):
        raise RuntimeError("check counters need the test build: set TPR_ROCM_DEV=1 before the library loads")
    v = ctypes.c_int64(0)
    _check(L.tpr_debug_get(key.encode(), ctypes.byref(v)))
    return v.value


TOPK_KINDS = {1: "short_small", 2: "rsel", 3: "rsel_seg", 4: "radix", 5: "short", 6: "wave", 7: "block", 8: "wave8"}


def topk_plan(dtype, rows, cols, k, row_stride=None, aligned=True):
    """(kernel family, segments per row, segment length, waves, workspace bytes)
    that tpr_topk plans for this call; launches nothing."""
    out = (ctypes.c_int64 * 5)()
    _check(lib().tpr_topk_plan(dtype, rows, cols, k, cols if row_stride is None else row_stride,
                               1 if aligned else 0, out))
    return TOPK_KINDS[out[0]], out[1], out[2], out[3], out[4]


def make_desc(op, shape, strides, reduce_dims, out_dtype, correction=1, count_override=0,
              in_dtype=FLOAT32, p=2.0):
    d = ReduceDesc()
    d.op = OP_NAMES[op] if isinstance(op, str) else op
    d.in_dtype = in_dtype
    d.out_dtype = out_dtype
    d.ndim = len(shape)
    if d.ndim > MAX_DIMS:
        raise ValueError("at most 8 dims")
    for i, (n, s) in enumerate(zip(shape, strides)):
        d.sizes[i] = n
        d.strides[i] = s
    m = 0
    for r in reduce_dims:
        m |= 1 << r
    d.reduce_mask = m
    d.correction = correction
    d.count_override = count_override
    d.p = p
    return d


def _stream(torch, device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def default_out_dtype(op, in_dtype=FLOAT32):
    op = OP_NAMES[op] if isinstance(op, str) else op
    if op in (ARGMAX, ARGMIN):
        return INT64
    if op in (ALL, ANY):
        return BOOL
    if in_dtype == FLOAT64:
        return FLOAT64   # sum / mean / prod / amax / amin / var / std / norm of float64
    if in_dtype != FLOAT32:
        if op in (SUM, PROD):
            return INT64
        if op in (AMAX, AMIN, MEDIAN):
            return in_dtype
    return FLOAT32


def _torch_dtypes():
    import torch
    m = {torch.float32: FLOAT32, torch.float64: FLOAT64, torch.int64: INT64, torch.int32: INT32,
         torch.int16: INT16, torch.int8: INT8, torch.uint8: UINT8, torch.bool: BOOL}
    for name, code in (("uint16", UINT16), ("uint32", UINT32), ("uint64", UINT64)):
        if hasattr(torch, name):
            m[getattr(torch, name)] = code
    return m


def reduce(x, op, dims=None, correction=1, out_dtype=None, count_override=0, p=2.0):
    """Reduce a float32 CUDA(ROCm) torch tensor over `dims` (None = all).

    Returns a dense torch tensor of the kept dims' shape (keepdim=False)."""
    import torch
    nd = x.dim()
    if dims is None:
        rd = list(range(nd))
    else:
        rd = sorted(set((d + nd) if d < 0 else d for d in dims))
    kept = [x.shape[i] for i in range(nd) if i not in rd]
    tmap = _torch_dtypes()
    idt = tmap[x.dtype]
    od = default_out_dtype(op, idt) if out_dtype is None else out_dtype
    tdt = {v: k for k, v in tmap.items()}[od]
    out = torch.empty(kept, dtype=tdt, device=x.device)
    desc = make_desc(op, list(x.shape), list(x.stride()), rd, od, correction, count_override, in_dtype=idt, p=p)
    L = lib()
    wsb = L.tpr_reduce_workspace_bytes(ctypes.byref(desc))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    _check(L.tpr_reduce(ctypes.byref(desc), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                        ctypes.c_void_p(ws.data_ptr()), wsb, _stream(torch, x.device)))
    return out


def reduce_noalloc(x, op, dims=None, correction=1, out=None, p=2.0):
    """reduce() through tpr_reduce_noalloc: no workspace, the library's fixed
    per-device scratch holds split partials.  `out` (dense, the kept dims'
    shape) may be passed in so the call itself allocates nothing."""
    import torch
    nd = x.dim()
    rd = list(range(nd)) if dims is None else sorted(set((d + nd) if d < 0 else d for d in dims))
    tmap = _torch_dtypes()
    idt = tmap[x.dtype]
    od = default_out_dtype(op, idt)
    if out is None:
        kept = [x.shape[i] for i in range(nd) if i not in rd]
        out = torch.empty(kept, dtype={v: k for k, v in tmap.items()}[od], device=x.device)
    desc = make_desc(op, list(x.shape), list(x.stride()), rd, od, correction, in_dtype=idt, p=p)
    _check(lib().tpr_reduce_noalloc(ctypes.byref(desc), ctypes.c_void_p(x.data_ptr()),
                                    ctypes.c_void_p(out.data_ptr()), _stream(torch, x.device)))
    return out


def topk(x2d, k, largest=True, sorted=True):
    """Top-k along the last dim of a 2-D device tensor of any supported dtype
    (unit inner stride).  Values keep the input dtype."""
    import torch
    assert x2d.dim() == 2 and (x2d.stride(1) == 1 or x2d.shape[1] <= 1)
    rows, cols = x2d.shape
    dt = _torch_dtypes()[x2d.dtype]
    vals = torch.empty((rows, k), dtype=x2d.dtype, device=x2d.device)
    idx = torch.empty((rows, k), dtype=torch.int64, device=x2d.device)
    L = lib()
    wsb = L.tpr_topk_workspace_bytes(dt, rows, cols, k)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x2d.device)
    _check(L.tpr_topk(ctypes.c_void_p(x2d.data_ptr()), dt, rows, cols, x2d.stride(0), k,
                      int(largest), int(sorted), ctypes.c_void_p(vals.data_ptr()),
                      ctypes.c_void_p(idx.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb,
                      _stream(torch, x2d.device)))
    return vals, idx


def make_copy_desc(shape, dst_strides, src_strides, dst_dtype, src_dtype):
    d = CopyDesc()
    d.ndim = len(shape)
    if d.ndim > MAX_DIMS:
        raise ValueError("at most 8 dims")
    d.dst_dtype, d.src_dtype = dst_dtype, src_dtype
    for i, n in enumerate(shape):
        d.sizes[i] = n
        d.dst_strides[i] = dst_strides[i]
        d.src_strides[i] = src_strides[i]
    return d


def copy_(dst, src):
    """dst[...] = src[...] cast to dst's dtype, both torch device tensors of one
    shape at any strides (src may be an expanded view).  Returns dst."""
    import torch
    tmap = _torch_dtypes()
    assert list(dst.shape) == list(src.shape), "copy_: shapes differ"
    d = make_copy_desc(list(dst.shape), list(dst.stride()), list(src.stride()), tmap[dst.dtype], tmap[src.dtype])
    _check(lib().tpr_copy(ctypes.byref(d), ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                          _stream(torch, dst.device)))
    return dst


def copy_plan(dst, src):
    tmap = _torch_dtypes()
    d = make_copy_desc(list(dst.shape), list(dst.stride()), list(src.stride()), tmap[dst.dtype], tmap[src.dtype])
    return lib().tpr_copy_plan(ctypes.byref(d), ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()))


def copy_strided(x):
    """Dense copy of any strided device tensor through tpr_copy_strided."""
    import torch
    out = torch.empty(list(x.shape), dtype=x.dtype, device=x.device)
    nd = x.dim()
    sizes = (ctypes.c_int64 * max(1, nd))(*x.shape)
    strides = (ctypes.c_int64 * max(1, nd))(*x.stride())
    _check(lib().tpr_copy_strided(ctypes.c_void_p(x.data_ptr()), x.element_size(), nd, sizes, strides,
                                  ctypes.c_void_p(out.data_ptr()), _stream(torch, x.device)))
    return out


def _view3(x, dim):
    """(outer, n, inner) extents and element strides of x around `dim`, or None
    when the outer or inner dims do not collapse to one stride."""
    nd = x.dim()
    if nd == 0:
        return (1, 1, 1), (1, 1, 1)
    d = dim % nd

    def collapse(lo, hi):
        size, stride, first = 1, 1, True
        for i in range(hi - 1, lo - 1, -1):
            if x.shape[i] == 1:
                continue
            if first:
                stride, first = x.stride(i), False
            elif x.stride(i) != stride * size:
                return None
            size *= x.shape[i]
        if any(x.shape[i] == 0 for i in range(lo, hi)):
            size = 0
        return size, stride
    o, i = collapse(0, d), collapse(d + 1, nd)
    if o is None or i is None:
        return None
    n = x.shape[d]
    so = o[1] if o[0] != 1 else n * i[0]
    si = i[1] if i[0] != 1 else 1
    return (o[0], n, i[0]), (so, x.stride(d), si)


def softmax(x, dim=-1, log=False, grad_of=None):
    """Softmax / log_softmax of a float32 or float64 device tensor along `dim` through
    tpr_softmax; with grad_of=y, the gradient given g = x and the forward
    output y.  Returns a dense tensor of x's shape."""
    import torch
    a, b = x, grad_of
    v = _view3(a, dim)
    if v is None:
        a = a.contiguous()
        v = _view3(a, dim)
    vb = None
    if b is not None:
        vb = _view3(b, dim)
        if vb is None:
            b = b.contiguous()
            vb = _view3(b, dim)
    out = torch.empty(list(x.shape), dtype=x.dtype, device=x.device)
    d = SoftmaxDesc()
    d.mode = (LOG_SOFTMAX_BWD if log else SOFTMAX_BWD) if b is not None else (LOG_SOFTMAX_FWD if log else SOFTMAX_FWD)
    d.dtype = FLOAT64 if x.dtype == torch.float64 else FLOAT32
    d.outer, d.n, d.inner = v[0]
    for k in range(3):
        d.a_strides[k] = v[1][k]
        d.b_strides[k] = vb[1][k] if vb is not None else 0
    L = lib()
    wsb = L.tpr_softmax_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    _check(L.tpr_softmax(ctypes.byref(d), ctypes.c_void_p(a.data_ptr()),
                         ctypes.c_void_p(b.data_ptr() if b is not None else 0),
                         ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb,
                         _stream(torch, x.device)))
    return out


def nll_loss(x, target, weight=None, reduction=1, ignore_index=-100):
    """(output, total_weight, status) of tpr_nll_loss on device tensors; status
    is the device int32 out-of-range flag (not synchronised)."""
    import torch
    n, c = x.shape
    out = torch.empty((n,) if reduction == 0 else (), dtype=torch.float32, device=x.device)
    tw = torch.empty((1,), dtype=torch.float32, device=x.device)
    status = torch.empty((1,), dtype=torch.int32, device=x.device)
    L = lib()
    wsb = L.tpr_nll_loss_workspace_bytes(n)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    _check(L.tpr_nll_loss(ctypes.c_void_p(x.data_ptr()), FLOAT32, n, c, x.stride(0), x.stride(1),
                          ctypes.c_void_p(target.data_ptr()), target.stride(0),
                          ctypes.c_void_p(weight.data_ptr() if weight is not None else 0), reduction, ignore_index,
                          ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(tw.data_ptr()),
                          ctypes.c_void_p(status.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb,
                          _stream(torch, x.device)))
    return out, tw, status


def nll_loss_backward(grad, target, n, c, weight=None, reduction=1, ignore_index=-100, total_weight=None,
                      device=None):
    """Dense [n, c] grad_input of tpr_nll_loss_backward."""
    import torch
    gi = torch.empty((n, c), dtype=torch.float32, device=device or grad.device)
    g = grad.reshape(-1)
    _check(lib().tpr_nll_loss_backward(ctypes.c_void_p(g.data_ptr()), g.stride(0) if g.numel() else 1,
                                       ctypes.c_void_p(target.data_ptr()), target.stride(0),
                                       ctypes.c_void_p(weight.data_ptr() if weight is not None else 0),
                                       ctypes.c_void_p(total_weight.data_ptr() if total_weight is not None else 0),
                                       n, c, reduction, ignore_index, ctypes.c_void_p(gi.data_ptr()),
                                       _stream(torch, gi.device)))
    return gi


def reduce_backward(grad, x, op, dims=None, correction=1, result=None, count_override=0):
    """Gradient of reduce(x, op, dims) for op in sum / mean / var / std given the
    output gradient `grad` (dense over the kept dims) and, for std, the forward
    result.  Returns a dense tensor of x's shape."""
    import torch
    nd = x.dim()
    rd = list(range(nd)) if dims is None else sorted(set((d + nd) if d < 0 else d for d in dims))
    desc = make_desc(op, list(x.shape), list(x.stride()), rd, FLOAT32, correction, count_override)
    gi = torch.empty(list(x.shape), dtype=torch.float32, device=x.device)
    g = grad.contiguous()
    r = result.contiguous() if result is not None else None
    L = lib()
    wsb = L.tpr_reduce_backward_workspace_bytes(ctypes.byref(desc))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    _check(L.tpr_reduce_backward(ctypes.byref(desc), ctypes.c_void_p(g.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                 ctypes.c_void_p(r.data_ptr() if r is not None else 0),
                                 ctypes.c_void_p(gi.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb,
                                 _stream(torch, x.device)))
    return gi


def sample(logits2d, uniforms, k, temperature=1.0, top_p=1.0):
    """One token id per row of a 2-D float32 device tensor (unit inner stride)
    through tpr_sample; uniforms: float32 device tensor [rows] in [0, 1)."""
    import torch
    rows, cols = logits2d.shape
    out = torch.empty((rows,), dtype=torch.int64, device=logits2d.device)
    L = lib()
    wsb = L.tpr_sample_workspace_bytes(FLOAT32, rows, cols, k)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=logits2d.device)
    u = uniforms.contiguous()
    _check(L.tpr_sample(ctypes.c_void_p(logits2d.data_ptr()), FLOAT32, rows, cols, logits2d.stride(0), k,
                        float(temperature), float(top_p), ctypes.c_void_p(u.data_ptr()),
                        ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb,
                        _stream(torch, logits2d.device)))
    return out
