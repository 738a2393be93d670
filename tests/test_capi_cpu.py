"""CPU-side checks of the C-ABI library: it loads, exports every function
declared in include/*.h, and validates arguments on the host without a GPU."""
import ctypes
import glob
import os
import re

import pytest

from tensorplay_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        for m in re.finditer(r"\b(tpr_[a-z_0-9]+)\s*\(", txt):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    declared = _declared_functions()
    assert declared == set(_capi.EXPORTED)
    dev = ctypes.CDLL(_capi.DEV_LIB_PATH)
    for name in declared:
        assert hasattr(dev, name), name
    # the shipped library: every entry point but the test build's hooks
    rel = ctypes.CDLL(_capi.LIB_PATH)
    for name in declared - _capi.TEST_BUILD_ONLY:
        assert hasattr(rel, name), name
    for name in _capi.TEST_BUILD_ONLY:
        assert not hasattr(rel, name), name


def test_release_build_has_no_plan_state():
    """The shipped library exports no tpr_debug_set and no knob symbols."""
    import subprocess
    syms = subprocess.run(["nm", "-D", "--defined-only", _capi.LIB_PATH], capture_output=True, text=True,
                          check=True).stdout
    assert "tpr_debug_set" not in syms and "tpr_debug_get" not in syms
    assert "knobs" not in syms
    dsyms = subprocess.run(["nm", "-D", "--defined-only", _capi.DEV_LIB_PATH], capture_output=True, text=True,
                           check=True).stdout
    assert "tpr_debug_set" in dsyms and "tpr_debug_get" in dsyms


def test_abi_version():
    assert _capi.lib().tpr_abi_version() >> 16 == 1


def test_descriptor_layout_matches_header():
    # int32 x4, int64[8] x2, uint32, int32, int64 x2
    assert ctypes.sizeof(_capi.ReduceDesc) == 16 + 128 + 8 + 16 + 8


def test_noalloc_rejects_plans_beyond_the_scratch_without_gpu():
    L = _capi.lib()
    # var over rows of 2^31 elements, 2^20 rows: 3 chunks x 2^20 rows x 24-byte states > 8 MiB
    n = (1 << 31) + 5
    d = _capi.make_desc("var", [1 << 20, n], [n, 1], [1], _capi.FLOAT32)
    need = L.tpr_reduce_workspace_bytes(ctypes.byref(d))
    assert need > _capi.REDUCE_SCRATCH_BYTES
    assert L.tpr_reduce_noalloc(ctypes.byref(d), None, None, None) == _capi.ERR_WORKSPACE
    assert b"scratch" in L.tpr_last_error()
    # an invalid descriptor is reported as by tpr_reduce
    d = _capi.make_desc("sum", [4, 4], [4, 1], [1], _capi.FLOAT32)
    d.in_dtype = 99
    assert L.tpr_reduce_noalloc(ctypes.byref(d), None, None, None) == _capi.ERR_UNSUPPORTED_DTYPE


def test_argument_validation_without_gpu():
    L = _capi.lib()
    d = _capi.make_desc("sum", [4, 4], [4, 1], [1], _capi.FLOAT32)
    d.in_dtype = _capi.INT32
    rc = L.tpr_reduce(ctypes.byref(d), None, None, None, 0, None)
    assert rc == _capi.ERR_UNSUPPORTED_DTYPE  # integral sums write Int64
    assert b"int64" in L.tpr_last_error()
    d = _capi.make_desc("var", [4, 4], [4, 1], [1], _capi.FLOAT32)
    d.in_dtype = _capi.INT32
    assert L.tpr_reduce(ctypes.byref(d), None, None, None, 0, None) == _capi.ERR_UNSUPPORTED_DTYPE
    assert b"float32" in L.tpr_last_error()
    # median of an integer input writes the input dtype (workspace for the radix passes)
    d = _capi.make_desc("median", [4, 4], [4, 1], [0, 1], _capi.INT32, in_dtype=_capi.INT32)
    assert L.tpr_reduce_workspace_bytes(ctypes.byref(d)) > 0
    d.out_dtype = _capi.FLOAT32
    assert L.tpr_reduce(ctypes.byref(d), None, None, None, 0, None) == _capi.ERR_INVALID_ARG
    d = _capi.make_desc("sum", [4, 4], [4, 1], [1], _capi.FLOAT32)
    d.in_dtype = 99
    assert L.tpr_reduce(ctypes.byref(d), None, None, None, 0, None) == _capi.ERR_UNSUPPORTED_DTYPE
    d = _capi.make_desc("argmax", [4, 4], [4, 1], [1], _capi.FLOAT32)
    assert L.tpr_reduce(ctypes.byref(d), None, None, None, 0, None) == _capi.ERR_INVALID_ARG
    rc = L.tpr_topk(None, _capi.FLOAT32, 2, 5, 5, 6, 1, 1, None, None, None, 0, None)
    assert rc == _capi.ERR_INVALID_ARG and b"k out of range" in L.tpr_last_error()
    rc = L.tpr_topk(None, 77, 2, 5, 5, 1, 1, 1, None, None, None, 0, None)
    assert rc == _capi.ERR_UNSUPPORTED_DTYPE  # every tpr_dtype is served; unknown codes are not
    rc = L.tpr_topk(None, _capi.FLOAT64, 2, 5, 5, 1, 1, 1, None, None, None, 0, None)
    assert rc == _capi.ERR_INVALID_ARG  # float64 is served: the null input is the error
    assert L.tpr_topk_workspace_bytes(_capi.INT64, 4, 10000, 2000) == 0          # 2048 composites in LDS
    assert L.tpr_topk_workspace_bytes(_capi.INT64, 4, 10000, 3000) == 4 * 4096 * 16  # sorted in the workspace
    assert L.tpr_topk_workspace_bytes(_capi.INT32, 4, 10000, 3000) == 0          # rows held in registers
    assert L.tpr_topk_workspace_bytes(_capi.FLOAT32, 4, 32768, 20000) == 0       # rows held in registers
    assert L.tpr_topk_workspace_bytes(_capi.INT32, 4, 40000, 3000) == 0          # streaming: 4096 in LDS
    assert L.tpr_topk_workspace_bytes(_capi.INT32, 4, 40000, 5000) == 4 * 8192 * 8  # streaming: workspace sort
    # sampling: k <= 1024 draws inside top-k; larger k adds the sorted values
    # and indices after top-k's own workspace (256-byte aligned parts)
    assert L.tpr_sample_workspace_bytes(_capi.FLOAT32, 4, 40000, 1024) == L.tpr_topk_workspace_bytes(
        _capi.FLOAT32, 4, 40000, 1024)
    tws = L.tpr_topk_workspace_bytes(_capi.FLOAT32, 4, 40000, 5000)
    assert tws == 4 * 8192 * 8
    assert L.tpr_sample_workspace_bytes(_capi.FLOAT32, 4, 40000, 5000) == tws + 80128 + 4 * 5000 * 8
    assert L.tpr_sample_workspace_bytes(_capi.FLOAT32, 3, 2000, 2000) == 24064 + 3 * 2000 * 8  # top-k needs none here
    with pytest.raises(_capi.TprError):
        _capi.debug_set("no_such_knob", 1)
    d = _capi.make_desc("sum", [4], [1], [0], _capi.FLOAT32)
    d.ndim = 9
    assert L.tpr_reduce(ctypes.byref(d), None, None, None, 0, None) == _capi.ERR_INVALID_ARG


def test_empty_output_is_a_no_op_without_gpu():
    L = _capi.lib()
    d = _capi.make_desc("sum", [0, 4], [4, 1], [1], _capi.FLOAT32)
    assert L.tpr_reduce(ctypes.byref(d), None, None, None, 0, None) == _capi.OK
    assert L.tpr_topk(None, _capi.FLOAT32, 3, 5, 5, 0, 1, 1, None, None, None, 0, None) == _capi.OK


def test_softmax_loss_validation_without_gpu():
    L = _capi.lib()
    assert ctypes.sizeof(_capi.SoftmaxDesc) == 8 + 24 + 48
    d = _capi.SoftmaxDesc()
    d.mode, d.dtype, d.outer, d.n, d.inner = 0, _capi.INT32, 2, 3, 1
    assert L.tpr_softmax(ctypes.byref(d), None, None, None, None, 0, None) == _capi.ERR_UNSUPPORTED_DTYPE
    d.dtype = _capi.FLOAT64  # float64 is served: a null pointer is the error now
    assert L.tpr_softmax(ctypes.byref(d), None, None, None, None, 0, None) == _capi.ERR_INVALID_ARG
    assert L.tpr_softmax_workspace_bytes(ctypes.byref(d)) == 0
    d.dtype, d.mode = _capi.FLOAT32, 7
    assert L.tpr_softmax(ctypes.byref(d), None, None, None, None, 0, None) == _capi.ERR_INVALID_ARG
    d.mode, d.n = _capi.SOFTMAX_FWD, 0
    assert L.tpr_softmax(ctypes.byref(d), None, None, None, None, 0, None) == _capi.OK  # empty: no launch
    d.n, d.mode = 3, _capi.SOFTMAX_BWD
    assert L.tpr_softmax(ctypes.byref(d), 16, None, 16, None, 0, None) == _capi.ERR_INVALID_ARG  # y missing
    d.mode, d.outer, d.n, d.inner = _capi.SOFTMAX_FWD, 64, 151936, 1
    d.a_strides[0], d.a_strides[1] = 151936, 1
    assert L.tpr_softmax_workspace_bytes(ctypes.byref(d)) == 64 * 19 * 8    # few long rows: split
    assert L.tpr_softmax(ctypes.byref(d), 16, None, 16, None, 0, None) == _capi.ERR_WORKSPACE
    d.outer = 4096
    assert L.tpr_softmax_workspace_bytes(ctypes.byref(d)) == 0              # one workgroup per row
    d.n = 1000
    assert L.tpr_softmax_workspace_bytes(ctypes.byref(d)) == 0              # register-resident rows
    assert L.tpr_nll_loss_workspace_bytes(1) > 0
    args = [None, _capi.FLOAT32, 4, 3, 3, 1, None, 1, None, 3, -100, None, None, None, None, 0, None]
    assert L.tpr_nll_loss(*args) == _capi.ERR_INVALID_ARG and b"reduction" in L.tpr_last_error()
    args[1] = _capi.FLOAT64
    assert L.tpr_nll_loss(*args) == _capi.ERR_UNSUPPORTED_DTYPE
    args[1], args[9] = _capi.FLOAT32, 1
    args[11], args[12], args[6], args[0] = 16, 16, 16, 16
    assert L.tpr_nll_loss(*args) == _capi.ERR_WORKSPACE
    assert L.tpr_nll_loss_backward(None, 1, None, 1, None, None, 0, 5, 1, -100, None, None) == _capi.OK
    assert L.tpr_nll_loss_backward(None, 1, None, 1, None, None, 2, 5, 4, -100, None, None) == _capi.ERR_INVALID_ARG
