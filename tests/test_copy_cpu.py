"""copy_ on the CPU: pins of the oracle's restatement of the reference's
copy_recursive (cpu/CopyKernels.cpp:27-55) and the C-ABI planner's kernel
choice (tpr_copy_plan launches nothing, so it runs without a GPU)."""
import ctypes
import itertools
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from tensorplay_amd import _capi
from tests.copy_util import DTYPES, as_bytes, expected, src_values


def _views(a):
    """(name, view) pairs of a 3-D base array."""
    yield "dense", a
    yield "transpose", a.transpose(0, 2, 1)
    yield "permute", a.transpose(2, 0, 1)
    yield "stepped", a[:, ::2, 1:]
    yield "broadcast", np.broadcast_to(a[:, :1, :], a.shape)


@pytest.mark.parametrize("src,dst", list(itertools.product(DTYPES, DTYPES)))
def test_oracle_copy_matches_numpy_astype(src, dst):
    rng = np.random.default_rng(zlib.crc32(f"{np.dtype(src).str}-{np.dtype(dst).str}".encode()))
    base = src_values(rng, src, dst, (3, 5, 7))
    for name, v in _views(base):
        out = np.empty(v.shape, dst)
        O.copy(out, v)
        np.testing.assert_array_equal(as_bytes(out), as_bytes(expected(v, dst)), err_msg=name)


def test_oracle_copy_into_strided_destination_brute_force():
    rng = np.random.default_rng(5)
    src = rng.standard_normal((4, 6)).astype(np.float32)[:, :3]
    big = np.zeros((6, 9), np.float64)
    dst = big[:4, ::2][:, :3]          # a strided window of a larger destination
    O.copy(dst, src)
    for i in range(4):
        for j in range(3):
            assert big[i, 2 * j] == np.float64(src[i, j])
    # untouched elements stay zero
    mask = np.zeros_like(big, bool)
    mask[:4, 0:6:2] = True
    assert (big[~mask] == 0).all()


def test_oracle_copy_scalar_and_empty():
    s = np.array(3.75, np.float32)
    d = np.array(0, np.int32)
    O.copy(d, s)
    assert int(d) == 3
    e = np.empty((0, 4), np.float32)
    O.copy(np.empty((0, 4), np.int64), e)


def _plan(shape, dst_strides, src_strides, ddt=_capi.FLOAT32, sdt=_capi.FLOAT32):
    d = _capi.make_copy_desc(shape, dst_strides, src_strides, ddt, sdt)
    return _capi.lib().tpr_copy_plan(ctypes.byref(d), ctypes.c_void_p(0), ctypes.c_void_p(0)) & 3


def test_planner_kernel_choice():
    C, R, T, E = _capi.COPY_CONTIG, _capi.COPY_ROWS, _capi.COPY_TILE, _capi.COPY_ELEM
    assert _plan([64, 1024, 1024], [1 << 20, 1024, 1], [1 << 20, 1024, 1]) == C           # dense: one run
    assert _plan([64, 1024, 1024], [1 << 20, 1024, 1], [1 << 20, 1024, 1], _capi.FLOAT64) == C  # cast
    assert _plan([64, 1024, 1024], [1 << 20, 1024, 1], [1 << 20, 1, 1024]) == T           # transpose(1,2)
    assert _plan([1024, 1024, 64], [65536, 64, 1], [1024, 1, 1 << 20]) == T               # permute(1,2,0)
    assert _plan([64, 1024, 512], [1 << 19, 512, 1], [1 << 20, 1024, 1]) == R             # sliced rows
    assert _plan([64, 1024, 8], [8192, 8, 1], [1 << 20, 1024, 1]) == E                    # short rows
    assert _plan([4096, 4096], [4096, 1], [0, 1]) == R                                    # broadcast rows
    assert _plan([4096, 4096], [4096, 1], [1, 0]) == T                                    # broadcast columns
    assert _plan([4096, 4096], [4096, 1], [0, 0]) == E                                    # broadcast scalar
    assert _plan([], [], []) == C                                                         # 0-dim
    bad = _capi.make_copy_desc([2], [1], [1], 99, _capi.FLOAT32)
    assert _capi.lib().tpr_copy_plan(ctypes.byref(bad), None, None) == -1


def test_copy_argument_validation_without_gpu():
    L = _capi.lib()
    d = _capi.make_copy_desc([2, 3], [3, 1], [3, 1], 42, _capi.FLOAT32)
    assert L.tpr_copy(ctypes.byref(d), None, None, None) == _capi.ERR_UNSUPPORTED_DTYPE
    d = _capi.make_copy_desc([2, -1], [3, 1], [3, 1], _capi.FLOAT32, _capi.FLOAT32)
    assert L.tpr_copy(ctypes.byref(d), None, None, None) == _capi.ERR_INVALID_ARG
    d = _capi.make_copy_desc([0, 3], [3, 1], [3, 1], _capi.FLOAT32, _capi.INT8)
    assert L.tpr_copy(ctypes.byref(d), None, None, None) == _capi.OK                      # empty: no launch
    d = _capi.make_copy_desc([2, 3], [3, 1], [3, 1], _capi.FLOAT32, _capi.INT8)
    assert L.tpr_copy(ctypes.byref(d), None, None, None) == _capi.ERR_INVALID_ARG         # null pointers
    assert L.tpr_copy(None, None, None, None) == _capi.ERR_INVALID_ARG


def test_planner_vector_variants():
    def plan(shape, ds, ss, ddt=_capi.FLOAT32, sdt=_capi.FLOAT32, dp=0, sp=0):
        d = _capi.make_copy_desc(shape, ds, ss, ddt, sdt)
        return _capi.lib().tpr_copy_plan(ctypes.byref(d), ctypes.c_void_p(dp), ctypes.c_void_p(sp))
    V = _capi.COPY_VEC
    assert plan([64, 1024, 1024], [1 << 20, 1024, 1], [1 << 20, 1, 1024]) == _capi.COPY_TILE | V
    assert plan([3, 300, 37], [11100, 37, 1], [11100, 1, 300]) == _capi.COPY_TILE          # 37-float rows: scalar
    assert plan([2, 272, 144], [39168, 144, 1], [39168, 1, 272], _capi.UINT8, _capi.UINT8) == _capi.COPY_TILE | V
    assert plan([2, 272, 140], [38080, 140, 1], [38080, 1, 272], _capi.UINT8, _capi.UINT8) == _capi.COPY_TILE
    assert plan([2, 272, 144], [39168, 144, 1], [39168, 1, 272], _capi.INT16, _capi.UINT8) == _capi.COPY_TILE | V
    assert plan([1 << 20], [1], [1]) == _capi.COPY_CONTIG | V
    assert plan([1 << 20], [1], [1], sp=4) == _capi.COPY_CONTIG                            # misaligned source
    assert plan([64, 1024, 1024], [1 << 20, 1024, 1], [1 << 20, 1, 1024], sp=8) == _capi.COPY_TILE
    assert plan([40, 300], [700, 1], [300, 1], _capi.FLOAT64) == _capi.COPY_ROWS | V
    assert plan([40, 301], [700, 1], [301, 1], _capi.FLOAT64) == _capi.COPY_ROWS           # odd row pitch
