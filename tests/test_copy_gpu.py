"""GPU parity of tpr_copy (copy_ / contiguous / to(dtype)) against the CPU
oracle's restatement of the reference's copy_recursive
(cpu/CopyKernels.cpp:27-55): bit-exact on the whole destination buffer,
untouched elements included, for all 121 dtype pairs and every kernel the
planner picks (dense run, rows, LDS tiles, per element)."""
import ctypes
import itertools
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from tensorplay_amd import _capi
from tests.copy_util import DTYPES, as_bytes, src_values

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

C, R, T, E = _capi.COPY_CONTIG, _capi.COPY_ROWS, _capi.COPY_TILE, _capi.COPY_ELEM


def _geom(view, base):
    off = view.__array_interface__["data"][0] - base.__array_interface__["data"][0]
    assert off % view.itemsize == 0
    return off, [s // view.itemsize for s in view.strides]


def gpu_copy(dst_base, dst_view, src_base, src_view, expect_kind=None):
    """Runs tpr_copy on device copies of the two base buffers with the views'
    geometry; returns the device result of the whole destination base."""
    print(f"case copy {src_view.dtype}{src_view.shape}{src_view.strides} -> "
          f"{dst_view.dtype}{dst_view.strides}", flush=True)
    sb = torch.from_numpy(np.ascontiguousarray(src_base).view(np.uint8).reshape(-1)).cuda()
    db = torch.from_numpy(np.ascontiguousarray(dst_base).view(np.uint8).reshape(-1).copy()).cuda()
    soff, sst = _geom(src_view, src_base)
    doff, dst_ = _geom(dst_view, dst_base)
    d = _capi.make_copy_desc(list(dst_view.shape), dst_, sst, O.DTYPE_CODES[dst_view.dtype],
                             O.DTYPE_CODES[src_view.dtype])
    sp, dp = ctypes.c_void_p(sb.data_ptr() + soff), ctypes.c_void_p(db.data_ptr() + doff)
    if expect_kind is not None:
        assert _capi.lib().tpr_copy_plan(ctypes.byref(d), dp, sp) & (3 if expect_kind < 4 else 7) == expect_kind
    rc = _capi.lib().tpr_copy(ctypes.byref(d), dp, sp, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, _capi.lib().tpr_last_error()
    return db.cpu().numpy()


def check(src_base, src_view, dst_dtype, dst_base=None, dst_view=None, expect_kind=None):
    if dst_base is None:
        dst_base = np.zeros(src_view.shape, dst_dtype)
        dst_view = dst_base
    got = gpu_copy(dst_base, dst_view, src_base, src_view, expect_kind)
    ref_base = dst_base.copy()
    # the oracle writes through the same view of its own copy of the destination base
    off = _geom(dst_view, dst_base)[0] // dst_base.itemsize
    ro = np.lib.stride_tricks.as_strided(ref_base.reshape(-1)[off:], dst_view.shape, dst_view.strides)
    O.copy(ro, src_view)
    np.testing.assert_array_equal(got, as_bytes(ref_base))


def _layouts(a):
    yield "dense", a, C
    yield "transpose", a.transpose(0, 2, 1), T
    yield "permute", a.transpose(2, 0, 1), T
    yield "stepped", a[:, ::2, ::3], E
    yield "broadcast", np.broadcast_to(a[:1], a.shape), R
    yield "misaligned-rows", a[:, 1:, 1:], R


@pytest.mark.parametrize("src", DTYPES, ids=lambda d: np.dtype(d).name)
def test_all_dtype_pairs_all_kernels(src):
    for dst in DTYPES:
        rng = np.random.default_rng(zlib.crc32(f"{np.dtype(src).str}-{np.dtype(dst).str}".encode()))
        base = src_values(rng, src, dst, (3, 37, 300))
        for name, v, kind in _layouts(base):
            check(base, v, dst, expect_kind=kind)


@pytest.mark.parametrize("src", DTYPES, ids=lambda d: np.dtype(d).name)
def test_vector_tiles_full_and_edge(src):
    """Transposes whose rows are 16-byte multiples on both sides take the
    vector tile kernel; 144 x 272 leaves partial edge tiles in both dims."""
    for dst in DTYPES:
        rng = np.random.default_rng(zlib.crc32(f"vt-{np.dtype(src).str}-{np.dtype(dst).str}".encode()))
        base = src_values(rng, src, dst, (2, 144, 272))
        t = base.transpose(0, 2, 1)
        vec_ok = 144 % (16 // np.dtype(dst).itemsize) == 0
        check(base, t, dst, expect_kind=T | (_capi.COPY_VEC if vec_ok else 0))
        p = base.transpose(2, 0, 1)   # permute: I = merged (2*144), J = 272
        check(base, p, dst, expect_kind=T | (_capi.COPY_VEC if vec_ok else 0))
        # I = 96 < 128: 4-byte pairs take 64 x 64 tiles instead of 128 x 64
        base = src_values(rng, src, dst, (3, 96, 208))
        vec_ok = 96 % (16 // np.dtype(dst).itemsize) == 0
        check(base, base.transpose(0, 2, 1), dst, expect_kind=T | (_capi.COPY_VEC if vec_ok else 0))


def test_ragged_and_tail_shapes():
    rng = np.random.default_rng(7)
    for shape in [(1,), (3,), (17,), (1000003,), (5, 255), (2, 257), (70, 65), (9, 16, 17), (2, 3, 4, 5, 6, 7)]:
        for src, dst in [(np.float32, np.float32), (np.float32, np.float64), (np.int8, np.int64),
                         (np.float64, np.float32), (np.uint8, np.float32), (np.int64, np.int16)]:
            a = src_values(rng, src, dst, shape)
            check(a, a, dst)
            if a.ndim >= 2:
                t = np.swapaxes(a, -1, -2)
                check(a, t, dst)


def test_destination_views():
    """copy_ into a strided / transposed window of a larger destination."""
    rng = np.random.default_rng(8)
    src = src_values(rng, np.float32, np.float64, (40, 300))
    big = np.full((120, 700), -1.0, np.float64)
    check(src, src, np.float64, big, big[10:50, 100:400], expect_kind=R)
    bigT = np.full((700, 120), -1.0, np.float64)
    check(src, src, np.float64, bigT, bigT[100:400, 10:50].T, expect_kind=T)
    check(src, src.T, np.float64, bigT, bigT[100:400, 10:50], expect_kind=None)
    big8 = np.zeros((90, 90, 4), np.int8)
    s8 = src_values(rng, np.float32, np.int8, (90, 90))
    check(s8, s8, np.int8, big8, big8[:, :, 2], expect_kind=E)


def test_scalar_and_empty():
    s = np.array(-2.5, np.float32)
    check(s, s, np.int32, expect_kind=C)
    e = np.zeros((0, 5), np.float32)
    d = _capi.make_copy_desc([0, 5], [5, 1], [5, 1], _capi.INT8, _capi.FLOAT32)
    assert _capi.lib().tpr_copy(ctypes.byref(d), None, None, None) == 0
    del e


def test_full_size_permutes_match_numpy():
    """BASELINE C2 geometry [64,1024,1024]: the CUDA argmax path's
    permute-to-last copy (ReductionKernels.cu:67-75) and a transpose, against
    numpy's own dense copy of the same views (bit-exact, a closed form)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    x = torch.randn((64, 1024, 1024), generator=g, device="cuda")
    xn = x.cpu().numpy()
    for perm, kind in (((1, 2, 0), T), ((0, 2, 1), T)):
        v = x.permute(*perm)
        out = torch.empty(v.shape, device="cuda")
        assert _capi.copy_plan(out, v) == kind | _capi.COPY_VEC
        _capi.copy_(out, v)
        np.testing.assert_array_equal(out.cpu().numpy(), np.ascontiguousarray(xn.transpose(perm)))
    # casts of the dense tensor: float32 -> float64 is exact
    o64 = torch.empty(x.shape, dtype=torch.float64, device="cuda")
    _capi.copy_(o64, x)
    assert torch.equal(o64.cpu(), x.cpu().double())
    # the dense clone (nontemporal accesses from 64 MiB)
    oc = torch.empty_like(x)
    assert _capi.copy_plan(oc, x) == C | _capi.COPY_VEC
    _capi.copy_(oc, x)
    assert torch.equal(oc, x)


def test_large_same_type_copies_other_widths():
    """Copies of 64 MiB or more between equal dtypes take nontemporal loads and
    stores: 1-, 2- and 8-byte tiles and dense runs, bit-exact against numpy."""
    rng = np.random.default_rng(12)
    cases = [(np.uint8, (64, 1024, 1024), (0, 2, 1)), (np.int16, (32, 1024, 1024), (1, 2, 0)),
             (np.int64, (16, 1024, 1024), (0, 2, 1)), (np.float64, (8, 1024, 1024), None)]
    for dt, shape, perm in cases:
        xn = rng.integers(-100, 100, size=shape).astype(dt)
        x = torch.from_numpy(xn).cuda()
        v = x if perm is None else x.permute(*perm)
        print(f"case large copy {np.dtype(dt).name} {shape} perm={perm}", flush=True)
        out = torch.empty(v.shape, dtype=x.dtype, device="cuda")
        _capi.copy_(out, v)
        ref = xn if perm is None else np.ascontiguousarray(xn.transpose(perm))
        np.testing.assert_array_equal(out.cpu().numpy(), ref)
        del x, v, out
