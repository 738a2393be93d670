"""GPU parity of tpr_reduce (via the C-ABI) against the CPU oracle.

  * amax/amin/argmax/argmin: bit-exact against the oracle (the reference CPU
    semantics: strict compare, first index wins, NaN ignored).  argmax over a
    non-last dim follows the permute layout (CUDA path, ReductionKernels.cu:67-75),
    i.e. oracle quirk=0.
  * sum/mean/var/std: max relative error <= 1e-5 against an fp64 host reference
    (numpy float64); the CPU oracle's own error is measured beside it.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from tensorplay_amd import _capi
from tests.gpu_util import assert_bits_equal, assert_close_rel, device_view, fp64_reference, rel_err

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(autouse=True)
def _reset_knobs():
    yield
    for k in ("splits", "lanes", "general", "tx", "unroll", "colblock", "nt", "rowreg"):
        _capi.debug_set(k, 0)


def gpu(t, op, dims, correction=1, p=2.0):
    out = _capi.reduce(t, op, dims, correction=correction, p=p)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(v, t, op, dims, correction=1, p=2.0):
    """Compare one reduction of the numpy view v / torch view t."""
    print(f"case op={op} shape={v.shape} strides={v.strides} dims={dims} p={p}", flush=True)
    got = gpu(t, op, dims, correction, p)
    full = dims is None or len(dims) == v.ndim
    if op in ("all", "any"):
        f = O.all_ if op == "all" else O.any_
        exp = f(v) if full else f(v, list(dims))
        np.testing.assert_array_equal(got.reshape(np.shape(exp)), exp)
    elif op == "median":
        assert_bits_equal(got.reshape(()), np.float32(O.median(v)))
    elif op == "norm" and np.isinf(p):
        if full and v.size == 0:
            return
        exp = np.float32(O.norm(v, p)) if full else O.norm(v, p, list(dims))
        assert_bits_equal(got.reshape(np.shape(exp)), exp)
    elif op in ("prod", "norm"):
        ref = fp64_reference(v, op, dims, correction, p)
        assert_close_rel(got.reshape(np.shape(ref)), ref)
    elif op in ("amax", "amin"):
        f = O.amax if op == "amax" else O.amin
        if dims is None or len(dims) == v.ndim:
            if v.size == 0:
                return
            exp = np.float32(f(v))
        else:
            exp = f(v, list(dims))
        assert_bits_equal(got.reshape(np.shape(exp)), exp)
    elif op in ("argmax", "argmin"):
        f = O.argmax if op == "argmax" else O.argmin
        if dims is None:
            exp = np.int64(f(v))
            assert int(got.reshape(())) == int(exp)
        else:
            assert_bits_equal(got, f(v, dims[0]))
    else:
        ref = fp64_reference(v, op, dims, correction)
        assert_close_rel(got.reshape(np.shape(ref)), ref)


KNOWN = json.load(open(os.path.join(HERE, "golden", "reference_known_answers.json")))


@pytest.mark.parametrize("case", KNOWN, ids=[c["src"] + ":" + c["op"] for c in KNOWN])
def test_reference_known_answers_on_device(case):
    # test_cuda_reductions.py / test_reduction.py known answers, on the ROCm device
    x = np.array(case["x"], np.float32).reshape(case["shape"])
    t = torch.from_numpy(x).cuda()
    got = gpu(t, case["op"], case.get("dims"))
    exp = case["expect"]
    if isinstance(exp, list):
        np.testing.assert_array_equal(got.ravel(), np.array(exp))
    elif "places" in case:
        assert round(float(got) - exp, case["places"]) == 0
    else:
        assert float(got) == exp


OPS = ["sum", "mean", "amax", "amin", "argmax", "argmin", "var", "std"]


def _views(rng):
    """(base, view) pairs covering the layout classes: rows, cols, general, full."""
    out = []
    for shape in [(7,), (33, 5), (5, 1000), (16, 4096), (3, 17, 129), (4, 8, 6, 5), (2, 3, 1, 64)]:
        b = rng.standard_normal(shape).astype(np.float32)
        out.append((b, b))
    b = rng.standard_normal((40, 64)).astype(np.float32)
    out.append((b, b.T))                 # transposed
    out.append((b, b[:, ::3]))           # stepped inner dim
    out.append((b, b[1:, 1:]))           # misaligned start (not 16B aligned)
    b = rng.standard_normal((6, 10, 12)).astype(np.float32)
    out.append((b, b.transpose(2, 0, 1)))
    out.append((b, b[:, 2:7, :]))
    b = rng.standard_normal(1 << 16).astype(np.float32)
    out.append((b, b[1:]))               # misaligned, odd length
    out.append((b, b[::2]))              # strided full
    return out


def _dim_sets(nd):
    sets = [None]
    for d in range(nd):
        sets.append([d])
    if nd >= 2:
        sets.append([0, nd - 1])
    if nd >= 3:
        sets.append([1, 2])
    return sets


@pytest.mark.parametrize("op", OPS)
def test_random_layouts(op):
    rng = np.random.default_rng(11)
    for base, v in _views(rng):
        t = device_view(torch, base, v)
        for dims in _dim_sets(v.ndim):
            if op in ("argmax", "argmin") and dims is not None and len(dims) > 1:
                continue
            check(v, t, op, dims)


@pytest.mark.parametrize("knob,values", [("general", [1]), ("splits", [1, 2, 3, 7, 64]),
                                         ("lanes", [16, 32, 64, 128, 256, 512, 1024]), ("tx", [64, 128, 256]),
                                         ("unroll", [1, 2, 4]), ("colblock", [256, 512, 1024]),
                                         ("nt", [1, -1])])
def test_forced_plans(knob, values):
    rng = np.random.default_rng(12)
    b = rng.standard_normal((37, 1029)).astype(np.float32)
    c = rng.standard_normal((5, 300, 36)).astype(np.float32)
    for val in values:
        _capi.debug_set(knob, val)
        for op in OPS:
            check(b, torch.from_numpy(b).cuda(), op, [1])
            check(b, torch.from_numpy(b).cuda(), op, None)
            if knob in ("tx", "splits", "unroll", "colblock"):
                d = rng.standard_normal((3, 9, 1030)).astype(np.float32)  # inner not a multiple of 4
                check(d, torch.from_numpy(d).cuda(), op, [1])
                check(d[:, :, 1:], device_view(torch, d, d[:, :, 1:]), op, [0])
            if knob != "lanes":
                check(c, torch.from_numpy(c).cuda(), op, [1])
                check(c, torch.from_numpy(c).cuda(), op, [0])


@pytest.mark.parametrize("rowreg", [0, 1, -1])
def test_var_rows_shifted_two_sums(rowreg):
    """var / std over rows of 1024 / 2048 / 4096 floats take k_rows_reg_var
    (every element shifted by the row's first element, fp64 two-sums); rowreg=1
    forces it for few rows, -1 takes k_rows.  Offsets far from zero, an outlier
    first element, tiny spread, NaN / inf rows, corrections 0-2."""
    rng = np.random.default_rng(23)
    _capi.debug_set("rowreg", rowreg)
    for rows, cols in ((3, 1024), (5, 2048), (2, 4096), (4096, 1024)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        x[0] += np.float32(1e4)                       # large mean, unit spread
        x[1] = np.float32(3.0) + x[1] * np.float32(1e-3)
        if rows > 2:
            x[2, 0] = np.float32(1e6)                 # the shift itself is an outlier
        t = torch.from_numpy(x).cuda()
        for op in ("var", "std"):
            for corr in (0, 1, 2):
                check(x, t, op, [1], correction=corr)
        y = x[:2].copy()
        y[0, 5] = np.nan
        y[1, 7] = np.inf
        g = gpu(torch.from_numpy(y).cuda(), "var", [1])
        assert np.isnan(g).all()


def test_rows_eight_vectors_in_flight():
    """k_rows with 32 lanes and 8 vectors per lane in flight (the planner's pick
    for rows of 1024 floats), forced on other lengths too: tails, partial tiles."""
    rng = np.random.default_rng(22)
    _capi.debug_set("lanes", 32)
    _capi.debug_set("unroll", 8)
    for rows, cols in ((33, 1024), (7, 1028), (5, 2048), (9, 1000), (3, 4100)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        x[0, [3, cols - 1]] = 9.0  # tie: the lowest index wins
        t = torch.from_numpy(x).cuda()
        for op in OPS:
            check(x, t, op, [1])


@pytest.mark.parametrize("rowreg", [1, -1])
def test_register_rows(rowreg):
    """k_rows_reg (zero-identity ops over rows of 65-1024 float4, loads past the
    row end read 0): row lengths 1-8 waves wide with ragged ends, row counts that
    leave the last workgroup partly empty, and a row stride wider than the row."""
    rng = np.random.default_rng(21)
    _capi.debug_set("rowreg", rowreg)
    for rows, cols in ((3, 260), (5, 516), (7, 1028), (9, 2052), (6, 4096), (1, 4092), (513, 2048)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        x[0] = 0.0
        x[0, -1] = -0.5  # any: only the last element of the row is nonzero
        if rows > 1:
            x[1] = 0.0   # any: all-zero row
        t = torch.from_numpy(x).cuda()
        for op in ("sum", "mean", "any"):
            check(x, t, op, [1])
        for p in (1.0, 2.0):
            check(x, t, "norm", [1], p=p)
        w = x[:, : cols - 4]  # rows 16-byte aligned, row stride > row length
        check(w, device_view(torch, x, w), "sum", [1])


def test_special_values():
    x = np.array([[np.nan, -0.0, 0.0, 1.0, 1.0],
                  [np.nan, np.nan, np.nan, np.nan, np.nan],
                  [-np.inf, -np.inf, -np.inf, -np.inf, -np.inf],
                  [0.0, -0.0, 0.0, -0.0, 0.0],
                  [3.0, np.inf, 2.0, np.inf, 1.0]], np.float32)
    t = torch.from_numpy(x).cuda()
    for op in ("amax", "amin", "argmax", "argmin"):
        for dims in ([1], [0], None):
            check(x, t, op, dims)
    # ties across threads: the lowest index wins wherever the equal values sit
    y = np.zeros((3, 5000), np.float32)
    y[0, [17, 4000, 4001]] = 7.0
    y[1, [4999, 256, 1024]] = -7.0
    for op in ("argmax", "argmin", "amax", "amin"):
        check(y, torch.from_numpy(y).cuda(), op, [1])
        check(y, torch.from_numpy(y).cuda(), op, None)


def test_empty_and_degenerate():
    e = np.zeros((0, 4), np.float32)
    t = torch.from_numpy(e).cuda()
    assert gpu(t, "sum", [1]).shape == (0,)
    s = gpu(t, "sum", [0])
    np.testing.assert_array_equal(s, np.zeros(4, np.float32))
    assert np.isnan(gpu(t, "mean", [0])).all()
    assert np.isnan(gpu(t, "var", [0])).all()
    assert (gpu(t, "amax", [0]) == -np.inf).all()
    assert (gpu(t, "argmax", [0]) == 0).all()
    one = np.array([2.5], np.float32)
    to = torch.from_numpy(one).cuda()
    assert np.isnan(gpu(to, "var", None))           # 0/0 as the reference
    assert gpu(to, "var", None, correction=0) == 0.0
    assert gpu(to, "sum", None) == 2.5


def test_mean_var_count_override_duplicates():
    # reference divides by the product over the listed dims, duplicates included
    x = np.random.default_rng(13).standard_normal((6, 9)).astype(np.float32)
    t = torch.from_numpy(x).cuda()
    m = _capi.reduce(t, "mean", [1], count_override=81).cpu().numpy()
    np.testing.assert_allclose(m, x.astype(np.float64).sum(1) / 81, rtol=1e-5)
    v = _capi.reduce(t, "var", [1], count_override=81).cpu().numpy()
    np.testing.assert_allclose(v, O.var(x, [1, 1]), rtol=1e-4)


# ---- BASELINE configurations at full size ---------------------------------------
def test_config1_sum_lastdim():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4096, 4096), dtype=np.float32)
    t = torch.from_numpy(x).cuda()
    got = gpu(t, "sum", [-1])
    ref = x.astype(np.float64).sum(1)
    e_gpu = assert_close_rel(got, ref)
    e_cpu = rel_err(O.sum(x, [-1]), ref)
    print(f"C1 sum dim=-1: gpu rel err {e_gpu:.2e}, reference-CPU-path rel err {e_cpu:.2e}")


def test_config2_strided():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 1024, 1024), dtype=np.float32)
    t = torch.from_numpy(x).cuda()
    got = gpu(t, "mean", [1])
    ref = x.astype(np.float64).mean(1)
    assert_close_rel(got, ref)
    print(f"C2 mean dim=1 cpu-path err {rel_err(O.mean(x, [1]), ref):.2e}")
    assert_bits_equal(gpu(t, "amax", [0]), O.amax(x, [0]))
    assert_bits_equal(gpu(t, "argmax", [0]), O.argmax(x, 0))
    for op in ("var", "std"):
        got = gpu(t, op, [-1])
        ref = fp64_reference(x, op, [2])
        assert_close_rel(got, ref)
        f = O.var if op == "var" else O.std
        print(f"C2 {op} dim=-1 cpu-path err {rel_err(f(x, [-1]), ref):.2e}")


def test_config4_full_tensor():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(1 << 28, dtype=np.float32) * np.float32(2.0) + np.float32(0.5))
    t = torch.from_numpy(x).cuda()
    x64 = x.astype(np.float64)
    s64 = x64.sum()
    assert_close_rel(gpu(t, "sum", None), s64)
    assert_close_rel(gpu(t, "mean", None), s64 / x.size)
    assert_bits_equal(gpu(t, "amax", None).reshape(()), np.float32(O.amax(x)))
    assert int(gpu(t, "argmax", None)) == int(O.argmax(x))
    v64 = x64.var(ddof=1)
    del x64
    assert_close_rel(gpu(t, "var", None), v64)
    assert_close_rel(gpu(t, "std", None), np.sqrt(v64))


def test_config5_argmax_logits():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((256, 151936), dtype=np.float32) * np.float32(3.0)
    for r in range(256):
        x[r, rng.choice(151936, 8, replace=False)] += np.float32(15.0)
    t = torch.from_numpy(x).cuda()
    assert_bits_equal(gpu(t, "argmax", [-1]), O.argmax(x, -1))


def test_few_long_rows():
    """Few long rows run one row per 512/1024-thread workgroup (no split)."""
    rng = np.random.default_rng(13)
    for rows, cols in ((3, 70001), (64, 151936), (1, 1 << 20)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        x[0, [5, cols - 1]] = 9.0  # tie far apart: lowest index wins
        t = torch.from_numpy(x).cuda()
        for op in OPS:
            check(x, t, op, [1])


# ---- prod / norm / all / any / median ----

NEW_OPS = [("prod", 2.0), ("all", 2.0), ("any", 2.0), ("norm", 2.0), ("norm", 1.0), ("norm", 3.0),
           ("norm", 0.5), ("norm", float("inf")), ("norm", float("-inf"))]


@pytest.mark.parametrize("op,p", NEW_OPS, ids=[f"{o}{p}" for o, p in NEW_OPS])
def test_new_ops_random_layouts(op, p):
    rng = np.random.default_rng(14)
    for base, v in _views(rng):
        if op == "prod":  # keep products representable: values near 1
            base[...] = rng.uniform(0.99, 1.01, size=base.shape).astype(np.float32)
        if op in ("all", "any"):  # plenty of exact zeros
            base[...] = np.where(rng.random(base.shape) < 0.3, np.float32(0.0), base)
        t = device_view(torch, base, v)
        for dims in _dim_sets(v.ndim):
            check(v, t, op, dims, p=p)


@pytest.mark.parametrize("knob,values", [("general", [1]), ("splits", [1, 3, 64]), ("lanes", [16, 256, 1024]),
                                         ("tx", [64, 256]), ("nt", [1])])
def test_new_ops_forced_plans(knob, values):
    rng = np.random.default_rng(15)
    b = rng.uniform(0.99, 1.01, size=(37, 1029)).astype(np.float32)
    b[5, 7] = 0.0
    b[9] = 0.0
    c = rng.uniform(0.99, 1.01, size=(5, 300, 36)).astype(np.float32)
    c[2, :, 3] = 0.0
    for val in values:
        _capi.debug_set(knob, val)
        for op, p in NEW_OPS:
            check(b, torch.from_numpy(b).cuda(), op, [1], p=p)
            check(b, torch.from_numpy(b).cuda(), op, None, p=p)
            check(c, torch.from_numpy(c).cuda(), op, [1], p=p)
            check(c, torch.from_numpy(c).cuda(), op, [0], p=p)


def test_new_ops_special_values():
    x = np.array([[np.nan, -0.0, 0.0, 1.0, 1.0],
                  [np.nan, np.nan, np.nan, np.nan, np.nan],
                  [0.0, -0.0, 0.0, -0.0, 0.0],
                  [3.0, -np.inf, 2.0, np.inf, 1.0]], np.float32)
    t = torch.from_numpy(x).cuda()
    for op in ("all", "any"):
        for dims in ([1], [0], None):
            check(x, t, op, dims)
    for p in (float("inf"), float("-inf")):
        for dims in ([1], [0], None):
            check(x, t, op="norm", dims=dims, p=p)
    # norm p=0: |x|^0 = 1 for every element, sum n, n^(1/0) = inf (the reference composite)
    z = np.array([[0.0, 2.0, 0.0]], np.float32)
    got = gpu(torch.from_numpy(z).cuda(), "norm", None, p=0.0)
    assert np.isinf(got) and got > 0
    # empty extents: prod 1, all true, any false, norm 0
    e = torch.zeros((0, 3), device="cuda")
    assert (gpu(e, "prod", [0]) == 1).all()
    assert gpu(e, "all", [0]).all() and not gpu(e, "any", [0]).any()
    assert (gpu(e, "norm", [0]) == 0).all()


@pytest.mark.parametrize("n", [1, 2, 3, 1000, 1001, 4096 + 3, 1 << 20, (1 << 22) + 5])
def test_median_sizes(n):
    rng = np.random.default_rng(16 + n % 97)
    x = rng.standard_normal(n).astype(np.float32)
    check(x, torch.from_numpy(x).cuda(), "median", None)
    # heavy ties and a misaligned start
    y = rng.integers(-3, 4, size=n + 1).astype(np.float32)
    check(y[1:], device_view(torch, y, y[1:]), "median", None)


@pytest.mark.parametrize("dt", ["float64", "int8", "uint8", "int16", "uint16", "int32", "uint32", "int64", "uint64",
                                "bool"])
def test_median_other_dtypes(dt):
    # median of every other dtype (radix select on the element width's key):
    # the lower median, bit-exact against numpy's sort, in the input dtype
    rng = np.random.default_rng(23)
    for n in (1, 2, 7, 1000, 4097, 100003):
        if dt == "bool":
            x = rng.random(n) < 0.4
        elif dt == "float64":
            x = rng.standard_normal(n) * 1e3
            x[: n // 7] = np.round(x[: n // 7])  # ties
            if n > 3:
                x[1], x[2] = -0.0, 0.0
        else:
            info = np.iinfo(dt)
            lo, hi = int(info.min), int(info.max)
            if dt == "uint64":
                x = rng.integers(0, hi, size=n, dtype=np.uint64, endpoint=True)
            elif dt == "int64":
                x = rng.integers(lo, hi, size=n, dtype=np.int64, endpoint=True)
            else:
                x = rng.integers(lo, hi + 1, size=n).astype(dt)
            x[: n // 5] = x[0]  # duplicates
        print(f"case median dtype={dt} n={n}", flush=True)
        got = _capi.reduce(torch.from_numpy(x).cuda(), "median", None).cpu().numpy()
        exp = np.sort(x, kind="stable")[(n - 1) // 2]
        assert got.dtype == x.dtype
        if dt == "float64" and exp == 0:
            assert float(got) == 0.0 and not np.signbit(got)  # a zero median comes back as +0.0
        else:
            assert_bits_equal(np.asarray(got).reshape(()), np.asarray(exp).reshape(()))


def test_median_special_values():
    x = np.array([np.nan, 1.0, np.nan, -np.inf, 2.0, -0.0, 0.0, np.inf, np.nan], np.float32)
    for k in range(1, len(x) + 1):
        v = np.ascontiguousarray(x[:k])
        check(v, torch.from_numpy(v).cuda(), "median", None)
    z = np.full(5, -0.0, np.float32)
    got = gpu(torch.from_numpy(z).cuda(), "median", None)
    assert got == 0.0 and not np.signbit(got)
    assert np.isnan(gpu(torch.zeros(0, device="cuda"), "median", None))
    m = torch.from_numpy(np.arange(24, dtype=np.float32).reshape(2, 3, 4)).cuda()
    check(m.cpu().numpy(), m, "median", None)
    with pytest.raises(_capi.TprError):  # strided views must be made dense first
        _capi.reduce(m[:, :, ::2], "median", None)
    with pytest.raises(_capi.TprError):  # full reductions only
        _capi.reduce(m, "median", [1])


def test_median_special_values_float64():
    # float64 keys: NaN ranks above every number (as numpy's sort places it),
    # +-inf at the ends, -0.0 == +0.0 with a zero median returned as +0.0
    x = np.array([np.nan, 1.0, np.nan, -np.inf, 2.0, -0.0, 0.0, np.inf, np.nan, -5e-324, 5e-324], np.float64)
    rng = np.random.default_rng(24)
    for k in range(1, len(x) + 1):
        for v in (np.ascontiguousarray(x[:k]), rng.permutation(x[:k])):
            print(f"case median float64 special n={k}", flush=True)
            got = np.asarray(_capi.reduce(torch.from_numpy(v).cuda(), "median", None).cpu().numpy()).reshape(())
            exp = np.sort(v)[(k - 1) // 2]
            if np.isnan(exp):
                assert np.isnan(got)
            elif exp == 0:
                assert float(got) == 0.0 and not np.signbit(got)
            else:
                assert_bits_equal(got, np.asarray(exp).reshape(()))


def test_new_ops_config_shapes():
    # the headline shape through the new ops (sizes the tests run in seconds)
    rng = np.random.default_rng(17)
    x = rng.uniform(0.999, 1.001, size=(64, 1024, 1024)).astype(np.float32)
    t = torch.from_numpy(x).cuda()
    check(x, t, "prod", [1])
    check(x, t, "norm", [2], p=2.0)
    check(x, t, "norm", [0], p=float("inf"))
    check(x, t, "any", [0])



# ---- integer and bool inputs ----
# Integer reductions are exact and order-independent (Int64 wrap-around sums
# and products; mean is a float sum of the fp32-converted values, within
# the float tolerance, strict-compare max/min/argmax with the first index, x != 0 for
# all/any), so numpy's own reductions are their closed forms: bit-exact.

INT_DTYPES = ["int32", "int64", "uint8", "int8", "int16", "uint16", "uint32", "uint64", "bool"]
INT_OPS = ["sum", "prod", "mean", "amax", "amin", "argmax", "argmin", "all", "any"]


def _np_int_ref(v, op, dims):
    ax = None if dims is None else tuple(dims)
    if op == "sum":
        return v.astype(np.int64).sum(axis=ax)
    if op == "prod":
        return v.astype(np.int64).prod(axis=ax)
    if op == "mean":  # the reference converts to Float32 before summing
        return v.astype(np.float32).astype(np.float64).mean(axis=ax)
    if op in ("amax", "amin"):
        if v.size == 0:
            return None
        return (np.max if op == "amax" else np.min)(v, axis=ax)
    if op in ("argmax", "argmin"):
        f = np.argmax if op == "argmax" else np.argmin
        if dims is None:
            return np.int64(f(v.ravel()))
        return f(v, axis=dims[0]).astype(np.int64)
    if op == "all":
        return (v != 0).all(axis=ax)
    return (v != 0).any(axis=ax)


def _int_view_data(rng, dt, shape):
    if dt == "bool":
        return rng.random(shape) < 0.7
    info = np.iinfo(dt)
    if dt in ("int32", "int64"):
        b = rng.integers(-5, 6, size=shape).astype(dt)  # ties for argmax
        big = rng.integers(info.min // 2, info.max // 2, size=shape, dtype=dt)
        return np.where(rng.random(shape) < 0.5, big, b)  # wrap-around sums / products
    if dt == "uint64":  # values on both sides of 2^63 (the kernel's key flips the top bit)
        b = rng.integers(0, 6, size=shape).astype(dt)
        big = rng.integers(0, info.max, size=shape, dtype=np.uint64, endpoint=True)
        return np.where(rng.random(shape) < 0.5, big, b)
    return rng.integers(info.min, int(info.max) + 1, size=shape).astype(dt)


def check_int(v, t, op, dims):
    print(f"case int op={op} dtype={v.dtype} shape={v.shape} strides={v.strides} dims={dims}", flush=True)
    if op in ("argmax", "argmin") and dims is not None and len(dims) > 1:
        return
    exp = _np_int_ref(v, op, dims)
    if exp is None:
        return
    got = _capi.reduce(t, op, dims).cpu().numpy()
    exp = np.asarray(exp)
    if op == "mean":
        assert_close_rel(got.reshape(exp.shape), exp)
    else:
        with np.errstate(over="ignore"):
            np.testing.assert_array_equal(got.reshape(exp.shape), exp.astype(got.dtype))


@pytest.mark.parametrize("dt", INT_DTYPES)
def test_integer_inputs_random_layouts(dt):
    rng = np.random.default_rng(18)
    tdt = getattr(torch, dt)
    for shape in [(7,), (33, 5), (5, 1000), (16, 4096), (3, 17, 129), (4, 8, 6, 5), (2, 70001)]:
        b = _int_view_data(rng, dt, shape)
        t = torch.from_numpy(b).cuda()
        views = [(b, t)]
        if b.ndim >= 2:
            views.append((b[:, 1:], t[:, 1:]))          # misaligned rows
            views.append((b.T, t.permute(*reversed(range(t.ndim)))))  # transposed (general / cols)
            views.append((b[:, ::3], t[:, ::3]))        # stepped inner dim
        for v, tv in views:
            for dims in _dim_sets(v.ndim):
                for op in INT_OPS:
                    check_int(v, tv, op, dims)


@pytest.mark.parametrize("knob,values", [("general", [1]), ("splits", [1, 3, 64]), ("lanes", [16, 64, 256, 1024]),
                                         ("tx", [64, 128, 256])])
def test_integer_forced_plans(knob, values):
    rng = np.random.default_rng(19)
    a = _int_view_data(rng, "int32", (37, 1029))
    c = _int_view_data(rng, "uint8", (5, 300, 36))
    for val in values:
        _capi.debug_set(knob, val)
        for op in INT_OPS:
            check_int(a, torch.from_numpy(a).cuda(), op, [1])
            check_int(a, torch.from_numpy(a).cuda(), op, None)
            check_int(c, torch.from_numpy(c).cuda(), op, [1])
            check_int(c, torch.from_numpy(c).cuda(), op, [0])


def test_integer_extremes_and_empty():
    x = np.array([[np.iinfo(np.int64).min] * 3, [np.iinfo(np.int64).max, 1, np.iinfo(np.int64).max]], np.int64)
    t = torch.from_numpy(x).cuda()
    for op in INT_OPS:
        for dims in (None, [0], [1]):
            check_int(x, t, op, dims)
    u = np.array([[0, 2**63, 2**64 - 1, 2**63 - 1], [2**63 - 1, 2**63, 1, 0], [5, 5, 5, 5]], np.uint64)
    for op in INT_OPS:
        for dims in (None, [0], [1]):
            check_int(u, torch.from_numpy(u).cuda(), op, dims)
    for dt in ("uint16", "uint32"):
        info = np.iinfo(dt)
        w = np.array([[0, info.max, info.max // 2 + 1], [info.max, 0, 1]], dt)
        for op in INT_OPS:
            for dims in (None, [0], [1]):
                check_int(w, torch.from_numpy(w).cuda(), op, dims)
    # all elements at the lowest value: argmax stays at index 0 (strict compare)
    y = np.full(1000, np.iinfo(np.int32).min, np.int32)
    assert int(_capi.reduce(torch.from_numpy(y).cuda(), "argmax", None).cpu()) == 0
    e = torch.zeros((0, 4), dtype=torch.int32, device="cuda")
    assert (_capi.reduce(e, "sum", [0]).cpu().numpy() == 0).all()
    assert (_capi.reduce(e, "prod", [0]).cpu().numpy() == 1).all()
    assert _capi.reduce(e, "all", [0]).cpu().numpy().all()
