"""Pins the CPU oracle (oracle/tp_cpu_reduce.c) before anything is checked
against it.  Every function is checked against something other than its own
formula: the reference tests' known answers, numpy closed forms (np.add.accumulate
is a strictly sequential fold, i.e. exactly the reference's accumulation order),
torch at the reference's own tolerance (test/test_statistical.py:10-17), or brute
force on tiny inputs."""
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
KNOWN = json.load(open(os.path.join(HERE, "golden", "reference_known_answers.json")))


def _call(case):
    x = np.array(case["x"], np.float32).reshape(case["shape"])
    op, dims, keep = case["op"], case.get("dims"), case.get("keepdim", False)
    if op == "sum":
        return O.sum(x, dims, keep)
    if op == "mean":
        return O.mean(x, dims, keep)
    if op == "amax":
        return O.amax(x, dims, keep)
    if op == "amin":
        return O.amin(x, dims, keep)
    if op in ("argmax", "argmin"):
        f = O.argmax if op == "argmax" else O.argmin
        return f(x, None if dims is None else dims[0], keep)
    if op == "var":
        return O.var(x, dims)
    if op == "std":
        return O.std(x, dims)
    if op == "prod":
        return O.prod(x, dims, keep)
    if op == "norm":
        return O.norm(x, case.get("p", 2.0), dims, keep)
    if op == "all":
        return O.all_(x, dims, keep)
    if op == "any":
        return O.any_(x, dims, keep)
    raise ValueError(op)


@pytest.mark.parametrize("case", KNOWN, ids=[c["src"] + ":" + c["op"] for c in KNOWN])
def test_reference_known_answers(case):
    got = _call(case)
    exp = case["expect"]
    if isinstance(exp, list):
        assert list(np.shape(got)) == case["expect_shape"]
        np.testing.assert_array_equal(np.asarray(got).ravel(), np.array(exp))
    elif "places" in case:
        assert round(float(got) - exp, case["places"]) == 0
    else:
        assert float(got) == exp


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("shape,dims", [((7, 5), [1]), ((7, 5), [0]), ((3, 4, 5), [1]), ((3, 4, 5), [0, 2]),
                                        ((2, 3, 4, 5), [1, 3]), ((6, 9), [-1])])
def test_sum_dim_is_sequential_fp32(shape, dims):
    # The reference accumulates each output in fp32, visiting reduced elements in
    # row-major order (ReductionKernels.cpp:157-178) == np.add.accumulate in fp32.
    x = (_rng(1).standard_normal(shape) * 1000).astype(np.float32)
    nd = len(shape)
    rd = [d % nd for d in dims]
    kept = [d for d in range(nd) if d not in rd]
    xt = np.transpose(x, kept + rd).reshape(int(np.prod([shape[d] for d in kept])), -1)
    expect = np.add.accumulate(xt, axis=1, dtype=np.float32)[:, -1]
    got = O.sum(x, dims).ravel()
    np.testing.assert_array_equal(got, expect)
    # a plausible mistake (pairwise / fp64 accumulation) differs on this data
    assert not np.array_equal(got, xt.astype(np.float64).sum(1).astype(np.float32)) or xt.shape[1] < 3


def test_sum_all_is_sequential_fp64():
    x = (_rng(2).standard_normal(10001) * 1e4).astype(np.float32)
    expect = np.float32(np.add.accumulate(x.astype(np.float64))[-1])
    assert O.sum(x) == expect
    assert O.mean(x) == np.float32(np.float64(expect) / np.float64(np.float32(x.size)))


def test_mean_dim_divides_in_double():
    x = _rng(3).standard_normal((5, 7)).astype(np.float32)
    s = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1]
    np.testing.assert_array_equal(O.mean(x, [1]), (s.astype(np.float64) / 7.0).astype(np.float32))
    # duplicate dims multiply the count (ReductionKernels.cpp:203-208)
    np.testing.assert_array_equal(O.mean(x, [1, 1]), (s.astype(np.float64) / 49.0).astype(np.float32))


def test_strided_views_walk_logical_order():
    base = _rng(4).standard_normal((6, 8)).astype(np.float32)
    v = base.T[::2]  # shape (4, 6), non-contiguous
    c = np.ascontiguousarray(v)
    for f in (O.sum, O.mean, O.amax, O.amin):
        np.testing.assert_array_equal(f(v, [1]), f(c, [1]))
        np.testing.assert_array_equal(f(v, [0]), f(c, [0]))
    assert O.argmax(v) == O.argmax(c) == np.argmax(c)
    assert O.sum(v) == O.sum(c)


def test_minmax_known_and_numpy():
    x = _rng(5).standard_normal((4, 5, 6)).astype(np.float32)
    np.testing.assert_array_equal(O.amax(x, [0]), x.max(0))
    np.testing.assert_array_equal(O.amin(x, [1, 2], True), x.min((1, 2), keepdims=True))
    assert O.amax(x) == x.max() and O.amin(x) == x.min()
    with pytest.raises(RuntimeError):
        O.amax(np.zeros((0,), np.float32))


def test_minmax_nan_and_signed_zero_brute_force():
    # strict '>' with -inf init: NaN never replaces; the first of +-0 is kept.
    x = np.array([np.nan, -0.0, 0.0, np.nan], np.float32)
    v = O.amax(x)
    assert v == 0 and math.copysign(1, v) < 0
    assert O.argmax(x) == 1
    y = np.array([np.nan, np.nan], np.float32)
    assert O.amax(y) == -np.inf and O.argmax(y) == 0
    assert O.amin(y) == np.inf and O.argmin(y) == 0
    z = np.array([[0.0, -0.0], [np.nan, 1.0]], np.float32)
    r = O.amax(z, [1])
    assert math.copysign(1, r[0]) > 0 and r[1] == 1.0


def test_argmax_dims_numpy_and_transpose_quirk():
    x = _rng(6).standard_normal((3, 4, 5)).astype(np.float32)
    for d in range(3):
        np.testing.assert_array_equal(O.argmax(x, d), np.argmax(x, d))
        np.testing.assert_array_equal(O.argmin(x, d), np.argmin(x, d))
    # CPU path quirk (ReductionKernels.cpp:714-735): rows of transpose(d,-1) written
    # linearly.  For d=0 of (3,4,5): rows enumerate (5,4) -> the transpose of the
    # correct (4,5) answer, reshaped into (4,5).
    q = O.argmax(x, 0, quirk=True)
    np.testing.assert_array_equal(q.reshape(5, 4), np.argmax(x, 0).T)
    np.testing.assert_array_equal(O.argmax(x, 2, quirk=True), np.argmax(x, 2))  # last dim: no quirk
    t = np.array([[1.0, 5.0, 5.0], [4.0, 4.0, 6.0]], np.float32)  # ties -> first index
    np.testing.assert_array_equal(O.argmax(t, 1), [1, 2])
    np.testing.assert_array_equal(O.argmax(t, 0), [1, 0, 1])


@pytest.mark.parametrize("shape", [(10,), (5, 5), (2, 3, 4)])
def test_var_std_against_torch_like_reference_test(shape):
    torch = pytest.importorskip("torch")
    g = torch.Generator().manual_seed(7)
    data = torch.randn(shape, dtype=torch.float32, generator=g)
    x = data.numpy()
    close = lambda a, b: np.testing.assert_allclose(a, b.numpy(), rtol=1e-5, atol=1e-8)
    close(O.var(x), data.var())
    close(O.var(x, correction=0), data.var(correction=0))
    close(O.std(x), data.std())
    close(O.std(x, correction=0), data.std(correction=0))
    if len(shape) > 1:
        close(O.var(x, [0]), data.var(dim=0))
        close(O.var(x, [1], keepdim=True), data.var(dim=1, keepdim=True))
        close(O.std(x, [0]), data.std(dim=0))
        close(O.std(x, [1], keepdim=True), data.std(dim=1, keepdim=True))


def test_var_edge_cases():
    assert np.isnan(O.var(np.zeros((0,), np.float32)))
    assert np.isnan(O.var(np.array([3.0], np.float32)))          # 0/0
    assert O.var(np.array([3.0], np.float32), correction=0) == 0.0
    assert O.var(np.array([1.0, 3.0], np.float32), correction=5) == np.inf  # x/0


def _topk_reference(x2d, k, largest):
    u = x2d.view(np.uint32).copy()
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    u[nan] = 0x7FC00000
    u[u == 0x80000000] = 0
    key = np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint64)
    if not largest:
        key = (~key.astype(np.uint32)).astype(np.uint64)
    order = np.argsort(-key.astype(np.int64), axis=1, kind="stable")[:, :k]
    return np.take_along_axis(x2d, order, 1), order


@pytest.mark.parametrize("largest", [True, False])
def test_topk_against_stable_argsort(largest):
    x = _rng(8).uniform(-1, 1, (16, 300)).astype(np.float32)
    x[:, 7] = x[:, 3]  # ties
    x[0, :] = 0.5      # all equal row
    x[1, 10] = np.nan
    x[2, 11] = -0.0
    x[2, 12] = 0.0
    x[3, :5] = np.inf
    for k in (1, 5, 64, 300):
        v, i = O.topk(x, k, largest)
        ev, ei = _topk_reference(x, k, largest)
        np.testing.assert_array_equal(i, ei)
        np.testing.assert_array_equal(v.view(np.uint32), ev.view(np.uint32))
        assert O.topk(x, k, largest, threads=4)[1].tolist() == i.tolist()


def test_topk_values_match_torch():
    torch = pytest.importorskip("torch")
    x = _rng(9).standard_normal((8, 1000)).astype(np.float32)
    v, i = O.topk(x, 50)
    tv, ti = torch.topk(torch.from_numpy(x), 50)
    np.testing.assert_array_equal(v, tv.numpy())
    np.testing.assert_array_equal(i, ti.numpy())  # no ties in continuous data


# ---- prod / all / any / norm / median ----

@pytest.mark.parametrize("shape,dims", [((9,), None), ((7, 5), [1]), ((7, 5), [0]), ((3, 4, 5), [0, 2])])
def test_prod_is_sequential_fp32(shape, dims):
    # prod_kernel multiplies sequentially in float: np.multiply.accumulate in
    # float32 is that fold, bit for bit
    x = _rng(40).uniform(0.5, 1.5, size=shape).astype(np.float32)
    got = O.prod(x, dims)
    if dims is None:
        assert got == np.multiply.accumulate(x.ravel(), dtype=np.float32)[-1]
    else:
        keep = [d for d in range(x.ndim) if d not in dims]
        xt = np.transpose(x, keep + dims).reshape(int(np.prod([shape[d] for d in keep])), -1)
        exp = np.multiply.accumulate(xt, axis=1, dtype=np.float32)[:, -1]
        np.testing.assert_array_equal(got.ravel(), exp)


def test_all_any_brute_force():
    x = np.array([[0.0, -0.0, np.nan, 1.0], [2.0, 3.0, -1.0, np.inf], [0.0, 0.0, -0.0, 0.0]], np.float32)
    nz = (x != 0)  # numpy: NaN != 0 is True, -0.0 != 0 is False
    assert O.all_(x) == nz.all() and O.any_(x) == nz.any()
    for d in (0, 1):
        np.testing.assert_array_equal(O.all_(x, [d]), nz.all(axis=d))
        np.testing.assert_array_equal(O.any_(x, [d]), nz.any(axis=d))
    e = np.zeros((0, 3), np.float32)
    assert O.all_(e) and not O.any_(e)
    np.testing.assert_array_equal(O.all_(e, [0]), [True, True, True])
    np.testing.assert_array_equal(O.any_(e, [0]), [False, False, False])


@pytest.mark.parametrize("p", [1.0, 2.0, 3.0, 0.5, np.inf, -np.inf])
@pytest.mark.parametrize("shape,dims", [((10,), None), ((5, 5), None), ((5, 5), [0]), ((5, 5), [1]),
                                        ((3, 4, 6), [0, 2])])
def test_norm_matches_torch(p, shape, dims):
    # the reference's own test compares norm with torch at rtol 1e-5
    # (test/test_statistical.py:51-66, tolerance :10-17)
    torch = pytest.importorskip("torch")
    x = _rng(41).standard_normal(shape).astype(np.float32)
    got = O.norm(x, p, dims)
    t = torch.from_numpy(x)
    exp = t.norm(p=p) if dims is None else t.norm(p=p, dim=dims)
    np.testing.assert_allclose(np.asarray(got), exp.numpy(), rtol=1e-5, atol=1e-8)


def test_norm_special_p():
    x = np.array([3.0, -4.0, 0.0], np.float32)
    assert O.norm(x, 2.0) == 5.0
    assert O.norm(x, np.inf) == 4.0 and O.norm(x, -np.inf) == 0.0
    assert O.norm(x, 1.0) == 7.0
    assert O.norm(x, 0.0) == np.inf            # pow(0, 0) = 1 -> sum 3 -> 3^(1/0)
    assert O.norm(x[:1], 0.0) == 1.0
    assert O.norm(np.array([np.nan, 1.0], np.float32), np.inf) == 1.0  # NaN never wins the max
    with pytest.raises(RuntimeError):
        O.norm(np.zeros(0, np.float32), np.inf)


def test_median_brute_force():
    rng = _rng(42)
    for n in range(1, 40):
        x = rng.integers(-5, 6, size=n).astype(np.float32)  # many ties
        assert O.median(x) == np.sort(x)[(n - 1) // 2]
    x = np.arange(1001, dtype=np.float32)[::-1].copy()
    assert O.median(x) == 500.0
    assert O.median(np.arange(1000, dtype=np.float32)) == 499.0  # lower median for even n
    assert np.isnan(O.median(np.zeros(0, np.float32)))
    # NaN ranks above every number (np.sort puts NaN last)
    y = np.array([np.nan, 1.0, np.nan, -np.inf, 2.0], np.float32)
    assert O.median(y) == np.sort(y)[2]
    z = np.array([-0.0, -0.0, -0.0], np.float32)
    m = O.median(z)
    assert m == 0.0 and not np.signbit(m)  # a zero median comes back as +0.0
    # strided view
    w = rng.standard_normal((6, 7)).astype(np.float32)[:, ::2]
    assert O.median(w) == np.sort(w.ravel())[(w.size - 1) // 2]

