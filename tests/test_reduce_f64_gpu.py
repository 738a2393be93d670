"""GPU parity of float64 reductions (tpr_reduce with in_dtype FLOAT64, through
the C-ABI and the dispatcher) against the oracle's float64 restatement.

Tolerances: amax / amin / argmax / argmin / all / any bit-exact; sum / mean
within 1e-13 of sum|x| (normwise: the accumulation order differs from the
reference's sequential one); prod, var, std and norm (p = 1, 2, +-inf) within
1e-12 relative; norm with another p within 1e-7 relative (the exponent reaches
the kernel as float32)."""
import numpy as np
import pytest

import tensorplay_amd as tp
from oracle import oracle as O
from tensorplay_amd import _capi

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

OPS = ["sum", "mean", "prod", "amax", "amin", "argmax", "argmin", "var", "std", "all", "any"]


def views(rng):
    out = []
    for shape in [(7,), (33, 5), (5, 1000), (16, 4096), (3, 17, 129), (2, 3, 1, 64)]:
        b = rng.standard_normal(shape)
        out.append((b, b))
    b = rng.standard_normal((40, 64))
    out += [(b, b.T), (b, b[:, ::3]), (b, b[1:, 1:])]
    return out


def expected(v, op, dims, c=1, p=2.0):
    if op in ("all", "any"):
        f = np.all if op == "all" else np.any
        return f(v != 0, axis=None if dims is None else tuple(dims))
    return O.reduce_f64(v, op, dims, c, p)


def check(base, v, op, dims, c=1, p=2.0):
    print(f"case f64 {op} shape={v.shape} strides={v.strides} dims={dims} c={c} p={p}", flush=True)
    t = torch.from_numpy(base).cuda()
    off = (v.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // 8
    tv = t.as_strided(v.shape, [s // 8 for s in v.strides], off)
    got = _capi.reduce(tv, op, dims, correction=c, p=p).cpu().numpy()
    exp = expected(v, op, dims, c, p)
    got = got.reshape(np.shape(exp))
    if op in ("amax", "amin", "argmax", "argmin", "all", "any"):
        np.testing.assert_array_equal(got, exp)
    elif op in ("sum", "mean"):
        ax = None if dims is None else tuple(dims)
        scale = np.abs(v).sum(axis=ax) / (1 if op == "sum" else max(1, v.size // max(1, np.size(exp))))
        assert np.all(np.abs(got - exp) <= 1e-13 * scale + 1e-300)
    else:
        rtol = 1e-7 if (op == "norm" and p not in (1.0, 2.0) and not np.isinf(p)) else 1e-12
        np.testing.assert_allclose(got, exp, rtol=rtol, atol=0)


@pytest.mark.parametrize("op", OPS)
def test_layouts(op):
    rng = np.random.default_rng(50)
    for base, v in views(rng):
        if op == "prod":
            base[...] = 1.0 + 0.01 * base      # keep products of thousands of factors finite (v views base)
        nd = v.ndim
        for dims in [None, [nd - 1], [0]] + ([[0, nd - 1]] if nd > 2 else []):
            for c in ((0, 1) if op in ("var", "std") else (1,)):
                check(base, v, op, dims, c)


@pytest.mark.parametrize("p", [1.0, 2.0, 3.0, np.inf, -np.inf])
def test_norm(p):
    rng = np.random.default_rng(51)
    for base, v in views(rng):
        for dims in [None, [v.ndim - 1]]:
            check(base, v, "norm", dims, p=p)


def test_large_and_nan():
    rng = np.random.default_rng(52)
    x = rng.standard_normal(1 << 22) * 2 + 0.5         # full reduction with split workgroups
    for op in ("sum", "mean", "amax", "argmax", "var", "std"):
        check(x, x, op, None)
    y = rng.standard_normal((64, 3000))
    y[3, 10] = np.nan
    y[5, :] = np.nan
    for op in ("amax", "amin", "argmax", "argmin"):
        check(y, y, op, [1])


def test_dispatcher_f64():
    rng = np.random.default_rng(53)
    x = rng.standard_normal((6, 500))
    t = tp.tensor(x, device="rocm")
    assert t.dtype == tp.float64
    s = t.sum(1)
    assert s.dtype == tp.float64
    np.testing.assert_allclose(s.numpy(), O.reduce_f64(x, "sum", [1]), rtol=1e-12)
    np.testing.assert_array_equal(t.max(1).numpy(), x.max(1))
    np.testing.assert_array_equal(t.argmax(1).numpy(), x.argmax(1))
    v = t.var([1])
    assert v.dtype == tp.float64
    np.testing.assert_allclose(v.numpy(), x.var(1, ddof=1), rtol=1e-12)
    np.testing.assert_allclose(t.std().item(), x.std(ddof=1), rtol=1e-12)
    np.testing.assert_allclose(t.norm(2.0).item(), np.linalg.norm(x), rtol=1e-12)
    assert t.mean().dtype == tp.float64
    m = t.median()  # lower median in float64
    assert m.dtype == tp.float64 and m.item() == np.sort(x.ravel())[(x.size - 1) // 2]


def test_median_float64_special_values():
    """float64 median: NaN ranks above every number (canonicalised), -inf/+inf at
    the ends, -0.0 == +0.0 (returned as +0.0); against np.sort for every prefix
    length, bit-exact."""
    x = np.array([np.nan, 1.0, np.nan, -np.inf, 2.0, -0.0, 0.0, np.inf, np.nan, -1e-310, 1e-310], np.float64)
    for k in range(1, len(x) + 1):
        v = np.ascontiguousarray(x[:k])
        print(f"case median f64 n={k}", flush=True)
        got = _capi.reduce(torch.from_numpy(v).cuda(), "median", None).cpu().numpy().reshape(())
        srt = np.sort(np.where(v == 0, 0.0, v))   # np.sort puts NaN last, as the key order
        exp = srt[(k - 1) // 2]
        if np.isnan(exp):
            assert np.isnan(got)
        else:
            assert got.view(np.uint64) == np.float64(exp).view(np.uint64), (k, got, exp)
    z = np.full(4, -0.0, np.float64)
    got = _capi.reduce(torch.from_numpy(z).cuda(), "median", None).cpu().numpy().reshape(())
    assert got == 0.0 and not np.signbit(got)
