"""Pins the oracle's float64 reductions (oracle.reduce_f64) against math.fsum,
numpy and torch in fp64.  CPU only."""
import math

import numpy as np
import pytest

from oracle import oracle as O

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("shape,dims", [((1000,), None), ((13, 17), [1]), ((13, 17), [0]), ((3, 4, 5), [0, 2]),
                                        ((3, 4, 5), None)])
def test_f64_oracle(shape, dims):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(shape) * 3 + 0.5
    ax = None if dims is None else tuple(dims)
    s = O.reduce_f64(x, "sum", dims)
    if ax is None:
        ref = math.fsum(x.ravel())
    else:
        y = np.moveaxis(x, ax, list(range(-len(ax), 0)))
        ref = np.apply_along_axis(math.fsum, -1, y.reshape(*np.sum(x, axis=ax).shape, -1))
    assert np.all(np.abs(s - ref) <= 1e-13 * np.abs(x).sum(axis=ax))
    np.testing.assert_allclose(O.reduce_f64(x, "mean", dims), np.mean(x, axis=ax), rtol=1e-13)
    np.testing.assert_array_equal(O.reduce_f64(x, "amax", dims), np.max(x, axis=ax))
    np.testing.assert_array_equal(O.reduce_f64(x, "amin", dims), np.min(x, axis=ax))
    if dims is None or len(dims) == 1:
        am = np.argmax(x) if dims is None else np.argmax(x, axis=dims[0])
        np.testing.assert_array_equal(O.reduce_f64(x, "argmax", dims), am)
    t = torch.from_numpy(x)
    kw = {} if dims is None else {"dim": tuple(dims)}
    for c in (0, 1, 2):
        np.testing.assert_allclose(O.reduce_f64(x, "var", dims, c), t.var(correction=c, **kw).numpy(), rtol=1e-12)
        np.testing.assert_allclose(O.reduce_f64(x, "std", dims, c), t.std(correction=c, **kw).numpy(), rtol=1e-12)
    for p in (1.0, 2.0, 3.0, np.inf, -np.inf):
        np.testing.assert_allclose(O.reduce_f64(x, "norm", dims, p=p),
                                   torch.linalg.vector_norm(t, ord=p, **kw).numpy(), rtol=1e-12)


def test_f64_nan_and_ties():
    x = np.array([[1.0, np.nan, 3.0, 3.0], [np.nan, np.nan, np.nan, np.nan]])
    np.testing.assert_array_equal(O.reduce_f64(x, "amax", [1]), [3.0, -np.inf])   # NaN ignored; all-NaN -> -inf
    np.testing.assert_array_equal(O.reduce_f64(x, "argmax", [1]), [2, 0])          # first of the tie
