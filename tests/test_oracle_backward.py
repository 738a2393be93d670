"""Pins the oracle's reduction gradients (oracle.reduce_backward, the
derivatives.yaml formulas op by op in float32) against torch.autograd in fp64,
full and along dims.  CPU only."""
import zlib

import numpy as np
import pytest

from oracle import oracle as O

torch = pytest.importorskip("torch")


def autograd(x, g, op, dims, correction):
    t = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    kw = {} if dims is None else {"dim": tuple(dims)}
    if op == "sum":
        y = t.sum(**kw)
    elif op == "mean":
        y = t.mean(**kw)
    elif op == "var":
        y = t.var(correction=correction, **kw)
    else:
        y = t.std(correction=correction, **kw)
    y.backward(torch.from_numpy(np.asarray(g, np.float64)).reshape(y.shape))
    return t.grad.numpy(), y.detach().numpy()


def tolerance(op, x, g, dims, correction, res):
    x = x.astype(np.float64)
    nd = x.ndim
    rd = tuple(range(nd)) if dims is None else tuple(d % nd for d in dims)
    n = int(np.prod([x.shape[d] for d in rd]))
    kshape = [1 if i in rd else x.shape[i] for i in range(nd)]
    g = np.abs(np.asarray(g, np.float64)).reshape(kshape)
    if op in ("sum", "mean"):
        return 1e-6 * g / (n if op == "mean" else 1) + 1e-38
    m = np.abs(x.mean(axis=rd, keepdims=True))
    scale = g * (np.abs(x) + m)
    if op == "var":
        return 1e-5 * 2 * scale / abs(n - correction)
    return 1e-5 * scale / (np.abs(np.asarray(res, np.float64)).reshape(kshape) * abs(n - correction))


CASES = [((1000,), None), ((33, 65), [1]), ((33, 65), [0]), ((4, 5, 6), [0, 2]), ((4, 5, 6), [1]),
         ((4, 5, 6), None), ((7, 3, 2, 5), [-1, 1])]


@pytest.mark.parametrize("op", ["sum", "mean", "var", "std"])
@pytest.mark.parametrize("shape,dims", CASES)
def test_reduce_backward_matches_torch_autograd(op, shape, dims):
    rng = np.random.default_rng(zlib.crc32(f"{op}-{shape}".encode()))
    x = (rng.standard_normal(shape) * 2 + 0.5).astype(np.float32)
    for correction in ((1,) if op in ("sum", "mean") else (0, 1, 2)):
        y_shape = np.sum(x, axis=None if dims is None else tuple(dims)).shape
        g = rng.standard_normal(y_shape).astype(np.float32)
        ref, res = autograd(x, g, op, dims, correction)
        got = O.reduce_backward(g, x, op, dims, correction, result=res.astype(np.float32))
        assert got.shape == x.shape and got.dtype == np.float32
        tol = tolerance(op, x, g, dims, correction, res)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= tol)


def test_reduce_backward_sum_mean_closed_forms():
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    np.testing.assert_array_equal(O.reduce_backward(np.float32(2.5), x, "sum"), np.full((3, 4), 2.5, np.float32))
    np.testing.assert_array_equal(O.reduce_backward(np.array([1, 2, 3], np.float32), x, "mean", [1]),
                                  np.repeat(np.array([0.25, 0.5, 0.75], np.float32)[:, None], 4, 1))
    # var of [1, 2, 3, 4] (unbiased): d/dx = 2 (x - 2.5) / 3
    v = O.reduce_backward(np.float32(1.0), np.array([1, 2, 3, 4], np.float32), "var")
    np.testing.assert_allclose(v, 2 * (np.array([1, 2, 3, 4]) - 2.5) / 3, rtol=1e-7)
