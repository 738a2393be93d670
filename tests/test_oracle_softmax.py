"""Pins the oracle's softmax / log_softmax, their gradients and nll_loss
(oracle/tp_cpu_softmax.c) against the reference tests' known answers, torch in
fp64 (softmax, log_softmax, autograd gradients, nll_loss) and brute force on
NaN / inf slices.  CPU only."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

torch = pytest.importorskip("torch")

HERE = os.path.dirname(os.path.abspath(__file__))
KNOWN = json.load(open(os.path.join(HERE, "golden", "reference_known_answers_softmax.json")))


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("case", KNOWN, ids=[c["src"] + ":" + c["op"] for c in KNOWN])
def test_reference_known_answers(case):
    x = np.array(case["x"], np.float32).reshape(case["shape"])
    y = O.softmax(x, case["dim"])
    got = y.sum(axis=case["dim"]) if case["op"] == "softmax_rowsum" else y
    assert list(got.shape) == case["expect_shape"]
    for a, b in zip(got.ravel().tolist(), case["expect"]):
        assert round(a - b, case["places"]) == 0


def softmax_tol_ok(y, x64, dim, log):
    """fp32 softmax within 1e-5 relative of the fp64 value; log_softmax within
    1e-5 of (|y64| + |log-sum-exp|) absolute (the two terms it subtracts)."""
    t = torch.from_numpy(x64)
    if log:
        ref = torch.log_softmax(t, dim).numpy()
        lse = torch.logsumexp(t - t.max(dim, keepdim=True).values, dim, keepdim=True).numpy()
        tol = 1e-5 * (np.abs(ref) + np.abs(lse))
    else:
        ref = torch.softmax(t, dim).numpy()
        tol = 1e-5 * np.abs(ref) + 1e-30
    err = np.abs(y.astype(np.float64) - ref)
    return bool(np.all(err <= tol)), float(np.max(err / np.maximum(tol, 1e-300)))


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("shape,dim", [((5, 7), 1), ((5, 7), 0), ((3, 4, 5), 1), ((3, 4, 5), -1), ((2, 3, 4, 5), 2),
                                       ((64,), 0), ((4, 300), 1)])
def test_softmax_matches_torch_fp64(shape, dim, log):
    x = (_rng(1).standard_normal(shape) * 3).astype(np.float32)
    y = O.softmax(x, dim, log=log)
    ok, worst = softmax_tol_ok(y, x.astype(np.float64), dim, log)
    assert ok, worst


def test_softmax_strided_input_walks_logical_order():
    b = _rng(2).standard_normal((6, 9)).astype(np.float32)
    v = b.T[::2]
    np.testing.assert_array_equal(O.softmax(v, 1), O.softmax(np.ascontiguousarray(v), 1))


def test_softmax_nan_inf_brute_force():
    inf, nan = np.inf, np.nan
    x = np.array([[1.0, nan, 2.0],      # a NaN makes the row NaN (it enters the sum)
                  [-inf, -inf, -inf],   # no value above -inf: max stays -inf, x - max is NaN
                  [nan, -inf, nan],
                  [1.0, inf, 2.0],      # inf - inf = NaN
                  [-inf, 0.0, 0.0],     # -inf entries are exp(-inf) = 0
                  [3.0, 3.0, 3.0]], np.float32)
    y = O.softmax(x, 1)
    ly = O.log_softmax(x, 1)
    for r in range(4):
        assert np.all(np.isnan(y[r])) and np.all(np.isnan(ly[r]))
    np.testing.assert_array_equal(y[4], np.array([0.0, 0.5, 0.5], np.float32))
    assert ly[4][0] == -inf and ly[4][1] == ly[4][2] == np.float32(-np.log(np.float32(2.0)))
    np.testing.assert_array_equal(y[5], np.full(3, np.float32(1.0) / np.float32(3.0)))


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("shape,dim", [((5, 7), 1), ((3, 4, 5), 1), ((3, 4, 5), 0), ((2, 130), 1)])
def test_softmax_backward_matches_torch_autograd(shape, dim, log):
    rng = _rng(3)
    x64 = rng.standard_normal(shape) * 2
    g64 = rng.standard_normal(shape)
    t = torch.from_numpy(x64).requires_grad_(True)
    yt = torch.log_softmax(t, dim) if log else torch.softmax(t, dim)
    yt.backward(torch.from_numpy(g64))
    ref = t.grad.numpy()
    y32 = yt.detach().numpy().astype(np.float32)
    g32 = g64.astype(np.float32)
    got = O.softmax_backward(g32, y32, dim, log=log).astype(np.float64)
    y = y32.astype(np.float64)
    g = g32.astype(np.float64)
    if log:
        tol = 1e-5 * (np.abs(g) + np.exp(y) * np.abs(g).sum(dim, keepdims=True))
    else:
        tol = 1e-5 * (np.abs(g) + np.abs(g * y).sum(dim, keepdims=True)) * np.abs(y) + 1e-30
    assert np.all(np.abs(got - ref) <= tol)


@pytest.mark.parametrize("reduction", [0, 1, 2])
@pytest.mark.parametrize("weighted", [False, True])
def test_nll_loss_matches_torch(reduction, weighted):
    rng = _rng(4)
    N, C = 37, 11
    x = rng.standard_normal((N, C)).astype(np.float32)
    t = rng.integers(0, C, N).astype(np.int64)
    t[[3, 9, 20]] = -100  # ignore_index
    w = rng.uniform(0.1, 2.0, C).astype(np.float32) if weighted else None
    out, tw = O.nll_loss(x, t, w, reduction, -100)
    ref = torch.nn.functional.nll_loss(torch.from_numpy(x.astype(np.float64)), torch.from_numpy(t),
                                       None if w is None else torch.from_numpy(w.astype(np.float64)),
                                       ignore_index=-100, reduction=["none", "mean", "sum"][reduction]).numpy()
    keep = t != -100
    wt = np.ones(C, np.float32) if w is None else w
    tw_ref = wt[t[keep]].astype(np.float64).sum()
    assert abs(float(tw[0]) - tw_ref) <= 1e-6 * tw_ref
    if reduction == 0:
        # closed form, bit-exact: -x[i, t_i] * w[t_i] in float32, 0 where ignored
        expect = np.zeros(N, np.float32)
        expect[keep] = -x[keep, t[keep]] * wt[t[keep]]
        np.testing.assert_array_equal(out, expect)
    else:
        assert abs(float(out) - float(ref)) <= 1e-6 * abs(float(ref))


def test_nll_loss_target_out_of_bounds_raises():
    x = np.zeros((2, 3), np.float32)
    with pytest.raises(RuntimeError, match="Target out of bounds"):
        O.nll_loss(x, np.array([0, 3], np.int64))
    with pytest.raises(RuntimeError, match="Target out of bounds"):
        O.nll_loss(x, np.array([-1, 0], np.int64))
    out, tw = O.nll_loss(x, np.array([-100, -100], np.int64), None, 1)  # all ignored: mean stays 0
    assert float(out) == 0.0 and float(tw[0]) == 0.0


@pytest.mark.parametrize("reduction", [0, 1, 2])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("pass_tw", [False, True])
def test_nll_loss_backward_matches_torch_autograd(reduction, weighted, pass_tw):
    rng = _rng(5)
    N, C = 29, 7
    x = rng.standard_normal((N, C)).astype(np.float32)
    t = rng.integers(0, C, N).astype(np.int64)
    t[[1, 5]] = 3 if C > 3 else 0
    t[7] = -100
    w = rng.uniform(0.1, 2.0, C).astype(np.float32) if weighted else None
    g = rng.standard_normal(N if reduction == 0 else ()).astype(np.float32)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    lt = torch.nn.functional.nll_loss(xt, torch.from_numpy(t), None if w is None else torch.from_numpy(
        w.astype(np.float64)), ignore_index=-100, reduction=["none", "mean", "sum"][reduction])
    lt.backward(torch.from_numpy(g.astype(np.float64)))
    ref = xt.grad.numpy()
    tw = O.nll_loss(x, t, w, 2)[1] if pass_tw else None
    got = O.nll_loss_backward(g, t, C, w, reduction, -100, tw)
    assert got.shape == (N, C)
    assert np.all((got != 0) == (ref != 0))
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=0)
