"""Randomised parity sweep of tpr_softmax (float32) against fp64: a fixed-seed
stream of softmax / log_softmax forward and gradient cases over unit-stride
rows (short, register-resident, one-CU-resident, row pieces, longer than the
pieces hold) and strided dims (scalar, float4 two-pass, held in registers,
row pieces), with NaN and -inf entries mixed in, so every forward and
gradient kernel the planner picks is reached on inputs no one chose by hand.

Bounds: the per-case tests' (softmax 1e-5 relative; log_softmax
1e-5 * (|y| + |log-sum-exp|); gradients 1e-5 of the formula's magnitudes),
with one stated addition for log_softmax, an absolute floor of 2^-20: when one
element dominates its slice, sum(exp(x - max)) = 1 + eps with eps within a few
fp32 ulps of 1, and the max element's -log(1 + eps) keeps that sum's rounding
(the reference's float32 composite, PointwiseKernels.cpp:533-545, rounds the
same way; e.g. for the slice [7.0556, -9.9746] both return 0 against -4.0e-8)."""
import numpy as np
import pytest

from tensorplay_amd import _capi
from tests.gpu_util import softmax_error

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

LOG_ABS_FLOOR = 2.0 ** -20


def _case(rng):
    kind = int(rng.integers(0, 3))
    if kind == 0:
        cols = int(rng.choice([int(rng.integers(2, 5000)), int(rng.integers(16000, 160000)),
                               int(rng.integers(150000, 700000))]))
        rows = int(rng.integers(1, max(2, min(400, 12_000_000 // cols)) + 1))
        return (rows, cols)
    n = int(rng.choice([int(rng.integers(2, 600)), int(rng.integers(500, 1100))]))
    inner = int(rng.choice([3, 64, 128, 200, 256, 1000, 1024]))
    outer = int(rng.integers(1, max(2, min(32, 6_000_000 // (n * inner))) + 1))
    return (outer, n, inner)


def test_random_sweep():
    rng = np.random.default_rng(20261204)
    for case in range(90):
        shape = _case(rng)
        dim = 1
        log = bool(rng.integers(0, 2))
        grad = rng.random() < 0.35
        x = (rng.standard_normal(shape) * 3).astype(np.float32)
        if not grad:
            if rng.random() < 0.3:
                x.reshape(-1)[rng.integers(0, x.size, 5)] = np.nan
            if rng.random() < 0.3:
                x.reshape(-1)[rng.integers(0, x.size, 5)] = -np.inf
        print(f"case {case}: shape={shape} dim={dim} log={log} grad={grad}", flush=True)
        if not grad:
            got = _capi.softmax(torch.from_numpy(x).cuda(), dim, log=log).cpu().numpy()
            r = softmax_error(got, x.astype(np.float64), dim, log, LOG_ABS_FLOOR if log else 0.0)
            assert r <= 1.0, f"case {case}: error {r:.2f}x the bound"
            continue
        tx = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
        ty = torch.log_softmax(tx, dim) if log else torch.softmax(tx, dim)
        g64 = rng.standard_normal(shape)
        ty.backward(torch.from_numpy(g64))
        ref = tx.grad.numpy()
        y = ty.detach().numpy().astype(np.float32)
        g = g64.astype(np.float32)
        got = _capi.softmax(torch.from_numpy(g).cuda(), dim, log=log,
                            grad_of=torch.from_numpy(y).cuda()).cpu().numpy().astype(np.float64)
        y64, gg = y.astype(np.float64), g.astype(np.float64)
        if log:
            tol = 1e-5 * (np.abs(gg) + np.exp(y64) * np.abs(gg).sum(dim, keepdims=True))
        else:
            tol = 1e-5 * (np.abs(gg) + np.abs(gg * y64).sum(dim, keepdims=True)) * np.abs(y64) + 1e-30
        assert np.all(np.abs(got - ref) <= tol), f"case {case}: gradient beyond the bound"
