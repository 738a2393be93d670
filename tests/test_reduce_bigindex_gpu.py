"""Reductions whose reduced run has 2^31 or more elements (indices past int32).

Such runs are cut into chunks of 2^30 elements, one row / column kernel launch
each, with the chunk's first index added to arg-op states and one finalize over
all partials.  Inputs are built so that every expected value is a closed form
(counts of ones, a few placed values), so no host copy of the 2-8 GiB tensors
is needed.
"""
import numpy as np
import pytest

from tensorplay_amd import _capi

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

N = (1 << 31) + 17  # elements in the reduced run
B = 1 << 31         # first index past int32


def red(t, op, dims=None):
    out = _capi.reduce(t, op, dims)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_int8_full_run_past_2_31():
    print("case int8 full n=2^31+17", flush=True)
    x = torch.ones(N, dtype=torch.int8, device="cuda")
    x[B + 5] = 100
    x[B + 9] = 100    # tie: the lower index wins
    x[B + 11] = -7
    assert int(red(x, "sum")) == N - 3 + 200 - 7
    assert int(red(x, "argmax")) == B + 5
    assert int(red(x, "amax")) == 100
    assert int(red(x, "argmin")) == B + 11
    assert int(red(x, "amin")) == -7
    assert bool(red(x, "all")) is True
    assert int(red(x, "median")) == 1
    x[B + 13] = 0
    assert bool(red(x, "all")) is False
    assert bool(red(x, "any")) is True
    del x
    torch.cuda.empty_cache()


def test_bool_any_past_2_31():
    print("case bool any n=2^31+17", flush=True)
    x = torch.zeros(N, dtype=torch.bool, device="cuda")
    assert bool(red(x, "any")) is False
    x[N - 1] = True   # only the very last element
    assert bool(red(x, "any")) is True
    assert bool(red(x, "all")) is False
    assert int(red(x, "argmax")) == N - 1
    assert int(red(x, "sum")) == 1
    del x
    torch.cuda.empty_cache()


def test_int8_rows_and_cols_past_2_31():
    print("case int8 rows [2, 2^31+17] and cols [2^31+17, 2]", flush=True)
    x = torch.ones((2, N), dtype=torch.int8, device="cuda")
    x[1, N - 1] = 50
    np.testing.assert_array_equal(red(x, "sum", [1]), [N, N + 49])
    np.testing.assert_array_equal(red(x, "argmax", [1]), [0, N - 1])
    del x
    torch.cuda.empty_cache()
    y = torch.zeros((N, 2), dtype=torch.int8, device="cuda")
    y[B + 3, 1] = 9
    y[B + 4, 1] = 9
    np.testing.assert_array_equal(red(y, "sum", [0]), [0, 18])
    np.testing.assert_array_equal(red(y, "argmax", [0]), [0, B + 3])
    np.testing.assert_array_equal(red(y, "amax", [0]), [0, 9])
    del y
    torch.cuda.empty_cache()


def test_float32_full_argmax_past_2_31():
    print("case float32 full n=2^31+17 (8 GiB)", flush=True)
    x = torch.zeros(N, dtype=torch.float32, device="cuda")
    x[5] = 0.5
    x[B + 3] = 1.0
    x[B + 9] = 1.0
    x[N - 1] = -2.0
    assert int(red(x, "argmax")) == B + 3
    assert float(red(x, "amax")) == 1.0
    assert int(red(x, "argmin")) == N - 1
    assert float(red(x, "sum")) == 0.5
    m = float(red(x, "mean"))
    assert abs(m - 0.5 / N) <= 1e-6 * (0.5 / N)
    del x
    torch.cuda.empty_cache()
