"""Randomised parity sweep of tpr_topk against the CPU oracle: a fixed-seed
stream of shapes, strides, k, direction and dtype that lands on every kernel the
planner picks (lane-group short rows, the wave and workgroup kernels with and
without row splits, the register-row and streaming radix kernels), with
duplicate-heavy, signed-zero, NaN and infinity rows mixed in.  Values are
compared bit for bit in the input dtype, indices exactly (ties to the lowest
index)."""
import numpy as np
import pytest

from oracle import oracle as O
from tensorplay_amd import _capi

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(autouse=True)
def _merge_contract():
    # the test build counts split-row merge outputs whose index lay past the row
    _capi.debug_get("topk_merge_clamped")
    yield
    assert _capi.debug_get("topk_merge_clamped") == 0

DTYPES = [np.float32] * 6 + [np.float64, np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint16, np.uint32,
                             np.uint64, np.bool_]


def _row_data(rng, dt, rows, cols):
    kind = rng.integers(0, 4)
    if dt == np.bool_:
        return rng.random((rows, cols)) < rng.random()
    if np.issubdtype(dt, np.floating):
        x = rng.standard_normal((rows, cols)).astype(dt) * dt(rng.choice([1e-3, 1.0, 1e3]))
        if kind == 1:
            x = np.round(x * 2) / 2                          # many ties
        elif kind == 2:
            x[:, ::7] = np.where(rng.random((rows, (cols + 6) // 7)) < 0.5, -0.0, 0.0).astype(dt)
            x[:, ::11] = np.nan
        elif kind == 3:
            x[:, ::13] = np.inf
            x[:, 5::17] = -np.inf
        return x
    info = np.iinfo(dt)
    if kind == 1:
        return rng.integers(0, 4, size=(rows, cols)).astype(dt)  # many ties
    return rng.integers(info.min, info.max, size=(rows, cols), dtype=dt, endpoint=True)


def test_random_sweep():
    rng = np.random.default_rng(20261202)
    for case in range(160):
        dt = DTYPES[rng.integers(0, len(DTYPES))]
        scale = rng.choice([8, 300, 3000, 40000, 200000])
        cols = int(rng.integers(1, scale + 1))
        rows = int(rng.integers(1, max(2, min(64, 2_000_000 // cols)) + 1))
        pad = int(rng.integers(0, 3)) if rng.random() < 0.3 else 0
        k = int(rng.choice([1, rng.integers(1, min(cols, 64) + 1), rng.integers(1, min(cols, 1100) + 1),
                            rng.integers(1, cols + 1)]))
        largest = bool(rng.integers(0, 2))
        base = _row_data(rng, dt, rows, cols + pad)
        x = base[:, pad:]
        print(f"case {case}: {np.dtype(dt).name} rows={rows} cols={cols} offset={pad} k={k} largest={largest}",
              flush=True)
        t = torch.from_numpy(base).cuda()[:, pad:]
        gv, gi = _capi.topk(t, k, largest)
        torch.cuda.synchronize()
        ev, ei = O.topk_any(np.ascontiguousarray(x), k, largest)
        np.testing.assert_array_equal(gi.cpu().numpy(), ei)
        g = gv.cpu().numpy()
        assert g.dtype == ev.dtype
        np.testing.assert_array_equal(g.view(np.uint8), ev.view(np.uint8))


def test_random_sweep_many_rows_float32():
    # float32 with many rows (the routing by rows per CU: lane groups, 4 / 8 /
    # 16-wave workgroups, two-per-CU 16-wave workgroups, the register and
    # segmented radix selects) and k up to 256 (512-entry wave lists)
    rng = np.random.default_rng(20261203)
    for case in range(40):
        cols = int(rng.choice([int(rng.integers(200, 4097)), int(rng.integers(4097, 16384)),
                               int(rng.integers(16384, 70000))]))
        rows = int(rng.integers(200, max(201, min(5000, 6_000_000 // cols)) + 1))
        k = int(min(cols, rng.choice([int(rng.integers(1, 65)), int(rng.integers(65, 129)),
                                      int(rng.integers(129, 257)), int(rng.integers(257, 1025))])))
        largest = bool(rng.integers(0, 2))
        x = _row_data(rng, np.float32, rows, cols)
        print(f"case {case}: float32 rows={rows} cols={cols} k={k} largest={largest}", flush=True)
        t = torch.from_numpy(x).cuda()
        gv, gi = _capi.topk(t, k, largest)
        torch.cuda.synchronize()
        ev, ei = O.topk(x, k, largest)
        np.testing.assert_array_equal(gi.cpu().numpy(), ei)
        np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint32), ev.view(np.uint32))
