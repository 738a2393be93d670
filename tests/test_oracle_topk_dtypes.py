"""oracle.topk_any (tpr_topk's order for every dtype) pinned without the
oracle's own formula: Python's sorted() on (value, index) pairs with the
ordering spelled out per dtype family, on small random rows with ties and
extremes; and equality with the C restatement (oracle.topk) on float32."""
import math

import numpy as np
import pytest

from oracle import oracle as O

INT_TYPES = [np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint16, np.uint32, np.uint64]


def brute(row, k, largest):
    def rank(v):
        if isinstance(v, float) and math.isnan(v):
            return (1, 0.0)              # NaN above every number
        return (0, 0.0 if v == 0 else v)  # -0.0 == +0.0
    items = [(rank(v), i) for i, v in enumerate(row.tolist())]
    if largest:
        items.sort(key=lambda t: (tuple(-a for a in t[0]), t[1]))
    else:
        items.sort(key=lambda t: (t[0], t[1]))
    return [i for _, i in items[:k]]


@pytest.mark.parametrize("dt", INT_TYPES + [np.bool_])
def test_integer_and_bool_rows(dt):
    rng = np.random.default_rng(40)
    if dt == np.bool_:
        x = rng.random((6, 37)) < 0.5
    else:
        info = np.iinfo(dt)
        x = rng.integers(info.min, info.max, size=(6, 37), dtype=dt, endpoint=True)
        x[0, :10] = info.max
        x[1, :10] = info.min
        x[2] = x[2] % 3            # heavy ties
    for k in (1, 5, 37):
        for largest in (True, False):
            v, i = O.topk_any(x, k, largest)
            for r in range(x.shape[0]):
                assert list(i[r]) == brute(x[r], k, largest)
                np.testing.assert_array_equal(v[r], x[r, i[r]])


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_float_rows(dt):
    rng = np.random.default_rng(41)
    x = rng.standard_normal((6, 40)).astype(dt)
    x[0, ::4] = np.nan
    x[1] = np.where(rng.random(40) < 0.5, -0.0, 0.0)
    x[2, :5] = np.inf
    x[2, 5:10] = -np.inf
    x[3] = np.round(x[3])
    for k in (1, 7, 40):
        for largest in (True, False):
            v, i = O.topk_any(x, k, largest)
            for r in range(x.shape[0]):
                assert list(i[r]) == brute(x[r], k, largest)
    if dt == np.float32:
        for largest in (True, False):
            v, i = O.topk_any(x, 7, largest)
            ev, ei = O.topk(x, 7, largest)
            np.testing.assert_array_equal(i, ei)
            np.testing.assert_array_equal(v.view(np.uint32), ev.view(np.uint32))
