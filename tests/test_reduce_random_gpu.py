"""Randomised parity sweep of tpr_reduce (float32) against the CPU oracle and
fp64: a fixed-seed stream of shapes (1-4 dims), strided and offset views,
reduced dim sets and ops that lands on every layout kernel (register rows,
rows, columns, general, split plans with their finalize).  amax / amin /
argmax / argmin / all / any bit-exact against the oracle, sum / mean / var /
std / norm within 1e-5 relative of numpy in float64 (the same checks as the
per-op tests)."""
import numpy as np
import pytest

from tests.test_reduce_gpu import check

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

OPS = ["sum", "mean", "amax", "amin", "argmax", "argmin", "var", "std", "norm", "all", "any"]


def test_random_sweep():
    rng = np.random.default_rng(1202)
    for case in range(150):
        nd = int(rng.integers(1, 5))
        shape = [int(rng.choice([1, 2, 3, 7, 31, 64, 100, 257, 1024, 4099])) for _ in range(nd)]
        while np.prod(shape) > 4_000_000:
            shape[int(rng.integers(0, nd))] //= 4
            shape = [max(1, s) for s in shape]
        op = OPS[int(rng.integers(0, len(OPS)))]
        # base with room for a leading offset and a stride-2 view on one dim
        step = [1] * nd
        if rng.random() < 0.3:
            step[int(rng.integers(0, nd))] = 2
        off = int(rng.integers(0, 2)) if rng.random() < 0.3 else 0
        bshape = [s * st for s, st in zip(shape, step)]
        bshape[-1] += off
        base = (rng.standard_normal(bshape) * 2 + 0.25).astype(np.float32)
        if rng.random() < 0.2:
            base = np.round(base)  # ties (arg ops) and zeros (all / any)
        sl = tuple(slice(0, s * st, st) for s, st in zip(shape, step))
        sl = sl[:-1] + (slice(off, off + shape[-1] * step[-1], step[-1]),)
        v = base[sl]
        if op in ("argmax", "argmin"):
            dims = None if rng.random() < 0.3 else [int(rng.integers(0, nd))]
        else:
            r = rng.random()
            dims = None if r < 0.2 else sorted(set(int(d) for d in rng.choice(nd, size=int(rng.integers(1, nd + 1)))))
        tb = torch.from_numpy(base).cuda()
        t = tb[sl]
        if op == "norm":
            check(v, t, op, dims, p=float(rng.choice([1.0, 2.0, 3.0, np.inf])))
        else:
            check(v, t, op, dims, correction=int(rng.integers(0, 2)))
        del tb, t
