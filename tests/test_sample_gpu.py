"""GPU parity of tpr_sample (top-k / top-p sampling) through the C-ABI and the
dispatcher, against the oracle.  The draw depends on float comparisons against
cumulative sums, which the GPU forms in float32 and the oracle in float64: ids
must be equal wherever both decision thresholds are further than 1e-5 (relative)
from every cumulative sum; closer than that, the GPU id must still lie in the
oracle's nucleus (a boundary draw).  Greedy and k = 1 cases are bit-exact."""
import numpy as np
import pytest

import tensorplay_amd as tp
from oracle import oracle as O
from tensorplay_amd import _capi

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def check(x, u, k, T, top_p):
    print(f"case sample shape={x.shape} k={k} T={T} top_p={top_p}", flush=True)
    got = _capi.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda(), k, T, top_p).cpu().numpy()
    exp, margin, m, j, cut_margin = O.sample(x, u, k, T, top_p, details=True)
    sure = margin > 1e-5
    np.testing.assert_array_equal(got[sure], exp[sure])
    if (~sure).any():
        _, idx = O.topk(x, k)
        for r in np.nonzero(~sure)[0]:
            # a boundary draw: the GPU's position in the top-k order is the
            # oracle's or a neighbour, and inside the oracle's nucleus 0..m
            # (0..m+1 when the top-p cut itself is within float32 rounding)
            pos = np.nonzero(idx[r] == got[r])[0]
            assert pos.size == 1, (r, got[r])
            m_hi = m[r] + (1 if cut_margin[r] <= 1e-5 else 0)
            assert pos[0] <= m_hi, (r, pos[0], m[r])
            assert abs(int(pos[0]) - int(j[r])) <= 1, (r, pos[0], j[r])
    return int((~sure).sum())


def test_boundary_draws_stay_in_the_nucleus():
    # u placed exactly on cumulative sums and top_p exactly on c_j / c_{k-1}:
    # every row is a boundary case, checked by the nucleus rule above
    rng = np.random.default_rng(33)
    x = (rng.standard_normal((64, 500)) * 2).astype(np.float32)
    _, _, m, j, _ = O.sample(x, np.full(64, 0.5, np.float32), 20, 1.0, 1.0, details=True)
    vals, _ = O.topk(x, 20)
    p = np.exp(vals.astype(np.float64) - vals[:, :1])
    c = np.cumsum(p, axis=1)
    u = (c[np.arange(64), rng.integers(0, 19, 64)] / c[:, -1]).astype(np.float32)
    n = check(x, u, 20, 1.0, 1.0)
    assert n > 0  # the construction produced boundary rows
    top_p = float(c[0, 9] / c[0, -1])
    check(x, rng.random(64).astype(np.float32), 20, 1.0, top_p)


def test_parameter_grid():
    rng = np.random.default_rng(30)
    for rows, cols in [(1, 1), (7, 10), (33, 1000), (16, 32768), (3, 40000)]:
        x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
        u = rng.random(rows).astype(np.float32)
        for k in sorted({1, min(cols, 7), min(cols, 50), min(cols, 64), min(cols, 100), min(cols, 1024)}):
            for T in (0.0, 0.7, 1.0, 2.0):
                for top_p in (0.1, 0.5, 0.9, 1.0):
                    check(x, u, k, T, top_p)


def test_llm_logits_c5_shape():
    # [256, 151936] N(0, 3) logits with 8 boosted positions per row, k = 50
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((256, 151936)) * 3).astype(np.float32)
    for r in range(256):
        x[r, rng.choice(151936, 8, replace=False)] += 15.0
    u = rng.random(256).astype(np.float32)
    for T, top_p in ((1.0, 0.9), (0.7, 0.95), (1.3, 1.0)):
        check(x, u, 50, T, top_p)


def test_ties_and_greedy():
    x = np.zeros((4, 300), np.float32)
    x[:, 5] = x[:, 17] = 2.0
    u = np.array([0.0, 0.4, 0.6, 0.99], np.float32)
    got = _capi.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda(), 2, 1.0, 1.0).cpu().numpy()
    np.testing.assert_array_equal(got, [5, 5, 17, 17])   # equal halves: u < 0.5 -> index 5
    got = _capi.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda(), 10, 0.0, 0.5).cpu().numpy()
    np.testing.assert_array_equal(got, [5, 5, 5, 5])


def test_dispatcher_op():
    rng = np.random.default_rng(32)
    x = rng.standard_normal((3, 4, 500)).astype(np.float32)
    u = rng.random(12).astype(np.float32)
    ids = tp.topk_topp_sample(tp.tensor(x, device="rocm"), tp.tensor(u.reshape(3, 4), device="rocm"), 20, 0.8, 0.9)
    assert ids.shape == [3, 4] and ids.dtype == tp.int64
    exp, margin = O.sample(x.reshape(12, 500), u, 20, 0.8, 0.9)
    got = ids.numpy().reshape(12)
    assert np.array_equal(got[margin > 1e-5], exp[margin > 1e-5])
    with pytest.raises(RuntimeError):
        tp.topk_topp_sample(tp.tensor(x, device="rocm"), tp.tensor(u, device="rocm"), 20, 1.0, 1.5)


def check_large_k(x, u, k, T, top_p, tol=1e-5):
    """k > 1024 (the sorted top k drawn by a second kernel).  Long tails hold
    many positions whose p_j lies below float32 rounding of the cumulative
    sums, so a boundary draw may land several positions from the oracle's;
    the rule: the GPU's position pos must satisfy the draw's inequalities on
    the oracle's float64 sums up to tol * c_{k-1}, i.e. pos <= m_hi (the last
    nucleus end the cut allows within tol), c_pos > u*c_m - tol and
    c_{pos-1} <= u*c_m + tol; rows with margin > tol must match exactly."""
    print(f"case sample_large shape={x.shape} k={k} T={T} top_p={top_p}", flush=True)
    got = _capi.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda(), k, T, top_p).cpu().numpy()
    exp, margin, m, _, _ = O.sample(x, u, k, T, top_p, details=True)
    sure = margin > tol
    np.testing.assert_array_equal(got[sure], exp[sure])
    if not T > 0:
        np.testing.assert_array_equal(got, exp)
        return
    vals, idx = O.topk(x, k)
    for r in np.nonzero(~sure)[0]:
        c = np.cumsum(np.exp(vals[r].astype(np.float64) / T - vals[r, 0] / T))
        e = tol * c[-1]
        hit = np.nonzero(c >= top_p * c[-1] + e)[0]
        m_hi = int(hit[0]) if hit.size else k - 1
        pos = np.nonzero(idx[r] == got[r])[0]
        assert pos.size == 1, (r, got[r])
        p = int(pos[0])
        thr = float(u[r]) * c[m[r]]
        assert p <= m_hi, (r, p, m_hi)
        assert c[p] > thr - e or p == m_hi, (r, p)
        assert p == 0 or c[p - 1] <= thr + e, (r, p)


def test_large_k_and_top_p_alone():
    rng = np.random.default_rng(34)
    for rows, cols, ks in [(33, 5000, (1025, 2000, 5000)), (5, 40000, (1025, 4096, 40000)), (2, 1025, (1025,))]:
        x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
        u = rng.random(rows).astype(np.float32)
        for k in ks:
            for T, top_p in ((1.0, 1.0), (0.7, 0.9), (1.5, 0.5), (0.0, 0.9), (1.0, 1e-6)):
                check_large_k(x, u, k, T, top_p)


def test_large_k_llm_logits_c5_shape():
    # top-p alone over the whole vocabulary of C5-shaped logits (k = cols)
    rng = np.random.default_rng(35)
    rows, cols = 16, 151936
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    for r in range(rows):
        x[r, rng.choice(cols, 8, replace=False)] += 15.0
    u = rng.random(rows).astype(np.float32)
    for T, top_p in ((1.0, 0.9), (0.7, 0.95), (1.3, 1.0)):
        check_large_k(x, u, cols, T, top_p)
    check_large_k(x, u, 2048, 1.0, 0.9)


def test_large_k_ties():
    # equal logits: ranks fall to the lowest index, the draw splits evenly
    x = np.zeros((4, 3000), np.float32)
    u = np.array([0.0, 0.25, 0.5, 0.999], np.float32)
    got = _capi.sample(torch.from_numpy(x).cuda(), torch.from_numpy(u).cuda(), 2000, 1.0, 1.0).cpu().numpy()
    exp, margin = O.sample(x, u, 2000, 1.0, 1.0)
    np.testing.assert_array_equal(got[margin > 1e-5], exp[margin > 1e-5])
    assert got[0] == 0 and np.all(got < 2000)


def test_random_sweep():
    """Fixed-seed sweep over row counts, row lengths, k on both sides of 1024
    (the draw inside top-k, and the sorted top-k plus the draw kernel),
    temperatures (greedy included) and top_p, with logits of three spreads."""
    rng = np.random.default_rng(20261202)
    for case in range(36):
        rows = int(rng.choice([1, 3, 17, 64, 300]))
        cols = int(rng.choice([50, 1000, 1500, 5000, 32768, 70000]))
        k = int(min(cols, rng.choice([1, 8, 50, 256, 1024, 1025, 3000, cols])))
        T = float(rng.choice([0.0, 0.5, 1.0, 1.7]))
        top_p = float(rng.choice([0.05, 0.5, 0.9, 0.99, 1.0]))
        scale = float(rng.choice([0.5, 2.0, 6.0]))
        x = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
        u = rng.random(rows).astype(np.float32)
        print(f"sweep case {case}", flush=True)
        if k > 1024:
            check_large_k(x, u, k, T, top_p)
        else:
            check(x, u, k, T, top_p)
