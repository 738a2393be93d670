"""Pins the oracle's top-k / top-p sampler (oracle.sample): it reduces to plain
inverse-CDF sampling of the full softmax when k = cols and top_p = 1, to argmax
when k = 1 or T <= 0, and over a dense grid of u its token frequencies are the
renormalised nucleus probabilities (brute force).  CPU only."""
import numpy as np

from oracle import oracle as O


def test_full_softmax_inverse_cdf():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((20, 37)) * 2).astype(np.float32)
    u = rng.random(20)
    ids, _ = O.sample(x, u, 37, 1.0, 1.0)
    for r in range(20):
        p = np.exp(x[r].astype(np.float64) - x[r].max())
        p /= p.sum()
        order = np.argsort(-x[r], kind="stable")
        c = np.cumsum(p[order])
        assert ids[r] == order[np.searchsorted(c, u[r] * c[-1], side="right")]


def test_greedy_cases():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((9, 100)).astype(np.float32)
    x[3, 10] = x[3, 20] = 9.0                     # tie: the lowest index wins
    u = rng.random(9)
    am = O.argmax(x, 1)
    assert np.array_equal(O.sample(x, u, 1, 1.0, 0.9)[0], am)
    assert np.array_equal(O.sample(x, u, 50, 0.0, 0.9)[0], am)
    assert O.sample(x, u, 50, -1.0, 0.5)[0][3] == 10
    assert np.array_equal(O.sample(x, np.zeros(9), 50, 1.0, 1.0)[0], am)   # u = 0 draws the top candidate


def test_grid_frequencies_are_the_nucleus_probabilities():
    x = np.array([[2.0, 1.0, 0.5, 0.0, -1.0, 3.0, -2.0, 1.5]], np.float32)
    k, T, top_p = 6, 0.7, 0.8
    n = 20000
    us = (np.arange(n) + 0.5) / n
    counts = {}
    for uu in us:
        t = int(O.sample(x, np.array([uu]), k, T, top_p)[0][0])
        counts[t] = counts.get(t, 0) + 1
    # expected: top-6 by value, softmax at T, smallest prefix with mass >= top_p, renormalised
    order = np.argsort(-x[0], kind="stable")[:k]
    p = np.exp(x[0][order].astype(np.float64) / T - x[0][order[0]] / T)
    c = np.cumsum(p) / p.sum()
    m = int(np.nonzero(c >= top_p)[0][0])
    q = p[: m + 1] / p[: m + 1].sum()
    assert set(counts) == set(order[: m + 1].tolist())
    for j, tok in enumerate(order[: m + 1]):
        assert abs(counts[tok] / n - q[j]) <= 1e-3
