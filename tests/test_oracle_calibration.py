"""Pins of the oracle's 1-D k-means (the GPU calibration fit's restatement)
and of the calibration's quantile definition, on the CPU.

The fit has no counterpart in the reference (which calls sklearn,
src/kvquant/calibration.py:106-123), so it is pinned by what the mathematics
fixes: known answers of the start and of well-separated clusters, the Lloyd
fixed point (every centre is the mean of the values nearest to it), and its
quality against sklearn's KMeans on the same values.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O

RNG = np.random.default_rng(17)


def test_padding_known_answers():
    # src/kvquant/calibration.py:113-119: no values -> zeros; n < k -> values + zeros, sorted
    assert np.array_equal(O.kmeans_1d(np.zeros(0, np.float32), 4, 20), np.zeros(4, np.float32))
    got = O.kmeans_1d(np.array([3.0, -1.0], np.float32), 4, 20)
    assert np.array_equal(got, np.array([-1.0, 0.0, 0.0, 3.0], np.float32))


def test_starts_known_answers():
    # order statistics floor((2l+1) n / 2k) of 0..99 at k = 4: 12, 37, 62, 87
    v = RNG.permutation(np.arange(100)).astype(np.float32)
    assert np.array_equal(O.kmeans_1d(v, 4, 0), np.array([12, 37, 62, 87], np.float32))
    # more than 8192 values: evenly over [0, 8] -> 1, 3, 5, 7
    w = np.concatenate([[0.0, 8.0], RNG.uniform(0, 8, 9000)]).astype(np.float32)
    assert np.array_equal(O.kmeans_1d(w, 4, 0), np.array([1, 3, 5, 7], np.float32))


def test_separated_clusters_are_their_means():
    parts = [c + RNG.uniform(-0.01, 0.01, 300) for c in (-10.0, 0.0, 10.0)]
    v = np.concatenate(parts).astype(np.float32)
    want = np.array([np.float32(p.astype(np.float32).astype(np.float64).mean()) for p in parts])
    assert np.array_equal(O.kmeans_1d(RNG.permutation(v), 3, 10), want)


@pytest.mark.parametrize("k", [2, 4, 16])
def test_lloyd_fixed_point(k):
    v = RNG.standard_normal(3000).astype(np.float32)
    c = O.kmeans_1d(v, k, 300)
    near = np.argmin(np.abs(v[:, None].astype(np.float64) - c[None, :]), axis=1)
    for l in range(k):
        members = v[near == l]
        assert members.size > 0
        assert c[l] == np.float32(members.astype(np.float64).mean()), l


@pytest.mark.parametrize("dist,k", [("normal", 4), ("normal", 16), ("t3clip", 4), ("t3clip", 16)])
def test_quality_against_sklearn(dist, k):
    from sklearn.cluster import KMeans

    x = RNG.standard_normal(5000) if dist == "normal" else RNG.standard_t(3, 5000)
    if dist == "t3clip":   # the calibration clips at the 0.5 / 99.5 % quantiles
        lo, up = np.quantile(x, [0.005, 0.995])
        x = x[(x >= lo) & (x <= up)]
    x = x.astype(np.float32)
    ours = O.kmeans_inertia(x, O.kmeans_1d(x, k, 50))
    sk = KMeans(n_clusters=k, n_init=3, max_iter=20, random_state=0).fit(x.reshape(-1, 1))
    assert ours <= 1.10 * O.kmeans_inertia(x, sk.cluster_centers_.ravel())


def test_row_quantiles_match_numpy():
    import torch
    from kvquant.calibration import row_quantiles

    # the reference calls np.quantile on float32 rows (calibration.py:141-142,
    # :176-177), which interpolates in float32; bit-equal on every row
    for n in (1, 2, 1001, 16384):
        X = RNG.standard_t(3, (64, n)).astype(np.float32)
        for q in (0.005, 0.5, 0.995, 0.0, 1.0, 0.025):
            got = row_quantiles(torch.from_numpy(X), q).numpy()
            want = np.quantile(X, q, axis=1)
            assert want.dtype == np.float32
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, q)


# ------------------------------------------------- the optimal fit (default)

def _sse(v: np.ndarray, labels: np.ndarray, k: int) -> float:
    s = 0.0
    for l in range(k):
        m = v[labels == l].astype(np.float64)
        if m.size:
            s += float(((m - m.mean()) ** 2).sum())
    return s


@pytest.mark.parametrize("n,k,seed", [(7, 2, 0), (8, 3, 1), (9, 3, 2), (6, 4, 3)])
def test_optimal_equals_brute_force_over_all_assignments(n, k, seed):
    """Every assignment of n values to k labels (k^n of them, no contiguity
    assumed): the least sum of squared deviations equals the oracle fit's
    inertia."""
    import itertools

    rng = np.random.default_rng(seed)
    v = rng.standard_normal(n).astype(np.float32)
    best = min(_sse(v, np.array(lab), k) for lab in itertools.product(range(k), repeat=n)
               if len(set(lab)) == k)
    got = O.kmeans_inertia(v, O.kmeans_optimal(v, k))
    assert abs(got - best) <= 1e-6 * max(1.0, best)


@pytest.mark.parametrize("dist,k", [("normal", 4), ("normal", 16), ("t3clip", 4), ("t3clip", 16)])
def test_optimal_never_worse_than_sklearn_or_lloyd(dist, k):
    """The calibration's problems (5000 in-threshold values): the optimal fit
    is at most sklearn's KMeans(n_init=3, max_iter=20) inertia (the
    reference's fit, calibration.py:121) and at most the Lloyd fit's."""
    from sklearn.cluster import KMeans

    for rep in range(3):
        x = RNG.standard_normal(5000) if dist == "normal" else RNG.standard_t(3, 5000)
        if dist == "t3clip":
            lo, up = np.quantile(x, [0.005, 0.995])
            x = x[(x >= lo) & (x <= up)]
        x = x.astype(np.float32)
        opt = O.kmeans_inertia(x, O.kmeans_optimal(x, k))
        sk = KMeans(n_clusters=k, n_init=3, max_iter=20, random_state=rep).fit(x.reshape(-1, 1))
        assert opt <= O.kmeans_inertia(x, sk.cluster_centers_.ravel()) * (1 + 1e-6)
        assert opt <= O.kmeans_inertia(x, O.kmeans_1d(x, k, 50)) * (1 + 1e-6)


def test_optimal_known_answers():
    # separated clusters: their means; padding as the reference; k = 1: the mean
    parts = [c + RNG.uniform(-0.01, 0.01, 300) for c in (-10.0, 0.0, 10.0)]
    v = np.concatenate(parts).astype(np.float32)
    want = np.array([np.float32(np.sort(p.astype(np.float32)).astype(np.float64).sum() / p.size)
                     for p in parts])
    got = O.kmeans_optimal(RNG.permutation(v), 3)
    assert np.allclose(got, want, rtol=0, atol=1e-6)
    assert np.array_equal(O.kmeans_optimal(np.array([3.0, -1.0], np.float32), 4),
                          np.array([-1.0, 0.0, 0.0, 3.0], np.float32))
    w = RNG.standard_normal(1000).astype(np.float32)
    assert abs(O.kmeans_optimal(w, 1)[0] - w.astype(np.float64).mean()) < 1e-6
    # the optimal partition of sorted values is contiguous: each centre is the
    # mean of the values nearest to it (a Lloyd fixed point)
    c = O.kmeans_optimal(w, 8)
    near = np.argmin(np.abs(w[:, None].astype(np.float64) - c[None, :]), axis=1)
    for l in range(8):
        assert abs(c[l] - w[near == l].astype(np.float64).mean()) < 1e-5
    # more than 6144 values: not solved
    assert np.isnan(O.kmeans_optimal(np.zeros(6145, np.float32), 4)).all()
