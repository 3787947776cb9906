"""Pins the oracle's fit functions (CPU only): ``kmeans`` (reference
codec.py:53-103), ``covariance_block_permutation`` (rotation.py:179-248) and
``fit_profileperm_baseline`` (codec.py:299-418 in baseline mode).

Each check is one a plausible mistake fails: hand-worked Lloyd steps with
the reference's initial rows, the Lloyd descent property, the fixed-point
property of converged centroids, empty clusters, the zero-padded short case;
a covariance whose greedy packing is worked out by hand (its seed changes if
the diagonal is not zeroed), uncorrelated dims (identity, the first-index
tie rule); the fit's per-block initial rows and seeds in closed form.
"""

import numpy as np
import pytest

from oracle import sunshape_oracle as O


def test_kmeans_one_hand_worked_step():
    """Six 2-D points, K = 2, seed 0: RandomState(0).permutation(6)[:2] =
    [5, 2], so C = (x5, x2) = ((10, 11), (0, 1)).  Every point goes to the
    nearer of the two: {x3, x4, x5} -> 0, {x0, x1, x2} -> 1, and the update
    gives their means (31/3, 31/3) and (1/3, 1/3), rounded to float32."""
    x = np.array([[0, 0], [1, 0], [0, 1], [10, 10], [11, 10], [10, 11]], np.float32)
    assert np.random.RandomState(0).permutation(6)[:2].tolist() == [5, 2]
    c0 = O.kmeans(x, 2, 0, seed=0)
    assert c0.tolist() == [[10, 11], [0, 1]]
    c1 = O.kmeans(x, 2, 1, seed=0)
    third = np.float32(1.0 / 3.0)
    big = np.float32(31.0 / 3.0)
    assert c1.dtype == np.float32
    assert c1.tolist() == [[big, big], [third, third]]
    # a second step changes nothing (fixed point)
    assert np.array_equal(O.kmeans(x, 2, 2, seed=0), c1)


def test_kmeans_seed_selects_initial_rows():
    """Seed 1 starts from rows (2, 1) = ((0, 1), (1, 0)): x0 and x3 are
    equidistant and go to centroid 0 (first index), x4 to 1, x5 to 0."""
    x = np.array([[0, 0], [1, 0], [0, 1], [10, 10], [11, 10], [10, 11]], np.float32)
    assert np.random.RandomState(1).permutation(6)[:2].tolist() == [2, 1]
    c = O.kmeans(x, 2, 1, seed=1)
    # cluster 0 = {x0, x2, x3, x5}, cluster 1 = {x1, x4}
    assert c.tolist() == [[np.float32(20 / 4), np.float32(22 / 4)], [6.0, 5.0]]


def test_kmeans_empty_cluster_keeps_its_centroid():
    """Seed 0 with N = 5 starts from rows (2, 0), which are the same point:
    every point ties and goes to centroid 0 (first index), centroid 1 gets
    no points and keeps its value."""
    x = np.array([[0, 0], [2, 0], [0, 0], [4, 4], [6, 2]], np.float32)
    assert np.random.RandomState(0).permutation(5)[:2].tolist() == [2, 0]
    c = O.kmeans(x, 2, 1, seed=0)
    assert c.tolist() == [[np.float32(12 / 5), np.float32(6 / 5)], [0.0, 0.0]]


def test_kmeans_short_data_is_zero_padded():
    x = np.arange(6, dtype=np.float32).reshape(3, 2) + 1
    c = O.kmeans(x, 4, 10, seed=3)
    assert c.tolist() == [[1, 2], [3, 4], [5, 6], [0, 0]]


def _inertia(x, c):
    d2 = ((x[:, None, :].astype(np.float64) - c[None].astype(np.float64)) ** 2).sum(-1)
    return d2.min(1).sum(), d2.argmin(1)


def test_kmeans_distortion_never_increases():
    """Lloyd's descent property: the distortion after i + 1 steps is at most
    the distortion after i (same seed, so the same trajectory)."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((300, 8)) * rng.uniform(0.5, 3.0, 8)).astype(np.float32)
    prev = np.inf
    for it in range(0, 12):
        cur, _ = _inertia(x, O.kmeans(x, 16, it, seed=7))
        assert cur <= prev * (1 + 1e-6)
        prev = cur


def test_kmeans_converged_centroids_are_cluster_means():
    """At convergence every non-empty cluster's centroid is the float64 mean
    of its points (to float32 rounding)."""
    rng = np.random.default_rng(6)
    x = rng.standard_normal((200, 4)).astype(np.float32)
    c = O.kmeans(x, 8, 200, seed=11)
    _, a = _inertia(x, c)
    for k in range(8):
        pts = x[a == k].astype(np.float64)
        if len(pts):
            assert np.allclose(c[k], pts.mean(0), rtol=1e-5, atol=1e-6)


def _hadamard8():
    h = np.array([[1]])
    for _ in range(3):
        h = np.block([[h, h], [h, -h]])
    return h.astype(np.float32)


def test_covariance_permutation_hand_worked_greedy():
    """Two orthogonal zero-mean factors (columns of an 8 x 8 Hadamard
    matrix), so the sample covariance is exactly (8 / 7) L^T L.  Factor A
    loads dims 1, 3, 5 with weights 1, 2, 4; factor B dims 0, 2, 4 with 3, 2,
    3.  Off-diagonal |cov| row sums (x 8/7): dim0 15, dim1 6, dim2 12, dim3
    10, dim4 15, dim5 12 -> seed dim0 (first of the two maxima, whose sums
    add the same two terms); gains to {0}: dim4 9, dim2 6 -> dim4; then
    dim2.  Three dims remain = block_dim -> sorted.  Expected [0, 4, 2, 1, 3,
    5].  (Without the zeroed diagonal the seed would be dim5: 12 + 16 = 28
    against dim0's 15 + 9.)"""
    z = _hadamard8()[:, 1:3]
    load = np.zeros((2, 6), np.float32)
    load[0, [1, 3, 5]] = [1, 2, 4]
    load[1, [0, 2, 4]] = [3, 2, 3]
    q = z @ load
    assert O.covariance_block_permutation(q, 3).tolist() == [0, 4, 2, 1, 3, 5]


def test_covariance_permutation_three_blocks():
    """Nine dims in three factors, block_dim 3: factor A dims 6, 7, 8 with
    weights 5, 4, 3 (row sums 35, 32, 27); B dims 0, 3, 4 with 1, 1, 2 (3, 3,
    4); C dims 1, 2, 5 with 2, 2, 2 (8, 8, 8).  Seed dim6, then dim7, dim8;
    among the rest the seed is dim1 (8, first of C), then dim2, dim5; B
    remains (3 dims) sorted."""
    z = _hadamard8()[:, 1:4]
    load = np.zeros((3, 9), np.float32)
    load[0, [6, 7, 8]] = [5, 4, 3]
    load[1, [0, 3, 4]] = [1, 1, 2]
    load[2, [1, 2, 5]] = [2, 2, 2]
    q = z @ load
    assert O.covariance_block_permutation(q, 3).tolist() == [6, 7, 8, 1, 2, 5, 0, 3, 4]


def test_covariance_permutation_uncorrelated_is_identity():
    """Uncorrelated dims (orthogonal zero-mean columns with distinct
    variances): every affinity is zero, every argmax takes the first
    remaining dim, so the packing is the identity."""
    z = _hadamard8()[:, 1:7] * np.array([1, 3, 2, 5, 4, 6], np.float32)
    assert O.covariance_block_permutation(z, 2).tolist() == [0, 1, 2, 3, 4, 5]


@pytest.mark.parametrize("d,bd", [(16, 8), (24, 8), (20, 8)])
def test_covariance_permutation_is_a_permutation(d, bd):
    rng = np.random.default_rng(d)
    q = (rng.standard_normal((64, 4)) @ rng.standard_normal((4, d))).astype(np.float32)
    p = O.covariance_block_permutation(q, bd)
    assert p.dtype == np.int32 and sorted(p.tolist()) == list(range(d))


def test_fit_initial_rows_and_block_seeds():
    """With no Lloyd step the fit's centroids are the k-means initial rows of
    each block: block b of the permuted keys at rows
    RandomState(seed + b).permutation(N)[:K] (codec.py:79, 391); the
    permutation is the covariance packing of q_cal."""
    rng = np.random.default_rng(9)
    q = rng.standard_normal((64, 16)).astype(np.float32)
    k = rng.standard_normal((40, 16)).astype(np.float32)
    perm, cents = O.fit_profileperm_baseline(q, k, block_dim=8, n_centroids=8, kmeans_iters=0,
                                             seed=5)
    assert np.array_equal(perm, O.covariance_block_permutation(q, 8))
    kp = k[:, perm]
    for b in range(2):
        rows = np.random.RandomState(5 + b).permutation(40)[:8]
        assert np.array_equal(cents[b], kp[rows, b * 8:(b + 1) * 8])
    # fewer keys than centroids: the permuted rows, zero-padded
    _, short = O.fit_profileperm_baseline(q, k[:3], block_dim=8, n_centroids=8,
                                          kmeans_iters=4, seed=5)
    for b in range(2):
        assert np.array_equal(short[b, :3], k[:3][:, perm][:, b * 8:(b + 1) * 8])
        assert not short[b, 3:].any()
