"""Pins the oracle's block-VQ encoder (CPU only).

Checks are chosen so that plausible mistakes fail: exact rational brute force
(wrong distance, dropped term, wrong tie order), the reference's seeded
known-answer test [13] (reference test_kernels.py:404-439), duplicate-centroid
ties, permutation handling, and agreement of the NumPy and C restatements.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import sunshape_oracle as O


def brute_force_exact(keys, cents, perm=None):
    """argmin over centroids in exact rational arithmetic, lowest index first."""
    k = np.asarray(keys, np.float32)
    if perm is not None:
        k = k[:, perm]
    nb, nc, bd = cents.shape
    out = np.zeros((k.shape[0], nb), np.int64)
    for t in range(k.shape[0]):
        for b in range(nb):
            best, bi = None, 0
            for c in range(nc):
                d = sum((Fraction(float(k[t, b * bd + j])) - Fraction(float(cents[b, c, j]))) ** 2
                        for j in range(bd))
                if best is None or d < best:
                    best, bi = d, c
            out[t, b] = bi
    return out


def test_encode_matches_exact_brute_force_tiny():
    rng = np.random.default_rng(11)
    keys = rng.standard_normal((6, 16)).astype(np.float32)
    cents = rng.standard_normal((2, 9, 8)).astype(np.float32)
    perm = rng.permutation(16).astype(np.int32)
    idx, near = O.encode_blockvq(keys, cents, perm)
    assert not near.any()
    assert np.array_equal(idx.astype(np.int64), brute_force_exact(keys, cents, perm))


def test_known_answer_13_seed_333():
    """Reference test [13]: keys/centroids from np.random.seed(333); the
    expected indices are the float32 NumPy argmin of the explicit distances
    (reference test_kernels.py:415-423), exact on every non-near-tie pair."""
    np.random.seed(333)
    n, nb, nc, bd = 32, 16, 256, 8
    keys = np.random.randn(n, nb * bd).astype(np.float32)
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    ref = np.zeros((n, nb), np.int32)
    for b in range(nb):
        diff = keys[:, b * bd:(b + 1) * bd][:, None, :] - cents[b][None]
        ref[:, b] = np.argmin(np.sum(diff ** 2, axis=-1), axis=1)
    idx, near = O.encode_blockvq(keys, cents)
    assert np.array_equal(idx[~near].astype(np.int32), ref[~near])
    assert near.sum() == 0


def test_duplicate_centroids_resolve_to_lowest_index():
    rng = np.random.default_rng(5)
    cents = rng.standard_normal((1, 6, 8)).astype(np.float32)
    cents[0, 4] = cents[0, 1]           # exact duplicate
    keys = cents[0, [1, 4, 2]] + 1e-3   # near the duplicated pair and near 2
    idx, near = O.encode_blockvq(keys.astype(np.float32), cents)
    assert idx[0, 0] == 1 and idx[1, 0] == 1 and idx[2, 0] == 2
    assert not near.any()               # exact ties are not near-ties


def test_zero_padded_codebook_ties():
    """k-means with N <= K zero-pads the codebook (reference codec.py:73-76):
    every padded centroid ties and the lowest index must win."""
    cents = np.zeros((1, 8, 8), np.float32)
    cents[0, :3] = np.eye(8, dtype=np.float32)[:3] * 5
    keys = np.zeros((2, 8), np.float32)
    keys[1, 0] = 4.9
    idx, near = O.encode_blockvq(keys, cents)
    assert idx[0, 0] == 3 and idx[1, 0] == 0 and not near.any()


def test_near_tie_is_flagged():
    cents = np.zeros((1, 2, 8), np.float32)
    cents[0, 0, 0] = 1.0
    cents[0, 1, 0] = -1.0
    keys = np.zeros((1, 8), np.float32)
    keys[0, 0] = 1e-8  # distances differ by ~4e-8 relative: a near-tie
    _, near = O.encode_blockvq(keys, cents)
    assert near[0, 0]
    keys[0, 0] = 0.5
    _, near = O.encode_blockvq(keys, cents)
    assert not near[0, 0]


def test_permutation_is_applied_before_blocking():
    rng = np.random.default_rng(2)
    keys = rng.standard_normal((50, 32)).astype(np.float32)
    cents = rng.standard_normal((4, 16, 8)).astype(np.float32)
    perm = rng.permutation(32).astype(np.int32)
    a, _ = O.encode_blockvq(keys, cents, perm)
    b, _ = O.encode_blockvq(keys[:, perm], cents)
    assert np.array_equal(a, b)
    c, _ = O.encode_blockvq(keys, cents)  # planted mistake: permutation dropped
    assert not np.array_equal(a, c)


def test_c_restatement_agrees_with_numpy():
    rng = np.random.default_rng(8)
    keys = rng.standard_normal((700, 128)).astype(np.float16)
    cents = rng.standard_normal((16, 256, 8)).astype(np.float32)
    cents[:, 9] = cents[:, 2]
    perm = rng.permutation(128).astype(np.int32)
    a, na = O.encode_blockvq(keys, cents, perm)
    b, nb_ = O.encode_blockvq_c(keys, cents, perm)
    assert np.array_equal(a, b) and np.array_equal(na, nb_)


def test_encode_decode_idempotent():
    """Encoding a reconstructed key returns the same indices (each block of
    k_hat IS a centroid), whenever the codebook has no duplicates."""
    rng = np.random.default_rng(4)
    cents = rng.standard_normal((16, 256, 8)).astype(np.float32)
    perm = rng.permutation(128).astype(np.int32)
    keys = rng.standard_normal((200, 128)).astype(np.float32)
    idx, _ = O.encode_blockvq(keys, cents, perm)
    k_hat = O.dequantize_blockvq(idx, cents, O.invert_permutation(perm))
    idx2, near = O.encode_blockvq(k_hat, cents, perm)
    assert not near.any()
    assert np.array_equal(idx, idx2)


@pytest.mark.parametrize("nc,dtype", [(256, np.uint8), (300, np.uint16)])
def test_index_dtype_follows_codebook_size(nc, dtype):
    """uint8 up to 256 centroids, uint16 above (reference codec.py:203-209)."""
    rng = np.random.default_rng(1)
    idx, _ = O.encode_blockvq(rng.standard_normal((3, 8)).astype(np.float32),
                              rng.standard_normal((1, nc, 8)).astype(np.float32))
    assert idx.dtype == dtype
