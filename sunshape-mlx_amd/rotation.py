"""Transforms and fit-time statistics.

Per-step transforms (``apply_permutation``) are applied inside the HIP
kernels on the hot path; the helpers here serve the Python API and the
offline fit.  Fit-time statistics (ProfilePerm packing, block metrics,
kurtosis masks, rotations) run once on calibration data, in NumPy float32,
like the reference's (rotation.py in gauravsaini/sunshape-mlx); they are
off the per-step path.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def _np32(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().float().cpu().numpy()
    return np.asarray(x, dtype=np.float32)


# ------------------------------------------------------------------ #
#  Rotations                                                          #
# ------------------------------------------------------------------ #


def generate_rotation_matrix(d: int, seed: int = 0) -> np.ndarray:
    """Haar-random orthogonal matrix: QR of a seeded Gaussian matrix, columns
    multiplied by sign(diag(R)).  Same construction as reference
    rotation.py:29-50; the Gaussian draw uses NumPy's ``default_rng(seed)``
    (the reference's MLX generator is not available), so the matrix is a
    different draw of the same distribution."""
    g = np.random.default_rng(seed).standard_normal((d, d))
    q, r = np.linalg.qr(g)
    q = q * np.sign(np.diag(r))[None, :]
    return q.astype(np.float32)


def _is_power_of_2(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def generate_wht_signs(d: int, seed: int = 0) -> np.ndarray:
    """Random +-1 signs for the randomized Walsh-Hadamard transform
    (reference rotation.py:65-83: ``RandomState(seed).choice([-1, 1], d)``)."""
    if not _is_power_of_2(d):
        raise ValueError(f"WHT requires d to be a power of 2, got {d}")
    return np.random.RandomState(seed).choice([-1.0, 1.0], size=d).astype(np.float32)


def _fwht(x: torch.Tensor) -> torch.Tensor:
    d = x.shape[-1]
    shape = x.shape
    y = x.reshape(-1, d)
    h = 1
    while h < d:
        y = y.reshape(-1, d // (2 * h), 2, h)
        a, b = y[:, :, 0, :], y[:, :, 1, :]
        y = torch.stack((a + b, a - b), dim=2)
        h *= 2
    return y.reshape(shape)


def apply_wht(x, signs, inverse: bool = False):
    """``R x`` with ``R = H_d diag(signs) / sqrt(d)`` (inverse: ``x R``),
    by the O(d log d) butterfly (reference rotation.py:86-163)."""
    t = x if isinstance(x, torch.Tensor) else torch.as_tensor(np.asarray(x, np.float32))
    d = t.shape[-1]
    if not _is_power_of_2(d):
        raise ValueError(f"WHT requires last dim to be a power of 2, got {d}")
    s = torch.as_tensor(np.asarray(signs, np.float32) if not isinstance(signs, torch.Tensor)
                        else signs, dtype=torch.float32, device=t.device)
    t = t.float()
    scale = 1.0 / math.sqrt(d)
    if inverse:
        return _fwht(t) * s * scale
    return _fwht(t * s) * scale


# ------------------------------------------------------------------ #
#  ProfilePerm                                                        #
# ------------------------------------------------------------------ #


def _covariance(x: np.ndarray) -> np.ndarray:
    c = x - x.mean(axis=0, keepdims=True)
    return (c.T @ c) / np.float32(max(1, x.shape[0] - 1))


def covariance_block_permutation(q_cal, block_dim: int) -> np.ndarray:
    """Greedy affinity packing of dimensions into blocks (ProfilePerm,
    reference rotation.py:186-248): affinity = |cov| with a zero diagonal;
    each block starts from the remaining dim with the largest total affinity
    to the remaining dims and grows by the candidate with the largest summed
    affinity to the block.  Returns int32 (d,)."""
    q = _np32(q_cal)
    aff = np.abs(_covariance(q))
    np.fill_diagonal(aff, 0.0)
    d = aff.shape[0]
    remaining = list(range(d))
    ordered: list[int] = []
    while remaining:
        if len(remaining) <= block_dim:
            ordered.extend(remaining)
            break
        rem = np.array(remaining)
        seed = int(rem[int(aff[rem].sum(axis=1).argmax())])
        block = [seed]
        remaining.remove(seed)
        while len(block) < block_dim and remaining:
            cand = np.array(remaining)
            gains = aff[cand][:, np.array(block)].sum(axis=1)
            best = int(cand[int(gains.argmax())])
            block.append(best)
            remaining.remove(best)
        ordered.extend(block)
    return np.array(ordered, dtype=np.int32)


def invert_permutation(perm):
    """Inverse permutation (reference rotation.py:251-259); numpy or torch in,
    same kind out."""
    if isinstance(perm, torch.Tensor):
        inv = torch.empty_like(perm)
        inv[perm.long()] = torch.arange(perm.numel(), dtype=perm.dtype, device=perm.device)
        return inv
    p = np.asarray(perm)
    inv = np.empty_like(p)
    inv[p] = np.arange(p.shape[0], dtype=p.dtype)
    return inv


def apply_permutation(x, perm):
    """``x[..., perm]`` (reference rotation.py:262-266)."""
    if perm is None:
        return x
    if isinstance(x, torch.Tensor):
        p = perm if isinstance(perm, torch.Tensor) else torch.as_tensor(np.asarray(perm))
        if p.numel() == 0:
            return x
        return x.index_select(-1, p.to(device=x.device, dtype=torch.long))
    p = np.asarray(perm)
    return x if p.size == 0 else np.asarray(x)[..., p]


# ------------------------------------------------------------------ #
#  Block statistics (fit time)                                        #
# ------------------------------------------------------------------ #


def block_local_cov_metric(q_cal, perm, block_dim: int) -> np.ndarray:
    """Block-diagonal metric whose blocks are the covariance of the permuted
    calibration queries (reference rotation.py:274-303)."""
    q = apply_permutation(_np32(q_cal), np.asarray(perm))
    cov = _covariance(q)
    d = cov.shape[0]
    out = np.zeros((d, d), dtype=np.float32)
    for b in range(d // block_dim):
        sl = slice(b * block_dim, (b + 1) * block_dim)
        out[sl, sl] = cov[sl, sl]
    return out


def _top_mass_mask(mass: np.ndarray, threshold: float) -> np.ndarray:
    ranked = np.argsort(mass)[::-1]
    cumulative = np.cumsum(mass[ranked])
    cutoff = int((cumulative < threshold).sum()) + 1
    cutoff = max(1, min(cutoff, mass.shape[0]))
    mask = np.zeros(mass.shape[0], dtype=bool)
    mask[ranked[:cutoff]] = True
    return mask


def block_affinity_gate(q_cal, block_dim: int):
    """Per-block variance share and the blocks covering >= 50% of it;
    affinities of active blocks normalised to max 1 (reference
    rotation.py:311-353).  Returns ``(affinity f32 (nb,), active bool (nb,))``."""
    q = _np32(q_cal)
    c = q - q.mean(axis=0, keepdims=True)
    var = (c * c).mean(axis=0)
    nb = var.shape[0] // block_dim
    mass = var.reshape(nb, block_dim).sum(axis=1)
    aff = mass / max(float(mass.sum()), 1e-12)
    active = _top_mass_mask(aff.astype(np.float64), 0.5)
    act_aff = aff * active.astype(np.float32)
    act_aff = act_aff / max(float(act_aff.max()), 1e-12)
    return act_aff.astype(np.float32), active


def positive_excess_kurtosis(q) -> np.ndarray:
    """max(E[c^4] / var^2 - 3, 0) per dimension (reference rotation.py:361-369)."""
    x = _np32(q)
    c = x - x.mean(axis=0, keepdims=True)
    var = np.maximum((c * c).mean(axis=0), 1e-12)
    excess = (c ** 4).mean(axis=0) / (var * var) - 3.0
    return np.maximum(excess, 0.0).astype(np.float32)


def mixed_precision_block_mask(q_cal, block_dim: int, mass_threshold: float = 0.5):
    """Heavy-tailed blocks: the top blocks by kurtosis mass covering
    ``mass_threshold`` of the total (reference rotation.py:372-404).
    Returns ``(heavy bool (nb,), block_mass f32 (nb,))``."""
    k = positive_excess_kurtosis(q_cal)
    nb = k.shape[0] // block_dim
    mass = k.reshape(nb, block_dim).sum(axis=1)
    normed = mass / max(float(mass.sum()), 1e-12)
    return _top_mass_mask(normed.astype(np.float64), mass_threshold), mass.astype(np.float32)


def safe_normalize(x, axis: int = -1, eps: float = 1e-8):
    """Unit vectors and norms; zero vectors are left unscaled (reference
    rotation.py:412-420)."""
    t = x if isinstance(x, torch.Tensor) else torch.as_tensor(np.asarray(x, np.float32))
    n = torch.linalg.vector_norm(t.float(), dim=axis, keepdim=True)
    safe = torch.where(n < eps, torch.ones_like(n), n)
    return t / safe, n
