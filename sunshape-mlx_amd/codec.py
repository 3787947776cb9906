"""SunShape block-VQ codec (keys -> uint8 centroid indices).

Same API as the reference's ``SunShapeBlockCodec`` (gauravsaini/sunshape-mlx
codec.py:217-650).  Codec state lives in torch tensors on one device; the
per-step operations run on the HIP kernels:

  quantize                    -> ss_encode_blockvq (permutation fused)
  dequantize / __call__       -> ss_dequantize_blockvq
  precompute_query_centroid_dots, attention_scores
                              -> ss_build_lut + ss_score_gather

``fit`` is offline calibration (ProfilePerm + per-block Lloyd k-means, DSQ
refinement for the local-metric mode) and, like the reference's, runs in
NumPy on the host.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import numpy as np
import torch

from . import _hip
from .rotation import (
    apply_permutation,
    block_affinity_gate,
    block_local_cov_metric,
    covariance_block_permutation,
    generate_rotation_matrix,
    invert_permutation,
    mixed_precision_block_mask,
)

PERM_MODES = ("profileperm_baseline", "profileperm_localmetric_dsq", "profileperm_mixed_precision")
MODES = PERM_MODES + ("rotated",)


class SunShapeQuantized(NamedTuple):
    """Quantized keys (reference codec.py:38-45)."""
    indices: torch.Tensor  # (n_tokens, n_blocks) uint8
    head_dim: int
    block_dim: int
    n_blocks: int
    passthrough_blocks: torch.Tensor | None = None   # (n_blocks,) bool
    passthrough_values: torch.Tensor | None = None   # (n_tokens, n_blocks, block_dim) f32


def _compact_index_dtype(n_centroids: int) -> torch.dtype:
    """Smallest dtype holding indices below n_centroids (codec.py:203-209)."""
    if n_centroids <= 256:
        return torch.uint8
    if n_centroids <= 65535:
        return torch.int32  # torch has no general uint16 arithmetic; indices fit
    return torch.int64


def _np(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().float().cpu().numpy()
    return np.asarray(x, dtype=np.float32)


def _kmeans(data: np.ndarray, n_centroids: int, n_iters: int = 25, seed: int = 0) -> np.ndarray:
    """Lloyd k-means (reference codec.py:53-103): zero-padded codebook when
    N <= K; initial centroids are the rows ``RandomState(seed).permutation(N)[:K]``;
    expanded-form float32 distances with first-index argmin; empty clusters
    keep their previous centroid."""
    x = np.asarray(data, dtype=np.float32)
    n, d = x.shape
    if n <= n_centroids:
        out = np.zeros((n_centroids, d), dtype=np.float32)
        out[:n] = x
        return out
    c = x[np.random.RandomState(seed).permutation(n)[:n_centroids]].copy()
    x_sq = np.sum(x ** 2, axis=1, keepdims=True)
    for _ in range(n_iters):
        dist = x_sq + np.sum(c ** 2, axis=1, keepdims=True).T - 2.0 * x @ c.T
        a = np.argmin(dist, axis=1)
        sums = np.zeros_like(c)
        np.add.at(sums, a, x)
        cnt = np.bincount(a, minlength=n_centroids).astype(np.float64)
        live = cnt > 0
        sums[live] /= cnt[live, None]
        sums[~live] = c[~live]
        c = sums
    return c.astype(np.float32)


def _softmax(x: np.ndarray) -> np.ndarray:
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def _refine_centroids(q_cal, k_cal, centroids, e_metric, block_dim, n_steps=3, step_size=0.1,
                      block_affinity=None, active_blocks=None) -> np.ndarray:
    """DSQ attention-aware centroid refinement (reference codec.py:111-189):
    gradient of (k_hat - k) + 0.5 * d(softmax error)/dk_hat on a calibration
    subset, applied per assigned centroid with a per-block step."""
    head_dim = k_cal.shape[-1]
    nb = head_dim // block_dim
    scale = math.sqrt(head_dim)
    q = np.asarray(q_cal[:min(128, q_cal.shape[0])], np.float32)
    k = np.asarray(k_cal[:min(1024, k_cal.shape[0])], np.float32)
    e = np.asarray(e_metric, np.float32)
    cents = np.array(centroids, np.float32, copy=True)
    ba = np.ones(nb, np.float32) if block_affinity is None else np.asarray(block_affinity)
    ab = np.ones(nb, bool) if active_blocks is None else np.asarray(active_blocks, bool)
    nc = cents.shape[1]

    def assign(b):
        sl = slice(b * block_dim, (b + 1) * block_dim)
        eb = e[sl, sl]
        ks = k[:, sl] @ eb.T
        cs = cents[b] @ eb.T
        return np.argmin(((ks[:, None, :] - cs[None]) ** 2).sum(-1), axis=1)

    k_hat = np.zeros_like(k)
    for b in range(nb):
        k_hat[:, b * block_dim:(b + 1) * block_dim] = cents[b][assign(b)]
    for _ in range(n_steps):
        p_orig = _softmax((q @ k.T) / scale)
        p_hat = _softmax((q @ k_hat.T) / scale)
        grad_attn = (((p_hat - p_orig) * p_hat * (1.0 - p_hat)).T @ q) / scale
        total = (k_hat - k) + 0.5 * grad_attn
        for b in range(nb):
            if not ab[b]:
                continue
            sl = slice(b * block_dim, (b + 1) * block_dim)
            a = assign(b)
            cnt = np.bincount(a, minlength=nc)
            gsum = np.zeros((nc, block_dim), np.float32)
            np.add.at(gsum, a, total[:, sl])
            live = cnt > 0
            new = cents[b].copy()
            new[live] -= step_size * float(ba[b]) * (gsum[live] / cnt[live, None])
            cents[b] = new
            k_hat[:, sl] = new[a]
    return cents


class SunShapeBlockCodec:
    """Block vector quantisation codec (reference codec.py:217-650).

    Modes: ``profileperm_baseline``, ``profileperm_localmetric_dsq``,
    ``profileperm_mixed_precision``, ``rotated``.
    """

    def __init__(self, head_dim: int, block_dim: int = 8, n_centroids: int = 256, c: float = 5.0,
                 n_refine_dsq: int = 3, mode: str = "profileperm_baseline",
                 use_rotation: bool = False, rotation_seed: int = 0, device=None,
                 heavy_fp16: bool = False):
        if head_dim % block_dim != 0:
            raise ValueError("head_dim must be divisible by block_dim")
        self.head_dim = head_dim
        self.block_dim = block_dim
        self.n_blocks = head_dim // block_dim
        self.n_centroids = n_centroids
        self.c = c
        self.mode = "rotated" if use_rotation else mode
        if self.mode not in MODES:
            raise ValueError(f"Unknown SunShapeBlockCodec mode: {self.mode}")
        self.n_refine_dsq = n_refine_dsq
        # mixed precision: keep the heavy blocks' key dims in fp16 and score
        # them exactly (the intent of README.md:87); False keeps the
        # reference's zero contribution (codec.py:381-388)
        self.heavy_fp16 = bool(heavy_fp16)
        self.use_rotation = self.mode == "rotated"
        self.last_score_backend = "none"
        if device is None:
            device = "cuda" if torch.cuda.is_available() else "cpu"
        self._device = torch.device(device)
        d, nb = head_dim, self.n_blocks
        rot = generate_rotation_matrix(d, seed=rotation_seed) if self.use_rotation \
            else np.eye(d, dtype=np.float32)
        self._set_state(
            E=np.eye(d, dtype=np.float32), E_inv=np.eye(d, dtype=np.float32),
            centroids=np.zeros((nb, n_centroids, block_dim), np.float32),
            dsq_block_affinity=np.ones(nb, np.float32), dsq_active_blocks=np.ones(nb, bool),
            mixed_high_precision_blocks=np.zeros(nb, bool),
            mixed_block_mass=np.zeros(nb, np.float32),
            permutation=np.arange(d, dtype=np.int32), rotation=rot)

    # ---------------------------------------------------------------- state
    _STATE_KEYS = ("E", "E_inv", "centroids", "dsq_block_affinity", "dsq_active_blocks",
                   "mixed_high_precision_blocks", "mixed_block_mass", "permutation", "rotation")

    def _set_state(self, **arrays):
        for k, v in arrays.items():
            t = v if isinstance(v, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(v))
            setattr(self, k, t.to(self._device).contiguous())
        if "permutation" in arrays:
            self.permutation = self.permutation.to(torch.int32)
            self.inv_permutation = invert_permutation(self.permutation)
        self._shaped_centroids = None

    @property
    def device(self) -> torch.device:
        return self._device

    def to(self, device) -> "SunShapeBlockCodec":
        self._device = torch.device(device)
        self._set_state(**{k: getattr(self, k) for k in self._STATE_KEYS})
        return self

    def state_dict(self) -> dict:
        """Codec state as CPU tensors plus the configuration (the reference
        codec has no serialisation; this is the format ``load_state_dict``
        reads)."""
        sd = {k: getattr(self, k).detach().cpu() for k in self._STATE_KEYS}
        sd["config"] = dict(head_dim=self.head_dim, block_dim=self.block_dim,
                            n_centroids=self.n_centroids, mode=self.mode, c=self.c,
                            n_refine_dsq=self.n_refine_dsq, heavy_fp16=self.heavy_fp16)
        return sd

    def load_state_dict(self, sd: dict) -> "SunShapeBlockCodec":
        cfg = sd.get("config", {})
        for k in ("head_dim", "block_dim", "n_centroids"):
            if k in cfg and cfg[k] != getattr(self, k):
                raise ValueError(f"state {k}={cfg[k]} does not match codec {getattr(self, k)}")
        if "heavy_fp16" in cfg:
            self.heavy_fp16 = bool(cfg["heavy_fp16"])
        if "mode" in cfg:
            self.mode = cfg["mode"]
            self.use_rotation = self.mode == "rotated"
        self._set_state(**{k: sd[k] for k in self._STATE_KEYS if k in sd})
        return self

    # ------------------------------------------------------------ transforms
    def _forward_transform(self, x: torch.Tensor) -> torch.Tensor:
        if self.mode in PERM_MODES:
            return apply_permutation(x, self.permutation)
        if self.use_rotation:
            return x.float() @ self.rotation.T
        return x

    def _inverse_transform(self, x: torch.Tensor) -> torch.Tensor:
        if self.mode in PERM_MODES:
            return apply_permutation(x, self.inv_permutation)
        if self.use_rotation:
            return x.float() @ self.rotation
        return x

    def kernel_permutation(self) -> torch.Tensor | None:
        """The permutation the kernels apply to raw queries/keys (None when the
        codec transform is not a permutation)."""
        return self.permutation if self.mode in PERM_MODES else None

    # ------------------------------------------------------------------ fit
    def fit(self, q_cal, k_cal, kmeans_iters: int = 25, seed: int = 0,
            kmeans_device=None) -> "SunShapeBlockCodec":
        """Fit from calibration queries/keys (reference codec.py:299-418).
        The per-block k-means runs on ``kmeans_device`` (default: the
        codec's device): on a GPU every block at once (``ss_kmeans_blocks``),
        else in NumPy; both start from the reference's initial rows."""
        q = _np(q_cal)
        k = _np(k_cal)
        d, bd, nb = self.head_dim, self.block_dim, self.n_blocks
        eye = np.eye(d, dtype=np.float32)
        E, E_inv = eye, eye
        perm = np.arange(d, dtype=np.int32)
        ba, ab = np.ones(nb, np.float32), np.ones(nb, bool)
        heavy, bmass = np.zeros(nb, bool), np.zeros(nb, np.float32)
        if self.mode == "rotated":
            r = self.rotation.detach().cpu().numpy()
            q, k = q @ r.T, k @ r.T
        else:
            perm = covariance_block_permutation(q, bd)
            q, k = q[:, perm], k[:, perm]
            if self.mode == "profileperm_localmetric_dsq":
                E = block_local_cov_metric(q, np.arange(d), bd)
                E_inv = np.linalg.pinv(E).astype(np.float32)
                ba, ab = block_affinity_gate(q, bd)
            elif self.mode == "profileperm_mixed_precision":
                heavy, bmass = mixed_precision_block_mask(q, bd, mass_threshold=0.5)
        dev = torch.device(kmeans_device) if kmeans_device is not None else self.device
        active = [b for b in range(nb)
                  if not (self.mode == "profileperm_mixed_precision" and heavy[b])]
        ks = {b: k[:, b * bd:(b + 1) * bd] @ E[b * bd:(b + 1) * bd, b * bd:(b + 1) * bd].T
              for b in active}
        fitted = {}
        n_pts = k.shape[0]
        if dev.type == "cuda" and active and n_pts > self.n_centroids:
            # reference initial centroids: rows RandomState(seed + b).permutation(N)[:K]
            init = np.stack([ks[b][np.random.RandomState(seed + b).permutation(n_pts)
                                   [:self.n_centroids]] for b in active])
            data = torch.from_numpy(np.ascontiguousarray(np.stack([ks[b] for b in active]),
                                                         dtype=np.float32)).to(dev)
            out = _hip.kmeans_blocks(data, torch.from_numpy(init.astype(np.float32)).to(dev),
                                     kmeans_iters).cpu().numpy()
            fitted = {b: out[i] for i, b in enumerate(active)}
        else:
            fitted = {b: _kmeans(ks[b], self.n_centroids, n_iters=kmeans_iters, seed=seed + b)
                      for b in active}
        cents = []
        for b in range(nb):
            sl = slice(b * bd, (b + 1) * bd)
            if b not in fitted:
                cents.append(np.zeros((self.n_centroids, bd), np.float32))
                continue
            cents.append((fitted[b] @ E_inv[sl, sl].T).astype(np.float32))
        working = np.stack(cents)
        if self.mode not in ("profileperm_baseline", "rotated") and self.n_refine_dsq > 0:
            working = _refine_centroids(q, k, working, E, bd, n_steps=self.n_refine_dsq,
                                        block_affinity=ba, active_blocks=ab)
        self._set_state(E=E, E_inv=E_inv, centroids=working.astype(np.float32),
                        dsq_block_affinity=ba, dsq_active_blocks=ab,
                        mixed_high_precision_blocks=heavy, mixed_block_mass=bmass,
                        permutation=perm)
        return self

    # ------------------------------------------------------------- quantize
    def _local_metric_blocks(self) -> torch.Tensor:
        nb, bd = self.n_blocks, self.block_dim
        e = self.E.reshape(nb, bd, nb, bd)
        return torch.stack([e[b, :, b, :] for b in range(nb)])  # (nb, bd, bd)

    def heavy_dims(self) -> torch.Tensor | None:
        """int32 codec-basis dims of the heavy blocks whose keys a cache keeps
        in fp16 (mixed-precision mode with ``heavy_fp16``), else None."""
        if self.mode != "profileperm_mixed_precision" or not self.heavy_fp16:
            return None
        hb = torch.nonzero(self.mixed_high_precision_blocks.to(torch.bool)).flatten()
        if hb.numel() == 0:
            return None
        bd = self.block_dim
        dims = (hb[:, None] * bd + torch.arange(bd, device=hb.device)[None]).flatten()
        return dims.to(torch.int32).to(self.device)

    def kernel_value_transform(self) -> torch.Tensor:
        """(D, D) float32 matrix taking a codec-space row to the original
        basis, ``x_orig = x_codec @ M`` (the inverse permutation as a 0/1
        matrix, the rotation, or the identity): the last step of the fused
        decode over values quantised with this codec.  Rebuilt when the
        transform changes."""
        if self.mode in PERM_MODES:
            src = self.inv_permutation
        elif self.use_rotation:
            src = self.rotation
        else:
            src = None
        key = (self.mode, None if src is None else (src.data_ptr(), src._version), str(self.device))
        cached = getattr(self, "_kernel_value_transform", None)
        if cached is None or cached[0] != key:
            d = self.head_dim
            if self.mode in PERM_MODES:
                m = torch.zeros((d, d), dtype=torch.float32, device=self.device)
                m[self.inv_permutation.long(), torch.arange(d, device=self.device)] = 1.0
            elif self.use_rotation:
                m = self.rotation.float().contiguous()
            else:
                m = torch.eye(d, dtype=torch.float32, device=self.device)
            cached = (key, m)
            self._kernel_value_transform = cached
        return cached[1]

    def scoring_centroids(self) -> torch.Tensor:
        """The centroids a cache's scores read.  With fp16 heavy blocks
        (``heavy_dims()`` not None) those blocks are scored exactly from
        their stored key dims, so their table entries must add nothing: a
        copy of the centroids with the heavy blocks zeroed (the fit's DSQ
        refinement moves a heavy block's centroid 0 away from zero,
        reference codec.py:400-410).  Otherwise the centroids themselves, so
        a heavy block's index 0 adds ``q . C[b][0]`` as in the reference
        (codec.py:575-637).  Cached until the centroids or the heavy mask
        change."""
        c = self.centroids
        if self.heavy_dims() is None:
            return c
        hb = self.mixed_high_precision_blocks
        key = (c.data_ptr(), c._version, hb.data_ptr(), hb._version, str(c.device))
        cached = getattr(self, "_scoring_centroids", None)
        if cached is None or cached[0] != key:
            z = c.clone()
            z[hb.to(torch.bool).to(z.device)] = 0.0
            cached = (key, z.contiguous())
            self._scoring_centroids = cached
        return cached[1]

    def kernel_codebook(self) -> torch.Tensor:
        """``scoring_centroids()`` as the split-fp16 buffer read by the
        matrix-core LUT build of the fused decodes, prepared once and rebuilt
        when the centroids change (new tensor, device or in-place update)."""
        c = self.scoring_centroids()
        cached = getattr(self, "_kernel_codebook", None)
        if cached is None or cached[0] is not c or cached[1] != c._version:
            cached = (c, c._version, _hip.codebook_f16x2(c))
            self._kernel_codebook = cached
        return cached[2]

    def encode_codebook(self, centroids: torch.Tensor | None = None) -> torch.Tensor | None:
        """The prepared codebook of the matrix-core encoder for ``centroids``
        (default: the codec's), built once and rebuilt when they change; None
        for shapes that encoder does not take (the plain encoder runs)."""
        c = self.centroids if centroids is None else centroids
        if not _hip.encode_codebook_supported(c):
            return None
        cached = getattr(self, "_encode_codebook", None)
        if cached is None or cached[0] is not c or cached[1] != c._version:
            cached = (c, c._version, _hip.encode_codebook(c))
            self._encode_codebook = cached
        return cached[2]

    def _encode_centroids(self) -> torch.Tensor:
        if self.mode == "profileperm_localmetric_dsq":
            if self._shaped_centroids is None:
                eb = self._local_metric_blocks()
                self._shaped_centroids = torch.einsum(
                    "bcd,bed->bce", self.centroids, eb).contiguous()
            return self._shaped_centroids
        return self.centroids

    def quantize(self, keys: torch.Tensor) -> SunShapeQuantized:
        """(N, head_dim) keys -> uint8 indices (N, n_blocks) (codec.py:424-514).
        Ties resolve to the lowest index.  Mixed-precision heavy blocks keep
        index 0 and carry the transformed key block in ``passthrough_values``."""
        _hip.require_gpu(keys)
        if self.n_centroids > 256:
            raise NotImplementedError("HIP encoder stores uint8 indices (n_centroids <= 256)")
        keys = keys.reshape(-1, self.head_dim)
        n = keys.shape[0]
        out = torch.empty((n, self.n_blocks), dtype=torch.uint8, device=keys.device)
        if self.mode == "profileperm_baseline":
            _hip.encode_blockvq(keys if keys.stride(-1) == 1 else keys.contiguous(),
                                self.permutation, self.centroids, out, self.block_dim,
                                prepared=self.encode_codebook())
        else:
            kt = self._forward_transform(keys.float())
            if self.mode == "profileperm_localmetric_dsq":
                kt = torch.einsum("nbd,bed->nbe", kt.reshape(n, self.n_blocks, self.block_dim),
                                  self._local_metric_blocks()).reshape(n, self.head_dim)
            ec = self._encode_centroids()
            _hip.encode_blockvq(kt.contiguous(), None, ec, out, self.block_dim,
                                prepared=self.encode_codebook(ec))
        passthrough_blocks = passthrough_values = None
        if self.mode == "profileperm_mixed_precision":
            passthrough_blocks = self.mixed_high_precision_blocks
            if bool(passthrough_blocks.any()):
                kt = self._forward_transform(keys.float()).reshape(n, self.n_blocks,
                                                                   self.block_dim)
                passthrough_values = kt * passthrough_blocks.reshape(1, -1, 1).float()
                out[:, passthrough_blocks] = 0
        return SunShapeQuantized(out, self.head_dim, self.block_dim, self.n_blocks,
                                 passthrough_blocks, passthrough_values)

    def dequantize(self, quantized: SunShapeQuantized) -> torch.Tensor:
        """Reconstructed keys (N, head_dim) float32 (codec.py:516-543)."""
        idx = quantized.indices.to(torch.uint8).contiguous()
        inv = self.inv_permutation if (self.mode in PERM_MODES
                                       and quantized.passthrough_values is None) else None
        k_hat = _hip.dequantize_blockvq(idx, self.centroids, inv)
        if inv is not None:
            return k_hat
        if quantized.passthrough_blocks is not None and quantized.passthrough_values is not None:
            n = k_hat.shape[0]
            kb = k_hat.reshape(n, self.n_blocks, self.block_dim)
            heavy = quantized.passthrough_blocks.to(kb.device)
            kb[:, heavy] = quantized.passthrough_values[:, heavy].to(kb.dtype)
            k_hat = kb.reshape(n, self.head_dim)
        elif quantized.passthrough_blocks is not None and bool(quantized.passthrough_blocks.any()):
            raise ValueError("Mixed-precision missing passthrough values.")
        return self._inverse_transform(k_hat)

    def __call__(self, keys: torch.Tensor) -> torch.Tensor:
        return self.dequantize(self.quantize(keys))

    # -------------------------------------------------------------- scores
    def precompute_query_centroid_dots(self, query: torch.Tensor) -> torch.Tensor:
        """LUT (n_qh, n_blocks, n_centroids) for queries already in codec
        space (codec.py:553-573)."""
        _hip.require_gpu(query)
        q = query.reshape(-1, self.head_dim)
        return _hip.build_lut(q if q.stride(-1) == 1 else q.contiguous(), None, 1.0,
                              self.centroids)

    def attention_scores(self, query: torch.Tensor, quantized: SunShapeQuantized, *,
                         prefer_metal: bool = True) -> torch.Tensor:
        """Unscaled scores (n_qh, n_tokens) = sum_b q_b . C[b][idx[t, b]] via
        the query x centroid table (codec.py:575-637).  As in the reference,
        the passthrough values are not read: a mixed-precision heavy block's
        index 0 adds ``q_b . C[b][0]``, which is zero after a fit without DSQ
        refinement (its centroids start at zero) and not after one.
        ``prefer_metal`` is accepted for signature compatibility."""
        _hip.require_gpu(query)
        q = query.reshape(-1, self.head_dim).float()
        if self.mode in PERM_MODES:
            lut = _hip.build_lut(q.contiguous(), self.permutation, 1.0, self.centroids)
        else:
            lut = _hip.build_lut(self._forward_transform(q).contiguous(), None, 1.0,
                                 self.centroids)
        scores = _hip.score_gather(lut, quantized.indices.to(torch.uint8).contiguous())
        self.last_score_backend = "hip"
        return scores

    def heldout_logit_mse(self, q_test: torch.Tensor, k_test: torch.Tensor) -> float:
        """E[(q . (k - k_hat))^2] (codec.py:639-650)."""
        q = q_test.float()
        k = k_test.float()
        delta = k - self(k)
        return float(((q * delta).sum(dim=1) ** 2).mean().item())
