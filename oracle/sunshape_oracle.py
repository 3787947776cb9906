"""NumPy restatement of the reference's SunShape compressed-KV attention path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker for the HIP
path, never the thing measured or shipped.

Each function cites the reference lines it restates
(``/root/reference/<file>:<line>``; the reference itself needs MLX and cannot
run here).  Where the reference's result is only defined up to rounding (its
Metal kernels run with fast-math), the oracle computes in float64 and the tests
compare with a stated tolerance; where it is integer/byte work (encode indices,
packing, grouped-quant codes, scalar quant) the oracle is exact and tests are
bit-exact.

Pinning (how each function is checked independently of its own formula; the
tests live in ``tests/test_oracle_*.py``):

=============================  ===============================================
function                       pinned by
=============================  ===============================================
invert/apply_permutation       round trip + explicit permutation matrix
encode_blockvq                 brute force over all centroids in exact
                               rational arithmetic (fractions) on tiny inputs;
                               known-answer test [13] (seed 333); duplicate-
                               centroid ties; C restatement ``encode_ref.c``;
                               idempotence encode(decode(i)) == i
query_centroid_dots            q_perm . k_hat_perm == q . k_hat (orig. basis)
gather_scores                  == q @ dequantize(idx).T ([6], seed 55) and the
                               cache-level invariant of test_sunshape_mlx
fused_attention(_grouped)      textbook softmax(q k_hat^T) V with k_hat from
                               dequantize ([7],[11],[12],[14]-[17]); literal
                               online-softmax loop of the reference kernel;
                               split-T log-sum-exp merge == whole
pack/unpack_indices            bit layout closed form, [1]-[3], [9]
quantize/dequantize_values     per-group min/max closed form, error bounds [4]
scalar_quantize                == searchsorted on sorted boundaries ([5])
lloyd_max_gaussian             the reference's literal table: symmetric,
                               midpoint boundaries, 1-bit closed form
                               sqrt(2/pi), within 1e-9 (2, 3 bits) and
                               4e-4 (4 bits) of the Lloyd-Max fixed point
turboquant_encode/decode       rotation orthogonality; round-trip MSE bound
sdpa                           per-head loop == fused_attention per (b,h,r);
                               GQA head mapping h*rep + r (attention.py:220)
sdpa_two_pass masks            boolean: == softmax over the kept keys only
                               (reconstructed keys), fully masked row == mean
                               of the values; additive: == softmax(q k^T + m)
                               over reconstructed keys; planted mistakes
                               (zero rows, a subtracted mask) fail the pins
kmeans                         hand-worked Lloyd steps from the reference's
                               initial rows (seeds 0, 1), empty cluster kept,
                               zero-padded short data, non-increasing
                               distortion, converged centroids = cluster
                               means (tests/test_oracle_fit.py)
covariance_block_permutation   hand-worked greedy packings of exact factor
                               covariances (2 and 3 blocks; the zeroed
                               diagonal decides the seed), identity for
                               uncorrelated dims, permutation validity
fit_profileperm_baseline       per-block initial rows RandomState(seed + b)
                               in closed form, zero-padded short data
=============================  ===============================================
"""

from __future__ import annotations

import math

import numpy as np

NEAR_TIE_REL = 1e-6


# --------------------------------------------------------------------------- #
#  Transforms                                                                  #
# --------------------------------------------------------------------------- #


def invert_permutation(perm: np.ndarray) -> np.ndarray:
    """Inverse permutation.  Restates rotation.py:251-259."""
    perm = np.asarray(perm)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.shape[0], dtype=perm.dtype)
    return inv


def apply_permutation(x: np.ndarray, perm) -> np.ndarray:
    """Gather along the last axis: ``x[..., perm]``.  Restates rotation.py:262-266."""
    if perm is None or np.size(perm) == 0:
        return x
    return np.asarray(x)[..., np.asarray(perm)]


# --------------------------------------------------------------------------- #
#  Block-VQ encode                                                             #
# --------------------------------------------------------------------------- #


def _duplicate_ids(cb: np.ndarray) -> np.ndarray:
    """For one block's codebook (NC, BD): id of the lowest centroid with an
    identical vector.  Identical centroids give identical distances in any
    arithmetic, so they are exact ties that must resolve to the lowest index
    (codec.py:73-76 zero-pads codebooks when N <= K, producing such ties)."""
    _, first, inverse = np.unique(cb, axis=0, return_index=True, return_inverse=True)
    return first[inverse.reshape(-1)]


def encode_blockvq(keys, centroids, perm=None, near_tie_rel: float = NEAR_TIE_REL,
                   chunk: int = 4096):
    """Block-VQ encode with lowest-index ties and near-tie flagging.

    Restates ``SunShapeBlockCodec.quantize`` (codec.py:424-470): cast keys to
    float32 (codec.py:435), apply the ProfilePerm permutation (codec.py:436,
    rotation.py:262-266), then per 8-dim block pick the centroid minimising
    sum_d (k_d - c_d)^2 (kernels.py:1013-1024).  The reference's strict ``<``
    (kernels.py:1020) keeps the lowest index on ties.  The reference kernel sums
    in float32 under Metal fast-math, so its rounding is not pinned; the truth
    here is float64, and a (token, block) whose second-best distance to a
    centroid with a *different* vector is within ``near_tie_rel`` (relative) of
    the best is flagged as a near-tie and excluded from bit-exact comparison.

    Returns ``(indices, near_tie)``: indices (N, n_blocks) uint8 when
    n_centroids <= 256 else uint16 (codec.py:203-209); near_tie bool (N, n_blocks).
    """
    k = np.asarray(keys).astype(np.float32)
    if perm is not None:
        k = apply_permutation(k, perm)
    cents = np.asarray(centroids, dtype=np.float32)
    n_blocks, n_cent, bd = cents.shape
    n = k.shape[0]
    kb = k.reshape(n, n_blocks, bd).astype(np.float64)
    c64 = cents.astype(np.float64)
    out = np.zeros((n, n_blocks), dtype=np.int64)
    near = np.zeros((n, n_blocks), dtype=bool)
    for b in range(n_blocks):
        dup = _duplicate_ids(cents[b])
        for s in range(0, n, chunk):
            e = min(n, s + chunk)
            diff = kb[s:e, b, None, :] - c64[b][None, :, :]
            d = np.einsum("ncd,ncd->nc", diff, diff)
            idx = np.argmin(d, axis=1)  # first occurrence == lowest index
            best = d[np.arange(e - s), idx]
            other = dup[None, :] != dup[idx][:, None]
            close = (d <= best[:, None] * (1.0 + near_tie_rel)) & other
            out[s:e, b] = idx
            near[s:e, b] = close.any(axis=1)
    dtype = np.uint8 if n_cent <= 256 else np.uint16
    return out.astype(dtype), near


def dequantize_blockvq(indices, centroids, inv_perm=None) -> np.ndarray:
    """k_hat[:, block b] = C[b, idx[:, b]], then the inverse permutation.
    Restates codec.py:516-543 (and the duplicate in cache.py:211-240)."""
    idx = np.asarray(indices).astype(np.int64)
    cents = np.asarray(centroids, dtype=np.float32)
    n_blocks = cents.shape[0]
    parts = [cents[b][idx[:, b]] for b in range(n_blocks)]
    k_hat = np.concatenate(parts, axis=1).astype(np.float32)
    if inv_perm is not None:
        k_hat = apply_permutation(k_hat, inv_perm)
    return k_hat


# --------------------------------------------------------------------------- #
#  LUT and score gather                                                        #
# --------------------------------------------------------------------------- #


def query_centroid_dots(q_transformed, centroids) -> np.ndarray:
    """LUT ``qd[r, b, c] = sum_d q[r, b*bd + d] * C[b, c, d]`` in float64.
    Restates codec.py:553-573 (einsum ``qbd,bcd->qbc``) and the in-kernel LUT
    build of kernels.py:178-190."""
    cents = np.asarray(centroids, dtype=np.float64)
    n_blocks, _, bd = cents.shape
    q = np.asarray(q_transformed, dtype=np.float64)
    q = q.reshape(q.shape[0], n_blocks, bd)
    return np.einsum("rbd,bcd->rbc", q, cents)


def gather_scores(lut, indices) -> np.ndarray:
    """``S[r, t] = sum_b lut[r, b, idx[t, b]]``.  Restates codec.py:617-634
    and the score kernel kernels.py:59-77."""
    lut = np.asarray(lut, dtype=np.float64)
    idx = np.asarray(indices).astype(np.int64)
    n_blocks = lut.shape[1]
    g = lut[:, np.arange(n_blocks)[None, :], idx]  # (R, T, NB)
    return g.sum(axis=-1)


def attention_scores(query, indices, centroids, perm=None) -> np.ndarray:
    """``SunShapeBlockCodec.attention_scores`` (codec.py:575-637): query cast
    to float32, permuted, *unscaled*; LUT; gather."""
    q = np.asarray(query).astype(np.float32)
    if perm is not None:
        q = apply_permutation(q, perm)
    return gather_scores(query_centroid_dots(q, centroids), indices)


# --------------------------------------------------------------------------- #
#  Fused attention                                                             #
# --------------------------------------------------------------------------- #


def _softmax_rows(scores, valid, values) -> np.ndarray:
    r_, _ = scores.shape
    out = np.zeros((r_, values.shape[1]), dtype=np.float64)
    for r in range(r_):
        v = valid[r]
        if not v.any():
            continue  # d_local == 0 -> output 0 (kernels.py:218-222)
        s = scores[r, v]
        p = np.exp(s - s.max())
        out[r] = (p @ values[v]) / p.sum()
    return out


def _softmax_rows_min_fill(scores, valid, values) -> np.ndarray:
    """The two-pass path's masking and softmax (attention.py:329-346): masked
    scores are replaced by float32's lowest finite value
    (``mx.where(mask, scores, finfo(float32).min)``, attention.py:336, 341),
    then an ordinary max-subtracted softmax runs over the whole row.  A row
    that keeps at least one key gives its masked keys weight exactly 0; a row
    with every key masked gets uniform weights, i.e. the mean of the values
    (the fused kernel's empty row gives 0 instead, ``_softmax_rows``)."""
    lo = float(np.finfo(np.float32).min)
    s = np.where(valid, np.asarray(scores, np.float64), lo)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    return (p @ values) / p.sum(axis=1, keepdims=True)


def causal_valid(n_rows: int, t_kv: int, causal: bool, q_offset: int) -> np.ndarray:
    """Row r may attend to key t iff ``t <= q_offset + r`` (kernels.py:322,353)."""
    t = np.arange(t_kv)[None, :]
    if not causal:
        return np.ones((n_rows, t_kv), dtype=bool)
    return t <= (q_offset + np.arange(n_rows))[:, None]


def fused_attention(q_transformed, centroids, indices, values, causal=False,
                    q_offset=0) -> np.ndarray:
    """Single-pass fused block-VQ attention, restated as an exact two-pass
    softmax in float64 (online and two-pass softmax are equal in exact
    arithmetic).  Restates kernels.py:142-223 (no mask), 303-378 (causal:
    row r keeps ``t <= q_offset + r``); values are upcast to float32 first as
    attention.py:91 does.  No scale inside: the caller pre-scales."""
    lut = query_centroid_dots(q_transformed, centroids)
    s = gather_scores(lut, indices)
    v = np.asarray(values).astype(np.float32).astype(np.float64)
    valid = causal_valid(s.shape[0], s.shape[1], causal, q_offset)
    return _softmax_rows(s, valid, v)


def fused_attention_online_literal(q_transformed, centroids, indices, values,
                                   causal=False, q_offset=0) -> np.ndarray:
    """Token-by-token online softmax exactly as the reference kernel loops
    (kernels.py:193-222): m0 = -1e30, d0 = 0, acc0 = 0; per token
    m' = max(s, m); d = d*e^(m-m') + e^(s-m'); acc = acc*e^(m-m') + e^(s-m')*v.
    Pure-Python loop for small inputs only; used to pin ``fused_attention``."""
    lut = query_centroid_dots(q_transformed, centroids)
    s_all = gather_scores(lut, indices)
    v = np.asarray(values).astype(np.float32).astype(np.float64)
    r_, t_ = s_all.shape
    out = np.zeros((r_, v.shape[1]))
    for r in range(r_):
        m, d, acc = -1e30, 0.0, np.zeros(v.shape[1])
        for t in range(t_):
            if causal and t > q_offset + r:
                continue
            s = s_all[r, t]
            m_new = s if s > m else m
            corr = math.exp(m - m_new)
            e = math.exp(s - m_new)
            d = d * corr + e
            acc = acc * corr + e * v[t]
            m = m_new
        out[r] = acc / d if d > 0 else 0.0
    return out


def fused_attention_grouped(q_transformed, centroids, indices, packed, scales,
                            zeros, head_dim, bits, group_size, causal=False,
                            q_offset=0) -> np.ndarray:
    """Fused attention with in-register grouped dequant of V.  Restates
    kernels.py:588-687 (and the causal variant 772-860):
    ``v = ((word >> (d % vpw) * bits) & mask) * scale[t, g] + zero[t, g]``.
    Scale/zero are used in the dtype they are stored in (float32 in the
    reference, cache.py:516-517; float16 when a cache stores them so)."""
    v = dequantize_values(packed, scales, zeros, head_dim, bits, group_size)
    return fused_attention(q_transformed, centroids, indices, v, causal, q_offset)


def lse_merge(parts):
    """Merge split-T partials ``(m, l, acc)`` (acc unnormalised) by
    log-sum-exp.  Used to pin the split-T decomposition the HIP kernel uses."""
    m = max(p[0] for p in parts)
    l_ = sum(p[1] * math.exp(p[0] - m) for p in parts)
    a = sum(p[2] * math.exp(p[0] - m) for p in parts)
    return a / l_ if l_ > 0 else np.zeros_like(a)


def materialized_block_vq_attention(qdots, indices, values, t_q, t_kv) -> np.ndarray:
    """``fused_block_vq_attention`` (kernels.py:514-563): scores from the LUT,
    causal mask applied iff ``T_kv >= T_q`` with q positions
    ``[T_kv - T_q, T_kv)``, softmax, ``@ values``."""
    s = gather_scores(qdots, indices)
    v = np.asarray(values).astype(np.float32).astype(np.float64)
    if t_kv >= t_q:
        valid = causal_valid(t_q, t_kv, True, t_kv - t_q)
    else:
        valid = np.ones(s.shape, dtype=bool)
    return _softmax_rows(s, valid, v)


# --------------------------------------------------------------------------- #
#  Bit packing and value codecs                                                #
# --------------------------------------------------------------------------- #


def values_per_word(bits: int) -> int:
    """2-bit: 16, 3-bit: 10, 4-bit: 8 per uint32 (kernels.py:1112-1135)."""
    if bits not in (2, 3, 4):
        raise ValueError(f"Unsupported bits: {bits}")
    return 32 // bits


def packed_dim(d: int, bits: int) -> int:
    """Words per row (cache.py:39-56)."""
    if bits == 2:
        if d % 16:
            raise ValueError("2-bit packing needs D % 16 == 0")
        return d // 16
    if bits == 3:
        return (d + 9) // 10
    if bits == 4:
        if d % 8:
            raise ValueError("4-bit packing needs D % 8 == 0")
        return d // 8
    raise ValueError(f"Unsupported bits: {bits}")


def pack_indices(indices, bits: int) -> np.ndarray:
    """Element i of each word group lives at bits [bits*i, bits*i + bits);
    values are masked to ``bits`` first; 3-bit rows are zero-padded to a
    multiple of 10.  Restates kernels.py:1102-1137."""
    idx = np.asarray(indices).astype(np.uint32)
    d = idx.shape[-1]
    vpw = values_per_word(bits)
    nw = packed_dim(d, bits)
    pad = nw * vpw - d
    if pad:
        idx = np.concatenate([idx, np.zeros(idx.shape[:-1] + (pad,), np.uint32)], axis=-1)
    idx = idx.reshape(idx.shape[:-1] + (nw, vpw)) & np.uint32((1 << bits) - 1)
    shifts = (np.arange(vpw, dtype=np.uint32) * np.uint32(bits))
    return np.bitwise_or.reduce(idx << shifts, axis=-1).astype(np.uint32)


def unpack_indices(packed, d: int, bits: int) -> np.ndarray:
    """Inverse of ``pack_indices``; returns uint32 (kernels.py:1140-1163)."""
    p = np.asarray(packed).astype(np.uint32)
    vpw = values_per_word(bits)
    shifts = (np.arange(vpw, dtype=np.uint32) * np.uint32(bits))
    e = (p[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    e = e.reshape(p.shape[:-1] + (p.shape[-1] * vpw,))
    return e[..., :d]


def quantize_values(values, bits: int = 4, group_size: int = 64):
    """Asymmetric per-group min-max quantization in float32.  Restates
    kernels.py:1173-1228: ``zero = min``, ``scale = (max - min) / (2^b - 1)``
    clamped below at 1e-8, ``q = clip(rint((v - zero) / scale), 0, 2^b - 1)``.
    Returns ``(packed uint32, scales f32 (T, G), zeros f32 (T, G), G)``."""
    v = np.asarray(values).astype(np.float32)
    t, d = v.shape
    g = d // group_size
    maxv = (1 << bits) - 1
    vg = v.reshape(t, g, group_size)
    mn = vg.min(axis=2, keepdims=True)
    mx = vg.max(axis=2, keepdims=True)
    sc = (mx - mn) / np.float32(maxv)
    sc = np.where(sc < np.float32(1e-8), np.float32(1e-8), sc).astype(np.float32)
    q = np.rint((vg - mn) / sc).astype(np.int32)
    q = np.clip(q, 0, maxv).astype(np.uint8)
    packed = pack_indices(q.reshape(t, d), bits)
    return packed, sc[..., 0], mn[..., 0], g


def quantize_value_codes(values, bits: int, group_size: int) -> np.ndarray:
    """The unpacked integer codes of ``quantize_values`` (T, D) uint8."""
    packed, _, _, _ = quantize_values(values, bits, group_size)
    d = np.asarray(values).shape[-1]
    return unpack_indices(packed, d, bits).astype(np.uint8)


def dequantize_values(packed, scales, zeros, d: int, bits: int = 4,
                      group_size: int = 64) -> np.ndarray:
    """``v = q * scale + zero`` per group (float32, separate multiply and add).
    Restates kernels.py:1231-1269."""
    q = unpack_indices(packed, d, bits).astype(np.float32)
    sc = np.asarray(scales).astype(np.float32)
    zr = np.asarray(zeros).astype(np.float32)
    g = d // group_size
    qg = q.reshape(q.shape[:-1] + (g, group_size))
    prod = (qg * sc[..., None]).astype(np.float32)
    return (prod + zr[..., None]).astype(np.float32).reshape(q.shape)


def scalar_quantize(values, boundaries) -> np.ndarray:
    """``idx = #{b : v > boundary[b]}`` as uint8 (kernels.py:453-463, 503-507)."""
    v = np.asarray(values).astype(np.float32)
    out = np.zeros(v.shape, dtype=np.uint8)
    for b in np.asarray(boundaries, dtype=np.float32):
        out += (v > b).astype(np.uint8)
    return out


# The reference's TurboQuant codebooks (value_codecs.py:20-87): Lloyd-Max
# levels and boundaries of N(0, 1), stored there as literal tables and kept
# here as the same data, levels then boundaries.
_REF_LLOYD_MAX = {
    1: ([-0.7978845608028654, 0.7978845608028654], [0.0]),
    2: ([-1.510417608611893, -0.4527800346911237, 0.4527800346911237, 1.510417608611893],
        [-0.9815988216515084, 0.0, 0.9815988216515084]),
    3: ([-2.151945705166112, -1.3439092791423422, -0.7560052816730181, -0.2450941791152904,
         0.2450941791152904, 0.7560052816730181, 1.3439092791423422, 2.151945705166112],
        [-1.7479274921542272, -1.0499572804076802, -0.5005497303941542, 0.0,
         0.5005497303941542, 1.0499572804076802, 1.7479274921542272]),
    4: ([-2.732896755154294, -2.069364258154187, -1.618400443227723, -1.2565648452462146,
         -0.9426291036999694, -0.6569817464411519, -0.38818871416000605,
         -0.12844300124876415, 0.12844300124876415, 0.38818871416000605,
         0.6569817464411519, 0.9426291036999694, 1.2565648452462146, 1.618400443227723,
         2.069364258154187, 2.732896755154294],
        [-2.4011305066542405, -1.8438823506909552, -1.4374826442369688, -1.099596974473092,
         -0.7998054250705606, -0.522585230300579, -0.2583158577043851, 0.0,
         0.2583158577043851, 0.522585230300579, 0.7998054250705606, 1.099596974473092,
         1.4374826442369688, 1.8438823506909552, 2.4011305066542405]),
}


def lloyd_max_gaussian(bits: int):
    """The reference's Lloyd-Max tables of N(0, 1) (value_codecs.py:20-87):
    ``(levels, boundaries)`` as float64 arrays."""
    lv, bd = _REF_LLOYD_MAX[bits]
    return np.array(lv, np.float64), np.array(bd, np.float64)


def turboquant_tables(bits: int, d: int):
    """Scaled float32 tables of ``TurboQuantValueCodec`` (value_codecs.py:
    148-151): python-float products ``x * (1 / sqrt(d))`` rounded to
    float32.  Returns ``(centroids, boundaries)``."""
    lv, bd = _REF_LLOYD_MAX[bits]
    s = 1.0 / math.sqrt(d)
    return (np.array([x * s for x in lv], np.float32), np.array([x * s for x in bd], np.float32))


def lloyd_max_fixed_point(bits: int, iters: int = 2000, tol: float = 1e-15):
    """Lloyd-Max quantizer of N(0, 1) computed by the classical fixed-point
    iteration (Max, 1960): boundaries are midpoints of adjacent levels; each
    level is the conditional mean of its cell,
    ``(phi(a) - phi(b)) / (Phi(b) - Phi(a))``.  Used to pin the literal
    tables above."""
    from scipy.stats import norm

    n = 1 << bits
    levels = norm.ppf((np.arange(n) + 0.5) / n)
    for _ in range(iters):
        b = 0.5 * (levels[1:] + levels[:-1])
        lo = np.concatenate([[-np.inf], b])
        hi = np.concatenate([b, [np.inf]])
        new = (norm.pdf(lo) - norm.pdf(hi)) / (norm.cdf(hi) - norm.cdf(lo))
        if np.max(np.abs(new - levels)) < tol:
            levels = new
            break
        levels = new
    return levels, 0.5 * (levels[1:] + levels[:-1])


def rotation_matrix(d: int, seed: int) -> np.ndarray:
    """Haar-random orthogonal matrix by QR of a Gaussian matrix with the
    column signs fixed by sign(diag(R)) (rotation.py:29-50).  The reference
    draws G from MLX's RNG, which is unavailable; the matrix here is data drawn
    from NumPy's ``default_rng(seed)``."""
    g = np.random.default_rng(seed).standard_normal((d, d)).astype(np.float32)
    q, r = np.linalg.qr(g.astype(np.float64))
    q = q * np.sign(np.diag(r))[None, :]
    return q.astype(np.float32)


def turboquant_encode(values, rotation, boundaries, bits):
    """TurboQuant value encode (value_codecs.py:159-171): ``n = ||v||``,
    ``u = v / max(n, 1e-8)``, ``r = u @ R^T``, ``idx = #(r > boundaries)``,
    pack.  float32 throughout.  Returns ``(packed, norms, idx)``."""
    v = np.asarray(values).astype(np.float32)
    n = np.sqrt((v.astype(np.float64) ** 2).sum(-1)).astype(np.float32)
    u = v / np.maximum(n, np.float32(1e-8))[..., None]
    r = u.astype(np.float64) @ np.asarray(rotation, np.float64).T
    idx = scalar_quantize(r.astype(np.float32), boundaries)
    return pack_indices(idx, bits), n, idx


def turboquant_decode(packed, norms, rotation, centroids, d, bits):
    """value_codecs.py:173-177: ``centroids[idx] @ R * n``."""
    idx = unpack_indices(packed, d, bits).astype(np.int64)
    rot = np.asarray(centroids, np.float64)[idx]
    u = rot @ np.asarray(rotation, np.float64)
    return u * np.asarray(norms, np.float64)[..., None]


# --------------------------------------------------------------------------- #
#  SDPA (GQA) semantics                                                        #
# --------------------------------------------------------------------------- #


def scale_query(queries, scale):
    """``queries * scale`` evaluated in the query dtype (attention.py:208):
    float32 product rounded to the query dtype."""
    q = np.asarray(queries)
    return (q.astype(np.float32) * np.float32(scale)).astype(q.dtype)


def sdpa(queries, key_indices, values, centroids, perm, scale, mask=None):
    """``sunshape_sdpa`` on a pure compressed cache (attention.py:166-305):
    q scaled in its own dtype, GQA reshape ``(B, Hkv, rep, Tq, D)`` so q head
    ``h*rep + r`` reads KV head h, permute, fused attention per (b, h, r) with
    causal offset ``T_kv - T_q`` when ``mask == "causal"``.  Returns float64
    (B, Hq, Tq, D); the reference casts to the query dtype."""
    q = scale_query(queries, scale)
    b_, hq, tq, d = q.shape
    hkv = key_indices.shape[1]
    rep = hq // hkv
    t_kv = key_indices.shape[2]
    qg = q.reshape(b_, hkv, rep, tq, d)
    qt = apply_permutation(qg, perm)
    causal = isinstance(mask, str) and mask == "causal"
    q_off = t_kv - tq if causal else 0
    out = np.zeros((b_, hq, tq, d))
    for b in range(b_):
        for h in range(hkv):
            for r in range(rep):
                out[b, h * rep + r] = fused_attention(
                    qt[b, h, r].astype(np.float32), centroids, key_indices[b, h],
                    values[b, h], causal, q_off)
    return out


def sdpa_two_pass(queries, scale, perm, centroids, key_indices, buffer_keys,
                  values_all, mask=None, heavy_keys=None, heavy_dims=None, rotation=None):
    """The two-pass fallback of attention.py:307-350 used when a hybrid cache
    has buffered fp16 tokens: compressed scores ``q_t . k_hat`` concatenated
    with ``q_scaled . k_buf^T`` (original basis), causal or additive/boolean
    mask (causal and boolean masks fill masked scores with float32's lowest
    value, attention.py:329-341, so a row with every key masked averages the
    values; an additive mask is added as is), softmax, ``@ values``
    (compressed values dequantized, then buffer).
    ``key_indices`` (B, Hkv, Tc, NB), ``buffer_keys`` (B, Hkv, Tb, D) or None,
    ``values_all`` (B, Hkv, Tc + Tb, D).

    ``heavy_keys`` (B, Hkv, Tc, nhd) with ``heavy_dims`` (nhd,): the build's
    extension for mixed-precision codecs (heavy blocks kept in fp16, the
    intent of README.md:87, where the reference zeroes their centroids,
    codec.py:381-388): the heavy blocks (those holding ``heavy_dims``) leave
    the centroid sum, whatever their centroids hold (the fit's DSQ
    refinement moves centroid 0, codec.py:400-410), and the exact dot
    products ``q_t[heavy_dims] . k_heavy`` take their place.

    ``rotation`` (D, D): a rotated codec's codec-space queries are
    ``q_scaled @ R^T`` (attention.py:229-230) in place of the permutation;
    buffered keys are still scored in the original basis (attention.py:323)."""
    if heavy_keys is not None:
        bd = np.asarray(centroids).shape[2]
        centroids = np.array(centroids, dtype=np.float32, copy=True)
        centroids[np.unique(np.asarray(heavy_dims, np.int64) // bd)] = 0.0
    q = scale_query(queries, scale)
    b_, hq, tq, d = q.shape
    hkv = values_all.shape[1]
    rep = hq // hkv
    t_kv = values_all.shape[2]
    qg = q.reshape(b_, hkv, rep, tq, d)
    if rotation is not None:
        qt = (qg.astype(np.float64) @ np.asarray(rotation, np.float64).T).astype(np.float32)
    else:
        qt = apply_permutation(qg, perm)
    out = np.zeros((b_, hq, tq, d))
    for b in range(b_):
        for h in range(hkv):
            for r in range(rep):
                parts = []
                if key_indices is not None and key_indices.shape[2] > 0:
                    lut = query_centroid_dots(qt[b, h, r].astype(np.float32), centroids)
                    sc = gather_scores(lut, key_indices[b, h])
                    if heavy_keys is not None:
                        hd = np.asarray(heavy_dims, np.int64)
                        sc = sc + (qt[b, h, r][:, hd].astype(np.float64)
                                   @ np.asarray(heavy_keys[b, h], np.float64).T)
                    parts.append(sc)
                if buffer_keys is not None and buffer_keys.shape[2] > 0:
                    parts.append(qg[b, h, r].astype(np.float64)
                                 @ np.asarray(buffer_keys[b, h], np.float64).T)
                s = np.concatenate(parts, axis=1)
                if isinstance(mask, str) and mask == "causal":
                    valid = causal_valid(tq, t_kv, True, t_kv - tq)
                elif mask is not None and not isinstance(mask, str):
                    m = np.asarray(mask)
                    if m.dtype == bool:
                        valid = np.broadcast_to(m, s.shape)
                    else:
                        s = s + m
                        valid = np.ones(s.shape, bool)
                else:
                    valid = np.ones(s.shape, bool)
                v = np.asarray(values_all[b, h], np.float32).astype(np.float64)
                out[b, h * rep + r] = _softmax_rows_min_fill(s, valid, v)
    return out


# --------------------------------------------------------------------------- #
#  Fit (fixture generation only; out of the hot path)                          #
# --------------------------------------------------------------------------- #


def kmeans(data, n_centroids: int, n_iters: int, seed: int) -> np.ndarray:
    """Lloyd k-means restating codec.py:53-103: zero-pad when N <= K; init
    rows ``RandomState(seed).permutation(N)[:K]``; float32 expanded-form
    distances, first-index argmin; empty clusters keep their centroid."""
    x = np.asarray(data, dtype=np.float32)
    n, d = x.shape
    if n <= n_centroids:
        out = np.zeros((n_centroids, d), dtype=np.float32)
        out[:n] = x
        return out
    rng = np.random.RandomState(seed)
    c = x[rng.permutation(n)[:n_centroids]].copy()
    for _ in range(n_iters):
        x_sq = np.sum(x ** 2, axis=1, keepdims=True)
        c_sq = np.sum(c ** 2, axis=1, keepdims=True).T
        dist = x_sq + c_sq - 2.0 * x @ c.T
        a = np.argmin(dist, axis=1)
        new = np.zeros_like(c)
        cnt = np.zeros(n_centroids, dtype=np.float64)
        np.add.at(new, a, x)
        np.add.at(cnt, a, 1.0)
        m = cnt > 0
        new[m] /= cnt[m, None]
        new[~m] = c[~m]
        c = new
    return c.astype(np.float32)


def covariance_block_permutation(q_cal, block_dim: int) -> np.ndarray:
    """Greedy ProfilePerm packing (rotation.py:179-248): seed = remaining dim
    with the largest total |cov| to the remaining dims (diagonal zeroed), then
    repeatedly add the candidate with the largest summed |cov| to the block."""
    q = np.asarray(q_cal, dtype=np.float32)
    c = q - q.mean(axis=0, keepdims=True)
    cov = (c.T @ c) / np.float32(max(1, q.shape[0] - 1))
    aff = np.abs(cov)
    np.fill_diagonal(aff, 0.0)
    d = aff.shape[0]
    remaining = set(range(d))
    ordered = []
    while remaining:
        rem = sorted(remaining)
        if len(rem) <= block_dim:
            ordered.extend(rem)
            break
        seed = rem[int(aff[rem].sum(axis=1).argmax())]
        block = [seed]
        remaining.remove(seed)
        while len(block) < block_dim and remaining:
            cand = sorted(remaining)
            gains = aff[np.array(cand)][:, np.array(block)].sum(axis=1)
            best = cand[int(gains.argmax())]
            block.append(best)
            remaining.remove(best)
        ordered.extend(block)
    return np.array(ordered, dtype=np.int32)


def fit_profileperm_baseline(q_cal, k_cal, block_dim: int = 8,
                             n_centroids: int = 256, kmeans_iters: int = 25,
                             seed: int = 0):
    """``fit`` in ``profileperm_baseline`` mode (codec.py:299-337, 377-397):
    permutation from q_cal, then per-block k-means on permuted k_cal with
    seed ``seed + b``.  Returns ``(perm int32, centroids (NB, K, bd) f32)``."""
    q = np.asarray(q_cal, np.float32)
    k = np.asarray(k_cal, np.float32)
    perm = covariance_block_permutation(q, block_dim)
    kp = k[:, perm]
    nb = k.shape[1] // block_dim
    cents = np.stack([
        kmeans(kp[:, b * block_dim:(b + 1) * block_dim], n_centroids,
               kmeans_iters, seed + b)
        for b in range(nb)
    ])
    return perm, cents.astype(np.float32)


# --------------------------------------------------------------------------- #
#  CPU baseline forms (timed by bench.py's cpu_baseline leg)                   #
# --------------------------------------------------------------------------- #


def decode_cpu_reference_shaped(q_t, centroids, key_indices, values):
    """Reference-shaped CPU decode (attention.py:268-350): loop over
    (b, h, r); per head: einsum LUT, gather, softmax, ``@ V`` in float32.
    ``q_t`` (B, Hkv, rep, D) already scaled+permuted."""
    b_, hkv, rep, d = q_t.shape
    nb = key_indices.shape[-1]
    cents = np.asarray(centroids, np.float32)
    out = np.zeros((b_, hkv * rep, d), np.float32)
    ar = np.arange(nb)[None, :]
    for b in range(b_):
        for h in range(hkv):
            idx = key_indices[b, h].astype(np.int64)
            v = values[b, h].astype(np.float32)
            for r in range(rep):
                qb = q_t[b, h, r].astype(np.float32).reshape(nb, -1)
                lut = np.einsum("bd,bcd->bc", qb, cents)
                s = lut[ar, idx].sum(-1)
                p = np.exp(s - s.max())
                out[b, h * rep + r] = (p @ v) / p.sum()
    return out


def decode_cpu_vectorised(q_t, centroids, key_indices, values):
    """Head-vectorised CPU decode in float32: one LUT einsum for all heads,
    one gather per KV head serving its rep query heads, batched softmax and
    matmul."""
    b_, hkv, rep, d = q_t.shape
    nb = key_indices.shape[-1]
    cents = np.asarray(centroids, np.float32)
    qb = q_t.astype(np.float32).reshape(b_, hkv, rep, nb, -1)
    lut = np.einsum("xhrbd,bcd->xhrbc", qb, cents)  # (B,Hkv,rep,NB,NC)
    out = np.zeros((b_, hkv, rep, d), np.float32)
    ar = np.arange(nb)[None, :]
    for b in range(b_):
        for h in range(hkv):
            idx = key_indices[b, h].astype(np.int64)
            s = lut[b, h][:, ar, idx].sum(-1)  # (rep, T)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[b, h] = (p @ values[b, h].astype(np.float32)) / p.sum(1, keepdims=True)
    return out.reshape(b_, hkv * rep, d)


def decode_cpu_parallel(q_t, centroids, key_indices, values, n_threads: int,
                        chunk: int = 4096):
    """The vectorised CPU decode spread over ``n_threads`` host threads:
    one LUT einsum for all heads, then every (b, KV head, token chunk) is an
    independent unit -- gather, chunk-local softmax partial (m, l, acc) in
    float32 -- and the chunks of a head are merged by log-sum-exp (the split
    scheme of the GPU kernels, on the host).  NumPy releases the GIL in the
    gather, exp and matmul, so the units run in parallel; run it with one
    BLAS thread per worker."""
    from concurrent.futures import ThreadPoolExecutor

    b_, hkv, rep, d = q_t.shape
    nb = key_indices.shape[-1]
    t_kv = key_indices.shape[2]
    cents = np.asarray(centroids, np.float32)
    qb = q_t.astype(np.float32).reshape(b_, hkv, rep, nb, -1)
    lut = np.einsum("xhrbd,bcd->xhrbc", qb, cents)
    ar = np.arange(nb)[None, :]
    units = [(b, h, t0) for b in range(b_) for h in range(hkv) for t0 in range(0, t_kv, chunk)]

    def part(u):
        b, h, t0 = u
        idx = key_indices[b, h, t0:t0 + chunk].astype(np.int64)
        s = lut[b, h][:, ar, idx].sum(-1)  # (rep, chunk)
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        return m[:, 0], p.sum(1), p @ values[b, h, t0:t0 + chunk].astype(np.float32)

    with ThreadPoolExecutor(max_workers=max(1, n_threads)) as ex:
        parts = list(ex.map(part, units))
    out = np.zeros((b_, hkv, rep, d), np.float32)
    n_ch = (t_kv + chunk - 1) // chunk
    for i in range(b_ * hkv):
        ms = np.stack([parts[i * n_ch + c][0] for c in range(n_ch)])  # (n_ch, rep)
        mx = ms.max(0)
        w = np.exp(ms - mx)
        l_ = sum(parts[i * n_ch + c][1] * w[c] for c in range(n_ch))
        acc = sum(parts[i * n_ch + c][2] * w[c][:, None] for c in range(n_ch))
        out[i // hkv, i % hkv] = acc / l_[:, None]
    return out.reshape(b_, hkv * rep, d)


# --------------------------------------------------------------------------- #
#  C restatement of the encoder (oracle/encode_ref.c)                          #
# --------------------------------------------------------------------------- #

_C_LIB = None


def _c_lib():
    global _C_LIB
    if _C_LIB is None:
        import ctypes
        import os

        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build",
                            "libss_oracle.so")
        if not os.path.exists(path):
            from oracle import build_oracle

            build_oracle.build()
        lib = ctypes.CDLL(path)
        lib.ss_oracle_encode.restype = ctypes.c_int
        lib.ss_oracle_encode.argtypes = [
            ctypes.c_void_p, ctypes.c_long, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double,
            ctypes.c_void_p, ctypes.c_void_p]
        _C_LIB = lib
    return _C_LIB


def encode_blockvq_c(keys, centroids, perm=None, near_tie_rel: float = NEAR_TIE_REL):
    """Same contract as ``encode_blockvq``, computed by ``encode_ref.c``
    (OpenMP-parallel float64 brute force): fast enough for full-size configs."""
    k = np.asarray(keys).astype(np.float32)
    if perm is not None:
        k = apply_permutation(k, perm)
    k = np.ascontiguousarray(k)
    cents = np.ascontiguousarray(np.asarray(centroids, dtype=np.float32))
    nb, nc, bd = cents.shape
    n, d = k.shape
    idx = np.zeros((n, nb), np.int32)
    near = np.zeros((n, nb), np.uint8)
    rc = _c_lib().ss_oracle_encode(k.ctypes.data, n, d, cents.ctypes.data, nb, nc,
                                   bd, float(near_tie_rel), idx.ctypes.data,
                                   near.ctypes.data)
    if rc != 0:
        raise ValueError(f"ss_oracle_encode failed ({rc})")
    dtype = np.uint8 if nc <= 256 else np.uint16
    return idx.astype(dtype), near.astype(bool)
