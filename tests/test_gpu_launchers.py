"""The reference's launcher surface on the GPU: known-answer tests [5]-[17] of
the reference's test_kernels.py (regenerated from their np.random.seed
streams, checked against the explicit references those tests write out),
the None-on-unsupported contract, the dispatch counters, and BASELINE
config 1 through the codec API (fit, quantize, attention_scores).

Each test calls the launcher names the reference exports (the ``*_metal``
aliases of ``sunshape_mlx_amd.kernels``), so a caller written against the
reference runs unchanged.
"""

import math

import numpy as np
import pytest
import torch

from oracle import sunshape_oracle as O
import sunshape_mlx_amd as S
from sunshape_mlx_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def k_hat_of(centroids, indices):
    """Keys rebuilt block by block from their centroids (as the reference's
    tests write it, test_kernels.py:212-216)."""
    n_blocks, _, bd = centroids.shape
    out = np.zeros((indices.shape[0], n_blocks * bd), np.float32)
    for b in range(n_blocks):
        out[:, b * bd:(b + 1) * bd] = centroids[b][indices[:, b]]
    return out


def explicit_attention(q, k, v, causal_offset=None, masked=-1e30):
    s = q.astype(np.float64) @ k.astype(np.float64).T
    if causal_offset is not None:
        q_pos = np.arange(causal_offset, causal_offset + q.shape[0])
        s = np.where(q_pos[:, None] >= np.arange(k.shape[0])[None, :], s, masked)
    w = np.exp(s - s.max(axis=-1, keepdims=True))
    return (w / w.sum(axis=-1, keepdims=True)) @ v.astype(np.float64)


def test_known_answer_5_scalar_quantize():
    np.random.seed(77)
    boundaries = np.array([-1.0, -0.5, 0.0, 0.5, 1.0], np.float32)
    values = np.random.randn(100, 64).astype(np.float32)
    ref = np.zeros(values.shape, np.uint8)
    for b in boundaries:
        ref += (values > b).astype(np.uint8)
    for prefer in (False, True):
        got, backend = K.quantize_scalar_to_indices(t(values), t(boundaries), prefer_metal=prefer)
        assert backend == "hip"
        assert np.array_equal(got.cpu().numpy(), ref)


def test_known_answer_6_block_vq_score():
    np.random.seed(55)
    t_q, nb, nc, t_kv = 4, 16, 256, 32
    qdots = np.random.randn(t_q, nb, nc).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.uint8)
    ref = qdots[:, np.arange(nb)[None, :], idx].sum(-1)  # (t_q, t_kv)
    got = K.block_vq_score_metal(t(qdots), t(idx), n_qh=t_q, T_kv=t_kv, n_blocks=nb,
                                 n_centroids=nc)
    assert got is not None and tuple(got.shape) == (t_q, t_kv)
    assert np.abs(got.cpu().numpy() - ref).max() < 1e-3


def test_known_answer_7_fused_block_vq_attention():
    np.random.seed(42)
    t_q, t_kv, nb, nc, bd = 4, 32, 16, 256, 8
    d = nb * bd
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.int32)
    vals = np.random.randn(t_kv, d).astype(np.float32)
    q = np.random.randn(t_q, d).astype(np.float32)
    ref = explicit_attention(q, k_hat_of(cents, idx), vals, causal_offset=t_kv - t_q, masked=-1e9)
    qdots = np.einsum("qbd,bcd->qbc", q.reshape(t_q, nb, bd), cents)
    got = K.fused_block_vq_attention(t(qdots), t(idx), t(vals), T_q=t_q, T_kv=t_kv, n_blocks=nb,
                                     n_centroids=nc, head_dim=d)
    assert np.abs(got.cpu().numpy() - ref).max() < 5e-3
    assert np.abs(got.cpu().numpy() - ref).max() <= 1e-3 * np.abs(ref).max()


def test_known_answer_9_3bit_overflow():
    idx = torch.full((1, 30), 7, dtype=torch.uint8, device=DEV)
    packed = K.pack_indices(idx, bits=3)
    assert (K.unpack_indices(packed, D=30, bits=3).cpu().numpy() == 7).all()
    assert int(packed.cpu().numpy().view(np.uint32)[0, 0]) >> 30 == 0


def test_known_answer_10_score_shape():
    np.random.seed(10)
    t_q, nb, nc, t_kv = 2, 8, 64, 16
    qdots = np.random.randn(t_q, nb, nc).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.uint8)
    got = K.block_vq_score_metal(t(qdots), t(idx), n_qh=t_q, T_kv=t_kv, n_blocks=nb,
                                 n_centroids=nc)
    assert got is not None and tuple(got.shape) == (t_q, t_kv)
    ref = qdots[:, np.arange(nb)[None, :], idx].sum(-1)
    assert np.abs(got.cpu().numpy() - ref).max() < 1e-4


@pytest.mark.parametrize("case", ["11", "12", "14"])
def test_known_answer_11_12_14_fused_attention(case):
    seed, t_q, t_kv, causal, vscale, tol = {
        "11": (111, 1, 64, False, 1.0, 5e-3),
        "12": (222, 4, 32, True, 1.0, 5e-3),
        "14": (444, 1, 512, False, 0.1, 0.01),
    }[case]
    np.random.seed(seed)
    nb, nc, bd = 16, 256, 8
    d = nb * bd
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.uint8)
    vals = (np.random.randn(t_kv, d) * vscale).astype(np.float32)
    q = (np.random.randn(t_q, d) * vscale).astype(np.float32)
    kw = dict(n_qh=t_q, T_kv=t_kv, n_blocks=nb, n_centroids=nc, head_dim=d)
    if causal:
        got = K.fused_attention_causal_metal(t(q), t(cents), t(idx), t(vals), q_offset=t_kv - t_q,
                                             **kw)
    else:
        got = K.fused_attention_metal(t(q), t(cents), t(idx), t(vals), **kw)
    assert got is not None and tuple(got.shape) == (t_q, d)
    ref = explicit_attention(q, k_hat_of(cents, idx), vals,
                             causal_offset=t_kv - t_q if causal else None)
    err = np.abs(got.cpu().numpy() - ref).max()
    assert err < tol and err <= 1e-3 * np.abs(ref).max()


def test_known_answer_13_block_vq_quantize():
    np.random.seed(333)
    n, nb, nc, bd = 32, 16, 256, 8
    d = nb * bd
    keys = np.random.randn(n, d).astype(np.float32)
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    ref = np.zeros((n, nb), np.int64)
    for b in range(nb):
        diff = keys[:, None, b * bd:(b + 1) * bd] - cents[b][None]
        ref[:, b] = np.argmin((diff ** 2).sum(-1), axis=1)
    got = K.block_vq_quantize_metal(t(keys), t(cents), n_blocks=nb, n_centroids=nc,
                                    block_dim=bd, head_dim=d)
    assert got is not None and got.dtype == torch.uint8
    assert np.array_equal(got.cpu().numpy().astype(np.int64), ref)


@pytest.mark.parametrize("case", ["15", "16", "17"])
def test_known_answer_15_16_17_fused_attention_dequant(case):
    seed, t_q, t_kv, bits, causal = {"15": (555, 1, 64, 4, False), "16": (666, 4, 32, 4, True),
                                     "17": (777, 1, 64, 2, False)}[case]
    np.random.seed(seed)
    nb, nc, bd, g = 16, 256, 8, 64
    d = nb * bd
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.uint8)
    q = np.random.randn(t_q, d).astype(np.float32)
    vals = np.random.randn(t_kv, d).astype(np.float32)
    packed, scales, zeros, n_groups = K.quantize_values(t(vals), bits=bits, group_size=g)
    assert n_groups == d // g
    # the codes and scale/zero equal the oracle's (bit-exact), so the
    # reference's dequantised values are the oracle's
    rp, rs, rz, _ = O.quantize_values(vals, bits, g)
    assert np.array_equal(packed.cpu().numpy().view(np.uint32), rp.view(np.uint32))
    assert np.array_equal(scales.cpu().numpy(), rs) and np.array_equal(zeros.cpu().numpy(), rz)
    deq = K.dequantize_values(packed, scales, zeros, D=d, bits=bits, group_size=g).cpu().numpy()
    ref = explicit_attention(q, k_hat_of(cents, idx), deq,
                             causal_offset=t_kv - t_q if causal else None)
    kw = dict(n_qh=t_q, T_kv=t_kv, n_blocks=nb, n_centroids=nc, head_dim=d, bits=bits,
              group_size=g)
    if causal:
        got = K.fused_attention_dequant_causal_metal(t(q), t(cents), t(idx), packed, scales, zeros,
                                                     q_offset=t_kv - t_q, **kw)
    else:
        got = K.fused_attention_dequant_metal(t(q), t(cents), t(idx), packed, scales, zeros, **kw)
    assert got is not None and tuple(got.shape) == (t_q, d)
    err = np.abs(got.cpu().numpy() - ref).max()
    assert err < 5e-3 and err <= 1e-3 * np.abs(ref).max()


def test_launchers_return_none_when_unsupported():
    """The reference's launchers return None for shapes their kernels do not
    take and the caller falls back (kernels.py:99-116, 259-291,
    1058-1082); the HIP launchers keep that contract."""
    rng = np.random.default_rng(3)
    q = t(rng.standard_normal((1, 96)).astype(np.float32))
    cents = t(rng.standard_normal((12, 256, 8)).astype(np.float32))
    idx = t(rng.integers(0, 256, (8, 12)).astype(np.uint8))
    vals = t(rng.standard_normal((8, 96)).astype(np.float32))
    kw = dict(n_qh=1, T_kv=8, n_blocks=12, n_centroids=256, head_dim=96)
    assert K.fused_attention_metal(q, cents, idx, vals, **kw) is None
    assert K.fused_attention_causal_metal(q, cents, idx, vals, **kw) is None
    big = t(rng.standard_normal((16, 512, 8)).astype(np.float32))
    keys = t(rng.standard_normal((4, 128)).astype(np.float32))
    assert K.block_vq_quantize_metal(keys, big, n_blocks=16, n_centroids=512, block_dim=8,
                                     head_dim=128) is None
    qd = t(rng.standard_normal((1, 16, 512)).astype(np.float32))
    assert K.block_vq_score_metal(qd, t(rng.integers(0, 256, (4, 16)).astype(np.uint8)), n_qh=1,
                                  T_kv=4, n_blocks=16, n_centroids=512) is None


def _config1_codec():
    """seed 42, q_cal (1024, 128) then k_cal (2048, 128)
    float32 N(0, 1), profileperm_baseline, kmeans_iters=15, k-means seed 42."""
    rng = np.random.default_rng(42)
    q_cal = rng.standard_normal((1024, 128)).astype(np.float32)
    k_cal = rng.standard_normal((2048, 128)).astype(np.float32)
    codec = S.SunShapeBlockCodec(128, block_dim=8, n_centroids=256,
                                 mode="profileperm_baseline", device=DEV).fit(
        q_cal, k_cal, kmeans_iters=15, seed=42)
    return codec, q_cal, k_cal


def test_config1_codec_api_against_oracle():
    """Config 1 through the API (reference codec.py:424-637): quantize
    (k_cal[:128]) is bit-exact against the oracle's encode with the fitted
    codebook (near-ties flagged by the oracle excepted); attention_scores
    (q_cal[:8]) matches the oracle's scores and the reference's own invariant
    scores == q @ dequantize(k).T (test_sunshape_mlx.py:172-182);
    precompute_query_centroid_dots matches the oracle's table."""
    codec, q_cal, k_cal = _config1_codec()
    perm = codec.permutation.cpu().numpy()
    assert np.array_equal(perm, O.covariance_block_permutation(q_cal, 8))
    cents = codec.centroids.cpu().numpy()
    qz = codec.quantize(t(k_cal[:128]))
    assert qz.indices.shape == (128, 16) and qz.indices.dtype == torch.uint8
    ref_idx, near = O.encode_blockvq(k_cal[:128], cents, perm)
    got_idx = qz.indices.cpu().numpy()
    assert near.sum() <= 2
    assert np.array_equal(got_idx[~near], ref_idx[~near])
    scores = codec.attention_scores(t(q_cal[:8]), qz)
    assert tuple(scores.shape) == (8, 128) and scores.dtype == torch.float32
    ref_scores = O.attention_scores(q_cal[:8], got_idx, cents, perm)
    sc = scores.cpu().numpy()
    assert np.abs(sc - ref_scores).max() <= 1e-4 * np.abs(ref_scores).max()
    k_hat = codec.dequantize(qz).cpu().numpy()
    assert np.array_equal(k_hat, O.dequantize_blockvq(got_idx, cents, O.invert_permutation(perm)))
    direct = q_cal[:8].astype(np.float64) @ k_hat.astype(np.float64).T
    assert np.abs(sc - direct).max() <= 1e-4 * np.abs(direct).max()
    lut = codec.precompute_query_centroid_dots(t(q_cal[:8][:, perm])).cpu().numpy()
    ref_lut = O.query_centroid_dots(q_cal[:8][:, perm], cents)
    assert np.abs(lut - ref_lut).max() <= 1e-5 * np.abs(ref_lut).max()
    assert codec.last_score_backend == "hip"


def test_config1_fit_against_oracle_fit():
    """The codec fit (k-means on the GPU, every block in one launch) against
    the oracle's fit (codec.py:299-418 restated): identical permutation; per
    block, the same k-means objective within 1 % (the GPU's float32 dot
    products may settle near-ties differently from NumPy's BLAS)."""
    codec, q_cal, k_cal = _config1_codec()
    perm, ref_cents = O.fit_profileperm_baseline(q_cal, k_cal, block_dim=8, n_centroids=256,
                                                 kmeans_iters=15, seed=42)
    assert np.array_equal(codec.permutation.cpu().numpy(), perm)
    kp = k_cal[:, perm].astype(np.float64)
    cents = codec.centroids.cpu().numpy().astype(np.float64)

    def inertia(x, c):
        d2 = ((x[:, None, :] - c[None]) ** 2).sum(-1)
        return d2.min(1).sum()

    for b in range(16):
        x = kp[:, b * 8:(b + 1) * 8]
        assert abs(inertia(x, cents[b]) / inertia(x, ref_cents[b].astype(np.float64)) - 1) <= 0.01


def test_kernel_stats_count_every_route():
    """Dispatch counters (reference kernels.py:33-47; test_kernel_stats_visible,
    test_sunshape_mlx.py:506-514) count the launches of every route: value
    codec quantize, codec quantize and attention_scores, cache append and a
    decode step through sunshape_sdpa."""
    tq = S.TurboQuantValueCodec(head_dim=128, bits=2, device=DEV)
    K.reset_kernel_stats()
    tq.quantize(torch.randn((8, 128), device=DEV))
    stats = K.get_kernel_stats()
    assert tq.last_quantize_backend == "hip"
    assert stats.get("sunshape_scalar_quantize_hip", 0) >= 1

    codec, q_cal, k_cal = _config1_codec()
    K.reset_kernel_stats()
    qz = codec.quantize(t(k_cal[:64]))
    codec.attention_scores(t(q_cal[:4]), qz)
    stats = K.get_kernel_stats()
    assert stats.get("sunshape_block_vq_quantize_hip") == 1
    assert stats.get("sunshape_query_centroid_dots_hip") == 1
    assert stats.get("sunshape_block_vq_score_hip") == 1

    cache = S.create_kv_cache(codec, n_kv_heads=2)
    k = torch.randn((1, 2, 100, 128), device=DEV).half()
    cache.update_and_fetch(k, torch.randn_like(k))
    K.reset_kernel_stats()
    S.sunshape_sdpa(torch.randn((1, 8, 1, 128), device=DEV).half(), cache, 0.088)
    assert K.get_kernel_stats() == {"sunshape_fused_attention_mfma_hip": 1}
    K.reset_kernel_stats()
    S.sunshape_sdpa(torch.randn((1, 8, 2, 128), device=DEV).half(), cache, 0.088, mask="causal")
    assert K.get_kernel_stats() == {"sunshape_fused_attention_mfma_causal_hip": 1}
    K.reset_kernel_stats()
    assert K.get_kernel_stats() == {}
