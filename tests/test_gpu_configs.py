"""BASELINE configs 4 and 5 at their full per-GPU shapes, built and decoded
through the drop-in API (``create_kv_cache`` -> ``update_and_fetch`` ->
``sunshape_sdpa``) and checked against the oracle on sampled (batch, KV head)
pairs (the oracle's float64 work over every head would take minutes).

Bars: stored codes, indices and scale/zero bit-exact against the oracle's
quantisation of the same inputs (encode excludes oracle-flagged near-ties);
attention outputs within 1e-3 of max |oracle| (the maximum over the compared
heads, not per element): the fp32 output (``out_dtype=torch.float32``, the
kernels' accumulation as it stands) against the float64 oracle, and the
drop-in fp16 output against the oracle rounded to fp16.
"""

import math

import numpy as np
import pytest
import torch

from oracle import sunshape_oracle as O
import sunshape_mlx_amd as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def rel_err16(got, ref):
    """max |got - fp16(ref)| / max |ref| for an fp16 output ``got``."""
    ref = np.asarray(ref, np.float64)
    r16 = ref.astype(np.float16).astype(np.float64)
    return float(np.abs(np.asarray(got, np.float64) - r16).max() / max(np.abs(ref).max(), 1e-30))


def _codec(seed, d=128, nc=256, mode="profileperm_baseline", heavy=None, block_dim=8):
    rng = np.random.default_rng(seed)
    nb = d // block_dim
    codec = S.SunShapeBlockCodec(d, block_dim=block_dim, n_centroids=nc, device=DEV, mode=mode,
                                 heavy_fp16=heavy is not None)
    state = {"centroids": rng.standard_normal((nb, nc, block_dim)).astype(np.float32),
             "permutation": rng.permutation(d).astype(np.int32)}
    if heavy is not None:
        hb = np.zeros(nb, bool)
        hb[heavy] = True
        state["mixed_high_precision_blocks"] = hb
    codec.load_state_dict(state)
    return codec


def _normal(seed, shape, dtype=torch.float16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV).to(dtype)


def test_config4_hybrid_full_shape():
    """Config 4: B=8, 32 query / 8 KV heads, head_dim 128, T_kv = 32768 per
    sequence (the default 128-token fp16 buffer holds the newest), 1-bit
    SunShape keys, 2-bit grouped values (group 64, fp16 scale/zero): one
    fused launch, checked on three (batch, KV head) pairs."""
    b, hq, hkv, d, t_kv, bits, g = 8, 32, 8, 128, 32768, 2, 64
    codec = _codec(4)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="grouped", value_bits=bits,
                              value_group_size=g, value_scale_dtype=torch.float16,
                              max_tokens=t_kv)
    k = _normal(40, (b, hkv, t_kv, d))
    v = _normal(41, (b, hkv, t_kv, d))
    cache.update_and_fetch(k, v)
    tc, tb = cache.compressed_offset, cache.buffer_offset
    assert tc + tb == t_kv and tb == 128
    q = _normal(42, (b, hq, 1, d))
    scale = 1.0 / math.sqrt(d)
    out = S.sunshape_sdpa(q, cache, scale)
    assert codec.last_score_backend == "hip_fused_mfma_dequant_buffer"
    assert out.shape == (b, hq, 1, d) and out.dtype == torch.float16
    out32 = S.sunshape_sdpa(q, cache, scale, out_dtype=torch.float32)
    assert codec.last_score_backend == "hip_fused_mfma_dequant_buffer"
    assert out32.dtype == torch.float32
    assert torch.equal(out32.to(torch.float16), out)  # one kernel, two output roundings
    cents = codec.centroids.cpu().numpy()
    perm = codec.permutation.cpu().numpy()
    rep = hq // hkv
    for bi, hi in ((0, 0), (3, 5), (7, 7)):
        kh = k[bi, hi].float().cpu().numpy()
        vh = v[bi, hi].float().cpu().numpy()
        idx = cache.key_indices[bi, hi].cpu().numpy()
        ref_idx, near = O.encode_blockvq_c(kh[:tc], cents, perm)
        assert np.array_equal(idx[~near], ref_idx[~near]) and near.mean() < 1e-3
        rp, rs, rz, _ = O.quantize_values(vh[:tc], bits, g)
        packed = cache.values_packed_raw[bi, hi].cpu().numpy()
        assert np.array_equal(packed.view(np.uint32), rp.view(np.uint32))
        sc = cache.value_scales_raw[bi, hi].cpu().numpy()
        zr = cache.value_zeros_raw[bi, hi].cpu().numpy()
        assert np.array_equal(sc, rs.astype(np.float16)) and np.array_equal(zr, rz.astype(np.float16))
        # fp16 scale/zero applied identically on both sides (config 4 stores them in fp16)
        vals = O.dequantize_values(rp, sc.astype(np.float32), zr.astype(np.float32), d, bits, g)
        vals_all = np.concatenate([vals, vh[tc:]], axis=0)[None, None]
        ref = O.sdpa_two_pass(q[bi:bi + 1, hi * rep:(hi + 1) * rep].cpu().numpy(), scale, perm,
                              cents, idx[None, None], kh[tc:][None, None], vals_all)
        got = out32[bi:bi + 1, hi * rep:(hi + 1) * rep].cpu().numpy()
        assert rel_err(got, ref) <= 1e-3
        got16 = out[bi:bi + 1, hi * rep:(hi + 1) * rep].float().cpu().numpy()
        assert rel_err16(got16, ref) <= 1e-3


def test_config5_one_layer_full_shape():
    """Config 5, one of its 28 layers: B=16, 32 query / 8 KV heads, head_dim
    128, T_kv = 131072, profileperm_mixed_precision keys with the 4 heavy
    blocks kept in fp16 (12 VQ blocks of 256 centroids), SunShape values
    (block_dim 4, 256 centroids, 32 bytes per token), random-init codebooks
    and N(0, 1) KV: one fused launch, checked on two (batch, KV head)
    pairs."""
    b, hq, hkv, d, t_kv = 16, 32, 8, 128, 131072
    heavy = [2, 5, 9, 14]
    codec = _codec(5, mode="profileperm_mixed_precision", heavy=heavy)
    vcodec = _codec(55, block_dim=4)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="sunshape", value_bits=8,
                              value_codec=vcodec, max_tokens=t_kv)
    k = _normal(50, (b, hkv, t_kv, d))
    v = _normal(51, (b, hkv, t_kv, d))
    cache.update_and_fetch(k, v)
    tc, tb = cache.compressed_offset, cache.buffer_offset
    assert tc + tb == t_kv
    q = _normal(52, (b, hq, 1, d))
    scale = 1.0 / math.sqrt(d)
    out = S.sunshape_sdpa(q, cache, scale)
    assert codec.last_score_backend == ("hip_fused_sunshape_v_buffer" if tb
                                        else "hip_fused_sunshape_v")
    out32 = S.sunshape_sdpa(q, cache, scale, out_dtype=torch.float32)
    assert out32.dtype == torch.float32
    assert torch.equal(out32.to(torch.float16), out)
    cents = codec.centroids.cpu().numpy()
    perm = codec.permutation.cpu().numpy()
    hd = codec.heavy_dims().cpu().numpy()
    assert hd.size == 32
    vcents = vcodec.centroids.cpu().numpy()
    vperm = vcodec.permutation.cpu().numpy()
    rep = hq // hkv
    for bi, hi in ((0, 3), (15, 6)):
        kh = k[bi, hi].float().cpu().numpy()
        vh = v[bi, hi].float().cpu().numpy()
        idx = cache.key_indices[bi, hi].cpu().numpy()
        ref_idx, near = O.encode_blockvq_c(kh[:tc], cents, perm)
        ref_idx[:, heavy] = 0  # heavy blocks keep index 0 (codec.py:472-514)
        near[:, heavy] = False
        assert np.array_equal(idx[~near], ref_idx[~near]) and near.mean() < 1e-3
        vi = cache._value_indices[bi, hi, :tc].cpu().numpy()
        ref_vi, vnear = O.encode_blockvq_c(vh[:tc], vcents, vperm)
        assert np.array_equal(vi[~vnear], ref_vi[~vnear]) and vnear.mean() < 1e-3
        k_heavy = kh[:tc][:, perm][:, hd].astype(np.float16)
        assert np.array_equal(cache._key_heavy[bi, hi, :tc].cpu().numpy(), k_heavy)
        vals = O.dequantize_blockvq(vi, vcents, O.invert_permutation(vperm))
        vals_all = np.concatenate([vals, vh[tc:]], axis=0)[None, None]
        ref = O.sdpa_two_pass(q[bi:bi + 1, hi * rep:(hi + 1) * rep].cpu().numpy(), scale, perm,
                              cents, idx[None, None], kh[tc:][None, None] if tb else None,
                              vals_all, heavy_keys=k_heavy[None, None], heavy_dims=hd)
        got = out32[bi:bi + 1, hi * rep:(hi + 1) * rep].cpu().numpy()
        assert rel_err(got, ref) <= 1e-3
        got16 = out[bi:bi + 1, hi * rep:(hi + 1) * rep].float().cpu().numpy()
        assert rel_err16(got16, ref) <= 1e-3


@pytest.mark.parametrize("t_kv", [4096, 32768])
def test_config2_fitted_anisotropic_decode(t_kv):
    """Config 2 as its recipe states (and, at T_kv = 32768, the metric
    workload): seed 2, per-dim scale s ~ U[0.5, 4]^128; the codec fitted on
    the GPU to 4096 anisotropic N(0, 1)·s keys and queries (15 k-means
    iterations); fresh N(0, 1)·s keys encoded through ``update_and_fetch``
    into an fp16-value cache (8 KV heads); one fp16 query token of 32
    heads, scale 1/sqrt(128).  The fitted codebook makes the per-block LUTs
    more peaked than random centroids do.  Every (KV head, query head) is
    compared with the oracle."""
    d, hq, hkv = 128, 32, 8
    rng = np.random.default_rng(2)
    s = rng.uniform(0.5, 4.0, d).astype(np.float32)
    k_cal = (rng.standard_normal((4096, d)) * s).astype(np.float32)
    q_cal = (rng.standard_normal((4096, d)) * s).astype(np.float32)
    codec = S.SunShapeBlockCodec(d, device=DEV).fit(q_cal, k_cal, kmeans_iters=15, seed=2)
    keys = (rng.standard_normal((1, hkv, t_kv, d)) * s).astype(np.float16)
    vals = rng.standard_normal((1, hkv, t_kv, d)).astype(np.float16)
    q = rng.standard_normal((1, hq, 1, d)).astype(np.float16)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, max_tokens=t_kv)
    assert isinstance(cache, S.SunShapeKVCache) and cache.values_interleaved
    cache.update_and_fetch(torch.from_numpy(keys).to(DEV), torch.from_numpy(vals).to(DEV))
    scale = 1.0 / math.sqrt(d)
    qd = torch.from_numpy(q).to(DEV)
    out = S.sunshape_sdpa(qd, cache, scale)
    assert codec.last_score_backend == "hip_fused_mfma"
    out32 = S.sunshape_sdpa(qd, cache, scale, out_dtype=torch.float32)
    assert torch.equal(out32.to(torch.float16), out)
    cents = codec.centroids.cpu().numpy()
    perm = codec.permutation.cpu().numpy()
    idx = cache.key_indices.cpu().numpy()
    # encoded keys: bit-exact against the float64 encoder away from near-ties
    # (every head at T = 4096, two heads at T = 32768 to bound the CPU work)
    for h in (range(hkv) if t_kv <= 4096 else (0, 5)):
        ref_idx, near = O.encode_blockvq_c(keys[0, h].astype(np.float32), cents, perm)
        assert np.array_equal(idx[0, h][~near], ref_idx[~near]) and near.mean() < 1e-3
    ref = O.sdpa(q, idx, vals, cents, perm, scale)
    assert rel_err(out32.cpu().numpy(), ref) <= 1e-3
    assert rel_err16(out.float().cpu().numpy(), ref) <= 1e-3
