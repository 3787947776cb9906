"""Codec and cache files (sunshape_mlx_amd.serialize): a saved object loads
back with identical arrays, offsets and configuration, decodes to the same
output and keeps appending like the original."""

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import sunshape_mlx_amd as S


def _codec(seed, mode="profileperm_baseline", device="cpu", d=128, bd=8):
    rng = np.random.default_rng(seed)
    codec = S.SunShapeBlockCodec(d, block_dim=bd, device=device,
                                 use_rotation=(mode == "rotated"), rotation_seed=seed,
                                 mode=mode if mode != "rotated" else "profileperm_baseline")
    state = {"centroids": rng.standard_normal((d // bd, 256, bd)).astype(np.float32)}
    if mode != "rotated":
        state["permutation"] = rng.permutation(d).astype(np.int32)
    return codec.load_state_dict(state)


@pytest.mark.parametrize("mode", ["profileperm_baseline", "rotated"])
def test_codec_roundtrip_cpu(tmp_path, mode):
    codec = _codec(3, mode)
    path = str(tmp_path / "codec.safetensors")
    S.save_codec(path, codec)
    back = S.load_codec(path, device="cpu")
    assert (back.mode, back.head_dim, back.block_dim, back.n_centroids) == \
        (codec.mode, codec.head_dim, codec.block_dim, codec.n_centroids)
    assert back.use_rotation == codec.use_rotation
    for k in S.SunShapeBlockCodec._STATE_KEYS:
        assert torch.equal(getattr(back, k).cpu(), getattr(codec, k).cpu()), k
    assert torch.equal(back.inv_permutation.cpu(), codec.inv_permutation.cpu())


def test_rejects_foreign_files(tmp_path):
    path = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(3)}, path, metadata={"format": "something-else"})
    with pytest.raises(ValueError, match="not a sunshape"):
        S.load_codec(path, device="cpu")
    codec_only = str(tmp_path / "codec.safetensors")
    S.save_codec(codec_only, _codec(4))
    with pytest.raises(ValueError, match="holds no cache"):
        S.load_cache(codec_only, device="cpu")


def _caches():
    return [
        ("fp16", lambda c: S.create_kv_cache(c, n_kv_heads=2)),
        ("hybrid-grouped-il", lambda c: S.create_kv_cache(c, n_kv_heads=2, value_backend="grouped",
                                                          value_bits=2, value_scale_dtype=torch.float16)),
        ("hybrid-grouped-3bit", lambda c: S.create_kv_cache(c, n_kv_heads=2, value_backend="grouped",
                                                            value_bits=3, buffer_size=32)),
        ("hybrid-turboquant", lambda c: S.create_kv_cache(c, n_kv_heads=2, value_backend="turboquant",
                                                          value_bits=2, buffer_size=64)),
        ("hybrid-sunshape", lambda c: S.create_kv_cache(c, n_kv_heads=2, value_backend="sunshape",
                                                        value_bits=8, value_codec=_codec(9, device="cuda",
                                                                                         bd=4),
                                                        buffer_size=16)),
        ("hybrid-fp16", lambda c: S.create_kv_cache(c, n_kv_heads=2, value_bits=None,
                                                    value_backend="fp16", buffer_size=48)),
        ("hybrid-sunshape-heavy-fp16", lambda c: S.create_kv_cache(
            _heavy_codec(c), n_kv_heads=2, value_backend="sunshape", value_bits=8,
            value_codec=_codec(10, device="cuda", bd=4), buffer_size=24)),
    ]


def _heavy_codec(base):
    """A mixed-precision codec with 4 heavy blocks kept in fp16, built from
    ``base``'s arrays."""
    heavy = np.zeros(16, bool)
    heavy[[1, 4, 9, 15]] = True
    cents = base.centroids.cpu().numpy().copy()
    cents[heavy] = 0.0
    codec = S.SunShapeBlockCodec(128, device=base.device, mode="profileperm_mixed_precision",
                                 heavy_fp16=True)
    return codec.load_state_dict({"centroids": cents,
                                  "permutation": base.permutation.cpu().numpy(),
                                  "mixed_high_precision_blocks": heavy})


@pytest.mark.gpu
@pytest.mark.parametrize("name,make", _caches(), ids=[n for n, _ in _caches()])
def test_cache_roundtrip_decodes_and_appends_alike(tmp_path, name, make):
    dev = torch.device("cuda")
    codec = _codec(5, device=dev)
    cache = make(codec)
    g = torch.Generator(device=dev).manual_seed(6)
    b, hq, hkv, d = 2, 8, 2, 128

    def kv(n):
        return (torch.randn((b, hkv, n, d), generator=g, device=dev).half(),
                torch.randn((b, hkv, n, d), generator=g, device=dev).half())

    k, v = kv(300)
    cache.update_and_fetch(k, v)
    path = str(tmp_path / f"{name}.safetensors")
    S.save_cache(path, cache)
    back = S.load_cache(path, device=dev)
    assert type(back) is type(cache) and back.offset == cache.offset
    q = torch.randn((b, hq, 1, d), generator=g, device=dev).half()
    o1 = S.sunshape_sdpa(q, cache, 0.088)
    be1 = cache.codec.last_score_backend
    o2 = S.sunshape_sdpa(q, back, 0.088)
    assert back.codec.last_score_backend == be1
    assert torch.equal(o1, o2)
    # both keep appending (flushes, growth) and stay identical
    k2, v2 = kv(290)
    cache.update_and_fetch(k2, v2)
    back.update_and_fetch(k2, v2)
    assert back.offset == cache.offset == 590
    assert torch.equal(S.sunshape_sdpa(q, cache, 0.088), S.sunshape_sdpa(q, back, 0.088))
    assert torch.equal(cache.values.cpu(), back.values.cpu())
