"""Codec and KV-cache state on disk (safetensors).

The reference exposes a cache's arrays for mlx-lm's prompt-cache helpers
(``state``, reference cache.py:256-262 and 988-1000) and its codec keeps its
fitted arrays as attributes (codec.py:228-267), but neither has a file format
of its own.  This module stores:

- a codec: every array of ``SunShapeBlockCodec.state_dict()`` plus its
  configuration;
- a cache: its codec (and a separate value codec, if any), every storage
  buffer at full capacity (so the restored cache keeps its layout, including
  the kernels' interleaved forms, and can be extended), its offsets and the
  constructor configuration.

Tensors go into one safetensors file under ``codec.*``, ``value_codec.*`` and
``cache.*``; configuration and offsets are JSON strings in the file's
metadata.  Loading executes nothing from the file.
"""

from __future__ import annotations

import json

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from . import _hip
from .cache import HybridSunShapeKVCache, SunShapeKVCache
from .codec import SunShapeBlockCodec

FORMAT = "sunshape-mlx-amd/1"

# storage buffers of each cache class (None when not allocated)
_CACHE_TENSORS = {
    "SunShapeKVCache": ("_key_indices", "_values"),
    "HybridSunShapeKVCache": ("_key_indices", "_values_packed", "_values_il", "_value_scales",
                              "_value_zeros", "_value_norms", "_value_indices", "_values_fp16",
                              "_values_il8", "_key_buffer", "_value_buffer", "_key_heavy"),
}
# integer bookkeeping restored alongside the buffers
_CACHE_SCALARS = {
    "SunShapeKVCache": ("offset", "_capacity"),
    "HybridSunShapeKVCache": ("_compressed_offset", "_buffer_offset", "_compressed_capacity",
                              "_value_n_groups", "_buf_start"),
}


def _dtype_name(dt: torch.dtype) -> str:
    return str(dt).split(".")[-1]


def _dtype(name: str) -> torch.dtype:
    dt = getattr(torch, name, None)
    if not isinstance(dt, torch.dtype):
        raise ValueError(f"unknown dtype {name!r} in cache metadata")
    return dt


def _codec_tensors(codec: SunShapeBlockCodec, prefix: str) -> tuple[dict, dict]:
    sd = codec.state_dict()
    cfg = dict(sd.pop("config"))
    cfg["rotation_seed"] = getattr(codec, "rotation_seed", 0)
    return {f"{prefix}.{k}": v.contiguous() for k, v in sd.items()}, cfg


def _codec_from(tensors: dict, prefix: str, cfg: dict, device) -> SunShapeBlockCodec:
    codec = SunShapeBlockCodec(cfg["head_dim"], block_dim=cfg["block_dim"],
                               n_centroids=cfg["n_centroids"], c=cfg.get("c", 5.0),
                               n_refine_dsq=cfg.get("n_refine_dsq", 3), mode=cfg["mode"],
                               use_rotation=cfg["mode"] == "rotated",
                               rotation_seed=cfg.get("rotation_seed", 0), device=device,
                               heavy_fp16=cfg.get("heavy_fp16", False))
    sd = {k[len(prefix) + 1:]: v for k, v in tensors.items() if k.startswith(prefix + ".")}
    sd["config"] = cfg
    return codec.load_state_dict(sd)


def save_codec(path: str, codec: SunShapeBlockCodec) -> None:
    """Write a codec's arrays and configuration to ``path``."""
    tensors, cfg = _codec_tensors(codec, "codec")
    save_file(tensors, path, metadata={"format": FORMAT, "codec": json.dumps(cfg)})


def _read(path: str) -> tuple[dict, dict]:
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path}: not a {FORMAT} file (format {meta.get('format')!r})")
    return tensors, meta


def load_codec(path: str, device=None) -> SunShapeBlockCodec:
    """Read a codec written by :func:`save_codec` (or the codec of a cache
    file) onto ``device``."""
    tensors, meta = _read(path)
    return _codec_from(tensors, "codec", json.loads(meta["codec"]), device)


def _cache_config(cache) -> dict:
    cfg = dict(n_kv_heads=cache.n_kv_heads, head_dim=cache.head_dim,
               dtype=_dtype_name(cache.dtype), max_tokens=cache.max_tokens)
    if isinstance(cache, HybridSunShapeKVCache):
        cfg.update(buffer_size=cache.buffer_size, value_backend=cache.value_backend,
                   value_bits=cache.value_bits, value_group_size=cache.value_group_size,
                   value_seed=cache.value_seed, prefer_metal_kernels=cache.prefer_metal_kernels,
                   value_scale_dtype=_dtype_name(cache.value_scale_dtype))
    else:
        cfg.update(return_dequantized_keys=cache.return_dequantized_keys)
    return cfg


def save_cache(path: str, cache) -> None:
    """Write a SunShape or hybrid cache (with its codecs) to ``path``."""
    kind = type(cache).__name__
    if kind not in _CACHE_TENSORS:
        raise TypeError(f"cannot serialise {kind}")
    if hasattr(cache, "flush"):
        cache.flush()  # a held decode step's tokens into storage first
    tensors, codec_cfg = _codec_tensors(cache.codec, "codec")
    meta = {"format": FORMAT, "codec": json.dumps(codec_cfg), "cache_class": kind,
            "cache_config": json.dumps(_cache_config(cache))}
    vc = getattr(cache, "value_codec", None)
    if vc is not None and vc is not cache.codec:
        vt, vcfg = _codec_tensors(vc, "value_codec")
        tensors.update(vt)
        meta["value_codec"] = json.dumps(vcfg)
    for name in _CACHE_TENSORS[kind]:
        t = getattr(cache, name)
        if t is not None:
            tensors[f"cache.{name}"] = t.detach().contiguous().cpu()
    meta["cache_scalars"] = json.dumps({k: int(getattr(cache, k)) for k in _CACHE_SCALARS[kind]})
    save_file({k: v.cpu() for k, v in tensors.items()}, path, metadata=meta)


def load_cache(path: str, device=None):
    """Read a cache written by :func:`save_cache` onto ``device`` (default:
    the current GPU).  Returns the cache; its codec is ``cache.codec``."""
    tensors, meta = _read(path)
    if "cache_class" not in meta:
        raise ValueError(f"{path}: holds no cache")
    dev = torch.device(device) if device is not None else torch.device("cuda")
    codec = _codec_from(tensors, "codec", json.loads(meta["codec"]), dev)
    cfg = json.loads(meta["cache_config"])
    cfg["dtype"] = _dtype(cfg["dtype"])
    kind = meta["cache_class"]
    if kind == "HybridSunShapeKVCache":
        cfg["value_scale_dtype"] = _dtype(cfg["value_scale_dtype"])
        vcodec = None
        if "value_codec" in meta:
            vcodec = _codec_from(tensors, "value_codec", json.loads(meta["value_codec"]), dev)
        cache = HybridSunShapeKVCache(codec, value_codec=vcodec, **cfg)
    elif kind == "SunShapeKVCache":
        cache = SunShapeKVCache(codec, **cfg)
    else:
        raise ValueError(f"{path}: unknown cache class {kind!r}")
    for name in _CACHE_TENSORS[kind]:
        key = f"cache.{name}"
        if key in tensors:
            setattr(cache, name, tensors[key].to(dev))
    for k, v in json.loads(meta["cache_scalars"]).items():
        setattr(cache, k, int(v))
    if kind == "HybridSunShapeKVCache" and cache._turbo_il and cache._values_packed is not None:
        # 2-bit TurboQuant codes written as packed rows (files of earlier
        # versions): interleave them as the cache now keeps them
        rows = cache._values_packed
        b_, h_, cap, _ = rows.shape
        cache._values_il = torch.zeros((b_, h_, cap // 16, cache.head_dim), dtype=torch.int32,
                                       device=rows.device)
        if cache._compressed_offset:
            _hip.pack_grouped_il(rows[:, :, :cache._compressed_offset], 2, cache._values_il, 0)
        cache._values_packed = None
    if kind == "HybridSunShapeKVCache" and cache._fp16_il8 and cache._values_fp16 is not None:
        # fp16 values written token-major (files of earlier versions): move
        # them into the interleaved layout the cache now keeps
        vf = cache._values_fp16
        b_, h_, cap, d = vf.shape
        cache._values_il8 = torch.zeros((b_, h_, (cap + 7) // 8, d, 8), dtype=torch.float16,
                                        device=vf.device)
        if cache._compressed_offset:
            _hip.append_values_il8(vf[:, :, :cache._compressed_offset].to(torch.float16),
                                   cache._values_il8, 0)
        cache._values_fp16 = None
    return cache
