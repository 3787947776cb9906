"""SDPA router (reference patch.py:1-109).

``scaled_dot_product_attention(queries, keys, values, cache, scale, mask,
sinks=None)`` has the signature of mlx-lm's ``models.base`` function that the
reference replaces: a SunShape cache goes to ``sunshape_sdpa``, anything else
to the original function of the patched module (or, with no original, plain
grouped-query softmax attention in torch).  ``apply()`` installs it as the
``scaled_dot_product_attention`` attribute of the target modules (by default
the reference's: ``mlx_lm.models.base`` and the qwen3 aliases; more with
``register_target``), ``revert()`` restores the originals.
"""

from __future__ import annotations

import importlib

import torch

from .attention import sunshape_sdpa
from .cache import HybridSunShapeKVCache, SunShapeKVCache

_BASE_MODULE = "mlx_lm.models.base"
_ALIAS_MODULES = ["mlx_lm.models.qwen3", "mlx_lm.models.qwen3_next", "mlx_lm.models.qwen3_moe"]

_patched = False
_originals: dict[str, object] = {}
_extra_targets: list[str] = []


def _plain_sdpa(queries, keys, values, scale, mask):
    """Grouped-query softmax attention in float32 (the non-SunShape path when
    the patched module had no original)."""
    hq, hkv = queries.shape[1], keys.shape[1]
    rep = hq // hkv
    k = keys.repeat_interleave(rep, dim=1).float()
    v = values.repeat_interleave(rep, dim=1).float()
    s = torch.matmul(queries.float() * scale, k.transpose(-1, -2).contiguous())
    t_q, t_kv = queries.shape[2], keys.shape[2]
    if isinstance(mask, str) and mask == "causal":
        q_pos = torch.arange(t_kv - t_q, t_kv, device=s.device)
        keep = q_pos[:, None] >= torch.arange(t_kv, device=s.device)[None, :]
        s = torch.where(keep, s, torch.finfo(torch.float32).min)
    elif mask is not None and not isinstance(mask, str):
        s = torch.where(mask, s, torch.finfo(torch.float32).min) if mask.dtype == torch.bool \
            else s + mask.float()
    return torch.matmul(torch.softmax(s, dim=-1), v).to(queries.dtype)


def _original_sdpa():
    """The base module's original SDPA (the aliases point at the same
    function), else the first patched module's."""
    if _BASE_MODULE in _originals:
        return _originals[_BASE_MODULE]
    return next(iter(_originals.values()), None)


def scaled_dot_product_attention(queries, keys, values, cache, scale, mask, sinks=None):
    """SDPA router: SunShape cache -> ``sunshape_sdpa`` (``sinks`` ignored, as
    the reference does); otherwise the original SDPA (patch.py:58-74)."""
    if isinstance(cache, (SunShapeKVCache, HybridSunShapeKVCache)):
        return sunshape_sdpa(queries, cache, scale, mask)
    original = _original_sdpa()
    if original is not None:
        return original(queries, keys, values, cache, scale, mask, sinks=sinks)
    return _plain_sdpa(queries, keys, values, scale, mask)


_patched_sdpa = scaled_dot_product_attention  # the reference's name for the router


def register_target(module_name: str) -> None:
    """Also patch ``module_name.scaled_dot_product_attention`` on ``apply()``."""
    if module_name not in _extra_targets:
        _extra_targets.append(module_name)


def _targets() -> list[str]:
    return [_BASE_MODULE] + _ALIAS_MODULES + _extra_targets


def apply() -> None:
    """Activate the router (idempotent).  Raises RuntimeError when no target
    module can be imported, as the reference does without mlx-lm
    (patch.py:77-88)."""
    global _patched
    if _patched:
        return
    found = []
    for name in _targets():
        try:
            module = importlib.import_module(name)
        except ImportError:
            continue
        if hasattr(module, "scaled_dot_product_attention"):
            found.append(module)
            _originals.setdefault(name, module.scaled_dot_product_attention)
    if not found:
        raise RuntimeError("no SDPA module to patch: mlx-lm style model code is not installed; "
                           "register one with register_target(module_name)")
    for module in found:
        module.scaled_dot_product_attention = scaled_dot_product_attention
    _patched = True


def revert() -> None:
    """Remove the router and restore every original (patch.py:91-104)."""
    global _patched
    if not _patched:
        return
    for name, original in _originals.items():
        try:
            module = importlib.import_module(name)
        except ImportError:
            continue
        module.scaled_dot_product_attention = original
    _originals.clear()
    _patched = False


def is_patched() -> bool:
    """Whether the router is installed (patch.py:107-109)."""
    return _patched
