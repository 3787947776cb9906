"""Value codecs for hybrid SunShape caches (reference value_codecs.py:1-201).

``GroupedValueCodec``: asymmetric per-group min-max 2/3/4-bit codes packed in
uint32 words, one scale/zero pair per group (HIP encode/decode kernels).
``TurboQuantValueCodec``: per-token norm, random rotation, Lloyd-Max scalar
codes of N(0, 1/D) coordinates, packed (rotation on torch, scalar quantise and
packing on HIP kernels).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from functools import lru_cache

import numpy as np
import torch

from . import _hip
from .kernels import (
    dequantize_values,
    pack_indices,
    quantize_scalar_to_indices,
    quantize_values,
    unpack_indices,
)
from .rotation import generate_rotation_matrix


# Positive levels of the Lloyd-Max quantiser of N(0, 1) (Max, 1960) at 1-4
# bits, the values the reference ships as literal tables
# (value_codecs.py:20-87).  Its tables are exactly symmetric and each
# boundary is exactly the midpoint of its two levels, so the full tables are
# rebuilt below bit for bit.  The 4-bit levels sit up to 3.5e-4 away from
# the exact fixed point of the Lloyd-Max conditions; they are kept as data
# (not recomputed) so that TurboQuant codes equal the reference's.
_LLOYD_MAX_POSITIVE: dict[int, tuple[float, ...]] = {
    1: (0.7978845608028654,),
    2: (0.4527800346911237, 1.510417608611893),
    3: (0.2450941791152904, 0.7560052816730181, 1.3439092791423422, 2.151945705166112),
    4: (0.12844300124876415, 0.38818871416000605, 0.6569817464411519, 0.9426291036999694,
        1.2565648452462146, 1.618400443227723, 2.069364258154187, 2.732896755154294),
}


@lru_cache(maxsize=None)
def lloyd_max_gaussian(bits: int) -> tuple[tuple[float, ...], tuple[float, ...]]:
    """Lloyd-Max quantiser of N(0, 1) at ``bits`` bits: ``(levels,
    boundaries)`` in ascending order, equal to the reference's
    ``_TURBOQUANT_CODEBOOKS[bits]`` (value_codecs.py:20-87)."""
    if bits not in _LLOYD_MAX_POSITIVE:
        raise ValueError(f"Lloyd-Max tables exist for 1-4 bits, got {bits}")
    pos = _LLOYD_MAX_POSITIVE[bits]
    levels = tuple(-x for x in reversed(pos)) + pos
    bounds = tuple(0.5 * (a + b) for a, b in zip(levels[:-1], levels[1:]))
    return levels, bounds


_CODES_PER_WORD = {2: 16, 3: 10, 4: 8}


def _packed_dim(head_dim: int, bits: int) -> int:
    """uint32 words per packed row: 16 two-bit, 10 three-bit (the last word
    zero-padded) or 8 four-bit codes per word; 2- and 4-bit rows must fill
    their words (the format rule of reference cache.py:39-56)."""
    per_word = _CODES_PER_WORD.get(bits)
    if per_word is None:
        raise ValueError(f"Unsupported bits: {bits} (must be 2, 3, or 4)")
    if bits != 3 and head_dim % per_word:
        raise ValueError(f"head_dim must be divisible by {per_word} for {bits}-bit packing, "
                         f"got {head_dim}")
    return -(-head_dim // per_word)


@dataclass
class GroupedValueCodec:
    """reference value_codecs.py:104-133."""
    head_dim: int
    bits: int
    group_size: int = 64
    name: str = "grouped"
    last_quantize_backend: str = "hip"

    @property
    def packed_dim(self) -> int:
        return _packed_dim(self.head_dim, self.bits)

    @property
    def n_groups(self) -> int:
        return self.head_dim // self.group_size

    def quantize(self, values: torch.Tensor):
        packed, scales, zeros, _ = quantize_values(values, bits=self.bits,
                                                   group_size=self.group_size)
        self.last_quantize_backend = "hip"
        return packed, scales, zeros

    def dequantize(self, packed, scales, zeros) -> torch.Tensor:
        return dequantize_values(packed, scales, zeros, D=self.head_dim, bits=self.bits,
                                 group_size=self.group_size)


@dataclass
class TurboQuantValueCodec:
    """reference value_codecs.py:136-177.  The rotation is drawn from NumPy's
    generator (see ``generate_rotation_matrix``)."""
    head_dim: int
    bits: int
    seed: int = 43
    prefer_metal: bool = True
    name: str = "turboquant"
    last_quantize_backend: str = "none"
    device: object = field(default=None, repr=False)

    def __post_init__(self) -> None:
        if self.bits not in (2, 3, 4):
            raise ValueError(f"TurboQuant values support 2, 3, or 4 bits, got {self.bits}")
        levels, bounds = lloyd_max_gaussian(self.bits)
        # python-float products rounded once to float32 (value_codecs.py:148-151)
        s = 1.0 / math.sqrt(self.head_dim)
        dev = self.device or ("cuda" if torch.cuda.is_available() else "cpu")
        self.centroids = torch.tensor([c * s for c in levels], dtype=torch.float32, device=dev)
        self.boundaries = torch.tensor([b * s for b in bounds], dtype=torch.float32, device=dev)
        self.rotation = torch.from_numpy(
            generate_rotation_matrix(self.head_dim, seed=self.seed)).to(dev)
        self.rotation_t = self.rotation.T.contiguous()

    @property
    def packed_dim(self) -> int:
        return _packed_dim(self.head_dim, self.bits)

    def levels_host(self) -> list[float]:
        """The scaled levels as host floats (the fused decode takes them as
        kernel arguments), read from the device once."""
        lv = getattr(self, "_levels_host", None)
        if lv is None:
            lv = self._levels_host = [float(x) for x in self.centroids.cpu().tolist()]
        return lv

    def _on(self, device):
        if self.rotation.device != device:
            self.centroids = self.centroids.to(device)
            self.boundaries = self.boundaries.to(device)
            self.rotation = self.rotation.to(device)
            self.rotation_t = self.rotation_t.to(device)

    def quantize(self, values: torch.Tensor):
        _hip.require_gpu(values)
        self._on(values.device)
        v = values.float()
        norms = torch.linalg.vector_norm(v, dim=-1, keepdim=True)
        unit = v / torch.clamp(norms, min=1e-8)
        rotated = unit @ self.rotation_t
        idx, backend = quantize_scalar_to_indices(rotated, self.boundaries,
                                                  prefer_metal=self.prefer_metal)
        self.last_quantize_backend = backend
        return pack_indices(idx, self.bits), norms.squeeze(-1)

    def dequantize(self, packed: torch.Tensor, norms: torch.Tensor) -> torch.Tensor:
        self._on(packed.device)
        idx = unpack_indices(packed, self.head_dim, self.bits).to(torch.int64)
        unit = self.centroids[idx] @ self.rotation
        return unit * norms[..., None]


def build_value_codec(value_backend: str, *, head_dim: int, value_bits: int,
                      value_group_size: int = 64, value_seed: int = 43,
                      prefer_metal: bool = True):
    """reference value_codecs.py:180-201."""
    if value_backend == "fp16":
        return None
    if value_backend == "grouped":
        return GroupedValueCodec(head_dim=head_dim, bits=value_bits, group_size=value_group_size)
    if value_backend == "turboquant":
        return TurboQuantValueCodec(head_dim=head_dim, bits=value_bits, seed=value_seed,
                                    prefer_metal=prefer_metal)
    raise ValueError(f"Unsupported value backend: {value_backend}")
