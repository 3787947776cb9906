"""Kernel launchers with the reference's names and argument meaning.

Mirrors the public launchers of the reference's ``kernels.py`` (Metal) on the
HIP C ABI.  Arrays are torch tensors on a ROCm device.  As in the reference, a
launcher returns ``None`` when the shape is outside what its kernel supports
(the caller then takes its slower path, which here also runs on the GPU);
unlike the reference, a missing library or a non-GPU tensor raises instead of
silently degrading.  The ``*_metal`` names are aliases kept so code written
against the reference runs unchanged.
"""

from __future__ import annotations

import torch

from . import _hip

# The dispatch counters live in the C-ABI binding layer, where every kernel
# launch of every route (launchers below, caches, SDPA, codecs) is counted
# (reference kernels.py:33-37).
_KERNEL_STATS: dict[str, int] = _hip._KERNEL_STATS
_record_kernel_dispatch = _hip.record_dispatch


def reset_kernel_stats() -> None:
    """Reset kernel dispatch counters (reference kernels.py:40-42)."""
    _KERNEL_STATS.clear()


def get_kernel_stats() -> dict[str, int]:
    """Kernel dispatch counters (reference kernels.py:45-47)."""
    return dict(_KERNEL_STATS)


def _as_u8_indices(indices: torch.Tensor) -> torch.Tensor:
    if indices.dtype != torch.uint8:
        indices = indices.to(torch.uint8)
    return indices.contiguous()


# --------------------------------------------------------------------------- #
#  Score gather                                                                #
# --------------------------------------------------------------------------- #


def block_vq_score_hip(qdots: torch.Tensor, indices: torch.Tensor, n_qh: int, T_kv: int,
                       n_blocks: int, n_centroids: int) -> torch.Tensor | None:
    """``scores[qh, t] = sum_b qdots[qh, b, indices[t, b]]`` -> (n_qh, T_kv) f32.
    Reference: block_vq_score_metal (kernels.py:87-116)."""
    _hip.require_gpu(qdots, indices)
    if n_centroids > 256 or n_blocks * n_centroids > 16384:
        return None
    q = qdots.reshape(n_qh, n_blocks, n_centroids).float()
    out = _hip.score_gather(q, _as_u8_indices(indices.reshape(T_kv, n_blocks)))
    return out


# --------------------------------------------------------------------------- #
#  Fused attention (one query group per call, reference signatures)           #
# --------------------------------------------------------------------------- #


def _fused_supported(head_dim: int, n_blocks: int, n_centroids: int) -> bool:
    return head_dim in (64, 128) and n_blocks * 8 == head_dim and 1 <= n_centroids <= 256


def _rows(queries: torch.Tensor, n_qh: int, head_dim: int) -> torch.Tensor:
    return queries.reshape(1, 1, n_qh, head_dim).contiguous()


def fused_attention_hip(queries, centroids, indices, values, n_qh: int, T_kv: int, n_blocks: int,
                        n_centroids: int, head_dim: int) -> torch.Tensor | None:
    """Single-pass online-softmax block-VQ attention over ``n_qh`` rows of
    already-transformed (and scaled) queries -> (n_qh, head_dim) float32.
    Reference: fused_attention_metal (kernels.py:233-291)."""
    return _fused_dense(queries, centroids, indices, values, n_qh, T_kv, n_blocks, n_centroids,
                        head_dim, False, 0)


def fused_attention_causal_hip(queries, centroids, indices, values, n_qh: int, T_kv: int,
                               n_blocks: int, n_centroids: int, head_dim: int,
                               q_offset: int = 0) -> torch.Tensor | None:
    """As ``fused_attention_hip`` with row r attending to keys t <= q_offset + r.
    Reference: fused_attention_causal_metal (kernels.py:388-446)."""
    return _fused_dense(queries, centroids, indices, values, n_qh, T_kv, n_blocks, n_centroids,
                        head_dim, True, q_offset)


def _fused_dense(queries, centroids, indices, values, n_qh, T_kv, n_blocks, n_centroids,
                 head_dim, causal, q_offset):
    _hip.require_gpu(queries, centroids, indices, values)
    if T_kv == 0:
        return torch.zeros((n_qh, head_dim), dtype=torch.float32, device=queries.device)
    if not _fused_supported(head_dim, n_blocks, n_centroids):
        return None
    q = _rows(queries, n_qh, head_dim)
    idx = _as_u8_indices(indices.reshape(1, 1, T_kv, n_blocks))
    v = values.reshape(1, 1, T_kv, head_dim).contiguous()
    out = _hip.decode_attn_dense(q, 1.0, None, centroids.float().contiguous(), idx, v, T_kv,
                                 causal=causal, q_offset=q_offset, out_dtype=torch.float32)
    return out.reshape(n_qh, head_dim)


def fused_attention_dequant_hip(queries, centroids, indices, packed_values, scales, zeros,
                                n_qh: int, T_kv: int, n_blocks: int, n_centroids: int,
                                head_dim: int, bits: int, group_size: int) -> torch.Tensor | None:
    """Fused attention with grouped values dequantised in registers.
    Reference: fused_attention_dequant_metal (kernels.py:697-765)."""
    return _fused_grouped(queries, centroids, indices, packed_values, scales, zeros, n_qh, T_kv,
                          n_blocks, n_centroids, head_dim, bits, group_size, False, 0)


def fused_attention_dequant_causal_hip(queries, centroids, indices, packed_values, scales, zeros,
                                       n_qh: int, T_kv: int, n_blocks: int, n_centroids: int,
                                       head_dim: int, bits: int, group_size: int,
                                       q_offset: int = 0) -> torch.Tensor | None:
    """Causal variant.  Reference: fused_attention_dequant_causal_metal
    (kernels.py:870-928)."""
    return _fused_grouped(queries, centroids, indices, packed_values, scales, zeros, n_qh, T_kv,
                          n_blocks, n_centroids, head_dim, bits, group_size, True, q_offset)


def _fused_grouped(queries, centroids, indices, packed, scales, zeros, n_qh, T_kv, n_blocks,
                   n_centroids, head_dim, bits, group_size, causal, q_offset):
    _hip.require_gpu(queries, centroids, indices, packed, scales, zeros)
    if T_kv == 0:
        return torch.zeros((n_qh, head_dim), dtype=torch.float32, device=queries.device)
    vpw = 32 // bits
    if not _fused_supported(head_dim, n_blocks, n_centroids) or bits not in (2, 3, 4) \
            or head_dim % group_size or group_size < vpw:
        return None
    q = _rows(queries, n_qh, head_dim)
    idx = _as_u8_indices(indices.reshape(1, 1, T_kv, n_blocks))
    p = packed.reshape(1, 1, T_kv, -1).contiguous()
    if p.dtype == torch.int32:
        p = p.view(torch.uint32)
    elif p.dtype != torch.uint32:
        p = p.to(torch.int64).to(torch.int32).view(torch.uint32)
    ng = head_dim // group_size
    sc = scales.reshape(1, 1, T_kv, ng).contiguous()
    zr = zeros.reshape(1, 1, T_kv, ng).to(sc.dtype).contiguous()
    if sc.dtype not in (torch.float32, torch.float16):
        sc, zr = sc.float(), zr.float()
    out = _hip.decode_attn_grouped(q, 1.0, None, centroids.float().contiguous(), idx, p, sc, zr,
                                   bits, group_size, T_kv, causal=causal, q_offset=q_offset,
                                   out_dtype=torch.float32)
    return out.reshape(n_qh, head_dim)


# --------------------------------------------------------------------------- #
#  Scalar quantisation                                                         #
# --------------------------------------------------------------------------- #


def quantize_scalar_to_indices(values: torch.Tensor, boundaries: torch.Tensor, *,
                               prefer_metal: bool = True) -> tuple[torch.Tensor, str]:
    """``idx = #{b : v > boundaries[b]}`` as uint8; returns ``(indices, backend)``.
    Reference: kernels.py:473-507.  ``prefer_metal`` is accepted for
    signature compatibility; the HIP kernel always runs."""
    out = _hip.scalar_quantize(values, boundaries.to(values.device))
    return out, "hip"


# --------------------------------------------------------------------------- #
#  Materialised path (reference kernels.py:514-563)                            #
# --------------------------------------------------------------------------- #


def fused_block_vq_attention(qdots, indices, values, T_q: int, T_kv: int, n_blocks: int,
                             n_centroids: int, head_dim: int) -> torch.Tensor:
    """Scores from a precomputed LUT, causal mask when ``T_kv >= T_q`` (query
    positions ``[T_kv - T_q, T_kv)``), softmax, ``@ values``.  Score gather on
    the HIP kernel, softmax/matmul with torch on the same device."""
    scores = block_vq_score_hip(qdots, indices, T_q, T_kv, n_blocks, n_centroids)
    if scores is None:
        raise ValueError("score gather unsupported for this LUT shape")
    if T_kv >= T_q:
        q_pos = torch.arange(T_kv - T_q, T_kv, device=scores.device)
        k_pos = torch.arange(T_kv, device=scores.device)
        causal = q_pos[:, None] >= k_pos[None, :]
        scores = torch.where(causal, scores, torch.finfo(scores.dtype).min)
    weights = torch.softmax(scores, dim=-1)
    return weights @ values.reshape(T_kv, head_dim).float()


# --------------------------------------------------------------------------- #
#  Block-VQ encode (reference kernels.py:1037-1082)                            #
# --------------------------------------------------------------------------- #


def block_vq_quantize_hip(keys_transformed: torch.Tensor, centroids: torch.Tensor, n_blocks: int,
                          n_centroids: int, block_dim: int, head_dim: int) -> torch.Tensor | None:
    """Nearest-centroid uint8 indices (N, n_blocks) for keys already in codec
    space.  Ties resolve to the lowest index."""
    _hip.require_gpu(keys_transformed, centroids)
    if n_centroids > 256 or block_dim not in (4, 8, 16) or n_blocks * block_dim != head_dim:
        return None
    k = keys_transformed.reshape(-1, head_dim)
    if k.stride(-1) != 1:
        k = k.contiguous()
    out = torch.empty((k.shape[0], n_blocks), dtype=torch.uint8, device=k.device)
    _hip.encode_blockvq(k, None, centroids.float().contiguous(), out, block_dim)
    return out


# --------------------------------------------------------------------------- #
#  Packing and grouped value quantisation (reference kernels.py:1102-1269)     #
# --------------------------------------------------------------------------- #


def _check_pack_shape(d: int, bits: int) -> None:
    if bits == 2 and d % 16:
        raise ValueError(f"Last dim must be divisible by 16 for 2-bit, got {d}")
    if bits == 4 and d % 8:
        raise ValueError(f"Last dim must be divisible by 8 for 4-bit, got {d}")
    if bits not in (2, 3, 4):
        raise ValueError(f"Unsupported bits: {bits}")


def pack_indices(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack 2/3/4-bit codes into uint32 words; element i of a word at bits
    [bits*i, bits*i+bits); 3-bit rows zero-padded to a multiple of 10."""
    _check_pack_shape(indices.shape[-1], bits)
    return _hip.pack_indices(indices, bits)


def unpack_indices(packed: torch.Tensor, D: int, bits: int) -> torch.Tensor:
    """Inverse of ``pack_indices`` -> uint32 (..., D)."""
    if bits not in (2, 3, 4):
        raise ValueError(f"Unsupported bits: {bits}")
    return _hip.unpack_indices(packed, D, bits)


def quantize_values(values: torch.Tensor, bits: int = 4, group_size: int = 64):
    """Asymmetric per-group min-max quantisation -> ``(packed, scales, zeros,
    n_groups)`` with float32 scales/zeros (T, n_groups)."""
    _hip.require_gpu(values)
    T, D = values.shape
    _check_pack_shape(D, bits)
    if D % group_size:
        raise ValueError(f"head_dim {D} not divisible by group_size {group_size}")
    ng = D // group_size
    nw = (D + 32 // bits - 1) // (32 // bits)
    packed = torch.empty((T, nw), dtype=torch.int32, device=values.device)
    scales = torch.empty((T, ng), dtype=torch.float32, device=values.device)
    zeros = torch.empty((T, ng), dtype=torch.float32, device=values.device)
    v = values if values.stride(-1) == 1 else values.contiguous()
    _hip.quantize_values_grouped(v, bits, group_size, packed, scales, zeros)
    return packed.view(torch.uint32), scales, zeros, ng


def dequantize_values(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, D: int,
                      bits: int = 4, group_size: int = 64) -> torch.Tensor:
    """``v = q * scale + zero`` per group -> float32 (..., D)."""
    return _hip.dequantize_values_grouped(packed, scales, zeros, D, bits, group_size)


# Reference names (drop-in aliases)
block_vq_score_metal = block_vq_score_hip
fused_attention_metal = fused_attention_hip
fused_attention_causal_metal = fused_attention_causal_hip
fused_attention_dequant_metal = fused_attention_dequant_hip
fused_attention_dequant_causal_metal = fused_attention_dequant_causal_hip
block_vq_quantize_metal = block_vq_quantize_hip
