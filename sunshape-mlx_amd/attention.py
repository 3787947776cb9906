"""SunShape SDPA: scaled dot-product attention over block-VQ keys
(reference attention.py:1-353).

Scores never need dequantised keys: with a fixed block codebook,
``score[q, t] = sum_b LUT[q, b, idx[t, b]]`` where ``LUT[q, b, c]`` is the dot
product of query block b with centroid c.  The fused HIP kernels build the LUT
in LDS and run gather + online softmax + value accumulation in one pass over
the cache, for every query head of every KV group in a single launch (the
reference loops over (batch, KV head, q head) with one Metal dispatch each,
attention.py:268-305).

Routing follows the reference (attention.py:236-246): a compressed-only cache
with no mask or a causal mask takes a fused kernel; a hybrid cache with
buffered full-precision tokens, or an explicit mask array, takes the two-pass
path (attention.py:307-350), which here also runs on the GPU (HIP LUT and
score kernels, torch softmax and matmul).
"""

from __future__ import annotations

import weakref

import torch

from . import _hip
from .cache import HybridSunShapeKVCache, SunShapeKVCache
from .codec import PERM_MODES, SunShapeBlockCodec


def _kernel_query(codec: SunShapeBlockCodec, queries: torch.Tensor, scale: float):
    """(q, scale, perm) for the fused kernels, which form
    ``round_to(q.dtype, q * scale)`` and then permute (attention.py:208, 228).
    The rotated mode rotates on the host: ``(q * scale) @ R^T`` in float32
    (attention.py:230), passed with scale 1 and no permutation."""
    if codec.mode in PERM_MODES:
        return queries, float(scale), codec.permutation
    if codec.use_rotation:
        q = (queries * scale).float() @ codec.rotation.t()
        return q.contiguous(), 1.0, None
    return queries, float(scale), None


def _transform_grouped(codec: SunShapeBlockCodec, q_grouped: torch.Tensor) -> torch.Tensor:
    """Codec-space queries from scaled, grouped queries (attention.py:223-232)."""
    if codec.mode in PERM_MODES:
        return q_grouped[..., codec.permutation.long()]
    if codec.use_rotation:
        return q_grouped.float() @ codec.rotation.t()
    return q_grouped


def _prepared_decode(cache, ops: dict, codec: SunShapeBlockCodec, q: torch.Tensor,
                     kscale: float, perm, buffered: bool = False):
    """The cache's prepared matrix-core decode (``_hip.PreparedDecode``, or
    ``PreparedDecodeBuffered`` for a hybrid cache holding buffered tokens)
    for queries shaped like ``q``: built on the first call and again whenever
    a cache buffer, the codebook or the query layout changes (the plan holds
    weak references, so it never keeps a replaced buffer alive)."""
    kind = ops["kind"]
    cb = codec.kernel_codebook()
    if kind == "il8":
        tensors = (ops["idx"], ops["values"], cb)
    else:
        tensors = (ops["idx"], ops["codes_il"], ops["scales"], ops["zeros"], cb)
    if perm is not None:
        tensors += (perm,)
    if buffered:  # the buffer stores (their windows move from call to call)
        tensors += (cache._key_buffer, cache._value_buffer)
    key = (kind, q.shape, q.dtype, q.device, kscale, ops.get("bits"), ops.get("group_size"),
           buffered)
    held = getattr(cache, "_decode_prepared", None)
    if held is not None and held[0] == key and len(held[1]) == len(tensors) and \
            all(r() is t for r, t in zip(held[1], tensors)):
        return held[2]
    nb, nc = codec.n_blocks, codec.n_centroids
    bk = ops["buf_keys"] if buffered else None
    if kind == "il8":
        plan = _hip.prepare_decode_il8(q, kscale, perm, cb, nb, nc, ops["idx"], ops["values"],
                                       buf_keys=bk)
    else:
        plan = _hip.prepare_decode_grouped_il(q, kscale, perm, cb, nb, nc, ops["idx"],
                                              ops["codes_il"], ops["scales"], ops["zeros"],
                                              ops["bits"], ops["group_size"], buf_keys=bk)
    cache._decode_prepared = (key, tuple(weakref.ref(t) for t in tensors), plan)
    return plan


def _fused_step(cache: SunShapeKVCache, queries: torch.Tensor, scale: float, causal: bool,
                q_offset: int, out_dtype: torch.dtype):
    """The decode step whose new tokens the cache holds back
    (``cache.fuse_steps``): one ``ss_decode_step_il8`` launch encodes them,
    attends every token and stores them; None (tokens still held) when that
    launch does not apply."""
    codec = cache.codec
    q, kscale, perm = _kernel_query(codec, queries, scale)
    tensors = (cache._key_indices, cache._values, codec.kernel_codebook(), codec.centroids)
    if perm is not None:
        tensors += (perm,)
    key = ("step", q.shape, q.dtype, q.device, kscale)
    held = getattr(cache, "_step_prepared", None)
    if held is not None and held[0] == key and len(held[1]) == len(tensors) and \
            all(r() is t for r, t in zip(held[1], tensors)):
        plan = held[2]
    else:
        try:
            plan = _hip.prepare_decode_step_il8(q, kscale, perm, tensors[2], codec.centroids,
                                                codec.n_blocks, codec.n_centroids,
                                                cache._key_indices, cache._values)
        except (_hip.SunShapeUnsupported, ValueError):
            return None
        cache._step_prepared = (key, tuple(weakref.ref(t) for t in tensors), plan)
    k, v, pos = cache._take_pending()
    try:
        out = plan(q, pos, k, v, causal, q_offset, out_dtype=out_dtype)
    except _hip.SunShapeUnsupported:
        cache._pending = (k, v, k._version, v._version, pos)
        return None
    codec.last_score_backend = "hip_fused_mfma_step"
    return out


def _fused_hybrid_step(cache: HybridSunShapeKVCache, queries: torch.Tensor, scale: float,
                       causal: bool, q_offset: int, out_dtype: torch.dtype):
    """The decode step a hybrid cache with 2/4-bit grouped or fp16 values
    holds back (``cache.fuse_steps``): one ``ss_decode_step_grouped_il_hybrid``
    (or ``ss_decode_step_il8_hybrid``) launch
    moves the tokens that leave the buffer into compressed storage, stores
    the new ones in the buffer and attends every token; None (step still
    held) when that launch does not apply."""
    codec = cache.codec
    q, kscale, perm = _kernel_query(codec, queries, scale)
    grouped = cache._grouped_il
    vals = ((cache._values_il, cache._value_scales, cache._value_zeros) if grouped
            else (cache._values_il8,))
    tensors = (cache._key_indices,) + vals + (codec.kernel_codebook(), codec.centroids,
                                               cache._key_buffer, cache._value_buffer)
    if perm is not None:
        tensors += (perm,)
    key = ("hstep", q.shape, q.dtype, q.device, kscale)
    held = getattr(cache, "_hstep_prepared", None)
    if held is not None and held[0] == key and len(held[1]) == len(tensors) and \
            all(r() is t for r, t in zip(held[1], tensors)):
        plan = held[2]
    else:
        cb = codec.kernel_codebook()
        try:
            if grouped:
                gc = cache._value_codec_impl
                plan = _hip.prepare_decode_step_grouped_il_hybrid(
                    q, kscale, perm, cb, codec.centroids, codec.n_blocks, codec.n_centroids,
                    cache._key_indices, cache._values_il, cache._value_scales,
                    cache._value_zeros, gc.bits, gc.group_size, cache._key_buffer)
            else:
                plan = _hip.prepare_decode_step_il8_hybrid(
                    q, kscale, perm, cb, codec.centroids, codec.n_blocks, codec.n_centroids,
                    cache._key_indices, cache._values_il8, cache._key_buffer)
        except (_hip.SunShapeUnsupported, ValueError):
            return None
        cache._hstep_prepared = (key, tuple(weakref.ref(t) for t in tensors), plan)
    pend = cache._pending
    k, v, tc, s0, n, nf = cache._take_pending()
    try:
        out = plan(q, tc, cache._key_buffer[:, :, s0:], cache._value_buffer[:, :, s0:], n, nf,
                   k, v, causal, q_offset, out_dtype=out_dtype)
    except (_hip.SunShapeUnsupported, ValueError):  # raised before any launch
        cache._pending = pend
        return None
    codec.last_score_backend = "hip_fused_mfma_dequant_step" if grouped else "hip_fused_mfma_step"
    return out


def _fused(cache, queries: torch.Tensor, scale: float, causal: bool, q_offset: int,
           out_dtype: torch.dtype):
    """One fused launch over the whole cache, or None when no fused kernel
    applies to this cache / shape (the reference's None-fallback,
    kernels.py:259-291)."""
    if getattr(cache, "_pending", None) is not None and queries.shape[2] <= _hip.MAX_STEP_TOKENS:
        if isinstance(cache, HybridSunShapeKVCache):
            out = _fused_hybrid_step(cache, queries, scale, causal, q_offset, out_dtype)
        else:
            out = _fused_step(cache, queries, scale, causal, q_offset, out_dtype)
        if out is not None:
            return out
    ops = cache.fused_operands()  # (stores held tokens first)
    if ops is None:
        return None
    codec = cache.codec
    buffered = cache.buffer_offset if isinstance(cache, HybridSunShapeKVCache) else 0
    q, kscale, perm = _kernel_query(codec, queries, scale)
    # a prompt against a hybrid cache (fp16, grouped or TurboQuant values):
    # compressed keys from the codebook, buffered keys whole, values
    # materialised once in the interleaved fp16 layout
    b_, hq, tq, d = queries.shape
    if buffered and cache.dtype == torch.bfloat16 and \
            ops["kind"] in ("grouped_il", "grouped", "turboquant_il", "turboquant", "sunshape_v"):
        # with buffered tokens the reference attends over cache.values, the
        # dequantised values rounded to the cache dtype (cache.py:754-784,
        # attention.py:307-350); the fused kernels keep them in float32,
        # which for bf16 (8 significant bits) moves outputs by ~2^-9 of
        # their scale, so bf16 caches keep the reference's two passes
        return None
    if isinstance(cache, HybridSunShapeKVCache) and tq > 1 and ops.get("k_heavy") is None and \
            cache.dtype == torch.float16 and \
            q.dtype in (torch.float16, torch.bfloat16) and \
            _hip.prefill_supported(hq, cache.n_kv_heads, tq, d, codec.n_blocks):
        pf = cache.prefill_operands()
        if pf is not None:
            vil8, rows, fac, t_raw0 = pf
            try:
                out = _hip.prefill_attn_il8_hybrid(q, kscale, perm, codec.kernel_codebook(),
                                                   codec.n_centroids, ops["idx"], vil8,
                                                   t_raw0 + buffered, rows, fac, t_raw0,
                                                   causal=causal, q_offset=q_offset,
                                                   out_dtype=out_dtype)
            except _hip.SunShapeUnsupported:
                out = None
            if out is not None:
                codec.last_score_backend = "hip_prefill_mfma_hybrid"
                return out
    # the buffer joins the fused softmax on every fused kernel
    if buffered and codec.mode not in PERM_MODES and codec.use_rotation:
        # the kernels score buffered keys against the query they are given,
        # here the rotated one: (q R^T) . (k R^T) = q . k for orthogonal R,
        # so the buffer's keys go in rotated (float32, with float32 values
        # to share their layout)
        nb_ = buffered
        ops = dict(ops, buf_keys=(ops["buf_keys"][:, :, :nb_].float()
                                  @ codec.rotation.t()).contiguous(),
                   buf_values=ops["buf_values"][:, :, :nb_].float().contiguous())
    t_kv = cache.compressed_offset if isinstance(cache, HybridSunShapeKVCache) else cache.offset
    kind = ops["kind"]
    # a prompt (many query rows per head) against an fp16 cache: keys
    # reconstructed from the codebook, both products on the matrix cores
    b_, hq, tq, d = queries.shape
    hv = {"k_heavy": ops.get("k_heavy"), "heavy_dims": ops.get("heavy_dims")}
    if not buffered and kind == "il8" and tq > 1 and hv["k_heavy"] is None and \
            _hip.prefill_supported(hq, cache.n_kv_heads, tq, d, codec.n_blocks):
        try:
            out = _hip.prefill_attn_il8(q, kscale, perm, codec.kernel_codebook(), codec.n_centroids,
                                        ops["idx"], ops["values"], t_kv, causal=causal,
                                        q_offset=q_offset, out_dtype=out_dtype)
        except _hip.SunShapeUnsupported:
            return None
        codec.last_score_backend = "hip_prefill_mfma"
        return out
    # the matrix-core decodes without a token buffer: one prepared launch
    # (argument checks, codebook and split plan done once per cache layout)
    if not buffered and kind in ("il8", "grouped_il") and hv["k_heavy"] is None:
        try:
            plan = _prepared_decode(cache, ops, codec, q, kscale, perm)
            out = plan(q, t_kv, causal, q_offset, out_dtype=out_dtype)
        except _hip.SunShapeUnsupported:
            return None
        codec.last_score_backend = "hip_fused_mfma" if kind == "il8" else "hip_fused_mfma_dequant"
        return out
    # the same with a hybrid cache's buffered tokens (the buffer window
    # passed per call); rotated codecs hand the kernel rotated buffer copies
    # and take the checked launch below
    if buffered and kind in ("il8", "grouped_il") and hv["k_heavy"] is None and \
            (codec.mode in PERM_MODES or not codec.use_rotation):
        try:
            plan = _prepared_decode(cache, ops, codec, q, kscale, perm, buffered=True)
            out = plan(q, t_kv, ops["buf_keys"], ops["buf_values"], buffered, causal, q_offset,
                       out_dtype=out_dtype)
        except _hip.SunShapeUnsupported:
            return None
        codec.last_score_backend = ("hip_fused_mfma_buffer" if kind == "il8"
                                    else "hip_fused_mfma_dequant_buffer")
        return out
    kw = dict(t_kv=t_kv, causal=causal, q_offset=q_offset, out_dtype=out_dtype)
    try:
        if kind == "il8":
            out = _hip.decode_attn_il8(q, kscale, perm, codec.scoring_centroids(), ops["idx"],
                                       ops["values"], codebook=codec.kernel_codebook(),
                                       buf_keys=ops["buf_keys"], buf_values=ops["buf_values"],
                                       buf_len=buffered, **hv, **kw)
            codec.last_score_backend = ("hip_fused_mfma_buffer" if buffered
                                        else "hip_fused_mfma_heavy")
        elif kind == "grouped_il":
            out = _hip.decode_attn_grouped_il(q, kscale, perm, codec.scoring_centroids(),
                                              ops["idx"], ops["codes_il"], ops["scales"],
                                              ops["zeros"], ops["bits"], ops["group_size"],
                                              codebook=codec.kernel_codebook(),
                                              buf_keys=ops["buf_keys"], buf_values=ops["buf_values"],
                                              buf_len=buffered, **hv, **kw)
            codec.last_score_backend = ("hip_fused_mfma_dequant_buffer" if buffered
                                        else "hip_fused_mfma_dequant")
        elif kind == "turboquant_il":
            out = _hip.decode_attn_turboquant_il(q, kscale, perm, codec.scoring_centroids(),
                                                 ops["idx"], ops["codes_il"], ops["norms"],
                                                 ops["levels"], ops["rotation"],
                                                 codebook=codec.kernel_codebook(),
                                                 buf_keys=ops["buf_keys"],
                                                 buf_values=ops["buf_values"], buf_len=buffered,
                                                 **hv, **kw)
            codec.last_score_backend = ("hip_fused_mfma_turboquant_buffer" if buffered
                                        else "hip_fused_mfma_turboquant")
        elif ops["kind"] == "turboquant":
            out = _hip.decode_attn_turboquant(q, kscale, perm, codec.centroids, ops["idx"],
                                              ops["packed"], ops["norms"], ops["levels"],
                                              ops["rotation"], ops["bits"],
                                              buf_keys=ops["buf_keys"], buf_values=ops["buf_values"],
                                              buf_len=buffered, **hv, **kw)
            codec.last_score_backend = ("hip_fused_turboquant_buffer" if buffered
                                        else "hip_fused_turboquant")
        elif ops["kind"] == "sunshape_v":
            out = _hip.decode_attn_sunshape_v(q, kscale, perm, codec.scoring_centroids(), ops["idx"],
                                              ops["v_idx"], ops["v_centroids"], ops["v_transform"],
                                              buf_keys=ops["buf_keys"], buf_values=ops["buf_values"],
                                              buf_len=buffered, **hv, **kw)
            codec.last_score_backend = ("hip_fused_sunshape_v_buffer" if buffered
                                        else "hip_fused_sunshape_v")
        elif ops["kind"] == "grouped":
            out = _hip.decode_attn_grouped(q, kscale, perm, codec.centroids, ops["idx"],
                                           ops["packed"], ops["scales"], ops["zeros"],
                                           ops["bits"], ops["group_size"],
                                           buf_keys=ops.get("buf_keys"),
                                           buf_values=ops.get("buf_values"), buf_len=buffered,
                                           **kw)
            codec.last_score_backend = "hip_fused_dequant_buffer" if buffered else "hip_fused_dequant"
        else:
            out = _hip.decode_attn_dense(q, kscale, perm, codec.centroids, ops["idx"],
                                         ops["values"], buf_keys=ops.get("buf_keys"),
                                         buf_values=ops.get("buf_values"), buf_len=buffered, **kw)
            codec.last_score_backend = "hip_fused_buffer" if buffered else "hip_fused"
    except _hip.SunShapeUnsupported:
        return None
    return out


def _compressed_scores(codec: SunShapeBlockCodec, q_t: torch.Tensor,
                       key_indices: torch.Tensor) -> torch.Tensor:
    """(B, Hkv, rep, Tq, Tc) float32 scores of codec-space queries q_t
    (B, Hkv, rep, Tq, D) against (B, Hkv, Tc, NB) indices
    (attention.py:44-73): one HIP LUT build for all rows and one gather
    launch over every (batch, KV head).  Fp16 heavy blocks add nothing here (their exact dot
    products are added by the caller)."""
    b_, hkv, rep, tq, d = q_t.shape
    rows = q_t.reshape(-1, d)
    if rows.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        rows = rows.float()
    lut = _hip.build_lut(rows.contiguous(), None, 1.0, codec.scoring_centroids())
    lut = lut.reshape(b_, hkv, rep * tq, codec.n_blocks, codec.n_centroids)
    tc = key_indices.shape[2]
    scores = _hip.score_gather_heads(lut, key_indices)  # every (batch, KV head) in one launch
    codec.last_score_backend = "hip"
    return scores.reshape(b_, hkv, rep, tq, tc)


def _two_pass(cache, queries: torch.Tensor, scale: float, mask,
              out_dtype: torch.dtype) -> torch.Tensor:
    """Scores (compressed, then buffered keys in the original basis), mask,
    float32 softmax, ``@ values`` (attention.py:307-350)."""
    b_, hq, tq, d = queries.shape
    hkv = cache.n_kv_heads
    rep = hq // hkv
    t_kv = cache.offset
    codec = cache.codec
    is_hybrid = isinstance(cache, HybridSunShapeKVCache)
    q_scaled = queries * scale
    q_grouped = q_scaled.reshape(b_, hkv, rep, tq, d)
    parts = []
    tc = cache.compressed_offset if is_hybrid else t_kv
    if tc > 0:
        q_t = _transform_grouped(codec, q_grouped)
        sc = _compressed_scores(codec, q_t, cache.key_indices)
        hd = getattr(cache, "_heavy_dims", None)
        if hd is not None:  # fp16 heavy blocks scored exactly (codec basis)
            kh = cache._key_heavy[:, :, :tc].float().transpose(-1, -2).contiguous()
            sc = sc + torch.matmul(q_t[..., hd.long()].float(), kh.unsqueeze(2))
        parts.append(sc)
    if is_hybrid and cache.buffer_offset > 0:
        kb_t = cache.buffer_keys.float().transpose(-1, -2).contiguous()  # (B, Hkv, D, Tb)
        parts.append(torch.matmul(q_grouped.float(), kb_t.unsqueeze(2)))
    scores = parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)
    scores = scores.reshape(b_, hq, tq, t_kv)
    if isinstance(mask, str):
        if mask == "causal":
            off = t_kv - tq
            q_pos = torch.arange(off, off + tq, device=queries.device)
            k_pos = torch.arange(t_kv, device=queries.device)
            keep = q_pos[:, None] >= k_pos[None, :]
            scores = torch.where(keep, scores, torch.finfo(torch.float32).min)
    elif mask is not None:
        mask = mask.to(queries.device)
        if mask.dtype == torch.bool:
            scores = torch.where(mask, scores, torch.finfo(torch.float32).min)
        else:
            scores = scores + mask.float()
    weights = torch.softmax(scores.float(), dim=-1)
    values = cache.values.float()  # (B, Hkv, T_kv, D)
    out = torch.matmul(weights.reshape(b_, hkv, rep * tq, t_kv), values)
    return out.reshape(b_, hq, tq, d).to(out_dtype)


def sunshape_sdpa(queries: torch.Tensor, cache: SunShapeKVCache | HybridSunShapeKVCache,
                  scale: float, mask: torch.Tensor | str | None = None, *,
                  out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Attention of ``queries`` (B, n_q_heads, T_q, D) against a SunShape cache
    (reference attention.py:166-353).  Query head ``h*rep + r`` reads KV head
    h; ``mask`` is None, ``"causal"`` (query i sees keys ``t <= T_kv - T_q + i``)
    or an additive / boolean array broadcastable to (B, n_q_heads, T_q, T_kv).
    Returns (B, n_q_heads, T_q, D) in the query dtype, as the reference does
    (attention.py:292, 304), or in ``out_dtype`` when given (an extension:
    float32 keeps the kernels' fp32 accumulation in the result)."""
    b_, hq, tq, d = queries.shape
    hkv = cache.n_kv_heads
    if hq % hkv != 0:
        raise ValueError(f"n_q_heads ({hq}) must be a multiple of the cache's n_kv_heads ({hkv})")
    if d != cache.head_dim:
        raise ValueError(f"query head_dim {d} != cache head_dim {cache.head_dim}")
    out_dtype = out_dtype or queries.dtype
    t_kv = cache.offset
    if t_kv == 0:
        return torch.zeros_like(queries, dtype=out_dtype)
    _hip.require_gpu(queries)
    is_hybrid = isinstance(cache, HybridSunShapeKVCache)
    use_causal = isinstance(mask, str) and mask == "causal"
    compressed = cache.compressed_offset if is_hybrid else t_kv
    # a non-empty hybrid buffer stays on the fused path where the kernel
    # takes it (_fused returns None otherwise)
    can_fuse = (mask is None or use_causal) and compressed > 0
    if can_fuse:
        out = _fused(cache, queries, scale, use_causal, t_kv - tq if use_causal else 0,
                     out_dtype)
        if out is not None:
            return out
    return _two_pass(cache, queries, scale, mask, out_dtype)
