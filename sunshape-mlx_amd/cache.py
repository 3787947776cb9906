"""SunShape KV caches on device memory (reference cache.py:1-1108).

``SunShapeKVCache``: keys as uint8 block-VQ indices (B, H, cap, n_blocks),
values in fp16.  For head_dim 64/128 the values are kept 8-token interleaved,
(B, H, cap/8, D, 8): element (t, d) at [t // 8][d][t % 8], the operand layout
of the MFMA decode kernel; ``values`` returns the token-major view the
reference returns.  ``HybridSunShapeKVCache``: a full-precision
recent-token buffer plus compressed storage whose value backend is fp16,
grouped 2/3/4-bit, TurboQuant or SunShape block-VQ.

Layout and growth follow the reference: capacity is a multiple of 256 tokens
and grows as needed, the first ``offset`` tokens of each (batch, head) row are
valid.  Everything stays on the GPU: appends are one encode launch for every
(batch, head) straight into the cache rows (the reference round-trips
through host NumPy arrays), and ``max_tokens`` preallocates the whole
capacity up front so a long decode never regrows.
"""

from __future__ import annotations

import torch

from . import _hip
from .codec import PERM_MODES, SunShapeBlockCodec
from .value_codecs import (GroupedValueCodec, TurboQuantValueCodec, _packed_dim,
                           build_value_codec)

_STEP = 256
_DEFAULT_BUFFER_SIZE = 128


def _round_capacity(n: int) -> int:
    return ((n + _STEP - 1) // _STEP) * _STEP


class DeferredTensor(torch.Tensor):
    """A tensor ``update_and_fetch`` returns but builds only if something
    reads it.  The reference returns the whole cache dequantised on every
    call (cache.py:156-205, 656-710), O(T) work per decode step that the
    patched SDPA never reads.  Shape, dtype and device are known at once;
    any torch operation on the tensor (indexing, arithmetic, ``.cpu()``,
    passing it to a torch function) builds it once, from the cache as it
    stood when ``update_and_fetch`` returned, and runs on the result.  The
    cache must not change in between: building it after a later append,
    trim or flush raises."""

    @staticmethod
    def __new__(cls, build, shape, dtype, device, cache):
        t = torch.Tensor._make_wrapper_subclass(cls, shape, dtype=dtype, device=device)
        t._build = build
        t._cache = cache
        t._stamp = cache._version
        t._value = None
        return t

    def materialize(self) -> torch.Tensor:
        """The tensor itself (built on first use)."""
        if self._value is None:
            if self._cache._version != self._stamp:
                raise RuntimeError(
                    "the cache has changed since update_and_fetch returned this tensor; use it "
                    "before the next append, trim or flush, or build the cache with "
                    "lazy_fetch=False")
            self._value = self._build()
        return self._value

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        def real(x):
            return x.materialize() if isinstance(x, DeferredTensor) else x
        args = torch.utils._pytree.tree_map(real, args)
        kwargs = torch.utils._pytree.tree_map(real, kwargs or {})
        return func(*args, **kwargs)

    def __repr__(self) -> str:
        return f"DeferredTensor({self.materialize()!r})"


def _fetched(cache, build, b_: int, last: int, dtype):
    """What ``update_and_fetch`` returns for one of keys / values (batch
    ``b_``): the built tensor with ``lazy_fetch`` off (the reference's
    behaviour), else a ``DeferredTensor`` over ``build``."""
    if not cache.lazy_fetch:
        return build()
    return DeferredTensor(build, (b_, cache.n_kv_heads, cache.offset, last), dtype,
                          cache.codec.device, cache)


def _grow(buf: torch.Tensor | None, shape, dtype, device, keep: int) -> torch.Tensor:
    """New zeroed buffer of ``shape`` holding the first ``keep`` tokens of ``buf``."""
    new = torch.zeros(shape, dtype=dtype, device=device)
    if buf is not None and keep > 0:
        new[:, :, :keep] = buf[:, :, :keep]
    return new


def _encode_into(codec: SunShapeBlockCodec, keys: torch.Tensor, out: torch.Tensor) -> None:
    """Encode (B, H, T, D) keys into the (B, H, T, n_blocks) uint8 view ``out``."""
    if codec.mode == "profileperm_baseline" and codec.n_centroids <= 256:
        k = keys if keys.stride(-1) == 1 else keys.contiguous()
        _hip.encode_blockvq(k, codec.permutation, codec.centroids, out, codec.block_dim,
                            prepared=codec.encode_codebook())
        return
    b_, h_, t_, d = keys.shape
    q = codec.quantize(keys.reshape(-1, d))
    out.copy_(q.indices.reshape(b_, h_, t_, -1).to(out.dtype))


def _dequantize_keys(codec: SunShapeBlockCodec, idx: torch.Tensor) -> torch.Tensor:
    """(B, H, T, NB) indices -> (B, H, T, D) float32 keys in the original basis
    (reference cache.py:211-240)."""
    b_, h_, t_, nb = idx.shape
    flat = idx.reshape(-1, nb).contiguous()
    inv = codec.inv_permutation if codec.mode in PERM_MODES else None
    k = _hip.dequantize_blockvq(flat, codec.centroids, inv)
    if codec.use_rotation:
        k = k @ codec.rotation
    return k.reshape(b_, h_, t_, codec.head_dim)


def _il8_ok(codec: SunShapeBlockCodec, head_dim: int, dtype: torch.dtype) -> bool:
    """Whether values go 8-token interleaved (the MFMA decode kernel's layout)."""
    return (dtype == torch.float16 and head_dim in (64, 128) and codec.block_dim == 8
            and codec.n_blocks * 8 == head_dim and codec.n_centroids <= 256)


def _grouped_il_ok(codec: SunShapeBlockCodec, head_dim: int, bits: int, group_size: int) -> bool:
    """Whether grouped value codes go token-interleaved (the layout of the
    matrix-core grouped decode kernel)."""
    return (bits in (2, 4) and head_dim in (64, 128) and group_size in (head_dim, head_dim // 2)
            and codec.block_dim == 8 and codec.n_blocks * 8 == head_dim
            and codec.n_centroids <= 256)


class SunShapeKVCache:
    """Block-VQ keys + fp16 values; drop-in for mlx-lm's KVCache protocol
    (reference cache.py:59-336)."""

    def __init__(self, codec: SunShapeBlockCodec, *, n_kv_heads: int = 1,
                 head_dim: int | None = None, dtype: torch.dtype = torch.float16,
                 max_tokens: int | None = None, return_dequantized_keys: bool = True,
                 lazy_fetch: bool = True):
        self.codec = codec
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim or codec.head_dim
        self.block_dim = codec.block_dim
        self.n_blocks = codec.n_blocks
        self.n_centroids = codec.n_centroids
        self.dtype = dtype
        self.offset = 0
        self.max_tokens = max_tokens
        # The reference returns dequantised keys from update_and_fetch (an
        # O(T) reconstruction per call that the patched SDPA never reads);
        # serving loops can switch it off.  With lazy_fetch (the default)
        # both returned tensors are DeferredTensors, built only if read.
        self.return_dequantized_keys = return_dequantized_keys
        self.lazy_fetch = lazy_fetch
        # With lazy_fetch, a decode step's few new fp16 tokens are held back
        # (their tensors, not copies) and stored by the next attention call
        # in its own launch (encode, attend, store); anything that reads the
        # storage first stores them.  Tensors passed to update_and_fetch
        # must then not be modified in place before that (checked: raises).
        self.fuse_steps = True
        self._pending = None  # (keys, values, their _version counters, position)
        self._version = 0  # bumped by every change of the stored tokens
        self._append_plan = None
        self._key_indices: torch.Tensor | None = None  # (B, H, cap, NB) uint8
        # (B, H, cap/8, D, 8) fp16 when interleaved, else (B, H, cap, D) dtype
        self._values: torch.Tensor | None = None
        self.values_interleaved = _il8_ok(codec, self.head_dim, dtype)
        self._capacity = 0

    # -------------------------------------------------------------- storage
    def _ensure_capacity(self, b_: int, new_tokens: int, device) -> None:
        needed = self.offset + new_tokens
        if needed <= self._capacity and self._key_indices is not None:
            return
        cap = _round_capacity(max(needed, self.max_tokens or 0))
        self._key_indices = _grow(self._key_indices, (b_, self.n_kv_heads, cap, self.n_blocks),
                                  torch.uint8, device, self.offset)
        if self.values_interleaved:
            # whole 8-token groups move; the tail of the last one is zero
            self._values = _grow(self._values, (b_, self.n_kv_heads, cap // 8, self.head_dim, 8),
                                 torch.float16, device, (self.offset + 7) // 8)
        else:
            self._values = _grow(self._values, (b_, self.n_kv_heads, cap, self.head_dim),
                                 self.dtype, device, self.offset)
        self._capacity = cap

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Encode new keys into the index cache, append values (reference
        cache.py:156-205).  Returns ``(keys, values)`` as stored: dequantised
        keys (float32) unless ``return_dequantized_keys`` is off (then None)."""
        b_, h_, t_, d = keys.shape
        assert h_ == self.n_kv_heads, f"Expected {self.n_kv_heads} kv heads, got {h_}"
        assert d == self.head_dim, f"Expected head_dim {self.head_dim}, got {d}"
        _hip.require_gpu(keys, values)
        self.flush()
        self._ensure_capacity(b_, t_, keys.device)
        plan = self._append_kv_plan()
        if plan is not None:  # encode + value store, one launch per decode step
            k = keys if keys.stride(-1) == 1 else keys.contiguous()
            v = values if values.stride(-1) == 1 else values.contiguous()
            if self.fuse_steps and self.lazy_fetch and self.offset > 0 and \
                    1 <= t_ <= _hip.MAX_STEP_TOKENS and k.dtype == torch.float16 and \
                    v.dtype == torch.float16 and k.stride()[:3] == v.stride()[:3] and \
                    tuple(v.shape) == tuple(k.shape):
                # held for the next attention call's fused step
                self._pending = (k, v, k._version, v._version, self.offset)
            else:
                plan(k, v, self.offset)
        else:
            sl = slice(self.offset, self.offset + t_)
            _encode_into(self.codec, keys, self._key_indices[:, :, sl])
            if self.values_interleaved:
                v = values if values.stride(-1) == 1 else values.contiguous()
                _hip.append_values_il8(v, self._values, self.offset)
            else:
                self._values[:, :, sl] = values.to(self.dtype)
        self.offset += t_
        self._version += 1
        keys_out = (_fetched(self, lambda: self.keys, b_, self.head_dim, torch.float32)
                    if self.return_dequantized_keys else None)
        return keys_out, _fetched(self, lambda: self.values, b_, self.head_dim, self.dtype)

    def _take_pending(self):
        """The held step's (keys, values, position), cleared; raises if a
        tensor was modified in place since update_and_fetch received it."""
        k, v, kv_, vv_, pos = self._pending
        self._pending = None
        if k._version != kv_ or v._version != vv_:
            raise RuntimeError("keys/values passed to update_and_fetch were modified in place "
                               "before the cache stored them; pass fresh tensors, or set "
                               "cache.fuse_steps = False")
        return k, v, pos

    def flush(self) -> None:
        """Store a held decode step's tokens now (one append launch)."""
        if self._pending is None:
            return
        k, v, pos = self._take_pending()
        self._append_kv_plan()(k, v, pos)

    def _append_kv_plan(self):
        """The prepared ``ss_append_kv_il8`` for the current buffers and
        codebook (None where that path does not apply: non-interleaved
        values, or codecs whose keys the HIP encoder does not take)."""
        c = self.codec
        if not self.values_interleaved or c.mode != "profileperm_baseline" or c.n_centroids > 256:
            return None
        cb, pm, pre = c.centroids, c.permutation, c.encode_codebook()
        key = (self._key_indices, self._values, cb, cb._version, pm,
               pm._version if pm is not None else 0, pre)
        held = self._append_plan
        if held is None or len(held[0]) != len(key) or \
                not all(a is b or (isinstance(a, int) and a == b) for a, b in zip(held[0], key)):
            held = (key, _hip.PreparedAppend(pm, cb, pre, self._key_indices, self._values))
            self._append_plan = held
        return held[1]

    # ----------------------------------------------------------- accessors
    @property
    def keys(self) -> torch.Tensor:
        """Dequantised keys up to ``offset`` (float32)."""
        self.flush()
        if self._key_indices is None or self.offset == 0:
            dev = self.codec.device
            return torch.zeros((1, self.n_kv_heads, 0, self.head_dim), dtype=torch.float32,
                               device=dev)
        return _dequantize_keys(self.codec, self._key_indices[:, :, :self.offset])

    @property
    def values(self) -> torch.Tensor:
        """Values up to ``offset``, token-major (B, H, T, D) (a copy when the
        storage is interleaved)."""
        self.flush()
        if self._values is None or self.offset == 0:
            return torch.zeros((1, self.n_kv_heads, 0, self.head_dim), dtype=self.dtype,
                               device=self.codec.device)
        if self.values_interleaved:
            return _hip.il8_to_dense(self._values, self.offset)
        return self._values[:, :, :self.offset]

    def fused_operands(self) -> dict | None:
        """Full-capacity device buffers for the fused decode kernels:
        {"kind": "il8"|"dense", "idx", "values"}; None when empty."""
        self.flush()
        if self._key_indices is None or self.offset == 0:
            return None
        return {"kind": "il8" if self.values_interleaved else "dense",
                "idx": self._key_indices, "values": self._values}

    @property
    def key_indices(self) -> torch.Tensor:
        self.flush()
        if self._key_indices is None or self.offset == 0:
            return torch.zeros((1, self.n_kv_heads, 0, self.n_blocks), dtype=torch.uint8,
                               device=self.codec.device)
        return self._key_indices[:, :, :self.offset]

    @property
    def state(self):
        self.flush()
        z = torch.zeros((1,))
        return (self._key_indices[:, :, :self.offset] if self._key_indices is not None else z,
                self.values if self._values is not None else z)

    # -------------------------------------------------------------- metrics
    @property
    def nbytes(self) -> int:
        if self._key_indices is None:
            return 0
        b_, t_ = self._key_indices.shape[0], self.offset
        idx_bytes = b_ * self.n_kv_heads * t_ * self.n_blocks * (1 if self.n_centroids <= 256 else 2)
        return idx_bytes + b_ * self.n_kv_heads * t_ * self.head_dim * 2

    @property
    def nbytes_equivalent_fp16(self) -> int:
        if self.offset == 0:
            return 0
        b_ = self._key_indices.shape[0] if self._key_indices is not None else 1
        return 2 * b_ * self.n_kv_heads * self.offset * self.head_dim * 2

    @property
    def compression_ratio(self) -> float:
        fp16 = self.nbytes_equivalent_fp16
        return 1.0 if fp16 == 0 else fp16 / max(1, self.nbytes)

    # ---------------------------------------------------- mlx-lm protocol
    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> None:
        self.flush()
        self.offset = max(0, self.offset - n)
        self._version += 1

    def empty(self) -> bool:
        return self.offset == 0

    def make_mask(self, N: int, return_array: bool = False, window_size: int | None = None,
                  **kwargs):
        return _make_mask(self.offset, N, return_array, self.codec.device)

    def __repr__(self) -> str:
        return (f"SunShapeKVCache(offset={self.offset}, head_dim={self.head_dim}, "
                f"n_blocks={self.n_blocks}, n_centroids={self.n_centroids}, "
                f"compression={self.compression_ratio:.1f}x)")


def _make_mask(t_: int, n: int, return_array: bool, device):
    """Causal mask for N new queries at positions [T, T+N) over keys [0, T+N)
    (reference cache.py:310-329)."""
    if t_ == 0 and n == 0:
        return "none"
    if not return_array:
        return "causal"
    q_pos = torch.arange(t_, t_ + n, device=device)
    k_pos = torch.arange(t_ + n, device=device)
    causal = q_pos[:, None] >= k_pos[None, :]
    return torch.where(causal, torch.tensor(0.0, device=device),
                       torch.tensor(torch.finfo(torch.float16).min, device=device)).to(torch.float16)


class HybridSunShapeKVCache:
    """Recent tokens in a full-precision buffer, older tokens compressed
    (reference cache.py:348-998).  ``value_scale_dtype`` selects how grouped
    scale/zero pairs are stored (float32 as the reference, or float16)."""

    def __init__(self, codec: SunShapeBlockCodec, *, n_kv_heads: int = 1,
                 head_dim: int | None = None, dtype: torch.dtype = torch.float16,
                 buffer_size: int = _DEFAULT_BUFFER_SIZE, value_backend: str | None = None,
                 value_bits: int | None = None, value_group_size: int = 64, value_seed: int = 43,
                 value_codec: SunShapeBlockCodec | None = None, prefer_metal_kernels: bool = True,
                 value_scale_dtype: torch.dtype = torch.float32, max_tokens: int | None = None,
                 lazy_fetch: bool = True):
        self.codec = codec
        # update_and_fetch returns DeferredTensors (built only if read)
        # unless lazy_fetch is off (the reference's eager O(T) return)
        self.lazy_fetch = lazy_fetch
        self._version = 0  # bumped by every change of the stored tokens
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim or codec.head_dim
        self.block_dim = codec.block_dim
        self.n_blocks = codec.n_blocks
        self.n_centroids = codec.n_centroids
        self.dtype = dtype
        self.buffer_size = buffer_size
        self.value_backend = value_backend or ("fp16" if value_bits is None else "grouped")
        self.value_bits = value_bits
        self.value_group_size = value_group_size
        self.value_seed = value_seed
        self.prefer_metal_kernels = prefer_metal_kernels
        self.value_codec = value_codec
        self.value_scale_dtype = value_scale_dtype
        self.max_tokens = max_tokens
        self.last_value_quant_backend = "none"
        if self.value_backend not in {"fp16", "grouped", "turboquant", "sunshape"}:
            raise ValueError(f"Unsupported value backend: {self.value_backend}")
        if self.value_backend != "fp16" and self.value_bits is None:
            raise ValueError(f"value_bits is required for value backend {self.value_backend}")
        if self.value_backend == "grouped" and self.head_dim % self.value_group_size != 0:
            raise ValueError(f"head_dim ({self.head_dim}) must be divisible by "
                             f"value_group_size ({self.value_group_size}) for value quantization")
        if value_scale_dtype not in (torch.float32, torch.float16):
            raise ValueError("value_scale_dtype must be float32 or float16")
        if self.value_backend == "sunshape":
            self.value_codec = self.value_codec or codec
            if self.value_codec.head_dim != self.head_dim:
                raise ValueError("SunShape value codec head_dim must match cache head_dim")
            self.value_n_blocks = self.value_codec.n_blocks
            self.value_n_centroids = self.value_codec.n_centroids
        else:
            self.value_n_blocks = 0
            self.value_n_centroids = 0
        self._value_codec_impl = None if self.value_backend == "sunshape" else build_value_codec(
            self.value_backend, head_dim=self.head_dim, value_bits=self.value_bits or 0,
            value_group_size=self.value_group_size, value_seed=self.value_seed,
            prefer_metal=self.prefer_metal_kernels)
        self._compressed_offset = 0
        self._buffer_offset = 0
        # the buffered tokens are the window [_buf_start, _buf_start +
        # _buffer_offset) of the buffer stores: a flush advances the start
        # instead of shifting the rest, and the window slides back to the
        # front only when it reaches the end of the store
        self._buf_start = 0
        self._key_buffer: torch.Tensor | None = None
        self._value_buffer: torch.Tensor | None = None
        self._step_plan = None
        # With lazy_fetch, a decode step of a grouped-value cache (a
        # few fp16 tokens) is held back (its tensors, not copies) and done by
        # the next attention call in its own launch (ss_decode_step_grouped_il_hybrid:
        # flush, store and attention); anything that reads the storage first
        # does it with flush().  The counters already include the step.
        self.fuse_steps = True
        self._pending = None  # (keys, values, _version counters, t_c, buf start, n_buf, n_flush)
        self._key_indices: torch.Tensor | None = None
        self._values_packed: torch.Tensor | None = None
        self._value_scales: torch.Tensor | None = None
        self._value_zeros: torch.Tensor | None = None
        self._value_norms: torch.Tensor | None = None
        self._value_indices: torch.Tensor | None = None
        self._values_fp16: torch.Tensor | None = None
        # fp16 values of compressed tokens kept 8-token interleaved ((B, H,
        # cap/8, D, 8), the matrix-core decode's layout) where the codec
        # allows it, else token-major in _values_fp16
        self._values_il8: torch.Tensor | None = None
        self._fp16_il8 = self.value_backend == "fp16" and _il8_ok(codec, self.head_dim, dtype)
        self._value_n_groups = 0
        self._compressed_capacity = 0
        # grouped codes held token-interleaved ((B, H, cap*bits/32, D) words)
        # for the matrix-core decode kernel; packed rows otherwise
        self._values_il: torch.Tensor | None = None
        # mixed-precision codecs with fp16 heavy blocks: those key dims
        # (codec basis) per token, (B, H, cap, n_heavy_dims) fp16
        self._key_heavy: torch.Tensor | None = None
        hd = codec.heavy_dims()
        self._heavy_dims = hd
        self._grouped_il = (self.value_backend == "grouped" and
                            _grouped_il_ok(codec, self.head_dim, self.value_bits or 0,
                                           self.value_group_size))
        # 2-bit TurboQuant codes held token-interleaved as well (the layout of
        # the matrix-core TurboQuant decode, whose level table must be affine
        # in the code bits)
        self._turbo_il = (self.value_backend == "turboquant" and self.value_bits == 2 and
                          _grouped_il_ok(codec, self.head_dim, 2, self.head_dim) and
                          _hip.turboquant_il_levels_ok(self._value_codec_impl.levels_host()))

    @property
    def offset(self) -> int:
        return self._compressed_offset + self._buffer_offset

    # ------------------------------------------------------------ storage
    def _grow_compressed(self, b_: int, needed: int, device) -> None:
        if needed <= self._compressed_capacity and self._key_indices is not None:
            return
        cap = _round_capacity(max(needed, self.max_tokens or 0))
        keep = self._compressed_offset
        h_ = self.n_kv_heads
        if self._heavy_dims is not None:
            self._key_heavy = _grow(self._key_heavy, (b_, h_, cap, self._heavy_dims.numel()),
                                    torch.float16, device, keep)
        self._key_indices = _grow(self._key_indices, (b_, h_, cap, self.n_blocks), torch.uint8,
                                  device, keep)
        if self.value_backend == "grouped":
            gc = self._value_codec_impl
            self._value_n_groups = gc.n_groups
            if self._grouped_il:
                tpw = 32 // gc.bits
                self._values_il = _grow(self._values_il, (b_, h_, cap // tpw, self.head_dim),
                                        torch.int32, device, (keep + tpw - 1) // tpw)
            else:
                self._values_packed = _grow(self._values_packed, (b_, h_, cap, gc.packed_dim),
                                            torch.int32, device, keep)
            self._value_scales = _grow(self._value_scales, (b_, h_, cap, gc.n_groups),
                                       self.value_scale_dtype, device, keep)
            self._value_zeros = _grow(self._value_zeros, (b_, h_, cap, gc.n_groups),
                                      self.value_scale_dtype, device, keep)
        elif self.value_backend == "turboquant":
            tc = self._value_codec_impl
            if self._turbo_il:
                self._values_il = _grow(self._values_il, (b_, h_, cap // 16, self.head_dim),
                                        torch.int32, device, (keep + 15) // 16)
            else:
                self._values_packed = _grow(self._values_packed, (b_, h_, cap, tc.packed_dim),
                                            torch.int32, device, keep)
            norms = self._value_norms
            self._value_norms = torch.zeros((b_, h_, cap), dtype=torch.float32, device=device)
            if norms is not None and keep:
                self._value_norms[:, :, :keep] = norms[:, :, :keep]
        elif self.value_backend == "sunshape":
            self._value_indices = _grow(self._value_indices, (b_, h_, cap, self.value_n_blocks),
                                        torch.uint8, device, keep)
        elif self._fp16_il8:
            # whole 8-token groups move; the tail of the last one is zero
            self._values_il8 = _grow(self._values_il8, (b_, h_, cap // 8, self.head_dim, 8),
                                     torch.float16, device, (keep + 7) // 8)
        else:
            self._values_fp16 = _grow(self._values_fp16, (b_, h_, cap, self.head_dim),
                                      self.dtype, device, keep)
        self._compressed_capacity = cap

    def _flush_buffer(self, b_: int, n_to_flush: int) -> None:
        """Move the oldest tokens of the buffer into compressed storage
        (reference cache.py:463-650)."""
        if n_to_flush <= 0 or self._key_buffer is None:
            return
        n = min(n_to_flush, self._buffer_offset)
        if n == 0:
            return
        dev = self._key_buffer.device
        self._grow_compressed(b_, self._compressed_offset + n, dev)
        c0, c1 = self._compressed_offset, self._compressed_offset + n
        s0 = self._buf_start
        kf = self._key_buffer[:, :, s0:s0 + n]
        vf = self._value_buffer[:, :, s0:s0 + n]
        _encode_into(self.codec, kf, self._key_indices[:, :, c0:c1])
        if self._heavy_dims is not None:
            kp = kf[..., self.codec.permutation.long()]
            self._key_heavy[:, :, c0:c1] = kp[..., self._heavy_dims.long()].to(torch.float16)
        if self.value_backend == "grouped":
            gc = self._value_codec_impl
            if self._grouped_il:
                # quantise into contiguous rows, then interleave the codes
                h_ = self.n_kv_heads
                rows = torch.empty((b_, h_, n, gc.packed_dim), dtype=torch.int32, device=dev)
                sc = torch.empty((b_, h_, n, gc.n_groups), dtype=self.value_scale_dtype, device=dev)
                zr = torch.empty_like(sc)
                _hip.quantize_values_grouped(vf, gc.bits, gc.group_size, rows, sc, zr)
                self._value_scales[:, :, c0:c1] = sc
                self._value_zeros[:, :, c0:c1] = zr
                _hip.pack_grouped_il(rows, gc.bits, self._values_il, c0)
            else:
                _hip.quantize_values_grouped(vf, gc.bits, gc.group_size,
                                             self._values_packed[:, :, c0:c1],
                                             self._value_scales[:, :, c0:c1],
                                             self._value_zeros[:, :, c0:c1])
            self.last_value_quant_backend = "hip"
        elif self.value_backend == "turboquant":
            tc = self._value_codec_impl
            packed, norms = tc.quantize(vf.float().reshape(-1, self.head_dim))
            rows = packed.view(torch.int32).reshape(b_, self.n_kv_heads, n, -1)
            if self._turbo_il:
                _hip.pack_grouped_il(rows, 2, self._values_il, c0)
            else:
                self._values_packed[:, :, c0:c1] = rows
            self._value_norms[:, :, c0:c1] = norms.reshape(b_, self.n_kv_heads, n)
            self.last_value_quant_backend = tc.last_quantize_backend
        elif self.value_backend == "sunshape":
            _encode_into(self.value_codec, vf, self._value_indices[:, :, c0:c1])
            self.last_value_quant_backend = "sunshape"
        elif self._fp16_il8:
            _hip.append_values_il8(vf, self._values_il8, c0)
            self.last_value_quant_backend = "fp16"
        else:
            self._values_fp16[:, :, c0:c1] = vf.to(self.dtype)
            self.last_value_quant_backend = "fp16"
        self._compressed_offset = c1
        self._buffer_offset -= n
        self._buf_start = s0 + n if self._buffer_offset else 0

    def _ensure_buffer(self, b_: int, t_: int, dev) -> None:
        """Room in the buffer stores for ``t_`` tokens after the window: the
        window slides to the front when it reaches the end of the store
        (at most buffer_size tokens moved once per store length of appends),
        and the store grows when the window itself would not fit."""
        h_, d = self.n_kv_heads, self.head_dim
        if self._key_buffer is None:
            size = max(2 * self.buffer_size, t_, 1)
            self._key_buffer = torch.zeros((b_, h_, size, d), dtype=self.dtype, device=dev)
            self._value_buffer = torch.zeros((b_, h_, size, d), dtype=self.dtype, device=dev)
            self._buf_start = 0
            return
        n, s0, cap = self._buffer_offset, self._buf_start, self._key_buffer.shape[2]
        if s0 + n + t_ <= cap:
            return
        if n + t_ > cap:
            size = max(n + t_, 2 * cap)
            for name in ("_key_buffer", "_value_buffer"):
                old = getattr(self, name)
                new = torch.zeros((b_, h_, size, d), dtype=self.dtype, device=dev)
                new[:, :, :n] = old[:, :, s0:s0 + n]
                setattr(self, name, new)
        elif n:
            self._key_buffer[:, :, :n] = self._key_buffer[:, :, s0:s0 + n].clone()
            self._value_buffer[:, :, :n] = self._value_buffer[:, :, s0:s0 + n].clone()
        self._buf_start = 0

    def _grouped_step_plan(self):
        """The C-ABI arguments of ss_hybrid_append_grouped_il that stay fixed
        for the current buffers and codebook (None where that fused step does
        not apply: other value backends, fp16 heavy blocks, codecs the HIP
        encoder does not take)."""
        c = self.codec
        if not self._grouped_il or self._heavy_dims is not None or \
                c.mode != "profileperm_baseline" or c.n_centroids > 256:
            return None
        cb, pm = c.centroids, c.permutation
        key = (self._key_buffer, self._value_buffer, self._key_indices, self._values_il,
               self._value_scales, self._value_zeros, cb, cb._version, pm,
               pm._version if pm is not None else 0)
        held = self._step_plan
        if held is not None and len(held[0]) == len(key) and \
                all(a is b or (isinstance(a, int) and a == b) for a, b in zip(held[0], key)):
            return held[1]
        gc = self._value_codec_impl
        for t in (self._key_buffer, self._value_buffer, self._key_indices, self._values_il,
                  self._value_scales, self._value_zeros):
            if not t.is_contiguous():
                return None
        nb, nc, bd = cb.shape
        args = {
            "buf": (self._key_buffer.data_ptr(), self._value_buffer.data_ptr(),
                    _hip.dtype_code(self.dtype), self._key_buffer.shape[2]),
            "codec": (self.head_dim, _hip.ptr(pm), cb.data_ptr(), nb, nc, bd,
                      self._key_indices.data_ptr(), gc.bits, gc.group_size,
                      self._values_il.data_ptr(), self._value_scales.data_ptr(),
                      self._value_zeros.data_ptr(), _hip.dtype_code(self.value_scale_dtype),
                      self._compressed_capacity),
            "fn": _hip.load_library().ss_hybrid_append_grouped_il,
        }
        self._step_plan = (key, args)
        return args

    def _held_step_ok(self, k: torch.Tensor, v: torch.Tensor, t_: int, n_flush: int) -> bool:
        """Whether update_and_fetch may hold this step for the fused
        attention launch: 1..4 fp16 tokens of an fp16 cache with compressed
        tokens, at most 4 of them flushed, whose values are 2- or 4-bit
        interleaved grouped codes or interleaved fp16, keys of the
        permutation codec (no fp16 heavy blocks)."""
        c = self.codec
        kind_ok = ((self._grouped_il and self.value_bits in (2, 4)) or self._fp16_il8) and \
            self._heavy_dims is None and c.mode == "profileperm_baseline" and c.n_centroids <= 256
        return (kind_ok and self.fuse_steps and self.lazy_fetch and
                self.dtype == torch.float16 and self._compressed_offset > 0 and
                1 <= t_ <= _hip.MAX_STEP_TOKENS and n_flush <= _hip.MAX_STEP_TOKENS and
                k.dtype == torch.float16 and v.dtype == torch.float16 and
                k.stride(-1) == 1 and v.stride(-1) == 1 and
                k.stride()[:3] == v.stride()[:3] and tuple(v.shape) == tuple(k.shape))

    def _run_grouped_step(self, plan, k, v, tc: int, s0: int, n: int, n_flush: int) -> None:
        """One ss_hybrid_append_grouped_il launch: the new tokens stored at
        buffer row s0 + n, the n_flush tokens from row s0 encoded and
        quantised into compressed positions tc .."""
        b_, h_, t_, _ = k.shape
        ks, vs = k.stride(), v.stride()
        rc = plan["fn"](k.data_ptr(), v.data_ptr(), _hip.dtype_code(k.dtype), b_, h_, t_,
                        ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], *plan["buf"], s0 + n,
                        s0, n_flush, *plan["codec"], tc, _hip.stream_handle(k.device))
        _hip._launched("sunshape_block_vq_quantize_hip", rc)

    def _take_pending(self):
        """The held step's (keys, values, t_c, buffer start, n_buf, n_flush)
        as it was received, cleared; raises if a tensor was modified in place
        since update_and_fetch received it."""
        k, v, kv_, vv_, tc, s0, n, nf = self._pending
        self._pending = None
        if k._version != kv_ or v._version != vv_:
            raise RuntimeError("keys/values passed to update_and_fetch were modified in place "
                               "before the cache stored them; pass fresh tensors, or set "
                               "cache.fuse_steps = False")
        return k, v, tc, s0, n, nf

    def flush(self) -> None:
        """Do a held decode step's buffer store and flush now: one
        ss_hybrid_append_grouped_il launch for grouped values; for fp16
        values the buffer store, then the flush of the oldest tokens as an
        unheld step does it."""
        if self._pending is None:
            return
        k, v, tc, s0, n, nf = self._take_pending()
        if self._grouped_il:
            self._run_grouped_step(self._grouped_step_plan(), k, v, tc, s0, n, nf)
            return
        after = (self._compressed_offset, self._buffer_offset, self._buf_start)
        t_ = k.shape[2]
        self._compressed_offset, self._buffer_offset, self._buf_start = tc, n + t_, s0
        self._key_buffer[:, :, s0 + n:s0 + n + t_] = k
        self._value_buffer[:, :, s0 + n:s0 + n + t_] = v
        self._flush_buffer(k.shape[0], nf)
        assert (self._compressed_offset, self._buffer_offset, self._buf_start) == after

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Append to the buffer; flush the overflow beyond ``buffer_size``
        (reference cache.py:656-710).  A decode step of a grouped-value cache
        (the new tokens fit beside the ones that leave) is one launch: the
        new tokens stored, the oldest buffered ones encoded and quantised
        into compressed storage.  Returns ``(keys, values)`` of every token,
        as DeferredTensors unless ``lazy_fetch`` is off."""
        b_, h_, t_, d = keys.shape
        assert h_ == self.n_kv_heads
        assert d == self.head_dim
        _hip.require_gpu(keys, values)
        self.flush()
        dev = keys.device
        self._ensure_buffer(b_, t_, dev)
        n_flush = max(0, self._buffer_offset + t_ - self.buffer_size)
        k = keys if keys.stride(-1) == 1 else keys.contiguous()
        v = values if values.stride(-1) == 1 else values.contiguous()
        hold = n_flush <= self._buffer_offset and self._held_step_ok(k, v, t_, n_flush)
        plan = None
        if self._grouped_il and 0 <= n_flush <= self._buffer_offset and t_ <= 64 and \
                (n_flush > 0 or hold):
            self._grow_compressed(b_, self._compressed_offset + n_flush, dev)
            plan = self._grouped_step_plan()
        if hold and (plan is not None or self._fp16_il8):
            # held for the next attention call's fused step (the counters
            # include it already; flush() stores it)
            self._grow_compressed(b_, self._compressed_offset + n_flush, dev)
            s0, n, tc = self._buf_start, self._buffer_offset, self._compressed_offset
            self._pending = (k, v, k._version, v._version, tc, s0, n, n_flush)
            self._compressed_offset += n_flush
            self._buffer_offset += t_ - n_flush
            self._buf_start = s0 + n_flush if self._buffer_offset else 0
            self.last_value_quant_backend = "hip" if plan is not None else "fp16"
        elif plan is not None and k.dtype == v.dtype:
            s0, n, tc = self._buf_start, self._buffer_offset, self._compressed_offset
            self._run_grouped_step(plan, k, v, tc, s0, n, n_flush)
            self._compressed_offset += n_flush
            self._buffer_offset += t_ - n_flush
            self._buf_start = s0 + n_flush if self._buffer_offset else 0
            self.last_value_quant_backend = "hip"
        else:
            sl = slice(self._buf_start + self._buffer_offset,
                       self._buf_start + self._buffer_offset + t_)
            self._key_buffer[:, :, sl] = keys.to(self.dtype)
            self._value_buffer[:, :, sl] = values.to(self.dtype)
            self._buffer_offset += t_
            if self._buffer_offset > self.buffer_size:
                self._flush_buffer(b_, self._buffer_offset - self.buffer_size)
        self._version += 1
        return (_fetched(self, lambda: self.keys, b_, self.head_dim, torch.float32),
                _fetched(self, lambda: self.values, b_, self.head_dim, self.dtype))

    # ---------------------------------------------------------- accessors
    def _zeros(self, last: int, dtype) -> torch.Tensor:
        return torch.zeros((1, self.n_kv_heads, 0, last), dtype=dtype, device=self.codec.device)

    @property
    def keys(self) -> torch.Tensor:
        self.flush()
        parts = []
        if self._compressed_offset > 0 and self._key_indices is not None:
            k = _dequantize_keys(self.codec, self._key_indices[:, :, :self._compressed_offset])
            if self._heavy_dims is not None:  # fp16 heavy dims: codec dim j is key dim perm[j]
                od = self.codec.permutation.long()[self._heavy_dims.long()]
                k[..., od] = self._key_heavy[:, :, :self._compressed_offset].float()
            parts.append(k)
        if self._buffer_offset > 0 and self._key_buffer is not None:
            parts.append(self.buffer_keys.float())
        if not parts:
            return self._zeros(self.head_dim, torch.float32)
        return torch.cat(parts, dim=2)

    def _compressed_values(self) -> torch.Tensor | None:
        tc_ = self._compressed_offset
        if tc_ == 0:
            return None
        if self.value_backend == "grouped" and self.values_packed_raw is not None:
            gc = self._value_codec_impl
            v = _hip.dequantize_values_grouped(self.values_packed_raw,
                                               self._value_scales[:, :, :tc_],
                                               self._value_zeros[:, :, :tc_], self.head_dim,
                                               gc.bits, gc.group_size)
            return v.to(self.dtype)
        if self.value_backend == "turboquant" and (self._values_packed is not None or
                                                   self._values_il is not None):
            tc = self._value_codec_impl
            if self._values_il is not None:
                p = _hip.grouped_il_to_packed(self._values_il, 2, tc_).contiguous()
            else:
                p = self._values_packed[:, :, :tc_].view(torch.uint32)
            v = tc.dequantize(p.reshape(-1, p.shape[-1]), self._value_norms[:, :, :tc_].reshape(-1))
            return v.reshape(p.shape[0], p.shape[1], tc_, self.head_dim).to(self.dtype)
        if self.value_backend == "sunshape" and self._value_indices is not None:
            return _dequantize_keys(self.value_codec,
                                    self._value_indices[:, :, :tc_]).to(self.dtype)
        if self._values_il8 is not None:
            return _hip.il8_to_dense(self._values_il8, tc_)
        if self._values_fp16 is not None:
            return self._values_fp16[:, :, :tc_]
        return None

    @property
    def values(self) -> torch.Tensor:
        self.flush()
        parts = []
        cv = self._compressed_values()
        if cv is not None:
            parts.append(cv)
        if self._buffer_offset > 0 and self._value_buffer is not None:
            parts.append(self.buffer_values)
        if not parts:
            return self._zeros(self.head_dim, self.dtype)
        return torch.cat(parts, dim=2)

    @property
    def key_indices(self) -> torch.Tensor:
        self.flush()
        if self._key_indices is None or self._compressed_offset == 0:
            return self._zeros(self.n_blocks, torch.uint8)
        return self._key_indices[:, :, :self._compressed_offset]

    @property
    def buffer_keys(self) -> torch.Tensor:
        self.flush()
        if self._key_buffer is None or self._buffer_offset == 0:
            return self._zeros(self.head_dim, self.dtype)
        s0 = self._buf_start
        return self._key_buffer[:, :, s0:s0 + self._buffer_offset]

    @property
    def buffer_values(self) -> torch.Tensor:
        self.flush()
        if self._value_buffer is None or self._buffer_offset == 0:
            return self._zeros(self.head_dim, self.dtype)
        s0 = self._buf_start
        return self._value_buffer[:, :, s0:s0 + self._buffer_offset]

    def _window(self, buf: torch.Tensor | None) -> torch.Tensor | None:
        """A buffer store from the window's first token on (the view the
        fused kernels read ``buffer_offset`` tokens of)."""
        return None if buf is None else buf[:, :, self._buf_start:]

    @property
    def compressed_offset(self) -> int:
        return self._compressed_offset

    @property
    def buffer_offset(self) -> int:
        return self._buffer_offset

    @property
    def values_packed_raw(self):
        """Grouped codes of the compressed tokens as reference packed rows
        (B, H, T, packed_dim) uint32 (converted from the interleaved words
        when the cache holds those)."""
        self.flush()
        if self.value_backend != "grouped" or self._compressed_offset == 0:
            return None
        if self._values_il is not None:
            return _hip.grouped_il_to_packed(self._values_il, self.value_bits,
                                             self._compressed_offset).contiguous()
        if self._values_packed is None:
            return None
        return self._values_packed[:, :, :self._compressed_offset].view(torch.uint32)

    @property
    def value_scales_raw(self):
        self.flush()
        if self.value_backend != "grouped" or self._value_scales is None \
                or self._compressed_offset == 0:
            return None
        return self._value_scales[:, :, :self._compressed_offset]

    @property
    def value_zeros_raw(self):
        self.flush()
        if self.value_backend != "grouped" or self._value_zeros is None \
                or self._compressed_offset == 0:
            return None
        return self._value_zeros[:, :, :self._compressed_offset]

    def fused_operands(self) -> dict | None:
        """Full-capacity compressed buffers for the fused decode kernels
        ({"kind": "grouped_il"|"grouped"|"turboquant_il"|"turboquant"|"sunshape_v"|"il8"|"dense",
        ...});
        None when there is nothing compressed or the value backend has no
        fused kernel."""
        self.flush()
        if self._key_indices is None or self._compressed_offset == 0:
            return None
        # fp16 heavy-block key dims of a mixed-precision codec, scored exactly
        # by every fused kernel of this cache's layouts but the reference-
        # layout grouped and token-major fp16 ones
        heavy = {"k_heavy": self._key_heavy, "heavy_dims": self._heavy_dims}
        if self.value_backend == "grouped" and self._values_il is not None:
            gc = self._value_codec_impl
            return {"kind": "grouped_il", "idx": self._key_indices, "codes_il": self._values_il,
                    "scales": self._value_scales, "zeros": self._value_zeros,
                    "bits": gc.bits, "group_size": gc.group_size,
                    "buf_keys": self._window(self._key_buffer),
                    "buf_values": self._window(self._value_buffer), **heavy}
        if self._heavy_dims is not None and (self.value_backend == "grouped" or
                                             (self.value_backend == "fp16" and
                                              self._values_il8 is None)):
            return None
        if self.value_backend == "grouped":
            gc = self._value_codec_impl
            return {"kind": "grouped", "idx": self._key_indices,
                    "packed": self._values_packed.view(torch.uint32),
                    "scales": self._value_scales, "zeros": self._value_zeros,
                    "bits": gc.bits, "group_size": gc.group_size,
                    "buf_keys": self._window(self._key_buffer),
                    "buf_values": self._window(self._value_buffer)}
        if self.value_backend == "turboquant" and self._values_il is not None:
            tc = self._value_codec_impl
            tc._on(self._values_il.device)
            return {"kind": "turboquant_il", "idx": self._key_indices, "codes_il": self._values_il,
                    "norms": self._value_norms, "levels": tc.levels_host(),
                    "rotation": tc.rotation,
                    "buf_keys": self._window(self._key_buffer),
                    "buf_values": self._window(self._value_buffer), **heavy}
        if self.value_backend == "turboquant" and self._values_packed is not None:
            tc = self._value_codec_impl
            tc._on(self._values_packed.device)
            return {"kind": "turboquant", "idx": self._key_indices,
                    "packed": self._values_packed, "norms": self._value_norms,
                    "levels": tc.levels_host(), "rotation": tc.rotation, "bits": tc.bits,
                    "buf_keys": self._window(self._key_buffer),
                    "buf_values": self._window(self._value_buffer), **heavy}
        if self.value_backend == "sunshape" and self._value_indices is not None \
                and self.value_codec.n_centroids <= 256:
            vc = self.value_codec
            return {"kind": "sunshape_v", "idx": self._key_indices, "v_idx": self._value_indices,
                    "v_centroids": vc.centroids.float().contiguous(),
                    "v_transform": vc.kernel_value_transform(),
                    "buf_keys": self._window(self._key_buffer),
                    "buf_values": self._window(self._value_buffer), **heavy}
        if self.value_backend == "fp16" and self._values_il8 is not None:
            return {"kind": "il8", "idx": self._key_indices, "values": self._values_il8,
                    "buf_keys": self._window(self._key_buffer),
                    "buf_values": self._window(self._value_buffer), **heavy}
        if self.value_backend == "fp16" and self._values_fp16 is not None:
            return {"kind": "dense", "idx": self._key_indices, "values": self._values_fp16,
                    "buf_keys": self._window(self._key_buffer),
                    "buf_values": self._window(self._value_buffer)}
        return None

    def prefill_operands(self):
        """What the prompt kernel (``ss_prefill_attn_il8_hybrid``) reads of
        this cache: ``(values_il8, key_rows, key_factors, t_raw0)`` -- every
        token's value in the 8-token interleaved fp16 layout (compressed values
        dequantised, then the buffer's), and the buffered keys whole in the
        codec's basis (``_hip.raw_key_rows``), which start at position t_raw0
        = compressed_offset.  O(T) work, against the prompt's O(T x T_q).
        None for SunShape-coded values (an fp16 copy of each value codeword
        would move every token that uses it the same way) and for fp16 heavy
        blocks."""
        self.flush()
        if self.value_backend == "sunshape" or self._heavy_dims is not None or \
                self._key_buffer is None:
            return None
        tc, tb = self._compressed_offset, self._buffer_offset
        t_kv = tc + tb
        b_, h_, d = self._key_buffer.shape[0], self.n_kv_heads, self.head_dim
        dev = self._key_buffer.device
        vil8 = torch.zeros((b_, h_, (t_kv + 7) // 8, d, 8), dtype=torch.float16, device=dev)
        if tc:
            if self._values_il8 is not None:
                nblk = (tc + 7) // 8
                vil8[:, :, :nblk] = self._values_il8[:, :, :nblk]
            elif self.value_backend == "grouped" and self._values_il is not None:
                gc = self._value_codec_impl
                _hip.grouped_il_to_il8(self._values_il, gc.bits, gc.group_size,
                                       self._value_scales, self._value_zeros, tc, vil8)
            else:
                dense = self._compressed_values()
                if dense is None:
                    return None
                _hip.append_values_il8(dense.to(torch.float16).contiguous(), vil8, 0)
        if tb:
            _hip.append_values_il8(self.buffer_values, vil8, tc)
            kb = self.buffer_keys
            c = self.codec
            if c.mode in PERM_MODES:
                rows, fac = _hip.raw_key_rows(kb, c.permutation)
            elif c.use_rotation:
                rows, fac = _hip.raw_key_rows((kb.float() @ c.rotation.t()).contiguous())
            else:
                rows, fac = _hip.raw_key_rows(kb)
        else:
            rows = torch.zeros((b_, h_, 1, 2, d), dtype=torch.float16, device=dev)
            fac = torch.ones((b_, h_, 1), dtype=torch.float32, device=dev)
        return vil8, rows, fac, tc

    @property
    def can_fuse_value_dequant(self) -> bool:
        return (self.value_backend == "grouped" and self._compressed_offset > 0
                and (self._values_packed is not None or self._values_il is not None)
                and self._value_scales is not None and self._value_zeros is not None)

    # ------------------------------------------------------------ metrics
    @property
    def nbytes(self) -> int:
        """Storage bytes with B taken as 1, as the reference does
        (cache.py:904-928)."""
        c, h_ = self._compressed_offset, self.n_kv_heads
        idx_bytes = h_ * c * self.n_blocks * (1 if self.n_centroids <= 256 else 2)
        if self.value_backend == "grouped" and c > 0:
            pd = _packed_dim(self.head_dim, self.value_bits)
            sz = 4 if self.value_scale_dtype == torch.float32 else 2
            val_bytes = h_ * c * pd * 4 + h_ * c * self._value_n_groups * sz * 2
        elif self.value_backend == "turboquant" and c > 0:
            val_bytes = h_ * c * _packed_dim(self.head_dim, self.value_bits) * 4 + h_ * c * 4
        elif self.value_backend == "sunshape" and c > 0:
            val_bytes = h_ * c * self.value_n_blocks * (1 if self.value_n_centroids <= 256 else 2)
        else:
            val_bytes = h_ * c * self.head_dim * 2
        return idx_bytes + val_bytes + h_ * self._buffer_offset * self.head_dim * 2 * 2

    @property
    def nbytes_equivalent_fp16(self) -> int:
        return 0 if self.offset == 0 else 2 * self.n_kv_heads * self.offset * self.head_dim * 2

    @property
    def compression_ratio(self) -> float:
        fp16 = self.nbytes_equivalent_fp16
        return 1.0 if fp16 == 0 else fp16 / max(1, self.nbytes)

    # ---------------------------------------------------- mlx-lm protocol
    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> None:
        """Trim the buffer first, then compressed storage (cache.py:954-963)."""
        self.flush()
        if n <= 0:
            return
        b = min(n, self._buffer_offset)
        self._buffer_offset -= b
        if self._buffer_offset == 0:
            self._buf_start = 0
        rest = n - b
        if rest > 0:
            self._compressed_offset = max(0, self._compressed_offset - rest)
        self._version += 1

    def empty(self) -> bool:
        return self.offset == 0

    def make_mask(self, N: int, return_array: bool = False, window_size: int | None = None,
                  **kwargs):
        return _make_mask(self.offset, N, return_array, self.codec.device)

    def __repr__(self) -> str:
        return (f"HybridSunShapeKVCache(offset={self.offset}, "
                f"compressed={self._compressed_offset}, buffer={self._buffer_offset}, "
                f"value_backend={self.value_backend}, "
                f"compression={self.compression_ratio:.1f}x)")

    @property
    def state(self):
        self.flush()
        parts = []
        if self._key_indices is not None and self._compressed_offset > 0:
            parts.append(self._key_indices[:, :, :self._compressed_offset])
        if self._key_buffer is not None and self._buffer_offset > 0:
            parts.append(self.buffer_keys)
        if not parts:
            parts.append(torch.zeros((1,)))
        return tuple(parts)


def create_kv_cache(codec: SunShapeBlockCodec, *, n_kv_heads: int = 1, head_dim: int | None = None,
                    dtype: torch.dtype = torch.float16, value_backend: str = "fp16",
                    value_bits: int | None = None, value_group_size: int = 64,
                    value_seed: int = 43, value_codec: SunShapeBlockCodec | None = None,
                    buffer_size: int = _DEFAULT_BUFFER_SIZE, prefer_metal_kernels: bool = True,
                    **kwargs):
    """Factory (reference cache.py:1006-1107): fp16 values with the default
    buffer -> ``SunShapeKVCache``; anything else -> ``HybridSunShapeKVCache``.
    Extra keywords (``max_tokens``, ``value_scale_dtype``) pass through."""
    if value_backend == "fp16" and buffer_size == _DEFAULT_BUFFER_SIZE:
        return SunShapeKVCache(codec, n_kv_heads=n_kv_heads, head_dim=head_dim, dtype=dtype,
                               max_tokens=kwargs.get("max_tokens"))
    return HybridSunShapeKVCache(codec, n_kv_heads=n_kv_heads, head_dim=head_dim, dtype=dtype,
                                 buffer_size=buffer_size, value_backend=value_backend,
                                 value_bits=value_bits, value_group_size=value_group_size,
                                 value_seed=value_seed, value_codec=value_codec,
                                 prefer_metal_kernels=prefer_metal_kernels, **kwargs)
