"""sunshape_mlx_amd -- SunShape compressed-KV attention on MI355X (gfx950).

A from-scratch HIP implementation of the compressed-KV attention path of
gauravsaini/sunshape-mlx behind that package's Python API: block-VQ key
encoding, the per-step query x centroid table, fused split-T gather-attention
decode over uint8 key indices with fp16 or grouped 2/3/4-bit values, KV-cache
append and value packing.  Compute runs in ``libsunshape_hip.so`` (C ABI in
``include/sunshape_hip.h``); torch supplies device memory and streams.

The source directory is ``sunshape-mlx_amd/``; it is imported under the name
``sunshape_mlx_amd``.
"""

from . import _hip
from .kernels import (
    block_vq_quantize_hip,
    block_vq_quantize_metal,
    block_vq_score_hip,
    block_vq_score_metal,
    dequantize_values,
    fused_attention_causal_hip,
    fused_attention_causal_metal,
    fused_attention_dequant_causal_hip,
    fused_attention_dequant_causal_metal,
    fused_attention_dequant_hip,
    fused_attention_dequant_metal,
    fused_attention_hip,
    fused_attention_metal,
    fused_block_vq_attention,
    get_kernel_stats,
    pack_indices,
    quantize_scalar_to_indices,
    quantize_values,
    reset_kernel_stats,
    unpack_indices,
)

__version__ = "0.1.0"

from . import codec, rotation  # noqa: E402
from .codec import SunShapeBlockCodec, SunShapeQuantized  # noqa: E402
from .rotation import (  # noqa: E402
    apply_permutation,
    apply_wht,
    block_affinity_gate,
    block_local_cov_metric,
    covariance_block_permutation,
    generate_rotation_matrix,
    generate_wht_signs,
    invert_permutation,
    mixed_precision_block_mask,
    positive_excess_kurtosis,
    safe_normalize,
)
from . import attention, cache, patch, value_codecs  # noqa: E402
from .attention import sunshape_sdpa  # noqa: E402
from .cache import HybridSunShapeKVCache, SunShapeKVCache, create_kv_cache  # noqa: E402
from .value_codecs import GroupedValueCodec, TurboQuantValueCodec, build_value_codec  # noqa: E402
from .serialize import load_cache, load_codec, save_cache, save_codec  # noqa: E402

__all__ = [
    "SunShapeBlockCodec", "SunShapeQuantized", "SunShapeKVCache", "HybridSunShapeKVCache",
    "create_kv_cache", "sunshape_sdpa", "GroupedValueCodec", "TurboQuantValueCodec",
    "build_value_codec", "block_vq_quantize_hip", "block_vq_score_hip", "fused_attention_hip",
    "fused_attention_causal_hip", "fused_attention_dequant_hip",
    "fused_attention_dequant_causal_hip", "fused_block_vq_attention", "quantize_scalar_to_indices",
    "pack_indices", "unpack_indices", "quantize_values", "dequantize_values", "get_kernel_stats",
    "reset_kernel_stats", "apply_permutation", "invert_permutation", "generate_rotation_matrix",
    "covariance_block_permutation", "save_codec", "load_codec", "save_cache", "load_cache",
]
