"""ctypes binding of ``libsunshape_hip.so`` (declared in ``include/sunshape_hip.h``).

Every wrapper takes torch tensors that live on a ROCm device, passes their
data pointers and the current HIP stream to the C ABI, and raises
``SunShapeHIPError`` on a non-zero status.  There is no CPU fallback: if the
library is missing or a tensor is not on the GPU the call raises.

torch is imported before the library is loaded so that the library binds to
the HIP runtime torch already loaded (both carry the SONAME libamdhip64.so.7).
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections import defaultdict

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsunshape_hip.so")

SS_OK = 0
SS_ERR_INVALID = -1
SS_ERR_UNSUPPORTED = -2
SS_ERR_HIP = -3
SS_ERR_WORKSPACE = -4
SS_ERR_WAIT = -5

SS_F32, SS_F16, SS_BF16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: SS_F32, torch.float16: SS_F16, torch.bfloat16: SS_BF16}


class SunShapeHIPError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


class SunShapeUnsupported(SunShapeHIPError):
    """Valid arguments the HIP kernels do not implement (status -2)."""


class SunShapeWaitError(SunShapeHIPError):
    """A bounded in-kernel wait of a fused decode gave up (status -5): the
    output of that launch is invalid."""


_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_size = ctypes.c_size_t

# name -> (restype, argtypes); the order follows include/sunshape_hip.h
_SIGNATURES = {
    "ss_version": (ctypes.c_char_p, []),
    "ss_last_error": (ctypes.c_char_p, []),
    "ss_encode_blockvq": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                                 _c_void_p, _c_void_p, _int, _int, _int, _c_void_p, _i64, _i64,
                                 _i64, _c_void_p]),
    "ss_encode_blockvq_prepared": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64,
                                          _int, _c_void_p, _c_void_p, _int, _int, _int, _c_void_p,
                                          _i64, _i64, _i64, _c_void_p, _c_void_p]),
    "ss_encode_codebook_bytes": (_size, [_int]),
    "ss_encode_codebook": (_int, [_c_void_p, _int, _int, _int, _c_void_p, _c_void_p]),
    "ss_build_lut": (_int, [_c_void_p, _int, _i64, _i64, _int, _c_void_p, _f32, _c_void_p,
                            _int, _int, _int, _c_void_p, _c_void_p]),
    "ss_score_gather": (_int, [_c_void_p, _i64, _int, _int, _c_void_p, _i64, _i64, _c_void_p,
                               _i64, _c_void_p]),
    "ss_score_gather_heads": (_int, [_c_void_p, _i64, _int, _int, _c_void_p, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _c_void_p, _c_void_p]),
    "ss_decode_workspace_bytes": (_size, [_i64, _int, _int, _i64, _int, _i64, _int]),
    "ss_decode_wait_failures": (_int, [_c_void_p, _int, ctypes.POINTER(ctypes.c_uint)]),
    "ss_decode_wait_flag_host": (_int, [ctypes.POINTER(ctypes.POINTER(ctypes.c_uint))]),
    "ss_debug_set_spin_limit": (_int, [_int]),
    "ss_stream_read": (_int, [_c_void_p, _i64, _int, _c_void_p, _c_void_p]),
    "ss_decode_default_splits": (_int, [_i64, _int, _int, _i64, _int, _i64]),
    "ss_decode_attn_dense": (_int, [_c_void_p, _int, _i64, _int, _int, _i64, _int, _f32,
                                    _c_void_p, _c_void_p, _int, _int, _c_void_p, _c_void_p, _int,
                                    _i64, _i64, _int, _i64, _c_void_p, _int, _c_void_p, _size,
                                    _int, _c_void_p]),
    "ss_decode_plan": (_int, [_int, _i64, _int, _int, _i64, _int, _i64, _int,
                              ctypes.POINTER(_int), ctypes.POINTER(_size)]),
    "ss_decode_attn_il8": (_int, [_c_void_p, _int, _i64, _int, _int, _i64, _int, _f32,
                                  _c_void_p, _c_void_p, _int, _int, _c_void_p, _c_void_p, _int,
                                  _i64, _i64, _int, _i64, _c_void_p, _int, _c_void_p, _size,
                                  _int, _c_void_p]),
    "ss_decode_attn_il8_hybrid": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _int, _int,
        _c_void_p, _c_void_p, _int, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _int,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_step_il8": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _c_void_p,
        _int, _int, _c_void_p, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_prefill_rows_per_workgroup": (_int, []),
    "ss_prefill_attn_il8": (_int, [_c_void_p, _int, _i64, _int, _int, _i64, _int, _f32,
                                   _c_void_p, _c_void_p, _int, _int, _c_void_p, _c_void_p, _int,
                                   _i64, _i64, _int, _i64, _c_void_p, _int, _c_void_p]),
    "ss_prefill_attn_il8_hybrid": (_int, [_c_void_p, _int, _i64, _int, _int, _i64, _int, _f32,
                                          _c_void_p, _c_void_p, _int, _int, _c_void_p, _i64,
                                          _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                          _int, _i64, _c_void_p, _int, _c_void_p]),
    "ss_decode_attn_il8_noalloc": (_int, [_c_void_p, _int, _i64, _int, _int, _i64, _int, _f32,
                                          _c_void_p, _c_void_p, _int, _int, _c_void_p, _c_void_p,
                                          _int, _i64, _i64, _int, _i64, _c_void_p, _int, _int,
                                          _c_void_p]),
    "ss_decode_static_scratch_bytes": (_size, []),
    "ss_codebook_f16x2_bytes": (_size, [_int, _int]),
    "ss_codebook_f16x2": (_int, [_c_void_p, _int, _int, _c_void_p, _c_void_p]),
    "ss_append_values_il8": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                                    _c_void_p, _i64, _i64, _c_void_p]),
    "ss_hybrid_append_grouped_il": (_int, [
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _int, _c_void_p, _c_void_p, _int,
        _int, _int, _c_void_p, _int, _int, _c_void_p, _c_void_p, _c_void_p, _int, _i64, _i64,
        _c_void_p]),
    "ss_append_kv_il8": (_int, [_c_void_p, _int, _c_void_p, _int, _i64, _i64, _i64, _i64, _i64,
                                _i64, _i64, _i64, _i64, _int, _c_void_p, _c_void_p, _int, _int,
                                _int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "ss_decode_attn_grouped": (_int, [_c_void_p, _int, _i64, _int, _int, _i64, _int, _f32,
                                      _c_void_p, _c_void_p, _int, _int, _c_void_p, _c_void_p,
                                      _c_void_p, _c_void_p, _int, _int, _int, _i64, _i64, _int,
                                      _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_attn_grouped_hybrid": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _int, _int,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _int, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_attn_dense_hybrid": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _int, _int,
        _c_void_p, _c_void_p, _int, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_attn_turboquant": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _int, _int,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _int,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_turboquant_workspace_bytes": (_size, [_i64, _int, _int, _i64, _int, _i64, _i64,
                                                     _int]),
    "ss_decode_attn_turboquant_il": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _int, _int,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _int,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_kmeans_blocks": (_int, [_c_void_p, _int, _i64, _int, _int, _int, _c_void_p, _c_void_p,
                                _c_void_p]),
    "ss_decode_attn_sunshape_v": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _int, _int,
        _c_void_p, _c_void_p, _c_void_p, _int, _int, _c_void_p, _c_void_p, _c_void_p, _int,
        _i64, _i64, _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _int, _i64,
        _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_attn_grouped_il": (_int, [_c_void_p, _int, _i64, _int, _int, _i64, _int, _f32,
                                         _c_void_p, _c_void_p, _int, _int, _c_void_p, _c_void_p,
                                         _c_void_p, _c_void_p, _int, _int, _int, _i64, _i64, _int,
                                         _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_attn_grouped_il_hybrid": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _int, _int,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _int, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _int,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_step_grouped_il_hybrid": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _c_void_p,
        _int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _int, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_decode_step_il8_hybrid": (_int, [
        _c_void_p, _int, _i64, _int, _int, _i64, _int, _f32, _c_void_p, _c_void_p, _c_void_p,
        _int, _int, _c_void_p, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _i64,
        _c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64,
        _int, _i64, _c_void_p, _int, _c_void_p, _size, _int, _c_void_p]),
    "ss_pack_grouped_il": (_int, [_c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int,
                                  _c_void_p, _i64, _i64, _c_void_p]),
    "ss_grouped_il_to_packed": (_int, [_c_void_p, _i64, _i64, _int, _int, _i64, _c_void_p,
                                       _c_void_p]),
    "ss_grouped_il_to_il8": (_int, [_c_void_p, _i64, _i64, _int, _int, _int, _c_void_p,
                                    _c_void_p, _int, _i64, _i64, _c_void_p, _i64, _c_void_p]),
    "ss_raw_key_rows": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                               _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "ss_quantize_values_grouped": (_int, [_c_void_p, _int, _i64, _i64, _i64, _i64, _i64, _i64,
                                          _int, _int, _int, _c_void_p, _c_void_p, _c_void_p, _int,
                                          _i64, _i64, _i64, _c_void_p]),
    "ss_dequantize_values_grouped": (_int, [_c_void_p, _c_void_p, _c_void_p, _int, _i64, _int,
                                            _int, _int, _c_void_p, _int, _c_void_p]),
    "ss_pack_indices": (_int, [_c_void_p, _i64, _int, _int, _c_void_p, _c_void_p]),
    "ss_unpack_indices": (_int, [_c_void_p, _i64, _int, _int, _c_void_p, _c_void_p]),
    "ss_scalar_quantize": (_int, [_c_void_p, _i64, _c_void_p, _int, _c_void_p, _c_void_p]),
    "ss_dequantize_blockvq": (_int, [_c_void_p, _i64, _i64, _c_void_p, _int, _int, _int,
                                     _c_void_p, _c_void_p, _int, _c_void_p]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib = None
_lock = threading.Lock()


def load_library(path: str | None = None):
    """Load (once) and return the ctypes handle.  Raises if the library is
    missing: build it with ``__graft_entry__.build()``."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"libsunshape_hip.so not found at {p}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repo root")
        lib = ctypes.CDLL(p)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def version() -> str:
    return load_library().ss_version().decode()


def _raise(rc: int):
    msg = load_library().ss_last_error().decode(errors="replace")
    if rc == SS_ERR_UNSUPPORTED:
        raise SunShapeUnsupported(rc, msg)
    if rc == SS_ERR_WAIT:
        raise SunShapeWaitError(rc, msg)
    raise SunShapeHIPError(rc, msg)


def check(rc: int) -> None:
    if rc != SS_OK:
        _raise(rc)


# Kernel dispatch counters (reference kernels.py:33-47, incremented at every
# Metal dispatch, kernels.py:113, 288, 443, 498, 762, 925, 1079): every
# wrapper below that launches a kernel counts its launch here once the call
# has been accepted, whichever Python route (cache, SDPA, codec, launcher)
# reached it.  ``kernels.get_kernel_stats`` reads this table.
_KERNEL_STATS: dict[str, int] = defaultdict(int)


def record_dispatch(name: str) -> None:
    _KERNEL_STATS[name] += 1


def _launched(name: str, rc: int) -> None:
    """``check(rc)``, then count one dispatch of ``name``."""
    check(rc)
    _KERNEL_STATS[name] += 1


def _attn_stat(stem: str, causal) -> str:
    return f"{stem}_causal_hip" if causal else f"{stem}_hip"


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt} (float32, float16, bfloat16)") from None


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError(
                "SunShape HIP kernels need tensors on a ROCm GPU device "
                f"(got device {t.device}); there is no CPU fallback")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def device_index(device) -> int:
    if isinstance(device, int):
        return device
    if device is None or device.index is None:
        return torch.cuda.current_device()
    return device.index


def stream_handle(device: torch.device | None = None) -> int:
    """hipStream_t of the current stream of ``device``."""
    if _raw_stream is not None:
        return _raw_stream(device_index(device))
    return torch.cuda.current_stream(device).cuda_stream


# --------------------------------------------------------------------------- #
#  Bounded-wait failures of the matrix-core decodes                           #
# --------------------------------------------------------------------------- #

# Check the wait-failure word after every matrix-core decode launch (one
# stream synchronisation per call); off by default, on with
# SUNSHAPE_CHECK_WAITS=1 or set_wait_checks(True).  Without it, every decode
# launch first polls the library's pinned host copy of the flags (a plain
# load, no synchronisation), so a give-up is raised by the first decode call
# made after the failing launch has run.
_check_waits = os.environ.get("SUNSHAPE_CHECK_WAITS", "0") == "1"
_wait_flag = None  # ctypes.c_uint over the pinned host word


def decode_wait_flag() -> int:
    """The pinned host copy of the wait-failure flags, read without
    synchronising (nonzero once a failed launch has finished running)."""
    global _wait_flag
    if _wait_flag is None:
        p = ctypes.POINTER(ctypes.c_uint)()
        check(load_library().ss_decode_wait_flag_host(ctypes.byref(p)))
        _wait_flag = p.contents
    return int(_wait_flag.value)


def _poll_waits(device) -> None:
    """Before a matrix-core decode launch: raise ``SunShapeWaitError`` if an
    earlier launch's bounded wait gave up (the host word is set; the
    synchronising check then reports and clears both words)."""
    if (_wait_flag.value if _wait_flag is not None else decode_wait_flag()):
        check_decode_waits(device)


def set_wait_checks(enabled: bool) -> bool:
    """Turn the per-call wait check on or off; returns the previous setting."""
    global _check_waits
    prev, _check_waits = _check_waits, bool(enabled)
    return prev


def decode_wait_failures(device: torch.device | None = None, clear: bool = True) -> int:
    """Synchronise the current stream of ``device`` and return the sticky
    wait-failure flags of the matrix-core decodes (0 if every wait ended in
    time; bit 1 compute barrier, 2 ring slot, 4 ring tile), clearing them
    when ``clear``."""
    flags = ctypes.c_uint(0)
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        rc = load_library().ss_decode_wait_failures(stream_handle(device), int(clear),
                                                    ctypes.byref(flags))
    if rc not in (SS_OK, SS_ERR_WAIT):
        _raise(rc)
    return int(flags.value)


def check_decode_waits(device: torch.device | None = None) -> None:
    """Raise ``SunShapeWaitError`` (and clear the flags) if a bounded wait
    of a matrix-core decode launched on ``device`` has given up."""
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        check(load_library().ss_decode_wait_failures(stream_handle(device), 1, None))


def set_spin_limit(limit: int | None) -> None:
    """Test hook: sleeps before a bounded wait gives up, for later launches
    (None restores the default)."""
    check(load_library().ss_debug_set_spin_limit(-1 if limit is None else int(limit)))


# --------------------------------------------------------------------------- #
#  Decode workspace (split-T partials)                                        #
# --------------------------------------------------------------------------- #

_ws_cache: dict[tuple[int, int], torch.Tensor] = {}


def decode_workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """Per (device, stream) scratch for split-T partials.  Calls on one stream
    are ordered, so they never overlap on the same buffer.  Allocated zeroed:
    its first 64 KiB hold the per-column split counters, which every call
    leaves at zero."""
    if nbytes <= 0:
        return None
    dev = device_index(device)
    key = (dev, stream if stream is not None else stream_handle(dev))
    ws = _ws_cache.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=torch.device("cuda", dev))
        _ws_cache[key] = ws
    return ws


class PreparedDecode:
    """A matrix-core decode (ss_decode_attn_il8 or ss_decode_attn_grouped_il)
    over fixed cache buffers, codebook and query shape: the C-ABI arguments
    that do not change between steps are checked and built once, and a call
    fills in the query, the output, the cache length, the causal offset and
    the current stream.  The split workspace is the per-(device, stream) one,
    passed at its allocated size; a call that needs more grows it and
    launches then (the library checks the size before it launches anything).
    The caller keeps the buffers alive (the cache that built the plan owns
    them) and builds a new plan when any of them changes."""

    __slots__ = ("fn", "pre", "dev", "shape", "dtype", "plan_args", "stat")

    def __init__(self, fn, pre: tuple, q: torch.Tensor, stat: str):
        self.fn = fn
        self.pre = pre
        self.dev = device_index(q.device)
        self.shape = tuple(q.shape)
        self.dtype = q.dtype
        self.plan_args = tuple(q.shape[:1]) + (pre[2], pre[3]) + tuple(q.shape[2:])
        self.stat = stat

    def __call__(self, q: torch.Tensor, t_kv: int, causal: bool = False, q_offset: int = 0,
                 out: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
        if q.shape != self.shape or q.dtype != self.dtype or not q.is_contiguous() or \
                q.device.index != self.dev:
            raise ValueError(f"query must be contiguous {self.dtype} {self.shape} on cuda:{self.dev}")
        if out is None:
            out = torch.empty(self.shape, dtype=out_dtype or self.dtype, device=q.device)
        elif tuple(out.shape) != self.shape or not out.is_contiguous() or out.device != q.device:
            raise ValueError(f"out must be contiguous {self.shape} on cuda:{self.dev}")
        _poll_waits(self.dev)
        st = stream_handle(self.dev)
        ws = _ws_cache.get((self.dev, st))
        if ws is None:
            ws = decode_workspace(self.dev, 1, st)
        tail = (int(t_kv), int(bool(causal)), int(q_offset), out.data_ptr(),
                dtype_code(out.dtype))
        rc = self.fn(q.data_ptr(), *self.pre, *tail, ws.data_ptr(), ws.numel(), 0, st)
        if rc == SS_ERR_WORKSPACE:
            _, need = decode_plan(KIND_IL8, *self.plan_args, int(t_kv), 0)
            ws = decode_workspace(self.dev, need, st)
            rc = self.fn(q.data_ptr(), *self.pre, *tail, ws.data_ptr(), ws.numel(), 0, st)
        _launched(_attn_stat(self.stat, causal), rc)
        if _check_waits:
            check_decode_waits(self.dev)
        return out


class PreparedDecodeBuffered(PreparedDecode):
    """:class:`PreparedDecode` of the hybrid-cache variants
    (ss_decode_attn_il8_hybrid, ss_decode_attn_grouped_il_hybrid): a call
    also passes the buffered tokens, ``buf_keys`` / ``buf_values`` (B, Hkv,
    >= buf_len, D) views of the cache's buffer stores (the window moves, the
    stores and their strides are fixed with the plan)."""

    __slots__ = ("buf_code", "buf_strides")

    def __init__(self, fn, pre: tuple, q: torch.Tensor, stat: str, buf_keys: torch.Tensor):
        super().__init__(fn, pre, q, stat)
        self.buf_code = dtype_code(buf_keys.dtype)
        self.buf_strides = tuple(buf_keys.stride()[:3])

    def __call__(self, q: torch.Tensor, t_kv: int, buf_keys: torch.Tensor,
                 buf_values: torch.Tensor, buf_len: int, causal: bool = False, q_offset: int = 0,
                 out: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
        if q.shape != self.shape or q.dtype != self.dtype or not q.is_contiguous() or \
                q.device.index != self.dev:
            raise ValueError(f"query must be contiguous {self.dtype} {self.shape} on cuda:{self.dev}")
        if tuple(buf_keys.stride()[:3]) != self.buf_strides or \
                tuple(buf_values.stride()[:3]) != self.buf_strides or \
                buf_keys.shape[2] < buf_len or buf_values.shape[2] < buf_len:
            raise ValueError("buffer views must keep the plan's strides and hold buf_len tokens")
        if out is None:
            out = torch.empty(self.shape, dtype=out_dtype or self.dtype, device=q.device)
        elif tuple(out.shape) != self.shape or not out.is_contiguous() or out.device != q.device:
            raise ValueError(f"out must be contiguous {self.shape} on cuda:{self.dev}")
        _poll_waits(self.dev)
        st = stream_handle(self.dev)
        ws = _ws_cache.get((self.dev, st))
        if ws is None:
            ws = decode_workspace(self.dev, 1, st)
        mid = (int(t_kv), buf_keys.data_ptr(), buf_values.data_ptr(), self.buf_code,
               *self.buf_strides, int(buf_len), None, None, 0, int(bool(causal)), int(q_offset),
               out.data_ptr(), dtype_code(out.dtype))
        rc = self.fn(q.data_ptr(), *self.pre, *mid, ws.data_ptr(), ws.numel(), 0, st)
        if rc == SS_ERR_WORKSPACE:
            _, need = decode_plan(KIND_IL8, *self.plan_args, int(t_kv), 0)
            ws = decode_workspace(self.dev, need, st)
            rc = self.fn(q.data_ptr(), *self.pre, *mid, ws.data_ptr(), ws.numel(), 0, st)
        _launched(_attn_stat(self.stat, causal), rc)
        if _check_waits:
            check_decode_waits(self.dev)
        return out


MAX_STEP_TOKENS = 4  # new tokens one fused decode step takes (kMaxStepTokens)


class PreparedDecodeStep(PreparedDecode):
    """One decode step of an fp16-value cache in one launch
    (``ss_decode_step_il8``): a call passes the step's new keys and values
    (B, Hkv, n_new, D) float16 (equal strides, unit last stride) and the
    number of tokens already in the cache; the kernel encodes the new keys,
    attends all tokens and stores the new ones at positions t_cache ..
    t_cache + n_new - 1."""

    __slots__ = ()

    def __call__(self, q: torch.Tensor, t_cache: int, k_new: torch.Tensor, v_new: torch.Tensor,
                 causal: bool = False, q_offset: int = 0, out: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
        if q.shape != self.shape or q.dtype != self.dtype or not q.is_contiguous() or \
                q.device.index != self.dev:
            raise ValueError(f"query must be contiguous {self.dtype} {self.shape} on cuda:{self.dev}")
        st3 = k_new.stride()[:3]
        if k_new.dtype != torch.float16 or v_new.dtype != torch.float16 or \
                k_new.shape != v_new.shape or v_new.stride()[:3] != st3 or \
                k_new.stride(-1) != 1 or v_new.stride(-1) != 1 or \
                k_new.device.index != self.dev or v_new.device.index != self.dev:
            raise ValueError("new keys and values must be float16 (B, Hkv, n, D) with equal "
                             "strides and unit last stride")
        if out is None:
            out = torch.empty(self.shape, dtype=out_dtype or self.dtype, device=q.device)
        elif tuple(out.shape) != self.shape or not out.is_contiguous() or out.device != q.device:
            raise ValueError(f"out must be contiguous {self.shape} on cuda:{self.dev}")
        _poll_waits(self.dev)
        st = stream_handle(self.dev)
        ws = _ws_cache.get((self.dev, st))
        if ws is None:
            ws = decode_workspace(self.dev, 1, st)
        mid = (int(t_cache), k_new.data_ptr(), v_new.data_ptr(), SS_F16, *st3,
               int(k_new.shape[2]), int(bool(causal)), int(q_offset), out.data_ptr(),
               dtype_code(out.dtype))
        rc = self.fn(q.data_ptr(), *self.pre, *mid, ws.data_ptr(), ws.numel(), 0, st)
        if rc == SS_ERR_WORKSPACE:
            _, need = decode_plan(KIND_IL8, *self.plan_args, int(t_cache), 0)
            ws = decode_workspace(self.dev, need, st)
            rc = self.fn(q.data_ptr(), *self.pre, *mid, ws.data_ptr(), ws.numel(), 0, st)
        _launched(_attn_stat(self.stat, causal), rc)
        if _check_waits:
            check_decode_waits(self.dev)
        return out


def prepare_decode_step_il8(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                            codebook: torch.Tensor, centroids: torch.Tensor, n_blocks: int,
                            n_centroids: int, idx: torch.Tensor,
                            values_il8: torch.Tensor) -> PreparedDecodeStep:
    """:class:`PreparedDecodeStep` for queries shaped like ``q`` over the
    cache buffers ``idx`` / ``values_il8`` (written by the call), with the
    float32 ``centroids`` (n_blocks, n_centroids, 8) for the exact encode and
    their prepared ``codebook`` for the LUT."""
    _check_decode_common(q, idx, None, perm)
    require_gpu(values_il8, codebook, centroids)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if nb != n_blocks or values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
            tuple(values_il8.shape) != (b_, hkv, cap // 8, d, 8):
        raise ValueError(f"values_il8 must be contiguous float16 {(b_, hkv, cap // 8, d, 8)}")
    if centroids.dtype != torch.float32 or not centroids.is_contiguous() or \
            tuple(centroids.shape) != (n_blocks, n_centroids, 8):
        raise ValueError(f"centroids must be contiguous float32 {(n_blocks, n_centroids, 8)}")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(n_blocks, n_centroids):
        raise ValueError("codebook does not match the centroids' shape")
    pre = (dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
           ptr(centroids), nb, n_centroids, ptr(idx), ptr(values_il8), cap)
    return PreparedDecodeStep(lib.ss_decode_step_il8, pre, q, "sunshape_fused_attention_mfma")


def decode_step_il8(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                    codebook: torch.Tensor, centroids: torch.Tensor, idx: torch.Tensor,
                    values_il8: torch.Tensor, t_cache: int, k_new: torch.Tensor,
                    v_new: torch.Tensor, causal: bool = False, q_offset: int = 0,
                    out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """One launch of :class:`PreparedDecodeStep` (checks every call)."""
    nb, nc = int(centroids.shape[0]), int(centroids.shape[1])
    plan = prepare_decode_step_il8(q, scale, perm, codebook, centroids, nb, nc, idx, values_il8)
    return plan(q, t_cache, k_new, v_new, causal, q_offset, out_dtype=out_dtype)


def prepare_decode_il8(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                       codebook: torch.Tensor, n_blocks: int, n_centroids: int,
                       idx: torch.Tensor, values_il8: torch.Tensor,
                       buf_keys: torch.Tensor | None = None) -> PreparedDecode:
    """:class:`PreparedDecode` of :func:`decode_attn_il8` for queries shaped
    like ``q`` (the same checks, done once); with ``buf_keys`` (a view of a
    hybrid cache's buffer store) the buffered variant,
    :class:`PreparedDecodeBuffered`."""
    _check_decode_common(q, idx, None, perm)
    require_gpu(values_il8, codebook)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if nb != n_blocks or values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
            tuple(values_il8.shape) != (b_, hkv, cap // 8, d, 8):
        raise ValueError(f"values_il8 must be contiguous float16 {(b_, hkv, cap // 8, d, 8)}")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(n_blocks, n_centroids):
        raise ValueError("codebook does not match the centroids' shape")
    pre = (dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
           nb, n_centroids, ptr(idx), ptr(values_il8), SS_F16, cap)
    if buf_keys is not None:
        _buffer_args(buf_keys, buf_keys, 1, b_, hkv, d)
        return PreparedDecodeBuffered(lib.ss_decode_attn_il8_hybrid, pre, q,
                                      "sunshape_fused_attention_mfma", buf_keys)
    return PreparedDecode(lib.ss_decode_attn_il8, pre, q, "sunshape_fused_attention_mfma")


def prepare_decode_grouped_il(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                              codebook: torch.Tensor, n_blocks: int, n_centroids: int,
                              idx: torch.Tensor, codes_il: torch.Tensor, scales: torch.Tensor,
                              zeros: torch.Tensor, bits: int, group_size: int,
                              buf_keys: torch.Tensor | None = None) -> PreparedDecode:
    """:class:`PreparedDecode` of :func:`decode_attn_grouped_il` for queries
    shaped like ``q``; with ``buf_keys`` the buffered variant."""
    _check_decode_common(q, idx, None, perm)
    require_gpu(codes_il, scales, zeros, codebook)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    tpw = 32 // bits if bits in (2, 4) else 0
    if nb != n_blocks or not tpw or codes_il.dim() != 4 or not codes_il.is_contiguous() or \
            tuple(codes_il.shape) != (b_, hkv, cap // tpw, d) or \
            codes_il.dtype not in (torch.int32, torch.uint32):
        raise ValueError("codes_il does not match the cache shape")
    for t in (scales, zeros):
        if t.dim() != 4 or not t.is_contiguous() or t.shape[:3] != idx.shape[:3]:
            raise ValueError("scales/zeros must be contiguous (B, n_kv_heads, cap, n_groups)")
    if scales.dtype != zeros.dtype or scales.dtype not in (torch.float32, torch.float16):
        raise ValueError("scales/zeros must share dtype float32 or float16")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(n_blocks, n_centroids):
        raise ValueError("codebook does not match the centroids' shape")
    pre = (dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
           nb, n_centroids, ptr(idx), ptr(codes_il), ptr(scales), ptr(zeros),
           dtype_code(scales.dtype), int(bits), int(group_size), cap)
    if buf_keys is not None:
        _buffer_args(buf_keys, buf_keys, 1, b_, hkv, d)
        return PreparedDecodeBuffered(lib.ss_decode_attn_grouped_il_hybrid, pre, q,
                                      "sunshape_fused_attention_dequant_mfma", buf_keys)
    return PreparedDecode(lib.ss_decode_attn_grouped_il, pre, q,
                          "sunshape_fused_attention_dequant_mfma")


class PreparedHybridStep(PreparedDecode):
    """One decode step of a hybrid cache with 2- or 4-bit interleaved
    grouped values (``ss_decode_step_grouped_il_hybrid``), or with fp16
    values held interleaved (``ss_decode_step_il8_hybrid``), in one launch: a call
    passes the buffer stores' window (``buf_keys`` / ``buf_values``, (B, Hkv,
    >= n_buf + n_new, D) float16 views starting at the oldest buffered
    token), the number of buffered tokens, how many of the oldest leave the
    buffer, and the step's new keys and values (B, Hkv, n_new, D) float16;
    the kernel writes the leaving tokens' index rows, codes, scales and
    zeros at compressed positions t_kv .., the new tokens at buffer rows
    n_buf .., and attends every token as the reference does after its
    append and flush."""

    __slots__ = ("buf_strides",)

    def __init__(self, fn, pre: tuple, q: torch.Tensor, stat: str, buf_keys: torch.Tensor):
        super().__init__(fn, pre, q, stat)
        self.buf_strides = tuple(buf_keys.stride()[:3])

    def __call__(self, q: torch.Tensor, t_kv: int, buf_keys: torch.Tensor,
                 buf_values: torch.Tensor, n_buf: int, n_flush: int, k_new: torch.Tensor,
                 v_new: torch.Tensor, causal: bool = False, q_offset: int = 0,
                 out: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
        if q.shape != self.shape or q.dtype != self.dtype or not q.is_contiguous() or \
                q.device.index != self.dev:
            raise ValueError(f"query must be contiguous {self.dtype} {self.shape} on cuda:{self.dev}")
        n_new = int(k_new.shape[2])
        if buf_keys.dtype != torch.float16 or buf_values.dtype != torch.float16 or \
                tuple(buf_keys.stride()[:3]) != self.buf_strides or \
                tuple(buf_values.stride()[:3]) != self.buf_strides or \
                buf_keys.shape[2] < n_buf + n_new or buf_values.shape[2] < n_buf + n_new:
            raise ValueError("buffer views must be float16, keep the plan's strides and hold "
                             "n_buf + n_new rows")
        st3 = k_new.stride()[:3]
        if k_new.dtype != torch.float16 or v_new.dtype != torch.float16 or \
                k_new.shape != v_new.shape or v_new.stride()[:3] != st3 or \
                k_new.stride(-1) != 1 or v_new.stride(-1) != 1 or \
                k_new.device.index != self.dev or v_new.device.index != self.dev:
            raise ValueError("new keys and values must be float16 (B, Hkv, n, D) with equal "
                             "strides and unit last stride")
        if out is None:
            out = torch.empty(self.shape, dtype=out_dtype or self.dtype, device=q.device)
        elif tuple(out.shape) != self.shape or not out.is_contiguous() or out.device != q.device:
            raise ValueError(f"out must be contiguous {self.shape} on cuda:{self.dev}")
        _poll_waits(self.dev)
        st = stream_handle(self.dev)
        ws = _ws_cache.get((self.dev, st))
        if ws is None:
            ws = decode_workspace(self.dev, 1, st)
        mid = (int(t_kv), buf_keys.data_ptr(), buf_values.data_ptr(), SS_F16, *self.buf_strides,
               int(n_buf), int(n_flush), k_new.data_ptr(), v_new.data_ptr(), SS_F16, *st3, n_new,
               int(bool(causal)), int(q_offset), out.data_ptr(), dtype_code(out.dtype))
        rc = self.fn(q.data_ptr(), *self.pre, *mid, ws.data_ptr(), ws.numel(), 0, st)
        if rc == SS_ERR_WORKSPACE:
            _, need = decode_plan(KIND_IL8, *self.plan_args, int(t_kv), 0)
            ws = decode_workspace(self.dev, need, st)
            rc = self.fn(q.data_ptr(), *self.pre, *mid, ws.data_ptr(), ws.numel(), 0, st)
        _launched(_attn_stat(self.stat, causal), rc)
        if _check_waits:
            check_decode_waits(self.dev)
        return out


def prepare_decode_step_grouped_il_hybrid(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                                          codebook: torch.Tensor, centroids: torch.Tensor,
                                          n_blocks: int, n_centroids: int, idx: torch.Tensor,
                                          codes_il: torch.Tensor, scales: torch.Tensor,
                                          zeros: torch.Tensor, bits: int, group_size: int,
                                          buf_keys: torch.Tensor) -> PreparedHybridStep:
    """:class:`PreparedHybridStep` for queries shaped like ``q`` over the
    compressed stores (``idx``, ``codes_il``, ``scales``, ``zeros``; written
    by the call) and buffer stores shaped like ``buf_keys``, with the float32
    ``centroids`` (n_blocks, n_centroids, 8) for the exact encode and their
    prepared ``codebook`` for the LUT."""
    _check_decode_common(q, idx, None, perm)
    require_gpu(codes_il, scales, zeros, codebook, centroids, buf_keys)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if bits not in (2, 4):
        raise SunShapeUnsupported(-2, "a fused hybrid step takes 2- or 4-bit grouped codes")
    if nb != n_blocks or codes_il.dim() != 4 or not codes_il.is_contiguous() or \
            tuple(codes_il.shape) != (b_, hkv, cap // (32 // bits), d) or \
            codes_il.dtype not in (torch.int32, torch.uint32):
        raise ValueError("codes_il does not match the cache shape")
    for t in (scales, zeros):
        if t.dim() != 4 or not t.is_contiguous() or t.shape[:3] != idx.shape[:3]:
            raise ValueError("scales/zeros must be contiguous (B, n_kv_heads, cap, n_groups)")
    if scales.dtype != zeros.dtype or scales.dtype not in (torch.float32, torch.float16):
        raise ValueError("scales/zeros must share dtype float32 or float16")
    if centroids.dtype != torch.float32 or not centroids.is_contiguous() or \
            tuple(centroids.shape) != (n_blocks, n_centroids, 8):
        raise ValueError(f"centroids must be contiguous float32 {(n_blocks, n_centroids, 8)}")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(n_blocks, n_centroids):
        raise ValueError("codebook does not match the centroids' shape")
    _buffer_args(buf_keys, buf_keys, 1, b_, hkv, d)
    pre = (dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
           ptr(centroids), nb, n_centroids, ptr(idx), ptr(codes_il), ptr(scales), ptr(zeros),
           dtype_code(scales.dtype), int(bits), int(group_size), cap)
    return PreparedHybridStep(lib.ss_decode_step_grouped_il_hybrid, pre, q,
                              "sunshape_fused_attention_dequant_mfma", buf_keys)


def prepare_decode_step_il8_hybrid(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                                   codebook: torch.Tensor, centroids: torch.Tensor, n_blocks: int,
                                   n_centroids: int, idx: torch.Tensor, values_il8: torch.Tensor,
                                   buf_keys: torch.Tensor) -> PreparedHybridStep:
    """:class:`PreparedHybridStep` of a hybrid cache with fp16 values held
    8-token interleaved (``ss_decode_step_il8_hybrid``): the flushed tokens'
    index rows and values are written into ``idx`` / ``values_il8``."""
    _check_decode_common(q, idx, None, perm)
    require_gpu(values_il8, codebook, centroids, buf_keys)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if nb != n_blocks or values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
            tuple(values_il8.shape) != (b_, hkv, cap // 8, d, 8):
        raise ValueError(f"values_il8 must be contiguous float16 {(b_, hkv, cap // 8, d, 8)}")
    if centroids.dtype != torch.float32 or not centroids.is_contiguous() or \
            tuple(centroids.shape) != (n_blocks, n_centroids, 8):
        raise ValueError(f"centroids must be contiguous float32 {(n_blocks, n_centroids, 8)}")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(n_blocks, n_centroids):
        raise ValueError("codebook does not match the centroids' shape")
    _buffer_args(buf_keys, buf_keys, 1, b_, hkv, d)
    pre = (dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
           ptr(centroids), nb, n_centroids, ptr(idx), ptr(values_il8), cap)
    return PreparedHybridStep(lib.ss_decode_step_il8_hybrid, pre, q,
                              "sunshape_fused_attention_mfma", buf_keys)


def decode_step_grouped_il_hybrid(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                                  codebook: torch.Tensor, centroids: torch.Tensor,
                                  idx: torch.Tensor, codes_il: torch.Tensor, scales: torch.Tensor,
                                  zeros: torch.Tensor, bits: int, group_size: int, t_kv: int,
                                  buf_keys: torch.Tensor, buf_values: torch.Tensor, n_buf: int,
                                  n_flush: int, k_new: torch.Tensor, v_new: torch.Tensor,
                                  causal: bool = False, q_offset: int = 0,
                                  out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """One launch of :class:`PreparedHybridStep` (checks every call)."""
    nb, nc = int(centroids.shape[0]), int(centroids.shape[1])
    plan = prepare_decode_step_grouped_il_hybrid(q, scale, perm, codebook, centroids, nb, nc, idx,
                                                 codes_il, scales, zeros, bits, group_size,
                                                 buf_keys)
    return plan(q, t_kv, buf_keys, buf_values, n_buf, n_flush, k_new, v_new, causal, q_offset,
                out_dtype=out_dtype)


# --------------------------------------------------------------------------- #
#  Typed wrappers                                                              #
# --------------------------------------------------------------------------- #


def encode_codebook(centroids: torch.Tensor) -> torch.Tensor:
    """Prepared codebook (flat uint8 buffer) of the matrix-core encoder for
    float32 centroids (n_blocks <= 16, n_centroids <= 256, 8): per block a
    power-of-two scale, the split-fp16 MFMA operands and the squared norms."""
    require_gpu(centroids)
    if centroids.dim() != 3 or centroids.dtype != torch.float32 or not centroids.is_contiguous():
        raise ValueError("centroids must be contiguous float32 (n_blocks, n_centroids, 8)")
    nb, nc, bd = centroids.shape
    lib = load_library()
    out = torch.empty(lib.ss_encode_codebook_bytes(nb), dtype=torch.uint8, device=centroids.device)
    check(lib.ss_encode_codebook(ptr(centroids), nb, nc, bd, ptr(out),
                                 stream_handle(centroids.device)))
    return out


def encode_codebook_supported(centroids: torch.Tensor) -> bool:
    """Shapes the prepared (matrix-core) encoder takes."""
    nb, nc, bd = centroids.shape
    return bd == 8 and 1 <= nb <= 16 and 1 <= nc <= 256


def encode_blockvq(keys: torch.Tensor, perm: torch.Tensor | None, centroids: torch.Tensor,
                   out: torch.Tensor, block_dim: int,
                   prepared: torch.Tensor | None = None) -> torch.Tensor:
    """Encode keys of shape (B, H, T, D) or (N, D) into ``out`` (same leading
    shape, last dim n_blocks, uint8; may be a strided view into a cache).
    With ``prepared`` (:func:`encode_codebook` of the same centroids) bulk
    encodes run on the matrix cores; the indices are the same."""
    require_gpu(keys, perm, centroids, out)
    if centroids.dtype != torch.float32 or not centroids.is_contiguous():
        raise ValueError("centroids must be contiguous float32 (n_blocks, n_centroids, block_dim)")
    if out.dtype != torch.uint8:
        raise ValueError("out must be uint8")
    k4 = keys.reshape((1, 1) + tuple(keys.shape)) if keys.dim() == 2 else keys
    o4 = out.reshape((1, 1) + tuple(out.shape)) if out.dim() == 2 else out
    if k4.dim() != 4 or o4.dim() != 4:
        raise ValueError("keys must be (N, D) or (B, H, T, D)")
    if k4.stride(-1) != 1 or o4.stride(-1) != 1:
        raise ValueError("keys and out must be contiguous in their last dimension")
    nb, nc, bd = centroids.shape
    b_, h_, t_, d = k4.shape
    if tuple(o4.shape) != (b_, h_, t_, nb):
        raise ValueError(f"out shape {tuple(out.shape)} does not match keys {tuple(keys.shape)}")
    if perm is not None and (perm.dtype != torch.int32 or perm.numel() != d):
        raise ValueError("perm must be int32 of length head_dim")
    lib = load_library()
    args = (ptr(k4), dtype_code(k4.dtype), b_, h_, t_, k4.stride(0), k4.stride(1), k4.stride(2), d,
            ptr(perm), ptr(centroids), nb, nc, bd, ptr(o4), o4.stride(0), o4.stride(1),
            o4.stride(2))
    if prepared is not None:
        require_gpu(prepared)
        if prepared.dtype != torch.uint8 or prepared.numel() < lib.ss_encode_codebook_bytes(nb):
            raise ValueError("prepared must be the uint8 buffer of encode_codebook(centroids)")
        st = lib.ss_encode_blockvq_prepared(*args, ptr(prepared), stream_handle(keys.device))
    else:
        st = lib.ss_encode_blockvq(*args, stream_handle(keys.device))
    _launched("sunshape_block_vq_quantize_hip", st)
    return out


def build_lut(q: torch.Tensor, perm: torch.Tensor | None, scale: float,
              centroids: torch.Tensor) -> torch.Tensor:
    """(n_rows, D) queries -> (n_rows, n_blocks, n_centroids) float32 LUT."""
    require_gpu(q, perm, centroids)
    if q.dim() != 2 or q.stride(-1) != 1:
        raise ValueError("q must be (n_rows, head_dim) with unit last stride")
    nb, nc, bd = centroids.shape
    lut = torch.empty((q.shape[0], nb, nc), dtype=torch.float32, device=q.device)
    _launched("sunshape_query_centroid_dots_hip", load_library().ss_build_lut(
        ptr(q), dtype_code(q.dtype), q.shape[0], q.stride(0), q.shape[1], ptr(perm), float(scale),
        ptr(centroids), nb, nc, bd, ptr(lut), stream_handle(q.device)))
    return lut


def score_gather(lut: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """lut (R, NB, NC) f32, idx (T, NB) uint8 -> scores (R, T) f32."""
    require_gpu(lut, idx)
    if idx.dtype != torch.uint8 or idx.dim() != 2 or idx.stride(-1) != 1:
        raise ValueError("indices must be uint8 (T, n_blocks) with unit last stride")
    lut = lut.contiguous().float()
    r_, nb, nc = lut.shape
    scores = torch.empty((r_, idx.shape[0]), dtype=torch.float32, device=lut.device)
    _launched("sunshape_block_vq_score_hip", load_library().ss_score_gather(
        ptr(lut), r_, nb, nc, ptr(idx), idx.shape[0], idx.stride(0), ptr(scores), idx.shape[0],
        stream_handle(lut.device)))
    return scores


def score_gather_heads(lut: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """lut (B, H, R, NB, NC) f32, idx (B, H, T, NB) uint8 (a strided view of a
    cache is fine) -> scores (B, H, R, T) f32, one launch for every head."""
    require_gpu(lut, idx)
    if idx.dtype != torch.uint8 or idx.dim() != 4 or idx.stride(-1) != 1:
        raise ValueError("indices must be uint8 (B, H, T, n_blocks) with unit last stride")
    lut = lut.contiguous().float()
    b_, h_, r_, nb, nc = lut.shape
    if tuple(idx.shape[:2]) != (b_, h_) or idx.shape[3] != nb:
        raise ValueError("lut and indices disagree on (B, H, n_blocks)")
    t_ = idx.shape[2]
    scores = torch.empty((b_, h_, r_, t_), dtype=torch.float32, device=lut.device)
    _launched("sunshape_block_vq_score_hip", load_library().ss_score_gather_heads(
        ptr(lut), r_, nb, nc, ptr(idx), b_, h_, idx.stride(0), idx.stride(1), idx.stride(2), t_,
        ptr(scores), stream_handle(lut.device)))
    return scores


def dequantize_blockvq(idx: torch.Tensor, centroids: torch.Tensor, inv_perm: torch.Tensor | None,
                       out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """idx (T, NB) uint8 -> (T, D) reconstructed vectors in the original basis."""
    require_gpu(idx, centroids, inv_perm)
    if idx.dtype != torch.uint8 or idx.dim() != 2 or idx.stride(-1) != 1:
        raise ValueError("indices must be uint8 (T, n_blocks) with unit last stride")
    nb, nc, bd = centroids.shape
    out = torch.empty((idx.shape[0], nb * bd), dtype=out_dtype, device=idx.device)
    _launched("sunshape_block_vq_dequantize_hip", load_library().ss_dequantize_blockvq(
        ptr(idx), idx.shape[0], idx.stride(0), ptr(centroids), nb, nc, bd, ptr(inv_perm), ptr(out),
        dtype_code(out_dtype), stream_handle(idx.device)))
    return out


def decode_workspace_bytes(batch, n_q_heads, n_kv_heads, t_q, head_dim, t_kv, n_splits=0) -> int:
    return int(load_library().ss_decode_workspace_bytes(batch, n_q_heads, n_kv_heads, t_q,
                                                        head_dim, t_kv, n_splits))


def default_splits(batch, n_q_heads, n_kv_heads, t_q, head_dim, t_kv) -> int:
    return int(load_library().ss_decode_default_splits(batch, n_q_heads, n_kv_heads, t_q,
                                                       head_dim, t_kv))


def _check_decode_common(q, idx, centroids, perm):
    require_gpu(q, idx, centroids, perm)
    if q.dim() != 4 or not q.is_contiguous():
        raise ValueError("queries must be contiguous (B, n_q_heads, T_q, D)")
    if idx.dim() != 4 or idx.dtype != torch.uint8 or not idx.is_contiguous():
        raise ValueError("key indices must be a contiguous uint8 (B, n_kv_heads, cap, n_blocks) buffer")
    if centroids is not None and (centroids.dtype != torch.float32 or not centroids.is_contiguous()):
        raise ValueError("centroids must be contiguous float32")
    if perm is not None and perm.dtype != torch.int32:
        raise ValueError("perm must be int32")


def decode_attn_dense(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                      centroids: torch.Tensor, idx: torch.Tensor, values: torch.Tensor,
                      t_kv: int, causal: bool = False, q_offset: int = 0,
                      out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                      n_splits: int = 0, buf_keys: torch.Tensor | None = None,
                      buf_values: torch.Tensor | None = None, buf_len: int = 0) -> torch.Tensor:
    """Fused decode over a (B, Hkv, cap, NB) index buffer and (B, Hkv, cap, D)
    dense values; returns (B, Hq, T_q, D).  A hybrid cache's recent tokens
    ``buf_keys``/``buf_values`` (B, Hkv, >= buf_len, D) join the same
    softmax as positions t_kv .. t_kv + buf_len - 1
    (``ss_decode_attn_dense_hybrid``)."""
    _check_decode_common(q, idx, centroids, perm)
    require_gpu(values)
    if values.dim() != 4 or not values.is_contiguous():
        raise ValueError("values must be a contiguous (B, n_kv_heads, cap, D) buffer")
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if values.shape[:3] != idx.shape[:3] or values.shape[3] != d:
        raise ValueError(f"values {tuple(values.shape)} do not match indices {tuple(idx.shape)}")
    nc = centroids.shape[1]
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    buf_len = int(buf_len)
    if buf_len > 0:
        buf_keys, buf_values, bdt, bsb, bsh, bst = _buffer_args(buf_keys, buf_values, buf_len,
                                                                b_, hkv, d)
        lib = load_library()
        ws_bytes = lib.ss_decode_turboquant_workspace_bytes(b_, hq, hkv, tq, d, int(t_kv),
                                                            buf_len, int(n_splits))
        ws = decode_workspace(q.device, ws_bytes)
        _launched(_attn_stat("sunshape_fused_attention", causal), lib.ss_decode_attn_dense_hybrid(
            ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm),
            ptr(centroids), nb, nc, ptr(idx), ptr(values), dtype_code(values.dtype), cap,
            int(t_kv), ptr(buf_keys), ptr(buf_values), bdt, bsb, bsh, bst, buf_len,
            int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype), ptr(ws),
            ws_bytes if ws is not None else 0, int(n_splits), stream_handle(q.device)))
        return out
    ws_bytes = decode_workspace_bytes(b_, hq, hkv, tq, d, t_kv, n_splits)
    ws = decode_workspace(q.device, ws_bytes)
    _launched(_attn_stat("sunshape_fused_attention", causal), load_library().ss_decode_attn_dense(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(centroids),
        nb, nc, ptr(idx), ptr(values), dtype_code(values.dtype), cap, int(t_kv), int(bool(causal)),
        int(q_offset), ptr(out), dtype_code(out.dtype), ptr(ws), ws_bytes if ws is not None else 0,
        int(n_splits), stream_handle(q.device)))
    return out


KIND_DENSE, KIND_IL8 = 0, 1


def decode_plan(kind, batch, n_q_heads, n_kv_heads, t_q, head_dim, t_kv, n_splits=0):
    """(splits, workspace_bytes) a decode call of ``kind`` would use."""
    sp = _int(0)
    wb = _size(0)
    check(load_library().ss_decode_plan(kind, batch, n_q_heads, n_kv_heads, t_q, head_dim, t_kv,
                                        n_splits, ctypes.byref(sp), ctypes.byref(wb)))
    return int(sp.value), int(wb.value)


def codebook_f16x2(centroids: torch.Tensor) -> torch.Tensor:
    """Split-fp16 codebook (flat uint8 buffer) read by :func:`decode_attn_il8`
    for float32 centroids (n_blocks, n_centroids, 8)."""
    require_gpu(centroids)
    if centroids.dim() != 3 or centroids.dtype != torch.float32 or not centroids.is_contiguous():
        raise ValueError("centroids must be contiguous float32 (n_blocks, n_centroids, 8)")
    nb, nc, _ = centroids.shape
    lib = load_library()
    out = torch.empty(lib.ss_codebook_f16x2_bytes(nb, nc), dtype=torch.uint8,
                      device=centroids.device)
    check(lib.ss_codebook_f16x2(ptr(centroids), nb, nc, ptr(out), stream_handle(centroids.device)))
    return out


def _heavy_args(k_heavy, heavy_dims, b_, hkv, cap, max_dims):
    """(k_heavy, heavy_dims, n) pointers of a mixed-precision codec's fp16
    heavy-block key dims (B, Hkv, cap, n) for the hybrid entry points."""
    if k_heavy is None:
        return None, None, 0
    require_gpu(k_heavy, heavy_dims)
    nhd = int(heavy_dims.numel())
    if k_heavy.dtype != torch.float16 or not k_heavy.is_contiguous() or \
            tuple(k_heavy.shape) != (b_, hkv, cap, nhd) or heavy_dims.dtype != torch.int32:
        raise ValueError(f"k_heavy must be contiguous fp16 {(b_, hkv, cap, nhd)} with int32 "
                         "heavy_dims")
    if nhd % 8 or nhd > max_dims:
        raise SunShapeUnsupported(-2, f"{nhd} heavy dims (a multiple of 8, at most {max_dims})")
    return ptr(k_heavy), ptr(heavy_dims), nhd


def _buffer_ptrs(b_, hkv, d, buf_keys, buf_values, buf_len):
    """The C-ABI buffer arguments (k_buf, v_buf, buf_dtype, buf_sb, buf_sh,
    buf_st, t_buf) of a hybrid cache's buffered tokens."""
    kb, vb, code, sb, sh, st = _buffer_args(buf_keys, buf_values, buf_len, b_, hkv, d)
    return ptr(kb), ptr(vb), code, sb, sh, st, int(buf_len)


def decode_attn_il8(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                    centroids: torch.Tensor, idx: torch.Tensor, values_il8: torch.Tensor,
                    t_kv: int, causal: bool = False, q_offset: int = 0,
                    out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                    n_splits: int = 0, codebook: torch.Tensor | None = None,
                    buf_keys: torch.Tensor | None = None,
                    buf_values: torch.Tensor | None = None, buf_len: int = 0,
                    k_heavy: torch.Tensor | None = None,
                    heavy_dims: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode (matrix-core LUT and P.V) over fp16 values in the 8-token
    interleaved layout ``values_il8`` (B, Hkv, cap/8, D, 8).  ``codebook`` is
    :func:`codebook_f16x2` of ``centroids`` (prepared here when None).  A
    hybrid cache's recent tokens ``buf_keys``/``buf_values`` (B, Hkv,
    >= buf_len, D, original basis) join the same softmax as positions t_kv ..
    t_kv + buf_len - 1, and a mixed-precision codec's fp16 heavy-block key
    dims ``k_heavy`` (B, Hkv, cap, nhd <= 32) with ``heavy_dims`` (nhd,)
    int32 are scored exactly (``ss_decode_attn_il8_hybrid``; the centroids
    must then hold zeros for those blocks)."""
    _check_decode_common(q, idx, centroids, perm)
    if codebook is None:
        codebook = codebook_f16x2(centroids)
    elif codebook.numel() != load_library().ss_codebook_f16x2_bytes(*centroids.shape[:2]):
        raise ValueError("codebook does not match the centroids' shape")
    require_gpu(values_il8)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
            tuple(values_il8.shape) != (b_, hkv, cap // 8, d, 8):
        raise ValueError(f"values_il8 must be contiguous float16 {(b_, hkv, cap // 8, d, 8)}")
    nc = centroids.shape[1]
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    _, ws_bytes = decode_plan(KIND_IL8, b_, hq, hkv, tq, d, t_kv, n_splits)
    ws = decode_workspace(q.device, ws_bytes)
    common = (ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm),
              ptr(codebook), nb, nc, ptr(idx), ptr(values_il8), SS_F16, cap, int(t_kv))
    tail = (int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype), ptr(ws),
            ws_bytes if ws is not None else 0, int(n_splits), stream_handle(q.device))
    stat = _attn_stat("sunshape_fused_attention_mfma", causal)
    heavy = _heavy_args(k_heavy, heavy_dims, b_, hkv, cap, 32)
    _poll_waits(q.device)
    if (buf_keys is None or buf_len == 0) and k_heavy is None:
        _launched(stat, load_library().ss_decode_attn_il8(*common, *tail))
    else:
        buf = _buffer_ptrs(b_, hkv, d, buf_keys, buf_values, buf_len if buf_keys is not None else 0)
        _launched(stat, load_library().ss_decode_attn_il8_hybrid(*common, *buf, *heavy, *tail))
    if _check_waits:
        check_decode_waits(q.device)
    return out


def prefill_attn_il8(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                     codebook: torch.Tensor, n_centroids: int, idx: torch.Tensor,
                     values_il8: torch.Tensor, t_kv: int, causal: bool = True, q_offset: int = 0,
                     out: torch.Tensor | None = None,
                     out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Prompt attention (``ss_prefill_attn_il8``) of queries (B, Hq, T_q,
    128) against an interleaved fp16 cache: keys reconstructed from the
    prepared ``codebook`` (:func:`codebook_f16x2`), Q.K^T and P.V on the
    matrix cores.  Row i of a head sees keys 0 .. q_offset + i when causal."""
    _check_decode_common(q, idx, None, perm)
    require_gpu(values_il8, codebook)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
            tuple(values_il8.shape) != (b_, hkv, cap // 8, d, 8):
        raise ValueError(f"values_il8 must be contiguous float16 {(b_, hkv, cap // 8, d, 8)}")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(nb, n_centroids):
        raise ValueError("codebook does not match the centroids' shape")
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    _launched(_attn_stat("sunshape_prefill_attention_mfma", causal), lib.ss_prefill_attn_il8(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
        nb, int(n_centroids), ptr(idx), ptr(values_il8), SS_F16, cap, int(t_kv),
        int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype),
        stream_handle(q.device)))
    return out


def prefill_attn_il8_hybrid(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                            codebook: torch.Tensor, n_centroids: int, idx: torch.Tensor,
                            values_il8: torch.Tensor, t_kv: int, kraw: torch.Tensor,
                            kfac: torch.Tensor, t_raw0: int, causal: bool = True,
                            q_offset: int = 0, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """:func:`prefill_attn_il8` over a hybrid cache (``ss_prefill_attn_il8_hybrid``):
    positions below ``t_raw0`` scored from ``idx``, the rest from the whole
    keys ``kraw`` (B, Hkv, t_kv - t_raw0, 2, 128) fp16 with factors ``kfac``
    (B, Hkv, t_kv - t_raw0) float32 (:func:`raw_key_rows`); ``values_il8``
    holds all t_kv tokens' values."""
    _check_decode_common(q, idx, None, perm)
    require_gpu(values_il8, codebook, kraw, kfac)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    cap_v = values_il8.shape[2] * 8
    n_raw = int(t_kv) - int(t_raw0)
    if values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
            tuple(values_il8.shape) != (b_, hkv, cap_v // 8, d, 8):
        raise ValueError(f"values_il8 must be contiguous float16 (B, Hkv, cap/8, {d}, 8)")
    if kraw.dtype != torch.float16 or not kraw.is_contiguous() or \
            tuple(kraw.shape) != (b_, hkv, max(n_raw, 1), 2, d) or \
            kfac.dtype != torch.float32 or not kfac.is_contiguous() or \
            tuple(kfac.shape) != (b_, hkv, max(n_raw, 1)):
        raise ValueError("kraw / kfac do not match the buffered tokens")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(nb, n_centroids):
        raise ValueError("codebook does not match the centroids' shape")
    out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    _launched(_attn_stat("sunshape_prefill_attention_mfma", causal), lib.ss_prefill_attn_il8_hybrid(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
        nb, int(n_centroids), ptr(idx), cap, ptr(values_il8), cap_v, int(t_kv), ptr(kraw),
        ptr(kfac), int(t_raw0), int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype),
        stream_handle(q.device)))
    return out


def raw_key_rows(keys: torch.Tensor, perm: torch.Tensor | None = None
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """Whole keys (B, H, T, D) -> (rows, factors) for
    :func:`prefill_attn_il8_hybrid` in one launch (``ss_raw_key_rows``), dim j
    taken from dim ``perm[j]`` of the key (the codec's basis).  Per token s
    brings max |key| * 2^-s into [2^14, 2^15) (s = 0 for a zero key); row 0 =
    fp16(key * 2^-s), row 1 = fp16(key * 2^-s - row 0), factor 2^s.  The
    rows hold the scaled key to 22 bits, exactly for fp16 and bf16 keys (at
    most 11 significant bits, row 1 = 0)."""
    require_gpu(keys)
    if keys.dim() != 4 or keys.stride(-1) != 1:
        raise ValueError("keys must be (B, H, T, D) with unit last stride")
    b_, h_, t_, d = keys.shape
    if perm is not None:
        require_gpu(perm)
        if perm.dtype != torch.int32 or not perm.is_contiguous() or perm.numel() != d:
            raise ValueError(f"perm must be a contiguous int32 vector of {d} entries")
    rows = torch.empty((b_, h_, t_, 2, d), dtype=torch.float16, device=keys.device)
    fac = torch.empty((b_, h_, t_), dtype=torch.float32, device=keys.device)
    check(load_library().ss_raw_key_rows(
        ptr(keys), dtype_code(keys.dtype), b_, h_, t_, keys.stride(0), keys.stride(1),
        keys.stride(2), d, ptr(perm), ptr(rows), ptr(fac), stream_handle(keys.device)))
    return rows, fac


def prefill_supported(n_q_heads: int, n_kv_heads: int, t_q: int, head_dim: int,
                      n_blocks: int) -> bool:
    """Whether :func:`prefill_attn_il8` takes this shape and is the better
    kernel for it (at least one workgroup's worth of positions)."""
    rows = int(load_library().ss_prefill_rows_per_workgroup())
    rep = n_q_heads // n_kv_heads
    return (head_dim == 128 and n_blocks == 16 and rows % rep == 0
            and t_q >= rows // rep)


def decode_attn_il8_noalloc(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                            centroids: torch.Tensor, idx: torch.Tensor, values_il8: torch.Tensor,
                            t_kv: int, out: torch.Tensor, codebook: torch.Tensor,
                            causal: bool = False, q_offset: int = 0,
                            n_splits: int = 0) -> torch.Tensor:
    """:func:`decode_attn_il8` through ``ss_decode_attn_il8_noalloc``: no
    workspace (the library's static per-GPU scratch holds the split
    partials), ``out`` and the prepared ``codebook`` supplied by the caller,
    so the call allocates nothing.  Calls that overlap on one GPU race."""
    _check_decode_common(q, idx, centroids, perm)
    require_gpu(values_il8, out, codebook)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
            tuple(values_il8.shape) != (b_, hkv, cap // 8, d, 8):
        raise ValueError(f"values_il8 must be contiguous float16 {(b_, hkv, cap // 8, d, 8)}")
    if tuple(out.shape) != (b_, hq, tq, d) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous {(b_, hq, tq, d)}")
    lib = load_library()
    if codebook.numel() != lib.ss_codebook_f16x2_bytes(*centroids.shape[:2]):
        raise ValueError("codebook does not match the centroids' shape")
    _poll_waits(q.device)
    _launched(_attn_stat("sunshape_fused_attention_mfma", causal), lib.ss_decode_attn_il8_noalloc(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
        nb, centroids.shape[1], ptr(idx), ptr(values_il8), SS_F16, cap, int(t_kv),
        int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype), int(n_splits),
        stream_handle(q.device)))
    if _check_waits:
        check_decode_waits(q.device)
    return out


def append_values_il8(values: torch.Tensor, out_il8: torch.Tensor, offset: int) -> None:
    """Write (B, H, T, D) values at cache positions [offset, offset+T) of the
    interleaved buffer (B, H, cap/8, D, 8)."""
    require_gpu(values, out_il8)
    if values.dim() != 4 or values.stride(-1) != 1:
        raise ValueError("values must be (B, H, T, D) with unit last stride")
    if out_il8.dim() != 5 or out_il8.dtype != torch.float16 or not out_il8.is_contiguous():
        raise ValueError("out_il8 must be a contiguous float16 (B, H, cap/8, D, 8) buffer")
    b_, h_, t_, d = values.shape
    if tuple(out_il8.shape[:2]) != (b_, h_) or out_il8.shape[3] != d:
        raise ValueError("values and cache shapes differ")
    cap = out_il8.shape[2] * 8
    check(load_library().ss_append_values_il8(
        ptr(values), dtype_code(values.dtype), b_, h_, t_, values.stride(0), values.stride(1),
        values.stride(2), d, ptr(out_il8), cap, int(offset), stream_handle(values.device)))


class PreparedAppend:
    """``ss_append_kv_il8`` into fixed cache buffers: the codebook, the
    permutation and the cache pointers are checked and packed once; a call
    passes the new keys and values (B, H, T, D, unit last stride) and the
    cache offset.  The caller (the cache that built it) keeps the buffers
    alive and builds a new one when they change."""

    __slots__ = ("fn", "mid", "tail", "shape_bh", "d", "cap", "dev")

    def __init__(self, perm: torch.Tensor | None, centroids: torch.Tensor,
                 prepared: torch.Tensor | None, idx_cache: torch.Tensor, values_il8: torch.Tensor):
        require_gpu(centroids, idx_cache, values_il8)
        if centroids.dtype != torch.float32 or not centroids.is_contiguous():
            raise ValueError("centroids must be contiguous float32 (n_blocks, n_centroids, block_dim)")
        nb, nc, bd = centroids.shape
        b_, h_, cap, nb2 = idx_cache.shape
        if nb2 != nb or idx_cache.dtype != torch.uint8 or not idx_cache.is_contiguous():
            raise ValueError("idx_cache must be contiguous uint8 (B, H, cap, n_blocks)")
        if values_il8.dtype != torch.float16 or not values_il8.is_contiguous() or \
                tuple(values_il8.shape) != (b_, h_, cap // 8, nb * bd, 8):
            raise ValueError(f"values_il8 must be contiguous float16 {(b_, h_, cap // 8, nb * bd, 8)}")
        if perm is not None and (perm.dtype != torch.int32 or perm.numel() != nb * bd):
            raise ValueError("perm must be int32 of length head_dim")
        lib = load_library()
        if prepared is not None and (prepared.dtype != torch.uint8 or
                                     prepared.numel() < lib.ss_encode_codebook_bytes(nb)):
            raise ValueError("prepared must be the uint8 buffer of encode_codebook(centroids)")
        self.fn = lib.ss_append_kv_il8
        self.mid = (nb * bd, ptr(perm), ptr(centroids), nb, nc, bd, ptr(prepared))
        self.tail = (ptr(idx_cache), ptr(values_il8), cap)
        self.shape_bh = (b_, h_)
        self.d = nb * bd
        self.cap = cap
        self.dev = device_index(idx_cache.device)

    def __call__(self, keys: torch.Tensor, values: torch.Tensor, offset: int) -> None:
        b_, h_, t_, d = keys.shape
        if (b_, h_) != self.shape_bh or d != self.d or tuple(values.shape) != (b_, h_, t_, d) or \
                keys.stride(3) != 1 or values.stride(3) != 1 or keys.device.index != self.dev or \
                values.device.index != self.dev:
            raise ValueError(f"keys/values must be {self.shape_bh + ('T', self.d)} with unit last "
                             f"stride on cuda:{self.dev}")
        ks, vs = keys.stride(), values.stride()
        rc = self.fn(keys.data_ptr(), dtype_code(keys.dtype), values.data_ptr(),
                     dtype_code(values.dtype), b_, h_, t_, ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
                     *self.mid, *self.tail, int(offset), stream_handle(self.dev))
        _launched("sunshape_block_vq_quantize_hip", rc)


def il8_to_dense(values_il8: torch.Tensor, t_kv: int | None = None) -> torch.Tensor:
    """(B, H, cap/8, D, 8) interleaved -> (B, H, cap, D) token-major copy."""
    b_, h_, c8, d, _ = values_il8.shape
    dense = values_il8.permute(0, 1, 2, 4, 3).reshape(b_, h_, c8 * 8, d)
    return dense[:, :, :t_kv] if t_kv is not None else dense


def decode_attn_grouped(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                        centroids: torch.Tensor, idx: torch.Tensor, packed: torch.Tensor,
                        scales: torch.Tensor, zeros: torch.Tensor, bits: int, group_size: int,
                        t_kv: int, causal: bool = False, q_offset: int = 0,
                        out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                        n_splits: int = 0, buf_keys: torch.Tensor | None = None,
                        buf_values: torch.Tensor | None = None,
                        buf_len: int = 0) -> torch.Tensor:
    """Fused decode with grouped-quantised values decoded in registers.  A
    hybrid cache's recent tokens join the softmax as in
    :func:`decode_attn_dense` (``ss_decode_attn_grouped_hybrid``)."""
    _check_decode_common(q, idx, centroids, perm)
    require_gpu(packed, scales, zeros)
    for name, t in (("packed", packed), ("scales", scales), ("zeros", zeros)):
        if t.dim() != 4 or not t.is_contiguous() or t.shape[:3] != idx.shape[:3]:
            raise ValueError(f"{name} must be a contiguous (B, n_kv_heads, cap, *) buffer")
    if packed.dtype not in (torch.int32, torch.uint32):
        raise ValueError("packed values must be 32-bit words")
    if scales.dtype != zeros.dtype or scales.dtype not in (torch.float32, torch.float16):
        raise ValueError("scales/zeros must share dtype float32 or float16")
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    nc = centroids.shape[1]
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    buf_len = int(buf_len)
    if buf_len > 0:
        buf_keys, buf_values, bdt, bsb, bsh, bst = _buffer_args(buf_keys, buf_values, buf_len,
                                                                b_, hkv, d)
        lib = load_library()
        ws_bytes = lib.ss_decode_turboquant_workspace_bytes(b_, hq, hkv, tq, d, int(t_kv),
                                                            buf_len, int(n_splits))
        ws = decode_workspace(q.device, ws_bytes)
        _launched(_attn_stat("sunshape_fused_attention_dequant", causal),
                  lib.ss_decode_attn_grouped_hybrid(
                      ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm),
                      ptr(centroids), nb, nc, ptr(idx), ptr(packed), ptr(scales), ptr(zeros),
                      dtype_code(scales.dtype), int(bits), int(group_size), cap, int(t_kv),
                      ptr(buf_keys), ptr(buf_values), bdt, bsb, bsh, bst, buf_len,
                      int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype), ptr(ws),
                      ws_bytes if ws is not None else 0, int(n_splits), stream_handle(q.device)))
        return out
    ws_bytes = decode_workspace_bytes(b_, hq, hkv, tq, d, t_kv, n_splits)
    ws = decode_workspace(q.device, ws_bytes)
    _launched(_attn_stat("sunshape_fused_attention_dequant", causal), load_library().ss_decode_attn_grouped(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(centroids),
        nb, nc, ptr(idx), ptr(packed), ptr(scales), ptr(zeros), dtype_code(scales.dtype),
        int(bits), int(group_size), cap, int(t_kv), int(bool(causal)), int(q_offset), ptr(out),
        dtype_code(out.dtype), ptr(ws), ws_bytes if ws is not None else 0, int(n_splits),
        stream_handle(q.device)))
    return out


def kmeans_blocks(data: torch.Tensor, init: torch.Tensor, iters: int,
                  return_assign: bool = False):
    """Lloyd k-means of every block at once: ``data`` (n_blocks, n, bd)
    float32, ``init`` (n_blocks, K, bd) float32 initial centroids.  Returns
    the fitted centroids (and the final uint8 assignments (n_blocks, n))."""
    require_gpu(data, init)
    if data.dim() != 3 or init.dim() != 3 or data.shape[0] != init.shape[0] or \
            data.shape[2] != init.shape[2]:
        raise ValueError("data (n_blocks, n, bd) and init (n_blocks, K, bd) must agree")
    data = data.float().contiguous()
    cents = init.float().contiguous().clone()
    nb, n, bd = data.shape
    k = cents.shape[1]
    assign = torch.empty((nb, n), dtype=torch.uint8, device=data.device) if return_assign else None
    _launched("sunshape_kmeans_hip", load_library().ss_kmeans_blocks(ptr(data), nb, n, bd, k, int(iters), ptr(cents),
                                          ptr(assign), stream_handle(data.device)))
    return (cents, assign) if return_assign else cents


def _buffer_args(buf_keys, buf_values, buf_len: int, b_: int, hkv: int, d: int):
    """(keys, values, dtype code, strides) of a hybrid buffer for the
    transformed-basis decodes; Nones and zeros when nothing is buffered."""
    if buf_len <= 0:
        return None, None, 0, 0, 0, 0
    require_gpu(buf_keys, buf_values)
    for name, tb in (("buf_keys", buf_keys), ("buf_values", buf_values)):
        if tb.dim() != 4 or tb.shape[0] != b_ or tb.shape[1] != hkv or tb.shape[3] != d or \
                tb.shape[2] < buf_len or tb.stride(3) != 1:
            raise ValueError(f"{name} must be (B, n_kv_heads, >= {buf_len}, {d}) with unit "
                             "element stride")
    if buf_keys.stride() != buf_values.stride() or buf_keys.dtype != buf_values.dtype:
        raise ValueError("buffer keys and values must share dtype and strides")
    bsb, bsh, bst = buf_keys.stride()[:3]
    return buf_keys, buf_values, dtype_code(buf_keys.dtype), bsb, bsh, bst


def decode_attn_sunshape_v(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                           centroids: torch.Tensor, idx: torch.Tensor, v_idx: torch.Tensor,
                           v_centroids: torch.Tensor, v_transform: torch.Tensor, t_kv: int,
                           causal: bool = False, q_offset: int = 0,
                           out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                           n_splits: int = 0, buf_keys: torch.Tensor | None = None,
                           buf_values: torch.Tensor | None = None,
                           buf_len: int = 0, k_heavy: torch.Tensor | None = None,
                           heavy_dims: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode over SunShape block-VQ values: ``v_idx`` (B, Hkv, cap,
    D / bd) uint8, ``v_centroids`` (D / bd, nc, bd) float32, ``v_transform``
    (D, D) float32 taking a codec-space row to the original basis.  Buffered
    tokens join the softmax as in :func:`decode_attn_turboquant`.
    ``k_heavy`` (B, Hkv, cap, nhd) fp16 with ``heavy_dims`` (nhd,) int32: a
    mixed-precision codec's heavy-block key dims, scored exactly."""
    _check_decode_common(q, idx, centroids, perm)
    require_gpu(v_idx, v_centroids, v_transform)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if v_centroids.dim() != 3 or v_centroids.dtype != torch.float32 or \
            not v_centroids.is_contiguous():
        raise ValueError("v_centroids must be contiguous float32 (n_blocks, n_centroids, block_dim)")
    nbv, vnc, vbd = v_centroids.shape
    if nbv * vbd != d:
        raise ValueError(f"value codebook covers {nbv * vbd} dims, head_dim is {d}")
    if v_idx.dtype != torch.uint8 or v_idx.dim() != 4 or not v_idx.is_contiguous() or \
            tuple(v_idx.shape) != (b_, hkv, cap, nbv):
        raise ValueError(f"v_idx must be contiguous uint8 {(b_, hkv, cap, nbv)}")
    if v_transform.dtype != torch.float32 or not v_transform.is_contiguous() or \
            tuple(v_transform.shape) != (d, d):
        raise ValueError(f"v_transform must be contiguous float32 ({d}, {d})")
    nc = centroids.shape[1]
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    nhd = 0
    if k_heavy is not None:
        require_gpu(k_heavy, heavy_dims)
        nhd = int(heavy_dims.numel())
        if k_heavy.dtype != torch.float16 or not k_heavy.is_contiguous() or \
                tuple(k_heavy.shape) != (b_, hkv, cap, nhd) or heavy_dims.dtype != torch.int32:
            raise ValueError(f"k_heavy must be contiguous fp16 {(b_, hkv, cap, nhd)} with int32 "
                             "heavy_dims")
    buf_len = int(buf_len)
    buf_keys, buf_values, bdt, bsb, bsh, bst = _buffer_args(buf_keys, buf_values, buf_len,
                                                            b_, hkv, d)
    lib = load_library()
    ws_bytes = lib.ss_decode_turboquant_workspace_bytes(b_, hq, hkv, tq, d, int(t_kv), buf_len,
                                                        int(n_splits))
    ws = decode_workspace(q.device, ws_bytes)
    _launched(_attn_stat("sunshape_fused_attention_sunshape_v", causal), lib.ss_decode_attn_sunshape_v(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(centroids),
        nb, nc, ptr(idx), ptr(v_idx), ptr(v_centroids), vbd, vnc, ptr(v_transform),
        ptr(k_heavy), ptr(heavy_dims), nhd, cap,
        int(t_kv), ptr(buf_keys), ptr(buf_values), bdt, bsb, bsh, bst, buf_len,
        int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype), ptr(ws),
        ws_bytes if ws is not None else 0, int(n_splits), stream_handle(q.device)))
    return out


def decode_attn_turboquant(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                           centroids: torch.Tensor, idx: torch.Tensor, packed: torch.Tensor,
                           norms: torch.Tensor, levels, rotation: torch.Tensor, bits: int,
                           t_kv: int, causal: bool = False, q_offset: int = 0,
                           out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                           n_splits: int = 0, buf_keys: torch.Tensor | None = None,
                           buf_values: torch.Tensor | None = None,
                           buf_len: int = 0, k_heavy: torch.Tensor | None = None,
                           heavy_dims: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode over TurboQuant values: ``packed`` (B, Hkv, cap,
    packed_dim) codes, ``norms`` (B, Hkv, cap) float32, ``levels`` the 2^bits
    scaled Lloyd-Max levels (any float sequence; copied to the kernel
    arguments), ``rotation`` (D, D) float32 with ``value = norm * (levels[code]
    @ rotation)``.  A hybrid cache's recent tokens ``buf_keys``/``buf_values``
    (B, Hkv, >= buf_len, D, original basis) join the same softmax as
    positions t_kv .. t_kv + buf_len - 1."""
    _check_decode_common(q, idx, centroids, perm)
    require_gpu(packed, norms, rotation)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if packed.dim() != 4 or not packed.is_contiguous() or packed.shape[:3] != idx.shape[:3] or \
            packed.dtype not in (torch.int32, torch.uint32):
        raise ValueError("packed must be contiguous 32-bit words (B, n_kv_heads, cap, packed_dim)")
    if norms.dtype != torch.float32 or not norms.is_contiguous() or \
            tuple(norms.shape) != tuple(idx.shape[:3]):
        raise ValueError("norms must be contiguous float32 (B, n_kv_heads, cap)")
    if rotation.dtype != torch.float32 or not rotation.is_contiguous() or \
            tuple(rotation.shape) != (d, d):
        raise ValueError(f"rotation must be contiguous float32 ({d}, {d})")
    lv = [float(x) for x in (levels.tolist() if isinstance(levels, torch.Tensor) else levels)]
    if len(lv) != (1 << int(bits)):
        raise ValueError(f"{1 << int(bits)} levels expected for {bits}-bit codes, got {len(lv)}")
    lv_host = (ctypes.c_float * len(lv))(*lv)
    nc = centroids.shape[1]
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    buf_len = int(buf_len)
    buf_keys, buf_values, bdt, bsb, bsh, bst = _buffer_args(buf_keys, buf_values, buf_len,
                                                            b_, hkv, d)
    lib = load_library()
    ws_bytes = lib.ss_decode_turboquant_workspace_bytes(b_, hq, hkv, tq, d, int(t_kv), buf_len,
                                                        int(n_splits))
    ws = decode_workspace(q.device, ws_bytes)
    _launched(_attn_stat("sunshape_fused_attention_turboquant", causal), lib.ss_decode_attn_turboquant(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(centroids),
        nb, nc, ptr(idx), ptr(packed), ptr(norms), ctypes.cast(lv_host, ctypes.c_void_p).value,
        ptr(rotation), int(bits), cap, int(t_kv), ptr(buf_keys), ptr(buf_values), bdt, bsb, bsh,
        bst, buf_len, *_heavy_args(k_heavy, heavy_dims, b_, hkv, cap, 64), int(bool(causal)), int(q_offset), ptr(out), dtype_code(out.dtype), ptr(ws),
        ws_bytes if ws is not None else 0, int(n_splits), stream_handle(q.device)))
    return out


def turboquant_il_levels_ok(levels) -> bool:
    """Whether a 2-bit level table is affine in the code bits (what the
    matrix-core TurboQuant decode needs): L3 = L2 + L1 - L0."""
    lv = [float(x) for x in (levels.tolist() if isinstance(levels, torch.Tensor) else levels)]
    return len(lv) == 4 and abs(lv[3] - (lv[2] + lv[1] - lv[0])) <= 1e-6 * max(abs(lv[0]),
                                                                               abs(lv[3]), 1e-30)


def decode_attn_turboquant_il(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                              centroids: torch.Tensor, idx: torch.Tensor, codes_il: torch.Tensor,
                              norms: torch.Tensor, levels, rotation: torch.Tensor, t_kv: int,
                              causal: bool = False, q_offset: int = 0,
                              out: torch.Tensor | None = None,
                              out_dtype: torch.dtype | None = None, n_splits: int = 0,
                              codebook: torch.Tensor | None = None,
                              buf_keys: torch.Tensor | None = None,
                              buf_values: torch.Tensor | None = None,
                              buf_len: int = 0, k_heavy: torch.Tensor | None = None,
                              heavy_dims: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode (matrix-core LUT and P.V) over 2-bit TurboQuant values
    whose codes are token-interleaved (``codes_il`` (B, Hkv, cap/16, D) words,
    written by :func:`pack_grouped_il`), ``norms`` (B, Hkv, cap) float32,
    ``levels`` the four scaled Lloyd-Max levels (affine in the code bits),
    ``rotation`` (D, D) with ``value = norm * (levels[code] @ rotation)``.
    ``codebook``: :func:`codebook_f16x2` of ``centroids`` (built if None).
    A hybrid cache's recent tokens join the softmax as in
    :func:`decode_attn_turboquant`."""
    _check_decode_common(q, idx, centroids, perm)
    require_gpu(codes_il, norms, rotation)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    if codes_il.dim() != 4 or not codes_il.is_contiguous() or \
            tuple(codes_il.shape) != (b_, hkv, cap // 16, d) or \
            codes_il.dtype not in (torch.int32, torch.uint32):
        raise ValueError("codes_il must be contiguous 32-bit words (B, n_kv_heads, cap/16, D)")
    if norms.dtype != torch.float32 or not norms.is_contiguous() or \
            tuple(norms.shape) != tuple(idx.shape[:3]):
        raise ValueError("norms must be contiguous float32 (B, n_kv_heads, cap)")
    if rotation.dtype != torch.float32 or not rotation.is_contiguous() or \
            tuple(rotation.shape) != (d, d):
        raise ValueError(f"rotation must be contiguous float32 ({d}, {d})")
    lv = [float(x) for x in (levels.tolist() if isinstance(levels, torch.Tensor) else levels)]
    if len(lv) != 4:
        raise ValueError(f"4 levels expected for 2-bit codes, got {len(lv)}")
    lv_host = (ctypes.c_float * 4)(*lv)
    nc = centroids.shape[1]
    if codebook is None:
        codebook = codebook_f16x2(centroids)
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    buf_len = int(buf_len)
    buf_keys, buf_values, bdt, bsb, bsh, bst = _buffer_args(buf_keys, buf_values, buf_len,
                                                            b_, hkv, d)
    lib = load_library()
    ws_bytes = lib.ss_decode_turboquant_workspace_bytes(b_, hq, hkv, tq, d, int(t_kv), buf_len,
                                                        int(n_splits))
    ws = decode_workspace(q.device, ws_bytes)
    _poll_waits(q.device)
    _launched(_attn_stat("sunshape_fused_attention_turboquant", causal),
              lib.ss_decode_attn_turboquant_il(
        ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm), ptr(codebook),
        nb, nc, ptr(idx), ptr(codes_il), ptr(norms), ctypes.cast(lv_host, ctypes.c_void_p).value,
        ptr(rotation), cap, int(t_kv), ptr(buf_keys), ptr(buf_values), bdt, bsb, bsh,
        bst, buf_len, *_heavy_args(k_heavy, heavy_dims, b_, hkv, cap, 32), int(bool(causal)),
        int(q_offset), ptr(out), dtype_code(out.dtype), ptr(ws),
        ws_bytes if ws is not None else 0, int(n_splits), stream_handle(q.device)))
    if _check_waits:
        check_decode_waits(q.device)
    return out


def decode_attn_grouped_il(q: torch.Tensor, scale: float, perm: torch.Tensor | None,
                           centroids: torch.Tensor, idx: torch.Tensor, codes_il: torch.Tensor,
                           scales: torch.Tensor, zeros: torch.Tensor, bits: int, group_size: int,
                           t_kv: int, causal: bool = False, q_offset: int = 0,
                           out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                           n_splits: int = 0, codebook: torch.Tensor | None = None,
                           buf_keys: torch.Tensor | None = None,
                           buf_values: torch.Tensor | None = None,
                           buf_len: int = 0, k_heavy: torch.Tensor | None = None,
                           heavy_dims: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode (matrix-core LUT and P.V) over grouped values whose codes
    are token-interleaved: ``codes_il`` (B, Hkv, cap * bits / 32, D) 32-bit
    words (see :func:`pack_grouped_il`), ``scales``/``zeros`` (B, Hkv, cap, D
    / group_size).  ``codebook`` is :func:`codebook_f16x2` of ``centroids``
    (prepared here when None).  A hybrid cache's recent tokens
    ``buf_keys``/``buf_values`` (B, Hkv, >= buf_len, D, original basis)
    join the same softmax as positions t_kv .. t_kv + buf_len - 1."""
    _check_decode_common(q, idx, centroids, perm)
    require_gpu(codes_il, scales, zeros)
    b_, hq, tq, d = q.shape
    _, hkv, cap, nb = idx.shape
    tpw = 32 // bits if bits in (2, 4) else 0
    if not tpw or codes_il.dim() != 4 or not codes_il.is_contiguous() or \
            tuple(codes_il.shape) != (b_, hkv, cap // tpw, d) or \
            codes_il.dtype not in (torch.int32, torch.uint32):
        raise ValueError(f"codes_il must be contiguous 32-bit words {(b_, hkv, cap // max(tpw, 1), d)}")
    for name, t in (("scales", scales), ("zeros", zeros)):
        if t.dim() != 4 or not t.is_contiguous() or t.shape[:3] != idx.shape[:3]:
            raise ValueError(f"{name} must be a contiguous (B, n_kv_heads, cap, n_groups) buffer")
    if scales.dtype != zeros.dtype or scales.dtype not in (torch.float32, torch.float16):
        raise ValueError("scales/zeros must share dtype float32 or float16")
    if codebook is None:
        codebook = codebook_f16x2(centroids)
    nc = centroids.shape[1]
    if out is None:
        out = torch.empty((b_, hq, tq, d), dtype=out_dtype or q.dtype, device=q.device)
    _, ws_bytes = decode_plan(KIND_IL8, b_, hq, hkv, tq, d, t_kv, n_splits)
    ws = decode_workspace(q.device, ws_bytes)
    common = (ptr(q), dtype_code(q.dtype), b_, hq, hkv, tq, d, float(scale), ptr(perm),
              ptr(codebook), nb, nc, ptr(idx), ptr(codes_il), ptr(scales), ptr(zeros),
              dtype_code(scales.dtype), int(bits), int(group_size), cap, int(t_kv))
    tail = (ptr(out), dtype_code(out.dtype), ptr(ws), ws_bytes if ws is not None else 0,
            int(n_splits), stream_handle(q.device))
    heavy = _heavy_args(k_heavy, heavy_dims, b_, hkv, cap, 32)
    _poll_waits(q.device)
    if (buf_keys is None or buf_len == 0) and k_heavy is None:
        _launched(_attn_stat("sunshape_fused_attention_dequant_mfma", causal), load_library().ss_decode_attn_grouped_il(
            *common, int(bool(causal)), int(q_offset), *tail))
        if _check_waits:
            check_decode_waits(q.device)
        return out
    buf = _buffer_ptrs(b_, hkv, d, buf_keys, buf_values, buf_len if buf_keys is not None else 0)
    _launched(_attn_stat("sunshape_fused_attention_dequant_mfma", causal), load_library().ss_decode_attn_grouped_il_hybrid(
        *common, *buf, *heavy, int(bool(causal)), int(q_offset), *tail))
    if _check_waits:
        check_decode_waits(q.device)
    return out


def pack_grouped_il(packed: torch.Tensor, bits: int, codes_il: torch.Tensor, offset: int) -> None:
    """Write the codes of reference-layout packed rows (B, H, T, D*bits/32)
    at cache positions [offset, offset + T) of the token-interleaved buffer
    (B, H, cap*bits/32, D); codes of other tokens sharing a word are kept."""
    require_gpu(packed, codes_il)
    if packed.dim() != 4 or packed.stride(-1) != 1:
        raise ValueError("packed must be (B, H, T, words) with unit last stride")
    if codes_il.dim() != 4 or not codes_il.is_contiguous():
        raise ValueError("codes_il must be a contiguous (B, H, cap*bits/32, D) buffer")
    b_, h_, t_, nw = packed.shape
    d = codes_il.shape[3]
    cap = codes_il.shape[2] * (32 // bits)
    if tuple(codes_il.shape[:2]) != (b_, h_) or nw * (32 // bits) != d:
        raise ValueError("packed rows and interleaved buffer shapes differ")
    check(load_library().ss_pack_grouped_il(
        ptr(packed), b_, h_, t_, packed.stride(0) // nw, packed.stride(1) // nw,
        packed.stride(2) // nw, d, int(bits), ptr(codes_il), cap, int(offset),
        stream_handle(packed.device)))


def grouped_il_to_packed(codes_il: torch.Tensor, bits: int, t: int | None = None) -> torch.Tensor:
    """(B, H, cap*bits/32, D) token-interleaved codes -> reference-layout
    packed rows (B, H, t, D*bits/32) uint32 of the first ``t`` tokens (all
    cap when None), one launch (``ss_grouped_il_to_packed``)."""
    require_gpu(codes_il)
    if codes_il.dim() != 4 or not codes_il.is_contiguous() or \
            codes_il.dtype not in (torch.int32, torch.uint32):
        raise ValueError("codes_il must be a contiguous 32-bit (B, H, cap*bits/32, D) buffer")
    b_, h_, nblk, d = codes_il.shape
    cap = nblk * (32 // bits)
    t = cap if t is None else int(t)
    out = torch.empty((b_, h_, t, d * bits // 32), dtype=torch.int32, device=codes_il.device)
    check(load_library().ss_grouped_il_to_packed(ptr(codes_il), b_ * h_, cap, d, int(bits), t,
                                                 ptr(out), stream_handle(codes_il.device)))
    return out.view(torch.uint32) if hasattr(torch, "uint32") else out


def grouped_il_to_il8(codes_il: torch.Tensor, bits: int, group_size: int, scales: torch.Tensor,
                      zeros: torch.Tensor, t: int, out_il8: torch.Tensor) -> None:
    """Dequantise the first ``t`` tokens of interleaved codes (scales/zeros
    (B, H, cap, n_groups), float16 or float32, contiguous) straight into the
    8-token interleaved fp16 buffer (B, H, cap_out/8, D, 8) at positions
    [0, t), one launch (``ss_grouped_il_to_il8``); v = fp16(q * scale + zero)
    as :func:`dequantize_values_grouped` then a cast.  Positions past t in
    the last 8-token group are set to zero."""
    require_gpu(codes_il, scales, zeros, out_il8)
    if codes_il.dim() != 4 or not codes_il.is_contiguous():
        raise ValueError("codes_il must be a contiguous (B, H, cap*bits/32, D) buffer")
    b_, h_, nblk, d = codes_il.shape
    cap = nblk * (32 // bits)
    if scales.dtype != zeros.dtype or scales.shape != zeros.shape or \
            not scales.is_contiguous() or not zeros.is_contiguous() or \
            tuple(scales.shape[:2]) != (b_, h_) or scales.shape[3] * group_size != d:
        raise ValueError("scales/zeros must be contiguous (B, H, cap, D/group_size) of one dtype")
    if out_il8.dtype != torch.float16 or not out_il8.is_contiguous() or out_il8.dim() != 5 or \
            tuple(out_il8.shape[:2]) != (b_, h_) or tuple(out_il8.shape[3:]) != (d, 8):
        raise ValueError(f"out_il8 must be a contiguous float16 (B, H, cap/8, {d}, 8) buffer")
    check(load_library().ss_grouped_il_to_il8(
        ptr(codes_il), b_ * h_, cap, d, int(bits), int(group_size), ptr(scales), ptr(zeros),
        dtype_code(scales.dtype), scales.shape[2], int(t), ptr(out_il8), out_il8.shape[2] * 8,
        stream_handle(codes_il.device)))


def quantize_values_grouped(values: torch.Tensor, bits: int, group_size: int,
                            packed: torch.Tensor, scales: torch.Tensor,
                            zeros: torch.Tensor) -> None:
    """values (B, H, T, D) (or (T, D)) -> packed/scales/zeros views of matching
    leading shape (token rows contiguous in their last dim)."""
    require_gpu(values, packed, scales, zeros)
    v4 = values.reshape((1, 1) + tuple(values.shape)) if values.dim() == 2 else values
    outs = []
    for t in (packed, scales, zeros):
        t4 = t.reshape((1, 1) + tuple(t.shape)) if t.dim() == 2 else t
        if t4.stride(-1) != 1:
            raise ValueError("outputs must be contiguous in their last dimension")
        outs.append(t4)
    p4, s4, z4 = outs
    if v4.stride(-1) != 1:
        raise ValueError("values must be contiguous in their last dimension")
    if s4.dtype != z4.dtype:
        raise ValueError("scales and zeros must share a dtype")
    b_, h_, t_, d = v4.shape
    nw = p4.shape[-1]
    ng = s4.shape[-1]
    # token-row strides of the outputs, in tokens
    o_sb, o_sh, o_st = p4.stride(0) // nw, p4.stride(1) // nw, p4.stride(2) // nw
    if (s4.stride(0) // ng, s4.stride(1) // ng, s4.stride(2) // ng) != (o_sb, o_sh, o_st):
        raise ValueError("packed and scales/zeros buffers must share the token layout")
    _launched("sunshape_quantize_values_hip", load_library().ss_quantize_values_grouped(
        ptr(v4), dtype_code(v4.dtype), b_, h_, t_, v4.stride(0), v4.stride(1), v4.stride(2), d,
        int(bits), int(group_size), ptr(p4), ptr(s4), ptr(z4), dtype_code(s4.dtype), o_sb, o_sh,
        o_st, stream_handle(values.device)))


def dequantize_values_grouped(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                              head_dim: int, bits: int, group_size: int,
                              out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    require_gpu(packed, scales, zeros)
    p2 = packed.reshape(-1, packed.shape[-1]).contiguous()
    s2 = scales.reshape(-1, scales.shape[-1]).contiguous()
    z2 = zeros.reshape(-1, zeros.shape[-1]).to(s2.dtype).contiguous()
    n = p2.shape[0]
    out = torch.empty((n, head_dim), dtype=out_dtype, device=packed.device)
    check(load_library().ss_dequantize_values_grouped(
        ptr(p2), ptr(s2), ptr(z2), dtype_code(s2.dtype), n, head_dim, int(bits), int(group_size),
        ptr(out), dtype_code(out_dtype), stream_handle(packed.device)))
    return out.reshape(tuple(packed.shape[:-1]) + (head_dim,))


def pack_indices(indices: torch.Tensor, bits: int) -> torch.Tensor:
    require_gpu(indices)
    d = indices.shape[-1]
    x = indices.reshape(-1, d).to(torch.uint8).contiguous()
    vpw = 32 // bits
    nw = (d + vpw - 1) // vpw
    out = torch.empty((x.shape[0], nw), dtype=torch.int32, device=indices.device)
    check(load_library().ss_pack_indices(ptr(x), x.shape[0], d, int(bits), ptr(out),
                                         stream_handle(indices.device)))
    return out.view(torch.uint32).reshape(tuple(indices.shape[:-1]) + (nw,))


def unpack_indices(packed: torch.Tensor, d: int, bits: int) -> torch.Tensor:
    require_gpu(packed)
    nw = packed.shape[-1]
    x = packed.reshape(-1, nw).contiguous()
    out = torch.empty((x.shape[0], d), dtype=torch.int32, device=packed.device)
    check(load_library().ss_unpack_indices(ptr(x), x.shape[0], int(d), int(bits), ptr(out),
                                           stream_handle(packed.device)))
    return out.view(torch.uint32).reshape(tuple(packed.shape[:-1]) + (d,))


def scalar_quantize(values: torch.Tensor, boundaries: torch.Tensor) -> torch.Tensor:
    require_gpu(values, boundaries)
    v = values.reshape(-1).float().contiguous()
    b = boundaries.reshape(-1).float().contiguous()
    out = torch.empty(v.shape, dtype=torch.uint8, device=values.device)
    _launched("sunshape_scalar_quantize_hip", load_library().ss_scalar_quantize(ptr(v), v.numel(), ptr(b), b.numel(), ptr(out),
                                            stream_handle(values.device)))
    return out.reshape(values.shape)
