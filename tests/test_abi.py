"""CPU checks of the C-ABI boundary and the host logic (no GPU, no kernel
launches): the shared library loads and exports every function that
``include/sunshape_hip.h`` declares, each with a ctypes signature in the
Python binding; status codes match the header; the SDPA router's error
behaviour without any target module matches the reference (patch.py:77-88).
"""

import os
import re

import pytest

import sunshape_mlx_amd as S
from sunshape_mlx_amd import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sunshape_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ss_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("ss_encode_blockvq", "ss_build_lut", "ss_score_gather", "ss_decode_attn_dense",
                 "ss_decode_attn_il8", "ss_decode_attn_grouped", "ss_decode_plan",
                 "ss_append_values_il8", "ss_quantize_values_grouped", "ss_pack_indices",
                 "ss_version", "ss_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _hip.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_every_declared_symbol_has_a_binding_signature():
    unbound = [n for n in declared_functions() if n not in _hip._SIGNATURES]
    assert not unbound, unbound


def test_version_and_status_codes():
    assert _hip.version().startswith("sunshape_hip")
    text = open(HEADER).read()
    codes = dict((k, int(v)) for k, v in re.findall(r"#define (SS_\w+)\s+\(?(-?\d+)\)?", text))
    assert codes["SS_OK"] == 0 and codes["SS_ERR_INVALID"] == -1
    assert codes["SS_ERR_UNSUPPORTED"] == -2 and codes["SS_F16"] == _hip.SS_F16


def test_router_apply_without_targets_raises_and_stays_unpatched():
    assert not S.patch.is_patched()
    with pytest.raises(RuntimeError):
        S.patch.apply()
    assert not S.patch.is_patched()
    S.patch.revert()  # no-op when not patched
    assert not S.patch.is_patched()


def test_product_path_refuses_cpu_tensors():
    import torch

    with pytest.raises(ValueError, match="no CPU fallback"):
        _hip.require_gpu(torch.zeros(4))
