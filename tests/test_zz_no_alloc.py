"""ss_decode_attn_il8_noalloc (the allocation-free variant of the
matrix-core fp16-value decode) against ss_decode_attn_il8 through the C ABI:
identical outputs on two calls in a row, the second with a smaller input
(the static scratch keeps the first call's contents), both within the
oracle's 1e-3 bar; shapes whose split scratch exceeds the static array are
rejected before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import sunshape_oracle as O
from sunshape_mlx_amd import _hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _il8(vals, cap):
    b, h, _, d = vals.shape
    v = np.zeros((b, h, cap, d), np.float16)
    v[:, :, :vals.shape[2]] = vals
    return _t(v.reshape(b, h, cap // 8, 8, d).transpose(0, 1, 2, 4, 3))


def _case(seed, b, hq, hkv, d, t_kv, t_q):
    rng = np.random.default_rng(seed)
    cents = rng.standard_normal((d // 8, 256, 8)).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    idx = rng.integers(0, 256, (b, hkv, t_kv, d // 8)).astype(np.uint8)
    vals = rng.standard_normal((b, hkv, t_kv, d)).astype(np.float16)
    q = rng.standard_normal((b, hq, t_q, d)).astype(np.float16)
    return cents, perm, idx, vals, q


def test_noalloc_decode_matches_workspace_entry_point():
    lib = _hip.load_library()
    assert lib.ss_decode_static_scratch_bytes() == 4 << 20
    cases = [  # seed, B, Hq, Hkv, D, T_kv, T_q (causal rows when > 1), splits
        (11, 2, 32, 8, 128, 32768, 1, 0),  # many splits: partials fill the static scratch
        (12, 1, 8, 2, 128, 1000, 3, 0),    # smaller input on the same scratch
    ]
    for seed, b, hq, hkv, d, t_kv, t_q, splits in cases:
        print(f"no-alloc case seed={seed} B={b} Hq={hq} Hkv={hkv} D={d} T={t_kv} Tq={t_q}",
              flush=True)
        cents, perm, idx, vals, q = _case(seed, b, hq, hkv, d, t_kv, t_q)
        causal = t_q > 1
        c_t = _t(cents)
        cb = _hip.codebook_f16x2(c_t)
        args = (_t(q), 1.0 / np.sqrt(d), _t(perm), c_t, _t(idx), _il8(vals, t_kv), t_kv)
        kw = dict(causal=causal, q_offset=t_kv - t_q if causal else 0, n_splits=splits)
        ref_out = _hip.decode_attn_il8(*args, out_dtype=torch.float32, codebook=cb, **kw)
        out = torch.full_like(ref_out, float("nan"))
        _hip.decode_attn_il8_noalloc(*args, out=out, codebook=cb, **kw)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out)
        ref = O.sdpa(q, idx, vals, cents, perm, 1.0 / np.sqrt(d),
                     mask="causal" if causal else None)
        got = out.cpu().numpy()
        assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max()


def test_noalloc_rejects_shapes_beyond_the_static_scratch():
    lib = _hip.load_library()
    # B=16, 8 KV heads, 512 splits over T=131072: 136 MB of split partials
    rc = lib.ss_decode_attn_il8_noalloc(None, _hip.SS_F16, 16, 32, 8, 1, 128, 1.0, None, None,
                                        16, 256, None, None, _hip.SS_F16, 131072, 131072, 0, 0,
                                        None, _hip.SS_F16, 512, None)
    assert rc == _hip.SS_ERR_WORKSPACE
    assert "static scratch" in lib.ss_last_error().decode()
