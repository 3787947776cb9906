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
        (11, 2, 32, 8, 128, 32768, 1, 0),  # the default split plan
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


def _splits_at_the_limit(b, hq, hkv, tq, d):
    """((S, T, bytes) under, (S, T, bytes) over): the largest split count
    whose partials fit the static array and the smallest that does not, each
    with a cache length T = 256 S (four tiles per split, so the plan takes
    exactly S), by the library's own sizing."""
    cap = _hip.load_library().ss_decode_static_scratch_bytes()
    under = over = None
    for s in range(2, 512):
        got, need = _hip.decode_plan(_hip.KIND_IL8, b, hq, hkv, tq, d, 256 * s, s)
        if got != s:
            continue
        if need <= cap:
            under = (s, 256 * s, need)
        elif over is None:
            over = (s, 256 * s, need)
    assert under is not None and over is not None
    return under, over


def test_noalloc_at_the_static_scratch_limit():
    """A split plan whose partials need just under the 4 MiB static array
    (within one split's share) runs and matches the workspace entry point
    bit for bit; the next split count, just over it, is rejected with
    SS_ERR_WORKSPACE before anything is launched."""
    b, hq, hkv, d = 2, 32, 8, 128
    (s_in, t_in, need_in), (s_out, t_out, need_out) = _splits_at_the_limit(b, hq, hkv, 1, d)
    cap = _hip.load_library().ss_decode_static_scratch_bytes()
    assert cap - need_in < 64 * 1024 and need_out > cap  # within one split of the limit
    print(f"no-alloc limit: {s_in} splits (T={t_in}) need {need_in} B, "
          f"{s_out} splits (T={t_out}) {need_out} B of {cap}", flush=True)
    for seed, s_, t_kv, fits in ((13, s_in, t_in, True), (14, s_out, t_out, False)):
        cents, perm, idx, vals, q = _case(seed, b, hq, hkv, d, t_kv, 1)
        c_t = _t(cents)
        cb = _hip.codebook_f16x2(c_t)
        args = (_t(q), 1.0 / np.sqrt(d), _t(perm), c_t, _t(idx), _il8(vals, t_kv), t_kv)
        ref_out = _hip.decode_attn_il8(*args, out_dtype=torch.float32, codebook=cb, n_splits=s_)
        out = torch.full_like(ref_out, float("nan"))
        if fits:
            _hip.decode_attn_il8_noalloc(*args, out=out, codebook=cb, n_splits=s_)
            torch.cuda.synchronize()
            assert torch.equal(out, ref_out)
        else:
            with pytest.raises(_hip.SunShapeHIPError) as err:
                _hip.decode_attn_il8_noalloc(*args, out=out, codebook=cb, n_splits=s_)
            assert err.value.status == _hip.SS_ERR_WORKSPACE
            assert torch.isnan(out).all()  # nothing launched


def test_noalloc_replays_under_graph_capture():
    """After one eager call (the per-device set-up: the scratch's device
    address and its zero fill), the entry point is captured in a HIP graph
    and every replay, with eager work and synchronisations between them,
    equals the eager output."""
    b, hq, hkv, d, t_kv = 1, 32, 8, 128, 8192
    cents, perm, idx, vals, q = _case(14, b, hq, hkv, d, t_kv, 1)
    c_t = _t(cents)
    cb = _hip.codebook_f16x2(c_t)
    args = (_t(q), 1.0 / np.sqrt(d), _t(perm), c_t, _t(idx), _il8(vals, t_kv), t_kv)
    eager = torch.empty((b, hq, 1, d), dtype=torch.float32, device=DEV)
    _hip.decode_attn_il8_noalloc(*args, out=eager, codebook=cb)
    torch.cuda.synchronize()
    out = torch.full_like(eager, float("nan"))
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _hip.decode_attn_il8_noalloc(*args, out=out, codebook=cb)  # warm on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            _hip.decode_attn_il8_noalloc(*args, out=out, codebook=cb)
    torch.cuda.synchronize()
    for i in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _hip.decode_attn_il8(*args, out_dtype=torch.float32, codebook=cb)  # eager work between
        torch.cuda.synchronize()
