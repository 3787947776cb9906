"""GPU parity of the C-ABI kernels against the CPU oracle.

Bars (written in each test):
  * integer/byte outputs (encode indices, packed words, codes, scalar
    indices, reconstructed centroids) are bit-exact; encode excludes only
    (token, block) pairs the oracle flags as near-ties (a centroid with a
    different vector within 1e-6 relative distance of the best);
  * attention outputs and scores: max |gpu - oracle| <= 1e-3 * max |oracle|
    (fp32 accumulation on the GPU, float64 oracle).
"""

import numpy as np
import pytest
import torch

from oracle import sunshape_oracle as O
from sunshape_mlx_amd import _hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
REL_TOL = 1e-3


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def decode_case(seed, b, hq, hkv, d, t_kv, t_q=1, cap=None, nc=256, v_dtype=np.float16):
    rng = np.random.default_rng(seed)
    nb = d // 8
    cap = cap or t_kv
    cents = rng.standard_normal((nb, nc, 8)).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    idx = np.zeros((b, hkv, cap, nb), np.uint8)
    idx[:, :, :t_kv] = rng.integers(0, nc, (b, hkv, t_kv, nb))
    vals = np.zeros((b, hkv, cap, d), v_dtype)
    vals[:, :, :t_kv] = rng.standard_normal((b, hkv, t_kv, d)).astype(v_dtype)
    q = rng.standard_normal((b, hq, t_q, d)).astype(np.float16)
    return cents, perm, idx, vals, q


@pytest.mark.parametrize(
    "b,hq,hkv,d,t_kv,t_q,causal,splits,cap",
    [
        (1, 32, 8, 128, 4096, 1, False, 0, None),    # config-2 shape (the metric decode)
        (1, 32, 8, 128, 4096, 1, True, 0, 4352),     # causal no-op at decode, padded cap
        (2, 8, 2, 128, 1000, 1, False, 0, 1024),     # ragged T, B=2
        (1, 4, 1, 128, 1, 1, False, 0, 256),         # single token
        (1, 4, 4, 128, 777, 1, False, 1, None),      # MHA (rep 1) -> R=1 path, no split
        (1, 4, 2, 128, 777, 1, False, 7, None),      # forced 7 splits
        (1, 8, 2, 64, 513, 1, False, 0, None),       # head_dim 64
        (1, 4, 1, 128, 64, 3, True, 0, None),        # prefill rows, causal q_offset
        (2, 6, 2, 64, 300, 5, True, 3, 320),         # rows spill over several row groups
    ])
def test_decode_dense_matches_oracle(b, hq, hkv, d, t_kv, t_q, causal, splits, cap):
    cents, perm, idx, vals, q = decode_case(b * 1000 + t_kv, b, hq, hkv, d, t_kv, t_q, cap)
    scale = 1.0 / np.sqrt(d)
    out = _hip.decode_attn_dense(t(q), scale, t(perm), t(cents), t(idx), t(vals), t_kv,
                                 causal=causal, q_offset=t_kv - t_q if causal else 0,
                                 out_dtype=torch.float32, n_splits=splits)
    torch.cuda.synchronize()
    ref = O.sdpa(q, idx[:, :, :t_kv], vals[:, :, :t_kv], cents, perm, scale,
                 mask="causal" if causal else None)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


def test_decode_dense_metric_shape_fp16_out_and_repeatability():
    """T_kv = 32768 (the metric shape): fp32 and fp16 outputs, and two calls
    in a row agree bit-for-bit (the split workspace carries no state)."""
    cents, perm, idx, vals, q = decode_case(42, 1, 32, 8, 128, 32768)
    scale = 1.0 / np.sqrt(128)
    args = (t(q), scale, t(perm), t(cents), t(idx), t(vals), 32768)
    o1 = _hip.decode_attn_dense(*args, out_dtype=torch.float32)
    o2 = _hip.decode_attn_dense(*args, out_dtype=torch.float32)
    o16 = _hip.decode_attn_dense(*args)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    ref = O.sdpa(q, idx, vals, cents, perm, scale)
    assert rel_err(o1.cpu().numpy(), ref) <= REL_TOL
    assert o16.dtype == torch.float16
    # fp16 output: the fp32 result rounded once more (half an fp16 ulp)
    assert rel_err(o16.float().cpu().numpy(), ref) <= REL_TOL


def test_decode_empty_cache_outputs_zero():
    cents, perm, idx, vals, q = decode_case(3, 1, 4, 1, 128, 0, cap=256)
    out = _hip.decode_attn_dense(t(q), 0.1, t(perm), t(cents), t(idx), t(vals), 0,
                                 out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0


def test_decode_bf16_and_f32_values():
    for vd, seed in ((np.float32, 5), (None, 6)):
        cents, perm, idx, vals, q = decode_case(seed, 1, 8, 2, 128, 600, v_dtype=np.float32)
        vt = t(vals) if vd is not None else t(vals).to(torch.bfloat16)
        vref = vals if vd is not None else vt.float().cpu().numpy()
        out = _hip.decode_attn_dense(t(q), 0.125, t(perm), t(cents), t(idx), vt, 600,
                                     out_dtype=torch.float32)
        torch.cuda.synchronize()
        ref = O.sdpa(q, idx, vref, cents, perm, 0.125)
        assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("bits,group,sz,d,t_kv,causal,t_q", [
    (2, 64, np.float16, 128, 2048, False, 1),   # config-4 value format
    (2, 64, np.float32, 128, 700, False, 1),    # reference storage (f32 scale/zero)
    (4, 64, np.float32, 128, 64, False, 1),     # known-answer [15] shape
    (4, 64, np.float32, 128, 32, True, 4),      # [16] shape
    (3, 16, np.float16, 128, 333, False, 1),    # 3-bit words straddle groups
    (4, 16, np.float32, 64, 500, True, 2),
    (2, 16, np.float16, 64, 129, False, 1),
])
def test_decode_grouped_matches_oracle(bits, group, sz, d, t_kv, causal, t_q):
    b, hq, hkv = 1, 8, 2
    cents, perm, idx, vals, q = decode_case(bits * 100 + t_kv, b, hq, hkv, d, t_kv, t_q,
                                            v_dtype=np.float32)
    flat = vals.reshape(-1, d)
    packed, sc, zr, _ = O.quantize_values(flat, bits, group)
    sc_s, zr_s = sc.astype(sz), zr.astype(sz)
    nw = packed.shape[-1]
    ng = d // group
    shp = (b, hkv, t_kv)
    deq = O.dequantize_values(packed, sc_s, zr_s, d, bits, group).reshape(shp + (d,))
    out = _hip.decode_attn_grouped(
        t(q), 0.1, t(perm), t(cents), t(idx), t(packed.reshape(shp + (nw,)).view(np.int32)),
        t(sc_s.reshape(shp + (ng,))), t(zr_s.reshape(shp + (ng,))), bits, group, t_kv,
        causal=causal, q_offset=t_kv - t_q if causal else 0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.sdpa(q, idx, deq, cents, perm, 0.1, mask="causal" if causal else None)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


def _kmeans_like_codebook(rng, nb, nc, bd, scale):
    # centroids drawn from the data distribution, with a duplicated pair per
    # block (exact ties must resolve to the lower index)
    c = (rng.standard_normal((nb, nc, bd)) * scale.reshape(nb, 1, bd)).astype(np.float32)
    c[:, 7] = c[:, 3]
    return c


@pytest.mark.parametrize("n_tok,bd,dtype", [
    (5, 8, np.float32),        # decode-step append path (wave per block)
    (300, 8, np.float16),      # small path, fp16 keys
    (4096, 8, np.float32),     # bulk path
    (2000, 4, np.float32),
    (1500, 16, np.float16),
])
def test_encode_bit_exact_except_near_ties(n_tok, bd, dtype):
    rng = np.random.default_rng(n_tok + bd)
    d = 128
    nb = d // bd
    s = np.exp(rng.uniform(np.log(0.25), np.log(8.0), d)).astype(np.float32)
    keys = (rng.standard_normal((n_tok, d)) * s).astype(dtype)
    perm = rng.permutation(d).astype(np.int32)
    cents = _kmeans_like_codebook(rng, nb, 256, bd, s[perm])
    out = torch.empty((n_tok, nb), dtype=torch.uint8, device=DEV)
    _hip.encode_blockvq(t(keys), t(perm), t(cents), out, bd)
    torch.cuda.synchronize()
    ref, near = O.encode_blockvq_c(keys, cents, perm)
    got = out.cpu().numpy()
    ok = ~near
    assert near.mean() < 1e-3
    assert np.array_equal(got[ok], ref[ok]), f"{(got[ok] != ref[ok]).sum()} mismatches"
    assert not (got == 7).any(), "duplicate centroid 7 must lose the tie to centroid 3"


@pytest.mark.parametrize("n_tok,dtype,nc,seed", [
    (4096, np.float16, 256, 1),
    (4000, np.float32, 256, 2),   # keys carry an fp16 lo part
    (3001, "bf16", 256, 3),
    (2500, np.float32, 100, 4),   # partial last centroid tile
    (2000, np.float16, 17, 5),
    (1030, np.float32, 1, 6),     # one centroid: nothing to beat
    (20000, np.float32, 256, 7),  # several tiles per persistent workgroup
])
def test_encode_prepared_matches_plain_encoder_and_oracle(n_tok, dtype, nc, seed):
    """Matrix-core encoder (prepared codebook): indices identical to the
    plain encoder on every (token, block), including rows that must take the
    exact path (keys equal to a centroid, a duplicated centroid pair, zero
    rows, keys beyond the scaled fp16 range, a NaN block); and bit-exact
    against the float64 oracle away from its flagged near-ties."""
    rng = np.random.default_rng(seed)
    d, bd = 128, 8
    nb = d // bd
    s = np.exp(rng.uniform(np.log(0.25), np.log(8.0), d)).astype(np.float32)
    keys = (rng.standard_normal((n_tok, d)) * s).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    cents = _kmeans_like_codebook(rng, nb, nc, bd, s[perm]) if nc >= 8 else \
        (rng.standard_normal((nb, nc, bd)) * s[perm].reshape(nb, 1, bd)).astype(np.float32)
    inv = np.argsort(perm)
    keys[10] = cents[np.arange(nb), 0].reshape(-1)[inv]   # exactly centroid 0 of every block
    keys[11] = 0.0
    if nc >= 8:
        keys[12] = cents[np.arange(nb), 3].reshape(-1)[inv]  # on the duplicated pair 3 / 7
    nan_row = dtype is np.float32
    if nan_row:
        keys[13, perm[:8]] = np.nan                       # block 0 of row 13
        keys[14, perm[8:16]] = 3.0e6                      # block 1 beyond the fp16 range
    if dtype == "bf16":
        kt = t(keys).to(torch.bfloat16)
        keys = kt.float().cpu().numpy()
    else:
        keys = keys.astype(dtype)
        kt = t(keys)
    # the rounded key rows become the centroids they were drawn from, so the
    # distances are exactly 0
    kp = keys.astype(np.float32)[:, perm].reshape(n_tok, nb, bd)
    cents[:, 0] = kp[10]
    if nc >= 8:
        cents[:, 3] = cents[:, 7] = kp[12]
    ct = t(cents)
    prep = _hip.encode_codebook(ct)
    plain = torch.empty((n_tok, nb), dtype=torch.uint8, device=DEV)
    fast = torch.full((n_tok, nb), 255, dtype=torch.uint8, device=DEV)
    _hip.encode_blockvq(kt, t(perm), ct, plain, bd)
    _hip.encode_blockvq(kt, t(perm), ct, fast, bd, prepared=prep)
    torch.cuda.synchronize()
    got, base = fast.cpu().numpy(), plain.cpu().numpy()
    assert np.array_equal(got, base), f"{(got != base).sum()} pairs differ from the plain encoder"
    finite = np.isfinite(keys).all(1)
    ref, near = O.encode_blockvq_c(keys[finite].astype(np.float32), cents, perm)
    ok = ~near
    assert np.array_equal(got[finite][ok], ref[ok]), f"{(got[finite][ok] != ref[ok]).sum()} mismatches"
    assert (got[10] == 0).all()
    if nc >= 8:
        assert (got[12] == 3).all() and not (got == 7).any()
    if nan_row:
        assert got[13, 0] == 0


def test_encode_config3_shape_and_cache_strides():
    """Config 3: fp16 K (8 heads x 8192 tokens x 128), ProfilePerm,
    encoded straight into a padded cache buffer (B, H, cap, 16) at an offset."""
    rng = np.random.default_rng(3)
    h, n, d, cap, off = 8, 8192, 128, 8192 + 512, 256
    s = np.exp(rng.uniform(np.log(0.25), np.log(8.0), d)).astype(np.float32)
    keys = (rng.standard_normal((1, h, n, d)) * s).astype(np.float16)
    perm = rng.permutation(d).astype(np.int32)
    cal = (rng.standard_normal((4096, d)) * s).astype(np.float32)[:, perm]
    cents = np.stack([cal[rng.permutation(4096)[:256], b * 8:(b + 1) * 8] for b in range(16)])
    ref, near = O.encode_blockvq_c(keys.reshape(-1, d), cents, perm)
    ok = ~near
    ct = t(cents)
    outs = []
    for prep in (None, _hip.encode_codebook(ct)):  # plain and matrix-core encoders
        cache = torch.full((1, h, cap, 16), 255, dtype=torch.uint8, device=DEV)
        _hip.encode_blockvq(t(keys), t(perm), ct, cache[:, :, off:off + n], 8, prepared=prep)
        torch.cuda.synchronize()
        got = cache.cpu().numpy()
        assert (got[:, :, :off] == 255).all() and (got[:, :, off + n:] == 255).all()
        g = got[0, :, off:off + n].reshape(-1, 16)
        assert np.array_equal(g[ok], ref[ok]), f"{(g[ok] != ref[ok]).sum()} mismatches"
        outs.append(g)
    assert np.array_equal(outs[0], outs[1])


def test_lut_and_score_gather():
    rng = np.random.default_rng(55)
    d, nb, nc = 128, 16, 256
    q = rng.standard_normal((8, d)).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    cents = rng.standard_normal((nb, nc, 8)).astype(np.float32)
    lut = _hip.build_lut(t(q), t(perm), 1.0, t(cents))
    torch.cuda.synchronize()
    ref_lut = O.query_centroid_dots(q[:, perm], cents)
    assert rel_err(lut.cpu().numpy(), ref_lut) <= 1e-5
    idx = rng.integers(0, nc, (1000, nb)).astype(np.uint8)
    sc = _hip.score_gather(lut, t(idx))
    torch.cuda.synchronize()
    ref = O.gather_scores(ref_lut, idx)
    assert rel_err(sc.cpu().numpy(), ref) <= REL_TOL
    # [10]: n_blocks 8, n_centroids 64, score shape (2, 16)
    qd = rng.standard_normal((2, 8, 64)).astype(np.float32)
    i2 = rng.integers(0, 64, (16, 8)).astype(np.uint8)
    s2 = _hip.score_gather(t(qd), t(i2))
    torch.cuda.synchronize()
    assert tuple(s2.shape) == (2, 16)
    assert rel_err(s2.cpu().numpy(), O.gather_scores(qd, i2)) <= 1e-6


def test_dequantize_blockvq_exact():
    rng = np.random.default_rng(9)
    cents = rng.standard_normal((16, 256, 8)).astype(np.float32)
    idx = rng.integers(0, 256, (321, 16)).astype(np.uint8)
    perm = rng.permutation(128).astype(np.int32)
    inv = O.invert_permutation(perm)
    out = _hip.dequantize_blockvq(t(idx), t(cents), t(inv))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.dequantize_blockvq(idx, cents, inv))


@pytest.mark.parametrize("bits,group,d", [(2, 64, 128), (4, 64, 128), (3, 16, 128), (4, 16, 64),
                                          (2, 16, 64)])
def test_quantize_values_bit_exact(bits, group, d):
    rng = np.random.default_rng(123 + bits)
    v = rng.standard_normal((257, d)).astype(np.float32)
    v[5] = 0.0  # constant group -> scale clamps to 1e-8
    nw = O.packed_dim(d, bits)
    p = torch.empty((257, nw), dtype=torch.int32, device=DEV)
    s = torch.empty((257, d // group), dtype=torch.float32, device=DEV)
    z = torch.empty_like(s)
    _hip.quantize_values_grouped(t(v), bits, group, p, s, z)
    torch.cuda.synchronize()
    rp, rs, rz, _ = O.quantize_values(v, bits, group)
    assert np.array_equal(p.cpu().numpy().view(np.uint32), rp)
    assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(z.cpu().numpy(), rz)
    deq = _hip.dequantize_values_grouped(p.view(torch.uint32), s, z, d, bits, group)
    torch.cuda.synchronize()
    assert np.array_equal(deq.cpu().numpy(), O.dequantize_values(rp, rs, rz, d, bits, group))


@pytest.mark.parametrize("bits,d", [(2, 128), (3, 100), (3, 27), (4, 128), (4, 32)])
def test_pack_unpack_bit_exact(bits, d):
    rng = np.random.default_rng(42 + d)
    x = rng.integers(0, 1 << bits, (32, d)).astype(np.uint8)
    p = _hip.pack_indices(t(x), bits)
    u = _hip.unpack_indices(p, d, bits)
    torch.cuda.synchronize()
    assert np.array_equal(p.cpu().numpy(), O.pack_indices(x, bits))
    assert np.array_equal(u.cpu().numpy(), x.astype(np.uint32))


def test_scalar_quantize_exact():
    rng = np.random.default_rng(77)
    v = rng.standard_normal((100, 64)).astype(np.float32)
    bnd = np.array([-1.0, -0.5, 0.0, 0.5, 1.0], np.float32)
    out = _hip.scalar_quantize(t(v), t(bnd))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.scalar_quantize(v, bnd))


def test_invalid_arguments_raise_before_launch():
    cents, perm, idx, vals, q = decode_case(1, 1, 6, 4, 128, 64)  # 6 % 4 != 0
    with pytest.raises(_hip.SunShapeHIPError):
        _hip.decode_attn_dense(t(q), 1.0, t(perm), t(cents), t(idx), t(vals), 64)
    cents, perm, idx, vals, q = decode_case(1, 1, 4, 4, 128, 64)
    with pytest.raises(_hip.SunShapeHIPError):
        _hip.decode_attn_dense(t(q), 1.0, t(perm), t(cents), t(idx), t(vals), 65)  # > cap


def to_il8(vals_np, cap):
    """Build the interleaved (B, H, cap/8, D, 8) cache with the append kernel."""
    b, h, t_kv, d = vals_np.shape
    buf = torch.zeros((b, h, cap // 8, d, 8), dtype=torch.float16, device=DEV)
    _hip.append_values_il8(t(vals_np.astype(np.float16)), buf, 0)
    return buf


def test_append_values_il8_roundtrip_and_offsets():
    rng = np.random.default_rng(0)
    v = rng.standard_normal((2, 3, 21, 64)).astype(np.float16)
    buf = torch.zeros((2, 3, 48 // 8, 64, 8), dtype=torch.float16, device=DEV)
    _hip.append_values_il8(t(v[:, :, :13]), buf, 0)
    _hip.append_values_il8(t(v[:, :, 13:]), buf, 13)   # unaligned offset
    torch.cuda.synchronize()
    dense = _hip.il8_to_dense(buf).cpu().numpy()
    assert np.array_equal(dense[:, :, :21], v)
    assert not dense[:, :, 21:].any()


@pytest.mark.parametrize(
    "b,hq,hkv,d,t_kv,t_q,causal,splits,cap",
    [
        (1, 32, 8, 128, 4096, 1, False, 0, None),    # config-2 shape (the metric decode)
        (1, 32, 8, 128, 32768, 1, False, 0, None),   # metric shape
        (2, 8, 2, 128, 1003, 1, False, 0, 1024),     # ragged T (partial 8-token block)
        (1, 4, 1, 128, 1, 1, False, 0, 256),         # single token
        (1, 4, 2, 128, 777, 1, False, 5, None),      # forced splits, rep 2 (rows 2-3 empty)
        (1, 8, 2, 64, 513, 1, False, 0, None),       # head_dim 64
        (1, 4, 1, 128, 64, 3, True, 0, None),        # prefill rows, causal
        (2, 6, 2, 64, 300, 5, True, 3, 320),         # several row groups
        (1, 8, 2, 128, 4096, 1, False, 48, None),    # 48 splits: the merge stages partials in LDS
        (1, 8, 2, 128, 4096, 1, False, 31, None),    # 31 splits: a register merge with one slot past the end
    ])
def test_decode_il8_matches_oracle(b, hq, hkv, d, t_kv, t_q, causal, splits, cap):
    cap = cap or ((t_kv + 7) // 8) * 8
    cents, perm, idx, vals, q = decode_case(b * 1000 + t_kv + 1, b, hq, hkv, d, t_kv, t_q, cap)
    vbuf = to_il8(vals, cap)
    if t_kv < cap:  # NaN padding after t_kv must not leak into the result
        tail = (t_kv // 8) * 8
        vbuf.view(b, hkv, cap // 8, d * 8)[:, :, tail // 8:] = float("nan")
        _hip.append_values_il8(t(vals[:, :, tail:t_kv]), vbuf, tail)
    scale = 1.0 / np.sqrt(d)
    out = _hip.decode_attn_il8(t(q), scale, t(perm), t(cents), t(idx), vbuf, t_kv,
                               causal=causal, q_offset=t_kv - t_q if causal else 0,
                               out_dtype=torch.float32, n_splits=splits)
    torch.cuda.synchronize()
    ref = O.sdpa(q, idx[:, :, :t_kv], vals[:, :, :t_kv], cents, perm, scale,
                 mask="causal" if causal else None)
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, ref) <= REL_TOL


def test_codebook_f16x2_reconstructs_the_centroids():
    """hi + lo * 2^-11, times the stored power of two, gives back every
    centroid to about 2^-22 of the codebook's largest magnitude, for codebooks
    far outside the fp16 range, tiny ones and an all-zero one; the squared
    norms that follow are every tile row's |C|^2 (float32)."""
    rng = np.random.default_rng(5)
    for mag, nc in ((1.0, 256), (3e6, 40), (2e-7, 16), (0.0, 8)):
        c = (rng.standard_normal((16, nc, 8)) * mag).astype(np.float32)
        c[0, 0, 0] = 0.0
        buf = _hip.codebook_f16x2(t(c))
        torch.cuda.synchronize()
        raw = buf.cpu().numpy()
        nct = (nc + 15) // 16
        body = 4 * nct * 2048
        assert raw.size == body + 16 + 4 * nct * 64 * 4
        # tile (bg, ct), part (hi, lo), lane l: centroid ct*16 + l%16 of block bg*4 + l/16
        hl = raw[:body].view(np.float16).reshape(4, nct, 2, 4, 16, 8).astype(np.float64)
        mul = float(raw[body:body + 4].view(np.float32)[0])
        assert mul > 0 and np.log2(mul) == np.round(np.log2(mul))  # a power of two
        assert np.isfinite(hl).all() and np.abs(hl[:, :, 0]).max() <= 2.0 ** 14
        full = (hl[:, :, 0] + hl[:, :, 1] / 2048.0) * mul          # (bg, ct, bs, n, 8)
        full = full.transpose(0, 2, 1, 3, 4).reshape(16, nct * 16, 8)
        back = full[:, :nc]
        assert not full[:, nc:].any()  # padding lanes are zero
        tol = max(np.abs(c).max(), 1e-30) * 2.0 ** -21
        assert np.abs(back - c).max() <= tol
        # |C|^2 per tile row, rows laid out as the hi parts
        nrm = raw[body + 16:].view(np.float32).reshape(4, nct, 4, 16)  # (bg, ct, bs, n)
        nrm = nrm.transpose(0, 2, 1, 3).reshape(16, nct * 16)
        want = (c.astype(np.float64) ** 2).sum(-1)
        assert not nrm[:, nc:].any()
        assert np.allclose(nrm[:, :nc], want, rtol=2e-6, atol=0.0)


@pytest.mark.parametrize("q_dtype,nc,d", [(np.float32, 256, 128), (np.float32, 40, 64),
                                          (np.float16, 40, 128), (np.float16, 8, 64)])
def test_decode_il8_query_dtypes_and_small_codebooks(q_dtype, nc, d):
    """fp32 queries take the split query operand of the matrix-core LUT
    build; codebooks with fewer than 16 centroids or a partial last tile of 16
    leave part of the LUT tiles unused."""
    cents, perm, idx, vals, q = decode_case(900 + nc, 1, 8, 2, d, 1500, cap=1504, nc=nc)
    q = (q.astype(np.float32) * 1.7).astype(q_dtype)
    if q_dtype == np.float32:
        q += np.float32(1e-4) * np.random.default_rng(3).standard_normal(q.shape).astype(np.float32)
    out = _hip.decode_attn_il8(t(q), 0.125, t(perm), t(cents), t(idx), to_il8(vals, 1504), 1500,
                               out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.sdpa(q, idx[:, :, :1500], vals[:, :, :1500], cents, perm, 0.125)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_decode_il8_misaligned_output(out_dtype):
    """An output view that starts one element past an aligned address takes
    the merge's element-wise stores instead of its packed ones, with the same
    result."""
    b, hq, hkv, d, t_kv = 1, 8, 2, 128, 3000
    cents, perm, idx, vals, q = decode_case(77, b, hq, hkv, d, t_kv)
    args = (t(q), 1.0 / np.sqrt(d), t(perm), t(cents), t(idx), to_il8(vals, t_kv), t_kv)
    ref = _hip.decode_attn_il8(*args, out_dtype=out_dtype, n_splits=8)
    n = b * hq * d
    base = torch.zeros(n + 1, dtype=out_dtype, device=DEV)
    out = base[1:].view(b, hq, 1, d)
    assert out.data_ptr() % 8 != 0
    _hip.decode_attn_il8(*args, out=out, n_splits=8)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref.cpu())
    assert base[0].item() == 0


def test_decode_il8_peaked_and_flat_softmax():
    """Probabilities spanning many orders of magnitude (the hi/lo fp16 split
    must keep small ones) and an almost flat softmax."""
    for qscale, seed in ((30.0, 1), (1e-3, 2)):
        cents, perm, idx, vals, q = decode_case(seed, 1, 4, 1, 128, 5000, cap=5000)
        q = (q.astype(np.float32) * qscale).astype(np.float16)
        out = _hip.decode_attn_il8(t(q), 0.0883883, t(perm), t(cents), t(idx), to_il8(vals, 5000),
                                   5000, out_dtype=torch.float32)
        torch.cuda.synchronize()
        ref = O.sdpa(q, idx, vals, cents, perm, 0.0883883)
        assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


def grouped_case(seed, b, hkv, t_kv, d, bits, group, cap, sz_dtype=torch.float16):
    """Grouped-quantised values of a (b, hkv, t_kv, d) N(0,1) cache: reference
    packed rows, scales/zeros of dtype sz_dtype (cap rows, zero past t_kv)
    and the token-interleaved codes built with the relayout kernel in three
    unaligned appends."""
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((b, hkv, t_kv, d)).astype(np.float16)
    nw, ng = d * bits // 32, d // group
    packed = torch.zeros((b, hkv, cap, nw), dtype=torch.int32, device=DEV)
    sc = torch.zeros((b, hkv, cap, ng), dtype=sz_dtype, device=DEV)
    ze = torch.zeros((b, hkv, cap, ng), dtype=sz_dtype, device=DEV)
    if t_kv:
        _hip.quantize_values_grouped(t(v), bits, group, packed[:, :, :t_kv], sc[:, :, :t_kv],
                                     ze[:, :, :t_kv])
    il = torch.zeros((b, hkv, cap * bits // 32, d), dtype=torch.int32, device=DEV)
    cuts = sorted({0, t_kv, min(t_kv, 7), min(t_kv, t_kv // 2 + 3)})
    for a0, a1 in zip(cuts[:-1], cuts[1:]):
        _hip.pack_grouped_il(packed[:, :, a0:a1], bits, il, a0)
    return v, packed, sc, ze, il


@pytest.mark.parametrize("bits,d,t_kv,cap", [(2, 128, 1000, 1024), (4, 128, 77, 96), (2, 64, 300, 320),
                                             (4, 64, 16, 16)])
def test_pack_grouped_il_roundtrip(bits, d, t_kv, cap):
    """Token-interleaved codes written in unaligned appends read back as the
    reference packed rows bit for bit; words past t_kv stay zero."""
    _, packed, _, _, il = grouped_case(11 + bits, 2, 3, t_kv, d, bits, d // 2, cap)
    torch.cuda.synchronize()
    back = _hip.grouped_il_to_packed(il, bits).view(torch.int32).cpu().numpy()
    assert np.array_equal(back[:, :, :t_kv], packed[:, :, :t_kv].cpu().numpy())
    assert not back[:, :, t_kv:].any()
    # the word layout itself: token i of a word at bit bits*(i//2) + 16*(i%2)
    tpw, mask = 32 // bits, (1 << bits) - 1
    pk = packed[:, :, :t_kv].cpu().numpy().view(np.uint32).astype(np.uint64)
    dims = np.arange(d)
    codes = (pk[..., dims // tpw] >> ((dims % tpw) * bits).astype(np.uint64)) & mask  # (B,H,T,D)
    want = np.zeros((2, 3, cap // tpw, d), dtype=np.uint64)
    for i in range(tpw):
        tok = np.arange(i, t_kv, tpw)
        want[:, :, tok // tpw, :] |= codes[:, :, tok, :] << np.uint64(bits * (i // 2) + 16 * (i % 2))
    assert np.array_equal(il.cpu().numpy().view(np.uint32).astype(np.uint64), want)


@pytest.mark.parametrize("bits,d,group,t_kv,cap,sz", [
    (2, 128, 64, 1000, 1024, torch.float16),    # config 4's codes, ragged end
    (4, 128, 128, 77, 96, torch.float32),       # 4-bit, one group, f32 scale/zero
    (2, 64, 32, 301, 320, torch.float16),       # head_dim 64
    (4, 64, 64, 8, 16, torch.float16),          # one 8-token group
])
def test_grouped_il_to_il8_equals_dequantise_then_interleave(bits, d, group, t_kv, cap, sz):
    """ss_grouped_il_to_il8 (one launch) writes the same fp16 words as the
    reference-layout dequantisation (float32) cast to fp16 and interleaved by
    ss_append_values_il8; positions past t_kv in the last 8-token group are
    zero and later groups are left alone."""
    _, packed, sc, ze, il = grouped_case(40 + bits, 2, 3, t_kv, d, bits, group, cap, sz_dtype=sz)
    dense = _hip.dequantize_values_grouped(packed[:, :, :t_kv].view(torch.uint32),
                                           sc[:, :, :t_kv], ze[:, :, :t_kv], d, bits, group)
    cap_out = cap + 16
    want = torch.zeros((2, 3, cap_out // 8, d, 8), dtype=torch.float16, device=DEV)
    _hip.append_values_il8(dense.to(torch.float16).contiguous(), want, 0)
    got = torch.full_like(want, 7.0)
    _hip.grouped_il_to_il8(il, bits, group, sc, ze, t_kv, got)
    torch.cuda.synchronize()
    n8 = (t_kv + 7) // 8
    assert torch.equal(got[:, :, :n8].view(torch.int16), want[:, :, :n8].view(torch.int16))
    assert bool((got[:, :, n8:] == 7.0).all())


@pytest.mark.parametrize("dtype,use_perm,d,t_", [
    (torch.float16, True, 128, 200),
    (torch.bfloat16, True, 128, 33),
    (torch.float32, False, 64, 65),
])
def test_raw_key_rows_are_the_power_of_two_split(dtype, use_perm, d, t_):
    """ss_raw_key_rows from a strided window of a buffer: per token the
    power of two 2^s with max |k| * 2^-s in [2^14, 2^15) (s = 0 for a zero
    key), row 0 = fp16(k * 2^-s), row 1 = fp16(k * 2^-s - row 0),
    written out with frexp / ldexp in float64; keys in the permuted basis.
    For 16-bit keys (row 0 + row 1) times 2^s is the key exactly."""
    g = torch.Generator(device=DEV).manual_seed(d + t_)
    buf = torch.randn((2, 3, t_ + 40, d), generator=g, device=DEV)
    e_lo, e_hi = (-8, 4) if dtype == torch.float16 else (-60, 60)  # per-token magnitudes
    buf *= torch.exp2(torch.randint(e_lo, e_hi, (2, 3, t_ + 40, 1), generator=g,
                                    device=DEV).float())
    buf[0, 1, 5] = 0.0  # a zero key
    buf = buf.to(dtype)
    win = buf[:, :, 17:17 + t_]  # a window view, as the hybrid buffer hands over
    perm = torch.randperm(d, generator=g, device=DEV).to(torch.int32) if use_perm else None
    rows, fac = _hip.raw_key_rows(win, perm)
    torch.cuda.synchronize()
    k = win.double().cpu().numpy()
    if use_perm:
        k = k[..., perm.long().cpu().numpy()]
    m = np.abs(k).max(axis=-1)
    _, e = np.frexp(m)  # m = f * 2^e, f in [0.5, 1)
    s = np.where(m > 0, e - 15, 0).clip(-126, 126)
    ks = np.ldexp(k, -s[..., None])
    hi = ks.astype(np.float32).astype(np.float16)
    lo = (ks - hi.astype(np.float64)).astype(np.float32).astype(np.float16)
    got = rows.cpu().numpy()
    assert np.array_equal(got[..., 0, :].view(np.int16), hi.view(np.int16))
    assert np.array_equal(got[..., 1, :].view(np.int16), lo.view(np.int16))
    assert np.array_equal(fac.cpu().numpy(), np.ldexp(1.0, s).astype(np.float32))
    if dtype != torch.float32:
        back = (got[..., 0, :].astype(np.float64) + got[..., 1, :]) * \
            fac.cpu().numpy()[..., None]
        assert np.array_equal(back, k)


@pytest.mark.parametrize(
    "b,hq,hkv,d,t_kv,t_q,bits,group,sz,causal,splits,cap",
    [
        (2, 32, 8, 128, 4096, 1, 2, 64, "f16", False, 0, None),   # config 4 shape, T=4096
        (1, 8, 2, 128, 1003, 1, 2, 64, "f32", False, 0, 1024),    # ragged T, f32 scale/zero
        (1, 4, 1, 128, 1, 1, 4, 128, "f16", False, 0, 16),        # single token, 4-bit, 1 group
        (1, 4, 2, 128, 777, 1, 4, 64, "f16", False, 5, 784),      # forced splits, rep 2
        (1, 8, 2, 64, 513, 1, 2, 32, "f16", False, 0, 528),       # head_dim 64, 2 groups
        (1, 4, 1, 64, 600, 1, 4, 64, "f32", False, 3, 608),       # head_dim 64, 1 group, f32
        (1, 4, 1, 128, 64, 3, 2, 64, "f16", True, 0, 64),         # prefill rows, causal
        (2, 6, 2, 128, 300, 5, 2, 64, "f16", True, 3, 320),       # several row groups
        (1, 8, 2, 128, 4096, 1, 2, 64, "f16", False, 40, 4096),   # 40 splits: partials staged in LDS
        (1, 8, 2, 128, 4000, 1, 2, 64, "f16", False, 29, 4000),   # 29 splits: four-part register merge
    ])
def test_decode_grouped_il_matches_oracle(b, hq, hkv, d, t_kv, t_q, bits, group, sz, causal, splits,
                                          cap):
    cap = cap or t_kv
    cents, perm, idx, _, q = decode_case(b * 7000 + t_kv + bits, b, hq, hkv, d, t_kv, t_q, cap)
    szt = torch.float16 if sz == "f16" else torch.float32
    _, packed, sc, ze, il = grouped_case(b + t_kv + bits, b, hkv, t_kv, d, bits, group, cap, szt)
    if t_kv < cap:  # unwritten scale/zero rows past t_kv must not leak into the result
        sc[:, :, t_kv:] = float("nan")
        ze[:, :, t_kv:] = float("nan")
    scale = 1.0 / np.sqrt(d)
    out = _hip.decode_attn_grouped_il(t(q), scale, t(perm), t(cents), t(idx), il, sc, ze, bits, group,
                                      t_kv, causal=causal, q_offset=t_kv - t_q if causal else 0,
                                      out_dtype=torch.float32, n_splits=splits)
    torch.cuda.synchronize()
    vals = np.stack([np.stack([
        O.dequantize_values(packed[bi, hi, :t_kv].cpu().numpy().view(np.uint32),
                            sc[bi, hi, :t_kv].float().cpu().numpy(),
                            ze[bi, hi, :t_kv].float().cpu().numpy(), d, bits, group)
        for hi in range(hkv)]) for bi in range(b)])
    ref = O.sdpa(q, idx[:, :, :t_kv], vals, cents, perm, scale, mask="causal" if causal else None)
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, ref) <= REL_TOL


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_grouped_il_peaked_and_flat_softmax(bits):
    """The grouped matrix-core decode carries softmax weights as a bf16 hi/lo
    pair: probabilities spanning many orders of magnitude (a peaked softmax,
    where the small weights must survive the split) and an almost flat one
    (thousands of near-equal weights summed) stay within the bar."""
    t_kv, cap, d, group = 5000, 5008, 128, 64
    for qscale, seed in ((30.0, 1), (1e-3, 2)):
        cents, perm, idx, _, q = decode_case(seed + 40 * bits, 1, 4, 1, d, t_kv, cap=cap)
        q = (q.astype(np.float32) * qscale).astype(np.float16)
        _, packed, sc, ze, il = grouped_case(seed + 50 * bits, 1, 1, t_kv, d, bits, group, cap)
        out = _hip.decode_attn_grouped_il(t(q), 0.0883883, t(perm), t(cents), t(idx), il, sc, ze,
                                          bits, group, t_kv, out_dtype=torch.float32)
        torch.cuda.synchronize()
        vals = O.dequantize_values(packed[0, 0, :t_kv].cpu().numpy().view(np.uint32),
                                   sc[0, 0, :t_kv].float().cpu().numpy(),
                                   ze[0, 0, :t_kv].float().cpu().numpy(), d, bits, group)[None, None]
        ref = O.sdpa(q, idx[:, :, :t_kv], vals, cents, perm, 0.0883883)
        assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


def ramp_case(seed, t_kv, cap, rise, t_q=1):
    """A cache whose scores climb steadily along the tokens by `rise` log2
    units in all (block 0's centroid c is c * step on every dim, the query
    constant, every other block's centroids small): tiles keep rising above
    the running maxima by less and by more than the kernels' lag before a
    wave-wide reduction."""
    d, scale = 128, 0.0883883
    cents, perm, idx, vals, q = decode_case(seed, 1, 4, 1, d, t_kv, t_q, cap=cap)
    cents[1:] *= 0.01
    qv = 0.5
    step = rise / (255 * scale * 1.4426950408889634 * qv * 8)
    cents[0] = (np.arange(256, dtype=np.float32) * step)[:, None] * np.ones(8, np.float32)
    idx[0, 0, :t_kv, 0] = (np.arange(t_kv) * 255 // max(t_kv - 1, 1)).astype(np.uint8)
    q = np.full_like(q, qv)
    q[:, 1::2] *= -1  # two rows fall along the ramp, two climb it
    return cents, perm, idx, vals, q, scale


@pytest.mark.parametrize("rise", [40.0, 600.0])
def test_decode_rising_scores(rise):
    """Scores that keep rising along the cache: the matrix-core decodes skip
    the wave-wide maximum while a tile stays within a few log2 units of the
    running maxima (staged probabilities above 1) and rescale past it; the
    fp16-value and grouped 2-bit kernels match the oracle, with two splits
    (many tiles per wave) and with the default split count."""
    t_kv, cap, d, bits, group = 5000, 5008, 128, 2, 64
    cents, perm, idx, vals, q, scale = ramp_case(17, t_kv, cap, rise)
    _, packed, sc, ze, il = grouped_case(18, 1, 1, t_kv, d, bits, group, cap)
    gvals = O.dequantize_values(packed[0, 0, :t_kv].cpu().numpy().view(np.uint32),
                                sc[0, 0, :t_kv].float().cpu().numpy(),
                                ze[0, 0, :t_kv].float().cpu().numpy(), d, bits, group)[None, None]
    ref = O.sdpa(q, idx[:, :, :t_kv], vals[:, :, :t_kv], cents, perm, scale)
    gref = O.sdpa(q, idx[:, :, :t_kv], gvals, cents, perm, scale)
    for splits in (2, 0):
        out = _hip.decode_attn_il8(t(q), scale, t(perm), t(cents), t(idx), to_il8(vals, cap), t_kv,
                                   out_dtype=torch.float32, n_splits=splits)
        gout = _hip.decode_attn_grouped_il(t(q), scale, t(perm), t(cents), t(idx), il, sc, ze, bits, group,
                                           t_kv, out_dtype=torch.float32, n_splits=splits)
        torch.cuda.synchronize()
        assert rel_err(out.cpu().numpy(), ref) <= REL_TOL, splits
        assert rel_err(gout.cpu().numpy(), gref) <= REL_TOL, splits


@pytest.mark.parametrize("b,hq,hkv,d,t_kv,t_buf,bits,group,splits", [
    (1, 8, 2, 128, 0, 40, 2, 64, 0),      # buffer only (no compressed tokens)
    (2, 8, 2, 64, 333, 70, 2, 32, 0),     # head_dim 64, buffer longer than one chunk
    (1, 4, 1, 128, 200, 5, 4, 128, 7),    # 4-bit (loader-wave ring), 7 splits sharing 5 tokens
])
def test_decode_grouped_il_hybrid_buffer(b, hq, hkv, d, t_kv, t_buf, bits, group, splits):
    """ss_decode_attn_grouped_il_hybrid: compressed tokens plus a token-major
    fp16 buffer in one softmax equals the two-pass oracle over both."""
    cap = max(((t_kv + 15) // 16) * 16, 16)
    cents, perm, idx, _, q = decode_case(t_kv + t_buf + bits, b, hq, hkv, d, t_kv, 1, cap)
    _, packed, sc, ze, il = grouped_case(t_kv + 5, b, hkv, t_kv, d, bits, group, cap)
    rng = np.random.default_rng(t_buf)
    kb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(np.float16)
    vb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    out = _hip.decode_attn_grouped_il(t(q), scale, t(perm), t(cents), t(idx), il, sc, ze, bits,
                                      group, t_kv, out_dtype=torch.float32, n_splits=splits,
                                      buf_keys=t(kb), buf_values=t(vb), buf_len=t_buf)
    torch.cuda.synchronize()
    vals = np.zeros((b, hkv, t_kv + t_buf, d), np.float64)
    for bi in range(b):
        for hi in range(hkv):
            if t_kv:
                vals[bi, hi, :t_kv] = O.dequantize_values(
                    packed[bi, hi, :t_kv].cpu().numpy().view(np.uint32),
                    sc[bi, hi, :t_kv].float().cpu().numpy(), ze[bi, hi, :t_kv].float().cpu().numpy(),
                    d, bits, group)
    vals[:, :, t_kv:] = vb[:, :, :t_buf]
    ref = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("b,hq,hkv,d,t_kv,t_buf,t_q,splits,bdt", [
    (1, 8, 2, 128, 0, 40, 1, 0, np.float16),       # buffer only (no compressed tokens)
    (2, 8, 2, 64, 333, 70, 1, 0, np.float16),      # head_dim 64, buffer longer than one chunk
    (1, 4, 1, 128, 200, 5, 1, 7, np.float32),      # 7 splits sharing 5 tokens, f32 buffer
    (1, 32, 8, 128, 4096, 128, 1, 0, np.float16),  # config-2 heads, default buffer
    (1, 8, 2, 128, 300, 64, 4, 3, np.float16),     # prefill rows, causal across the buffer
])
def test_decode_il8_hybrid_buffer(b, hq, hkv, d, t_kv, t_buf, t_q, splits, bdt):
    """ss_decode_attn_il8_hybrid: compressed fp16 tokens (interleaved) plus a
    token-major buffer in one softmax equals the two-pass oracle over both
    (causal rows see the buffer up to their own position)."""
    cap = max(((t_kv + 7) // 8) * 8, 8)
    cents, perm, idx, vals, q = decode_case(t_kv + t_buf + 3, b, hq, hkv, d, t_kv, t_q, cap)
    rng = np.random.default_rng(t_buf + 1)
    kb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(bdt)
    vb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(bdt)
    scale = 1.0 / np.sqrt(d)
    causal = t_q > 1
    out = _hip.decode_attn_il8(t(q), scale, t(perm), t(cents), t(idx), to_il8(vals, cap), t_kv,
                               causal=causal, q_offset=t_kv + t_buf - t_q if causal else 0,
                               out_dtype=torch.float32, n_splits=splits, buf_keys=t(kb),
                               buf_values=t(vb), buf_len=t_buf)
    torch.cuda.synchronize()
    vals_all = np.concatenate([vals[:, :, :t_kv].astype(np.float64),
                               vb[:, :, :t_buf].astype(np.float64)], axis=2)
    ref = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals_all,
                          mask="causal" if causal else None)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("b,hq,hkv,d,t_kv,t_q,causal,bits,splits,cap", [
    (1, 32, 8, 128, 4096, 1, False, 2, 0, None),   # config-2 heads, 2-bit
    (2, 8, 2, 128, 1000, 1, False, 3, 0, 1024),    # 3-bit words (10 codes, 2 pad bits)
    (1, 8, 2, 128, 777, 1, False, 4, 7, None),     # 4-bit, forced 7 splits
    (1, 8, 2, 64, 513, 1, False, 2, 1, None),      # head_dim 64, one split
    (2, 6, 2, 64, 300, 5, True, 4, 3, 320),        # prefill rows, causal
    (1, 4, 1, 128, 1, 1, False, 3, 0, 16),         # single token
    (1, 4, 1, 128, 0, 1, False, 2, 0, 16),         # empty cache: zeros
])
def test_decode_turboquant_matches_oracle(b, hq, hkv, d, t_kv, t_q, causal, bits, splits, cap):
    """ss_decode_attn_turboquant: softmax(q.k) over norm * (levels[code] @ R)
    values equals the oracle SDPA over the TurboQuant-dequantised cache."""
    cap = cap or t_kv
    cents, perm, idx, _, q = decode_case(40 + bits + t_kv, b, hq, hkv, d, t_kv, t_q, cap)
    rng = np.random.default_rng(bits * 1000 + t_kv)
    codes = rng.integers(0, 1 << bits, (b, hkv, cap, d)).astype(np.uint8)
    packed = O.pack_indices(codes, bits).astype(np.uint32)
    norms = (rng.random((b, hkv, cap)) * 3 + 0.1).astype(np.float32)
    levels = (O.lloyd_max_gaussian(bits)[0] / np.sqrt(d)).astype(np.float32)
    rot = O.rotation_matrix(d, 43)
    scale = 1.0 / np.sqrt(d)
    out = _hip.decode_attn_turboquant(t(q), scale, t(perm), t(cents), t(idx),
                                      t(packed.view(np.int32)), t(norms), levels, t(rot), bits,
                                      t_kv, causal=causal, q_offset=t_kv - t_q if causal else 0,
                                      out_dtype=torch.float32, n_splits=splits)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if t_kv == 0:
        assert not got.any()
        return
    vals = O.turboquant_decode(packed[:, :, :t_kv], norms[:, :, :t_kv], rot, levels, d, bits)
    ref = O.sdpa(q, idx[:, :, :t_kv], vals, cents, perm, scale, mask="causal" if causal else None)
    assert rel_err(got, ref) <= REL_TOL


@pytest.mark.parametrize("b,hq,hkv,d,t_kv,t_buf,t_q,bits,splits", [
    (1, 32, 8, 128, 2048, 128, 1, 2, 0),   # default hybrid buffer
    (2, 8, 2, 64, 333, 300, 1, 4, 3),      # buffer longer than one 256-token chunk
    (1, 4, 1, 128, 0, 40, 1, 3, 0),        # buffer only
    (1, 8, 2, 128, 200, 20, 4, 2, 1),      # prefill rows, causal across the buffer
])
def test_decode_turboquant_with_buffer(b, hq, hkv, d, t_kv, t_buf, t_q, bits, splits):
    """Buffered fp16 tokens join the TurboQuant decode as one more split
    partial (taken into the rotated basis); the result equals the two-pass
    oracle over the dequantised cache followed by the buffer."""
    cap = max(((t_kv + 15) // 16) * 16, 16)
    cents, perm, idx, _, q = decode_case(60 + bits + t_buf, b, hq, hkv, d, t_kv, t_q, cap)
    rng = np.random.default_rng(t_buf + 7)
    codes = rng.integers(0, 1 << bits, (b, hkv, cap, d)).astype(np.uint8)
    packed = O.pack_indices(codes, bits).astype(np.uint32)
    norms = (rng.random((b, hkv, cap)) * 3 + 0.1).astype(np.float32)
    levels = (O.lloyd_max_gaussian(bits)[0] / np.sqrt(d)).astype(np.float32)
    rot = O.rotation_matrix(d, 43)
    kb = rng.standard_normal((b, hkv, t_buf + 5, d)).astype(np.float16)
    vb = rng.standard_normal((b, hkv, t_buf + 5, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    causal = t_q > 1
    total = t_kv + t_buf
    out = _hip.decode_attn_turboquant(t(q), scale, t(perm), t(cents), t(idx),
                                      t(packed.view(np.int32)), t(norms), levels, t(rot), bits,
                                      t_kv, causal=causal, q_offset=total - t_q if causal else 0,
                                      out_dtype=torch.float32, n_splits=splits,
                                      buf_keys=t(kb), buf_values=t(vb), buf_len=t_buf)
    torch.cuda.synchronize()
    vals = np.zeros((b, hkv, total, d), np.float64)
    if t_kv:
        vals[:, :, :t_kv] = O.turboquant_decode(packed[:, :, :t_kv], norms[:, :, :t_kv], rot,
                                                levels, d, bits)
    vals[:, :, t_kv:] = vb[:, :, :t_buf]
    ref = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals,
                          mask="causal" if causal else None)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("b,hq,hkv,d,t_kv,t_buf,t_q,causal,splits,peak", [
    (1, 32, 8, 128, 4096, 0, 1, False, 0, False),   # config-2 heads
    (8, 32, 8, 128, 2000, 128, 1, False, 0, False),  # config-4 heads, hybrid buffer
    (1, 8, 2, 64, 517, 0, 1, False, 3, False),      # head_dim 64, ragged T, 3 splits
    (2, 6, 2, 128, 300, 20, 5, True, 1, False),     # prefill rows, causal across the buffer
    (1, 8, 2, 128, 1000, 0, 1, False, 0, True),     # sharper softmax (query x 4)
    (1, 4, 1, 128, 0, 40, 1, False, 0, False),      # buffer only
    (1, 4, 1, 128, 0, 0, 1, False, 0, False),       # empty cache: zeros
])
def test_decode_turboquant_il_matches_oracle(b, hq, hkv, d, t_kv, t_buf, t_q, causal, splits,
                                             peak):
    """ss_decode_attn_turboquant_il (2-bit codes token-interleaved, P.V on the
    matrix cores through the bit-affine split of the level table): equals the
    oracle over the TurboQuant-dequantised cache, with the hybrid buffer as the
    two-pass oracle's trailing tokens."""
    cap = max(((t_kv + 15) // 16) * 16, 16)
    cents, perm, idx, _, q = decode_case(80 + t_kv + t_buf, b, hq, hkv, d, t_kv, t_q, cap)
    rng = np.random.default_rng(t_kv + 3 * t_buf + 11)
    codes = rng.integers(0, 4, (b, hkv, cap, d)).astype(np.uint8)
    packed = O.pack_indices(codes, 2).astype(np.uint32)
    norms = (rng.random((b, hkv, cap)) * 3 + 0.1).astype(np.float32)
    levels = (O.lloyd_max_gaussian(2)[0] / np.sqrt(d)).astype(np.float32)
    rot = O.rotation_matrix(d, 43)
    scale = 1.0 / np.sqrt(d)
    if peak and t_kv:
        # row r of every head sees one token whose key scores far above the rest
        q = q.astype(np.float32) * 4
        q = q.astype(np.float16)
    codes_il = torch.zeros((b, hkv, cap // 16, d), dtype=torch.int32, device=DEV)
    _hip.pack_grouped_il(t(packed.view(np.int32)), 2, codes_il, 0)
    kb = rng.standard_normal((b, hkv, t_buf + 5, d)).astype(np.float16)
    vb = rng.standard_normal((b, hkv, t_buf + 5, d)).astype(np.float16)
    total = t_kv + t_buf
    out = _hip.decode_attn_turboquant_il(t(q), scale, t(perm), t(cents), t(idx), codes_il,
                                         t(norms), levels, t(rot), t_kv, causal=causal,
                                         q_offset=total - t_q if causal else 0,
                                         out_dtype=torch.float32, n_splits=splits,
                                         buf_keys=t(kb) if t_buf else None,
                                         buf_values=t(vb) if t_buf else None, buf_len=t_buf)
    torch.cuda.synchronize()
    _hip.check_decode_waits()
    got = out.cpu().numpy()
    if total == 0:
        assert not got.any()
        return
    vals = np.zeros((b, hkv, total, d), np.float64)
    if t_kv:
        vals[:, :, :t_kv] = O.turboquant_decode(packed[:, :, :t_kv], norms[:, :, :t_kv], rot,
                                                levels, d, 2)
    vals[:, :, t_kv:] = vb[:, :, :t_buf]
    ref = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals,
                          mask="causal" if causal else None)
    assert rel_err(got, ref) <= REL_TOL
    # the interleaved words hold the packed rows' codes
    back = _hip.grouped_il_to_packed(codes_il, 2, cap).cpu().numpy().view(np.uint32)
    assert np.array_equal(back, packed)


@pytest.mark.parametrize("b,hq,hkv,d,t_kv,t_buf,t_q,bd,vnc,transform,splits", [
    (1, 32, 8, 128, 2048, 0, 1, 4, 256, "perm", 0),     # config-5 value codec (block_dim 4)
    (2, 8, 2, 128, 700, 128, 1, 8, 256, "perm", 0),     # block_dim 8, with a buffer
    (1, 8, 2, 64, 513, 0, 1, 4, 100, "rot", 3),         # head_dim 64, rotated codec, 100 centroids
    (2, 6, 2, 128, 300, 20, 5, 8, 256, "rot", 1),       # prefill rows, causal across the buffer
    (1, 8, 2, 128, 999, 0, 1, 4, 100, "rot", 5),        # matrix-core path: ragged T, 100 centroids
    (2, 8, 2, 128, 64, 7, 3, 4, 256, "perm", 0),        # matrix-core path: one unit, causal rows
])
def test_decode_sunshape_v_matches_oracle(b, hq, hkv, d, t_kv, t_buf, t_q, bd, vnc, transform,
                                          splits):
    """ss_decode_attn_sunshape_v: values given as block-VQ indices of a value
    codec (gathered centroids taken back to the original basis by the codec's
    inverse permutation or rotation) equal the oracle SDPA over the oracle's
    block-VQ dequantisation."""
    cap = max(((t_kv + 15) // 16) * 16, 16)
    cents, perm, idx, _, q = decode_case(80 + bd + t_kv, b, hq, hkv, d, t_kv, t_q, cap)
    rng = np.random.default_rng(bd * 100 + t_buf)
    nbv = d // bd
    v_cents = rng.standard_normal((nbv, vnc, bd)).astype(np.float32)
    v_idx = rng.integers(0, vnc, (b, hkv, cap, nbv)).astype(np.uint8)
    if transform == "perm":
        vperm = rng.permutation(d).astype(np.int32)
        inv = O.invert_permutation(vperm)
        m = np.zeros((d, d), np.float32)
        m[inv, np.arange(d)] = 1.0
    else:
        inv = None
        m = O.rotation_matrix(d, 5)
    kb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(np.float16)
    vb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    causal = t_q > 1
    total = t_kv + t_buf
    out = _hip.decode_attn_sunshape_v(t(q), scale, t(perm), t(cents), t(idx), t(v_idx),
                                      t(v_cents), t(m), t_kv, causal=causal,
                                      q_offset=total - t_q if causal else 0,
                                      out_dtype=torch.float32, n_splits=splits,
                                      buf_keys=t(kb), buf_values=t(vb), buf_len=t_buf)
    torch.cuda.synchronize()
    vals = np.zeros((b, hkv, total, d), np.float64)
    for bi in range(b):
        for hi in range(hkv):
            kc = O.dequantize_blockvq(v_idx[bi, hi, :t_kv], v_cents, inv)
            vals[bi, hi, :t_kv] = kc if inv is not None else kc.astype(np.float64) @ m
    vals[:, :, t_kv:] = vb[:, :, :t_buf]
    ref = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals,
                          mask="causal" if causal else None)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


def _inertia(x, c):
    x = np.asarray(x, np.float64)
    c = np.asarray(c, np.float64)
    return float(((x[:, None, :] - c[None]) ** 2).sum(-1).min(1).mean())


@pytest.mark.parametrize("bd,n,k", [(8, 2048, 256), (4, 4096, 256), (8, 700, 100)])
def test_kmeans_blocks_matches_oracle(bd, n, k):
    """ss_kmeans_blocks: from the oracle's initial rows, one Lloyd step gives
    the oracle's assignments away from near-ties and bit-identical centroids
    for every cluster no near-tie point touches; 15 steps reach the oracle's
    inertia within 1 %."""
    rng = np.random.default_rng(bd + n)
    nbk = 3
    scales = rng.uniform(0.5, 4, (nbk, 1, bd))
    data = (rng.standard_normal((nbk, n, bd)) * scales).astype(np.float32)
    init = np.stack([data[b][np.random.RandomState(7 + b).permutation(n)[:k]] for b in range(nbk)])
    c1, a1 = _hip.kmeans_blocks(t(data), t(init), 1, return_assign=True)
    c1, a1 = c1.cpu().numpy(), a1.cpu().numpy()
    for b in range(nbk):
        x, c = data[b], init[b]
        # the oracle's float32 expanded-form distances and argmin
        dist = (np.sum(x ** 2, axis=1, keepdims=True) + np.sum(c ** 2, axis=1, keepdims=True).T
                - 2.0 * x @ c.T)
        a_ref = np.argmin(dist, axis=1)
        d64 = ((x.astype(np.float64)[:, None, :] - c.astype(np.float64)[None]) ** 2).sum(-1)
        srt = np.sort(d64, axis=1)
        scale = (x.astype(np.float64) ** 2).sum(1) + (c.astype(np.float64) ** 2).sum(1).max()
        near = (srt[:, 1] - srt[:, 0]) <= 1e-5 * scale
        assert near.mean() < 0.01
        assert np.array_equal(a1[b][~near], a_ref[~near])
        touched = set(a1[b][near].tolist()) | set(a_ref[near].tolist())
        ref1 = O.kmeans(x, k, 1, 7 + b)
        keep = np.array([kk not in touched for kk in range(k)])
        assert np.array_equal(c1[b][keep], ref1[keep])
    c15 = _hip.kmeans_blocks(t(data), t(init), 15).cpu().numpy()
    for b in range(nbk):
        ref = O.kmeans(data[b], k, 15, 7 + b)
        assert abs(_inertia(data[b], c15[b]) / _inertia(data[b], ref) - 1.0) <= 0.01


@pytest.mark.parametrize("b,hq,hkv,t_kv,t_buf,t_q,n_heavy,splits", [
    (2, 32, 8, 1500, 0, 1, 4, 0),    # config-5 shape: 4 heavy blocks (32 fp16 dims)
    (1, 8, 2, 333, 40, 3, 1, 2),     # one heavy block, buffer, causal prefill rows
    (1, 8, 2, 700, 0, 1, 2, 0),      # two heavy blocks
    (1, 4, 1, 257, 16, 1, 8, 3),     # eight heavy blocks (64 dims), a partial last unit
])
def test_decode_sunshape_v_heavy_blocks(b, hq, hkv, t_kv, t_buf, t_q, n_heavy, splits):
    """Mixed-precision keys with their heavy blocks in fp16: the fused decode
    scores the heavy blocks from their fp16 dims in place of the LUT (their
    centroids are nonzero, as after a fit with DSQ refinement, and must add
    nothing), as the oracle's two-pass SDPA with heavy keys does."""
    d, bd = 128, 4
    cap = ((t_kv + 15) // 16) * 16
    cents, perm, idx, _, q = decode_case(90 + n_heavy, b, hq, hkv, d, t_kv, t_q, cap)
    rng = np.random.default_rng(91 + n_heavy)
    heavy = np.sort(rng.permutation(16)[:n_heavy])
    hd = np.concatenate([np.arange(x * 8, x * 8 + 8) for x in heavy]).astype(np.int32)
    kh = np.zeros((b, hkv, cap, hd.size), np.float16)
    kh[:, :, :t_kv] = rng.standard_normal((b, hkv, t_kv, hd.size)).astype(np.float16)
    nbv = d // bd
    v_cents = rng.standard_normal((nbv, 256, bd)).astype(np.float32)
    v_idx = rng.integers(0, 256, (b, hkv, cap, nbv)).astype(np.uint8)
    vperm = rng.permutation(d).astype(np.int32)
    inv = O.invert_permutation(vperm)
    m = np.zeros((d, d), np.float32)
    m[inv, np.arange(d)] = 1.0
    kb = rng.standard_normal((b, hkv, t_buf + 2, d)).astype(np.float16)
    vb = rng.standard_normal((b, hkv, t_buf + 2, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    causal = t_q > 1
    total = t_kv + t_buf
    out = _hip.decode_attn_sunshape_v(t(q), scale, t(perm), t(cents), t(idx), t(v_idx),
                                      t(v_cents), t(m), t_kv, causal=causal,
                                      q_offset=total - t_q if causal else 0,
                                      out_dtype=torch.float32, n_splits=splits,
                                      buf_keys=t(kb), buf_values=t(vb), buf_len=t_buf,
                                      k_heavy=t(kh), heavy_dims=t(hd))
    torch.cuda.synchronize()
    vals = np.zeros((b, hkv, total, d), np.float64)
    for bi in range(b):
        for hi in range(hkv):
            vals[bi, hi, :t_kv] = O.dequantize_blockvq(v_idx[bi, hi, :t_kv], v_cents, inv)
    vals[:, :, t_kv:] = vb[:, :, :t_buf]
    ref = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals,
                          mask="causal" if causal else None, heavy_keys=kh[:, :, :t_kv],
                          heavy_dims=hd)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL
    # without k_heavy the kernel keeps the reference's scores (a heavy block's
    # index adds its centroid's dot product like any other block)
    out0 = _hip.decode_attn_sunshape_v(t(q), scale, t(perm), t(cents), t(idx), t(v_idx),
                                       t(v_cents), t(m), t_kv, causal=causal,
                                       q_offset=total - t_q if causal else 0,
                                       out_dtype=torch.float32, n_splits=splits,
                                       buf_keys=t(kb), buf_values=t(vb), buf_len=t_buf)
    torch.cuda.synchronize()
    ref0 = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals,
                           mask="causal" if causal else None)
    assert rel_err(out0.cpu().numpy(), ref0) <= REL_TOL


@pytest.mark.parametrize("kind,bits,b,hq,hkv,d,t_kv,t_buf,t_q,n_heavy,splits", [
    ("il8", 16, 2, 32, 8, 128, 1500, 0, 1, 4, 0),      # config-5 heads, 4 heavy blocks
    ("il8", 16, 1, 8, 2, 128, 333, 40, 3, 1, 2),       # buffer, causal prefill rows
    ("il8", 16, 1, 8, 2, 64, 517, 0, 1, 3, 3),         # head_dim 64, 24 heavy dims
    ("grouped_il", 2, 1, 8, 2, 128, 700, 20, 1, 2, 0),
    ("grouped_il", 4, 1, 8, 2, 64, 300, 0, 4, 4, 3),   # 4-bit at head_dim 64, causal rows
    ("turboquant_il", 2, 8, 32, 8, 128, 2000, 128, 1, 4, 0),  # config-4 heads, hybrid buffer
    ("turboquant_il", 2, 2, 6, 2, 128, 300, 20, 5, 3, 1),     # causal across the buffer
    ("turboquant", 3, 1, 8, 2, 128, 777, 16, 1, 8, 0),  # vector-ALU kernel, 64 heavy dims
    ("turboquant", 4, 1, 8, 2, 128, 400, 0, 4, 2, 2),   # vector-ALU kernel, causal rows
])
def test_decode_mfma_heavy_blocks(kind, bits, b, hq, hkv, d, t_kv, t_buf, t_q, n_heavy, splits):
    """fp16 heavy-block keys on the interleaved fp16, grouped and TurboQuant
    decodes: the heavy blocks' exact dot products replace their table
    entries (the matrix-core kernels read a codebook whose heavy blocks are
    zero; the vector-ALU TurboQuant kernel skips them in its own table), as
    the oracle's two-pass SDPA with heavy keys does."""
    cap = max(((t_kv + 15) // 16) * 16, 16)
    cents, perm, idx, vals16, q = decode_case(200 + n_heavy + t_kv, b, hq, hkv, d, t_kv, t_q, cap)
    rng = np.random.default_rng(201 + n_heavy + t_buf)
    heavy = np.sort(rng.permutation(d // 8)[:n_heavy])
    hd = np.concatenate([np.arange(x * 8, x * 8 + 8) for x in heavy]).astype(np.int32)
    kh = np.zeros((b, hkv, cap, hd.size), np.float16)
    kh[:, :, :t_kv] = rng.standard_normal((b, hkv, t_kv, hd.size)).astype(np.float16)
    scoring = cents.copy()
    scoring[heavy] = 0.0
    kb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(np.float16)
    vb = rng.standard_normal((b, hkv, t_buf + 3, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    causal = t_q > 1
    total = t_kv + t_buf
    kw = dict(causal=causal, q_offset=total - t_q if causal else 0, out_dtype=torch.float32,
              n_splits=splits, buf_keys=t(kb) if t_buf else None,
              buf_values=t(vb) if t_buf else None, buf_len=t_buf, k_heavy=t(kh),
              heavy_dims=t(hd))
    vals = np.zeros((b, hkv, total, d), np.float64)
    vals[:, :, t_kv:] = vb[:, :, :t_buf]
    if kind == "il8":
        out = _hip.decode_attn_il8(t(q), scale, t(perm), t(scoring), t(idx),
                                   to_il8(vals16, cap), t_kv, **kw)
        vals[:, :, :t_kv] = vals16[:, :, :t_kv]
    elif kind == "grouped_il":
        group = d // 2
        _, packed, sc, ze, il = grouped_case(t_kv + 9, b, hkv, t_kv, d, bits, group, cap)
        out = _hip.decode_attn_grouped_il(t(q), scale, t(perm), t(scoring), t(idx), il, sc, ze,
                                          bits, group, t_kv, **kw)
        for bi in range(b):
            for hi in range(hkv):
                vals[bi, hi, :t_kv] = O.dequantize_values(
                    packed[bi, hi, :t_kv].cpu().numpy().view(np.uint32),
                    sc[bi, hi, :t_kv].float().cpu().numpy(),
                    ze[bi, hi, :t_kv].float().cpu().numpy(), d, bits, group)
    else:
        codes = rng.integers(0, 1 << bits, (b, hkv, cap, d)).astype(np.uint8)
        packed = O.pack_indices(codes, bits).astype(np.uint32)
        norms = (rng.random((b, hkv, cap)) * 3 + 0.1).astype(np.float32)
        levels = (O.lloyd_max_gaussian(bits)[0] / np.sqrt(d)).astype(np.float32)
        rot = O.rotation_matrix(d, 43)
        if kind == "turboquant_il":
            codes_il = torch.zeros((b, hkv, cap // 16, d), dtype=torch.int32, device=DEV)
            _hip.pack_grouped_il(t(packed.view(np.int32)), 2, codes_il, 0)
            out = _hip.decode_attn_turboquant_il(t(q), scale, t(perm), t(scoring), t(idx),
                                                 codes_il, t(norms), levels, t(rot), t_kv, **kw)
        else:
            # the raw centroids: this kernel leaves the heavy blocks out itself
            out = _hip.decode_attn_turboquant(t(q), scale, t(perm), t(cents), t(idx),
                                              t(packed.view(np.int32)), t(norms), levels,
                                              t(rot), bits, t_kv, **kw)
        vals[:, :, :t_kv] = O.turboquant_decode(packed[:, :, :t_kv], norms[:, :, :t_kv], rot,
                                                levels, d, bits)
    torch.cuda.synchronize()
    _hip.check_decode_waits()
    ref = O.sdpa_two_pass(q, scale, perm, cents, idx[:, :, :t_kv], kb[:, :, :t_buf], vals,
                          mask="causal" if causal else None, heavy_keys=kh[:, :, :t_kv],
                          heavy_dims=hd)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL
    # the heavy dims change the result (the check above is not vacuous)
    ref0 = O.sdpa_two_pass(q, scale, perm, scoring, idx[:, :, :t_kv], kb[:, :, :t_buf], vals,
                           mask="causal" if causal else None)
    assert rel_err(ref0, ref) > 10 * REL_TOL


def test_decode_mfma_heavy_blocks_limits():
    """The matrix-core decodes take at most 32 heavy dims, and none on the
    loader-wave shape (4-bit grouped codes at head_dim 128): both report
    SunShapeUnsupported, the cue for the caller's two-pass path."""
    b, hq, hkv, d, t_kv = 1, 8, 2, 128, 300
    cap = 304
    cents, perm, idx, vals16, q = decode_case(210, b, hq, hkv, d, t_kv, 1, cap)
    hd40 = np.arange(40, dtype=np.int32)
    kh40 = np.zeros((b, hkv, cap, 40), np.float16)
    with pytest.raises(_hip.SunShapeUnsupported):
        _hip.decode_attn_il8(t(q), 0.088, t(perm), t(cents), t(idx), to_il8(vals16, cap), t_kv,
                             k_heavy=t(kh40), heavy_dims=t(hd40))
    hd8 = np.arange(8, dtype=np.int32)
    kh8 = np.zeros((b, hkv, cap, 8), np.float16)
    _, _, sc, ze, il = grouped_case(211, b, hkv, t_kv, d, 4, 64, cap)
    with pytest.raises(_hip.SunShapeUnsupported):
        _hip.decode_attn_grouped_il(t(q), 0.088, t(perm), t(cents), t(idx), il, sc, ze, 4, 64,
                                    t_kv, k_heavy=t(kh8), heavy_dims=t(hd8))


@pytest.mark.parametrize("q_dtype", [np.float32, "bf16"])
def test_decode_sunshape_v_heavy_blocks_wide_queries(q_dtype):
    """bf16 and fp32 queries on the matrix-core SunShape-value decode: the
    heavy-dim products take the query as an fp16 hi/lo pair (exact for fp32
    only to ~22 bits, within the bar), the LUT takes it in fp32."""
    b, hq, hkv, t_kv, d, bd = 1, 8, 2, 900, 128, 4
    cap = 912
    cents, perm, idx, _, q16 = decode_case(95, b, hq, hkv, d, t_kv, 1, cap)
    rng = np.random.default_rng(96)
    q = (q16.astype(np.float32) * 1.3 + 1e-3 * rng.standard_normal(q16.shape)).astype(np.float32)
    hd = np.concatenate([np.arange(x * 8, x * 8 + 8) for x in (1, 6, 9, 12)]).astype(np.int32)
    kh = np.zeros((b, hkv, cap, hd.size), np.float16)
    kh[:, :, :t_kv] = rng.standard_normal((b, hkv, t_kv, hd.size)).astype(np.float16)
    v_cents = rng.standard_normal((d // bd, 256, bd)).astype(np.float32)
    v_idx = rng.integers(0, 256, (b, hkv, cap, d // bd)).astype(np.uint8)
    vperm = rng.permutation(d).astype(np.int32)
    inv = O.invert_permutation(vperm)
    m = np.zeros((d, d), np.float32)
    m[inv, np.arange(d)] = 1.0
    # bf16 queries come pre-scaled (scale 1): q * 1 rounds to itself in bf16
    # and in the float32 the oracle sees
    qt, scale = (t(q), 0.088) if q_dtype == np.float32 else (t(q * 0.088).to(torch.bfloat16), 1.0)
    qref = qt.float().cpu().numpy()
    out = _hip.decode_attn_sunshape_v(qt, scale, t(perm), t(cents), t(idx), t(v_idx), t(v_cents),
                                      t(m), t_kv, out_dtype=torch.float32, k_heavy=t(kh),
                                      heavy_dims=t(hd))
    torch.cuda.synchronize()
    vals = np.stack([np.stack([O.dequantize_blockvq(v_idx[0, hi, :t_kv], v_cents, inv)
                               for hi in range(hkv)])])
    ref = O.sdpa_two_pass(qref, scale, perm, cents, idx[:, :, :t_kv], None, vals,
                          heavy_keys=kh[:, :, :t_kv], heavy_dims=hd)
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


def test_transformed_decode_leaves_split_counters_zero():
    """Regression: a single-split TurboQuant / SunShape-value decode keeps its
    transformed-basis rows clear of the workspace's split counters, so a
    matrix-core decode with an in-kernel merge on the same (per-stream)
    workspace still merges correctly afterwards."""
    b, hq, hkv, d, t_small, t_big = 2, 8, 2, 128, 200, 4000
    cents, perm, idx, vals, q = decode_case(123, b, hq, hkv, d, t_big, 1, t_big)
    rng = np.random.default_rng(124)
    packed = O.pack_indices(rng.integers(0, 4, (b, hkv, t_big, d)), 2).astype(np.uint32)
    norms = (rng.random((b, hkv, t_big)) + 0.5).astype(np.float32)
    levels = (O.lloyd_max_gaussian(2)[0] / np.sqrt(d)).astype(np.float32)
    rot = O.rotation_matrix(d, 43)
    scale = 1.0 / np.sqrt(d)
    for _ in range(2):
        _hip.decode_attn_turboquant(t(q), scale, t(perm), t(cents), t(idx),
                                    t(packed.view(np.int32)), t(norms), levels, t(rot), 2,
                                    t_small, out_dtype=torch.float32, n_splits=1)
        out = _hip.decode_attn_il8(t(q), scale, t(perm), t(cents), t(idx), to_il8(vals, t_big),
                                   t_big, out_dtype=torch.float32, n_splits=8)
        torch.cuda.synchronize()
        ws = _hip.decode_workspace(torch.device(DEV), 1)
        assert not ws[:64 * 1024].any()
        ref = O.sdpa(q, idx, vals, cents, perm, scale)
        assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


def test_bounded_wait_failure_reaches_python():
    """A bounded in-kernel wait that gives up is reported, not hidden: with
    the spin limit forced to 0 from the host (every wait gives up after one
    sleep while every wave still ends normally) the matrix-core decode sets
    the sticky wait-failure word and its pinned host copy; the next decode
    call raises SunShapeWaitError before launching (a plain load of the host
    copy, no synchronisation), ss_decode_wait_failures returns SS_ERR_WAIT,
    and with wait checks on the failing call itself raises.  With the default limit restored the same decode is correct and
    reports nothing."""
    b, hq, hkv, d, t_kv = 1, 32, 8, 128, 32768
    cents, perm, idx, vals, q = decode_case(71, b, hq, hkv, d, t_kv)
    args = (t(q), 1.0 / np.sqrt(d), t(perm), t(cents), t(idx), to_il8(vals, t_kv), t_kv)
    assert _hip.decode_wait_failures() == 0 and _hip.decode_wait_flag() == 0
    prev = _hip.set_wait_checks(False)
    try:
        _hip.set_spin_limit(0)
        _hip.decode_attn_il8(*args, out_dtype=torch.float32)
        torch.cuda.synchronize()
        # the pinned host copy is set once the failed launch has run ...
        assert _hip.decode_wait_flag() != 0
        # ... so the next decode call raises before it launches, without a
        # per-call synchronisation (the check clears both words)
        with pytest.raises(_hip.SunShapeWaitError):
            _hip.decode_attn_il8(*args, out_dtype=torch.float32)
        assert _hip.decode_wait_flag() == 0 and _hip.decode_wait_failures() == 0
        _hip.decode_attn_il8(*args, out_dtype=torch.float32)
        flags = _hip.decode_wait_failures(clear=False)
        assert flags != 0 and flags & ~7 == 0
        with pytest.raises(_hip.SunShapeWaitError):
            _hip.check_decode_waits()
        assert _hip.decode_wait_failures() == 0  # cleared by the check
        assert _hip.decode_wait_flag() == 0
        _hip.set_wait_checks(True)
        with pytest.raises(_hip.SunShapeWaitError):
            _hip.decode_attn_il8(*args, out_dtype=torch.float32)
    finally:
        _hip.set_spin_limit(None)
        _hip.set_wait_checks(prev)
        _hip.decode_wait_failures()
    out = _hip.decode_attn_il8(*args, out_dtype=torch.float32)
    assert _hip.decode_wait_failures() == 0
    _hip.check_decode_waits()
    ref = O.sdpa(q, idx, vals, cents, perm, 1.0 / np.sqrt(d))
    assert rel_err(out.cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("rise,qdt", [(40.0, "f16"), (600.0, "f16"), (40.0, "f32")])
def test_prefill_rising_scores(rise, qdt):
    """Causal prefill over scores that keep rising along the prompt: rows keep
    their running maxima while a sub-tile stays within a few log2 units of
    them (probabilities above 1 in the fp16 staging) and rescale past it."""
    t_kv = 1000
    cap = ((t_kv + 15) // 16) * 16
    cents, perm, idx, vals, q, scale = ramp_case(19, t_kv, cap, rise, t_q=t_kv)
    qt = t(q) if qdt == "f16" else t(q.astype(np.float32))
    cb = _hip.codebook_f16x2(t(cents))
    out = _hip.prefill_attn_il8(qt, scale, t(perm), cb, 256, t(idx), to_il8(vals, cap), t_kv, causal=True,
                                q_offset=0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.sdpa(q, idx[:, :, :t_kv], vals[:, :, :t_kv], cents, perm, scale, mask="causal")
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, ref) <= REL_TOL


@pytest.mark.parametrize("b,hq,hkv,t_q,t_kv,causal,qdt,nc", [
    (1, 32, 8, 200, 200, True, "f16", 256),      # rep 4: 32 positions per workgroup, ragged
    (2, 8, 8, 96, 300, True, "f16", 256),        # rep 1, chunked prefill after 204 cached tokens
    (1, 16, 2, 64, 64, False, "f16", 256),       # rep 8, unmasked
    (1, 8, 2, 130, 1000, True, "bf16", 100),     # bf16 queries (32-row kernel), 100 centroids
    (1, 4, 1, 33, 77, True, "f32", 256),         # f32 queries, partial tiles everywhere
])
def test_prefill_il8_matches_oracle(b, hq, hkv, t_q, t_kv, causal, qdt, nc):
    """ss_prefill_attn_il8: a prompt's rows (keys reconstructed from the
    prepared codebook, both products on the matrix cores) equal the oracle
    SDPA, causal rows seeing keys up to q_offset + i, and agree with the
    decode kernel on the same inputs."""
    d = 128
    cap = ((t_kv + 15) // 16) * 16
    cents, perm, idx, vals, q16 = decode_case(700 + t_q + t_kv, b, hq, hkv, d, t_kv, t_q, cap, nc=nc)
    scale = 1.0 / np.sqrt(d)
    if qdt == "f16":
        qt = t(q16)
    elif qdt == "bf16":  # pre-scaled: q * 1 rounds to itself in bf16 and in the oracle's float32
        qt = t(q16.astype(np.float32) * scale).to(torch.bfloat16)
        scale = 1.0
    else:
        qt = t(q16.astype(np.float32) * 1.3 + 1e-3)
    qref = qt.float().cpu().numpy() if qdt != "f16" else q16
    v8 = to_il8(vals, cap)
    cb = _hip.codebook_f16x2(t(cents))
    q_off = t_kv - t_q if causal else 0
    out = _hip.prefill_attn_il8(qt, scale, t(perm), cb, nc, t(idx), v8, t_kv, causal=causal,
                                q_offset=q_off, out_dtype=torch.float32)
    ref_dec = _hip.decode_attn_il8(qt, scale, t(perm), t(cents), t(idx), v8, t_kv, causal=causal,
                                   q_offset=q_off, out_dtype=torch.float32, codebook=cb)
    torch.cuda.synchronize()
    ref = O.sdpa(qref, idx[:, :, :t_kv], vals[:, :, :t_kv], cents, perm, scale,
                 mask="causal" if causal else None)
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, ref) <= REL_TOL
    assert rel_err(got, ref_dec.cpu().numpy()) <= REL_TOL


@pytest.mark.parametrize("b,hq,hkv,d,t_cache,n_new,t_q,causal", [
    (1, 32, 8, 128, 4096, 1, 1, False),   # the metric shape's decode step
    (2, 16, 2, 128, 1003, 3, 1, False),   # rep 8: two row groups of a head, one writes
    (1, 8, 2, 64, 515, 4, 4, True),       # head_dim 64, four new tokens as causal rows
    (2, 8, 8, 128, 40, 2, 1, False),      # a short cache (one split), rep 1
])
def test_decode_step_il8_equals_append_then_decode(b, hq, hkv, d, t_cache, n_new, t_q, causal):
    """ss_decode_step_il8 (encode the new tokens, attend every token, store
    the new ones, one launch) leaves the cache exactly as ss_append_kv_il8
    does (index rows and interleaved values, bit for bit) and returns the
    decode over the appended cache (the new tokens attended in float32
    instead of through the matrix cores: within a few 1e-6), which matches
    the oracle."""
    rng = np.random.default_rng(900 + t_cache + n_new)
    nb = d // 8
    cents = t(rng.standard_normal((nb, 256, 8)).astype(np.float32))
    perm = t(rng.permutation(d).astype(np.int32))
    t_all = t_cache + n_new
    cap = ((t_all + 31) // 8) * 8
    keys = t(rng.standard_normal((b, hkv, t_all, d)).astype(np.float16))
    vals = t(rng.standard_normal((b, hkv, t_all, d)).astype(np.float16))
    q = t(rng.standard_normal((b, hq, t_q, d)).astype(np.float16))
    idx_a = torch.zeros((b, hkv, cap, nb), dtype=torch.uint8, device=DEV)
    v8_a = torch.zeros((b, hkv, cap // 8, d, 8), dtype=torch.float16, device=DEV)
    app = _hip.PreparedAppend(perm, cents, None, idx_a, v8_a)
    app(keys[:, :, :t_cache], vals[:, :, :t_cache], 0)
    idx_b, v8_b = idx_a.clone(), v8_a.clone()
    k_new, v_new = keys[:, :, t_cache:].contiguous(), vals[:, :, t_cache:].contiguous()
    app(k_new, v_new, t_cache)
    cb = _hip.codebook_f16x2(cents)
    scale = 1.0 / np.sqrt(d)
    q_off = t_all - t_q if causal else 0
    ref = _hip.decode_attn_il8(q, scale, perm, cents, idx_a, v8_a, t_all, causal=causal,
                               q_offset=q_off, out_dtype=torch.float32, codebook=cb)
    got = _hip.decode_step_il8(q, scale, perm, cb, cents, idx_b, v8_b, t_cache, k_new, v_new,
                               causal=causal, q_offset=q_off, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(idx_b, idx_a)
    assert torch.equal(v8_b.view(torch.int16), v8_a.view(torch.int16))
    assert rel_err(got.cpu().numpy(), ref.cpu().numpy()) <= 2e-5
    oref = O.sdpa(q.cpu().numpy(), idx_a[:, :, :t_all].cpu().numpy(),
                  vals.cpu().numpy(), cents.cpu().numpy(), perm.cpu().numpy(), scale,
                  mask="causal" if causal else None)
    assert rel_err(got.cpu().numpy(), oref) <= REL_TOL


def test_decode_step_il8_ties_take_the_exact_ranking():
    """New keys exactly halfway between two centroids of every block (an exact
    tie, which no float error bound can clear) and keys a hair closer to the
    second: the step's encode falls back to the exact ranking, giving the
    lower index on the tie and the nearer centroid otherwise, as the encoder
    does (ss_append_kv_il8)."""
    rng = np.random.default_rng(77)
    b, hq, hkv, d, t_cache, nb = 1, 8, 2, 128, 300, 16
    c = rng.standard_normal((nb, 256, 8)).astype(np.float32) * 0.5
    c[:, 3, :] = 1.0   # the two centroids every new key sits between
    c[:, 7, :] = 3.0
    cents = t(c)
    perm = t(rng.permutation(d).astype(np.int32))
    keys = t(rng.standard_normal((b, hkv, t_cache + 2, d)).astype(np.float16))
    vals = t(rng.standard_normal((b, hkv, t_cache + 2, d)).astype(np.float16))
    keys[:, :, t_cache] = 2.0                                  # tie: index 3
    near = np.full(d, 2.0, np.float32)
    near[perm.cpu().numpy()[0::8]] = np.float16(2.0 + 2.0 ** -9)  # block dim 0 a hair nearer 7
    keys[:, :, t_cache + 1] = t(near.astype(np.float16))
    cap = t_cache + 12 - (t_cache + 12) % 8
    idx_a = torch.zeros((b, hkv, cap, nb), dtype=torch.uint8, device=DEV)
    v8_a = torch.zeros((b, hkv, cap // 8, d, 8), dtype=torch.float16, device=DEV)
    app = _hip.PreparedAppend(perm, cents, None, idx_a, v8_a)
    app(keys[:, :, :t_cache], vals[:, :, :t_cache], 0)
    idx_b, v8_b = idx_a.clone(), v8_a.clone()
    k_new, v_new = keys[:, :, t_cache:].contiguous(), vals[:, :, t_cache:].contiguous()
    app(k_new, v_new, t_cache)
    q = t(rng.standard_normal((b, hq, 1, d)).astype(np.float16))
    cb = _hip.codebook_f16x2(cents)
    _hip.decode_step_il8(q, 0.088, perm, cb, cents, idx_b, v8_b, t_cache, k_new, v_new)
    torch.cuda.synchronize()
    assert torch.equal(idx_b, idx_a)
    got = idx_b[:, :, t_cache:t_cache + 2].cpu().numpy()
    assert (got[:, :, 0] == 3).all() and (got[:, :, 1] == 7).all()


def test_decode_step_il8_rejects_what_it_cannot_take():
    """Host checks before any launch: no new tokens or more than
    MAX_STEP_TOKENS, an empty cache, tokens past the capacity, non-fp16 new
    tokens."""
    rng = np.random.default_rng(5)
    cents = t(rng.standard_normal((16, 256, 8)).astype(np.float32))
    idx = torch.zeros((1, 2, 64, 16), dtype=torch.uint8, device=DEV)
    v8 = torch.zeros((1, 2, 8, 128, 8), dtype=torch.float16, device=DEV)
    cb = _hip.codebook_f16x2(cents)
    q = torch.randn((1, 8, 1, 128), device=DEV).half()

    def new(n, dt=torch.float16):
        return (torch.randn((1, 2, n, 128), device=DEV).to(dt),
                torch.randn((1, 2, n, 128), device=DEV).to(dt))
    for t_cache, kv_, err in ((10, new(_hip.MAX_STEP_TOKENS + 1), _hip.SunShapeUnsupported),
                              (0, new(1), _hip.SunShapeHIPError),
                              (60, new(5), _hip.SunShapeHIPError),
                              (10, new(1, torch.float32), ValueError)):
        with pytest.raises(err):
            _hip.decode_step_il8(q, 0.088, None, cb, cents, idx, v8, t_cache, *kv_)
    torch.cuda.synchronize()
    assert not idx.any() and not v8.any()


def test_hybrid_steps_reject_what_they_cannot_take():
    """Host checks of the one-launch hybrid steps before any launch: no new
    tokens or more than MAX_STEP_TOKENS, more tokens flushed than buffered
    or than a step takes, an empty compressed part, flushed positions past
    the capacity, non-fp16 new tokens, 3-bit codes; nothing is written."""
    rng = np.random.default_rng(6)
    cents = t(rng.standard_normal((16, 256, 8)).astype(np.float32))
    cb = _hip.codebook_f16x2(cents)
    cap = 64
    idx = torch.zeros((1, 2, cap, 16), dtype=torch.uint8, device=DEV)
    il = torch.zeros((1, 2, cap // 16, 128), dtype=torch.int32, device=DEV)
    sc = torch.zeros((1, 2, cap, 2), dtype=torch.float16, device=DEV)
    ze = torch.zeros_like(sc)
    v8 = torch.zeros((1, 2, cap // 8, 128, 8), dtype=torch.float16, device=DEV)
    bk = torch.zeros((1, 2, 32, 128), dtype=torch.float16, device=DEV)
    bv = torch.zeros_like(bk)
    q = torch.randn((1, 8, 1, 128), device=DEV).half()

    def new(n, dt=torch.float16):
        return (torch.randn((1, 2, n, 128), device=DEV).to(dt),
                torch.randn((1, 2, n, 128), device=DEV).to(dt))
    cases = ((10, 8, 1, new(_hip.MAX_STEP_TOKENS + 1), _hip.SunShapeUnsupported),
             (10, 8, 5, new(1), _hip.SunShapeUnsupported),      # more than a step flushes
             (10, 2, 3, new(1), _hip.SunShapeHIPError),         # more than buffered
             (0, 8, 1, new(1), _hip.SunShapeHIPError),          # nothing compressed
             (63, 8, 2, new(1), _hip.SunShapeHIPError),         # flushed past the capacity
             (10, 8, 1, new(1, torch.float32), ValueError))
    plan_g = _hip.prepare_decode_step_grouped_il_hybrid(q, 0.088, None, cb, cents, 16, 256, idx, il,
                                                        sc, ze, 2, 64, bk)
    plan_f = _hip.prepare_decode_step_il8_hybrid(q, 0.088, None, cb, cents, 16, 256, idx, v8, bk)
    for plan in (plan_g, plan_f):
        for t_kv, n_buf, n_flush, kv_, err in cases:
            with pytest.raises(err):
                plan(q, t_kv, bk, bv, n_buf, n_flush, *kv_)
    with pytest.raises(_hip.SunShapeUnsupported):
        _hip.prepare_decode_step_grouped_il_hybrid(q, 0.088, None, cb, cents, 16, 256, idx, il, sc,
                                                   ze, 3, 64, bk)
    torch.cuda.synchronize()
    for x in (idx, il, sc, ze, v8, bk, bv):
        assert not x.any()


def test_prefill_il8_at_the_benchmarked_prompt():
    """The prefill kernel at the benchmarked shape (B=1, 32 query / 8 KV
    heads, a causal 4096-token prompt against its own cache): every row of
    every head agrees with the decode kernel over the same prompt, and two
    query heads (on different KV heads, all 4096 rows) with the oracle."""
    b, hq, hkv, d, t_kv = 1, 32, 8, 128, 4096
    cents, perm, idx, vals, q16 = decode_case(4096, b, hq, hkv, d, t_kv, t_kv)
    scale = 1.0 / np.sqrt(d)
    v8 = to_il8(vals, t_kv)
    cb = _hip.codebook_f16x2(t(cents))
    out = _hip.prefill_attn_il8(t(q16), scale, t(perm), cb, 256, t(idx), v8, t_kv, causal=True,
                                q_offset=0, out_dtype=torch.float32)
    ref_dec = _hip.decode_attn_il8(t(q16), scale, t(perm), t(cents), t(idx), v8, t_kv,
                                   causal=True, q_offset=0, out_dtype=torch.float32, codebook=cb)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, ref_dec.cpu().numpy()) <= REL_TOL
    for qh in (3, 21):
        kh = qh // (hq // hkv)
        ref = O.sdpa(q16[:, qh:qh + 1], idx[:, kh:kh + 1], vals[:, kh:kh + 1], cents, perm,
                     scale, mask="causal")
        assert rel_err(got[:, qh:qh + 1], ref) <= REL_TOL


@pytest.mark.parametrize("e2", [20, -20])
def test_queries_beyond_fp16_range_prefill_and_decode(e2):
    """bf16 and float32 queries whose scaled elements lie beyond fp16's range
    (2^20 times larger than usual, past +-65504) or below its normal range
    (2^20 times smaller, under 2^-14), against centroids scaled the other
    way so the scores stay of order one: the prefill kernels (32-row for
    bf16, 16-row for float32) and the matrix-core decode's LUT take each
    query row scaled by a power of two into fp16's range, so the outputs
    match the oracle at the usual bar instead of saturating or flushing."""
    b, hq, hkv, d, t_q, t_kv = 1, 8, 2, 128, 96, 700
    cap = 704
    cents, perm, idx, vals, q16 = decode_case(880 + e2, b, hq, hkv, d, t_kv, t_q, cap)
    cents = (cents * np.float32(2.0 ** -e2)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    v8 = to_il8(vals, cap)
    cb = _hip.codebook_f16x2(t(cents))
    for qdt in (torch.bfloat16, torch.float32):
        # pre-scaled so q * 1 rounds to itself in the query dtype and the oracle
        qt = t(q16.astype(np.float32) * np.float32(scale * 2.0 ** e2)).to(qdt)
        qref = qt.float().cpu().numpy()
        big = np.abs(qref).max()
        assert (big > 65504) if e2 > 0 else (big < 2.0 ** -14)
        out = _hip.prefill_attn_il8(qt, 1.0, t(perm), cb, 256, t(idx), v8, t_kv, causal=True,
                                    q_offset=t_kv - t_q, out_dtype=torch.float32)
        dec = _hip.decode_attn_il8(qt[:, :, -4:].contiguous(), 1.0, t(perm), t(cents), t(idx), v8,
                                   t_kv, causal=True, q_offset=t_kv - 4, out_dtype=torch.float32,
                                   codebook=cb)
        torch.cuda.synchronize()
        ref = O.sdpa(qref, idx[:, :, :t_kv], vals[:, :, :t_kv], cents, perm, 1.0, mask="causal")
        got = out.cpu().numpy()
        assert np.isfinite(got).all() and rel_err(got, ref) <= REL_TOL, qdt
        gd = dec.cpu().numpy()
        assert np.isfinite(gd).all() and rel_err(gd, ref[:, :, -4:]) <= REL_TOL, qdt


def test_score_gather_heads_matches_per_head_and_oracle():
    """ss_score_gather_heads: every (batch, KV head) of a cache-shaped,
    strided index view in one launch -- bit-identical to the per-head
    ss_score_gather (same sums in the same order), and the oracle's gather
    within float32 rounding; also rows not a multiple of the row group and
    a codebook of 100 centroids (the byte-wise index path)."""
    rng = np.random.default_rng(91)
    for (b, hkv, rows, t_kv, cap, nb, nc) in ((2, 3, 4, 1000, 1024, 16, 256),
                                               (1, 2, 7, 333, 512, 16, 100),
                                               (2, 2, 3, 200, 256, 8, 256)):
        lut = t(rng.standard_normal((b, hkv, rows, nb, nc)).astype(np.float32))
        idx_full = t(rng.integers(0, nc, (b, hkv, cap, nb)).astype(np.uint8))
        idx = idx_full[:, :, :t_kv]
        got = _hip.score_gather_heads(lut, idx)
        for bi in range(b):
            for h in range(hkv):
                one = _hip.score_gather(lut[bi, h], idx[bi, h])
                assert torch.equal(got[bi, h], one)
        ref = np.stack([np.stack([O.gather_scores(lut[bi, h].cpu().numpy(), idx[bi, h].cpu().numpy())
                                  for h in range(hkv)]) for bi in range(b)])
        assert np.abs(got.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
