"""GPU parity of the drop-in Python surface (caches, ``sunshape_sdpa``, value
codecs, SDPA router) against the CPU oracle.

Bars: key indices bit-exact except oracle-flagged near-ties; stored values
bit-exact; attention outputs max |gpu - oracle| <= 1e-3 * max |oracle| (fp32
accumulate, float64 oracle; the maximum is over every compared element, not
per element).  The drop-in API returns the query dtype, fp16 here, so those
outputs are compared with the oracle rounded to fp16 (``rel_err16``): the two
roundings differ by at most one fp16 step, below 2^-10 = 9.8e-4 of the
largest element, so the 1e-3 bar still holds the accumulation to a few
1e-5.
"""

import sys
import types

import numpy as np
import pytest
import torch

from oracle import sunshape_oracle as O
import sunshape_mlx_amd as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
REL_TOL = 1e-3


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def rel_err16(got, ref):
    """max |got - fp16(ref)| / max |ref| for an fp16 output ``got``."""
    ref = np.asarray(ref, np.float64)
    r16 = ref.astype(np.float16).astype(np.float64)
    return float(np.abs(np.asarray(got, np.float64) - r16).max() / max(np.abs(ref).max(), 1e-30))


def make_codec(seed, d=128, nc=256, mode="profileperm_baseline"):
    rng = np.random.default_rng(seed)
    nb = d // 8
    codec = S.SunShapeBlockCodec(d, n_centroids=nc, device=DEV,
                                 use_rotation=(mode == "rotated"), rotation_seed=seed)
    state = {"centroids": rng.standard_normal((nb, nc, 8)).astype(np.float32)}
    if mode != "rotated":
        state["permutation"] = rng.permutation(d).astype(np.int32)
    codec.load_state_dict(state)
    return codec


def kv(seed, b, hkv, t_, d, dtype=torch.float16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn((b, hkv, t_, d), generator=g, device=DEV).to(dtype)
    v = torch.randn((b, hkv, t_, d), generator=g, device=DEV).to(dtype)
    return k, v


def oracle_indices(codec, keys):
    cents = codec.centroids.cpu().numpy()
    perm = codec.permutation.cpu().numpy()
    b_, h_, t_, d = keys.shape
    res = O.encode_blockvq(keys.float().cpu().numpy().reshape(-1, d), cents, perm)
    idx, near = res[0], res[1]
    return idx.reshape(b_, h_, t_, -1), near.reshape(b_, h_, t_, -1)


@pytest.mark.parametrize("d,prefill,steps", [(128, 300, 5), (64, 17, 9)])
def test_fp16_cache_store_and_fused_decode(d, prefill, steps):
    codec = make_codec(1, d=d)
    b, hq, hkv = 2, 8, 2
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, head_dim=d)
    assert isinstance(cache, S.SunShapeKVCache) and cache.values_interleaved
    k, v = kv(2, b, hkv, prefill + steps, d)
    cache.update_and_fetch(k[:, :, :prefill], v[:, :, :prefill])
    for s in range(steps):
        sl = slice(prefill + s, prefill + s + 1)
        keys_out, vals_out = cache.update_and_fetch(k[:, :, sl], v[:, :, sl])
    t_kv = prefill + steps
    assert cache.offset == t_kv
    # stored values round-trip bit-exactly through the interleaved layout
    assert torch.equal(cache.values, v)
    assert torch.equal(vals_out, v)
    # key indices: bit-exact except near-ties
    idx_ref, near = oracle_indices(codec, k)
    got = cache.key_indices.cpu().numpy()
    assert np.array_equal(got[~near], idx_ref[~near])
    # returned keys are the dequantised indices
    cents = codec.centroids.cpu().numpy()
    inv = codec.inv_permutation.cpu().numpy()
    khat = O.dequantize_blockvq(got.reshape(-1, d // 8), cents, inv).reshape(b, hkv, t_kv, d)
    assert np.array_equal(keys_out.cpu().numpy(), khat.astype(np.float32))
    # one decode step through the fused MFMA path
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 1.0 / np.sqrt(d), mask=None)
    assert codec.last_score_backend == "hip_fused_mfma"
    ref = O.sdpa(q.cpu().numpy(), got, v.cpu().numpy(), cents, codec.permutation.cpu().numpy(),
                 1.0 / np.sqrt(d))
    assert out.dtype == torch.float16
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL


def test_fp16_cache_causal_prefill_and_capacity_growth():
    codec = make_codec(3)
    b, hq, hkv, d = 1, 8, 2, 128
    cache = S.create_kv_cache(codec, n_kv_heads=hkv)
    k, v = kv(4, b, hkv, 600, d)
    cache.update_and_fetch(k[:, :, :250], v[:, :, :250])   # capacity 256
    cache.update_and_fetch(k[:, :, 250:600], v[:, :, 250:600])  # grows to 768
    assert torch.equal(cache.values, v)
    tq = 16
    q = torch.randn((b, hq, tq, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.1, mask="causal")
    ref = O.sdpa(q.cpu().numpy(), cache.key_indices.cpu().numpy(), v.cpu().numpy(),
                 codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), 0.1,
                 mask="causal")
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL


def test_prompt_prefill_takes_the_prefill_kernel():
    """A prompt (32 query / 8 KV heads, 300 tokens, mask "causal") through
    update_and_fetch and sunshape_sdpa, as mlx-lm's prefill runs it: the
    prefill kernel serves it and matches the oracle; a second chunk of 70
    tokens (chunked prefill, rows offset by the 300 cached ones) too."""
    codec = make_codec(51)
    b, hq, hkv, d = 1, 32, 8, 128
    cache = S.create_kv_cache(codec, n_kv_heads=hkv)
    k, v = kv(52, b, hkv, 370, d)
    q = torch.randn((b, hq, 370, d), device=DEV).to(torch.float16)
    cache.update_and_fetch(k[:, :, :300], v[:, :, :300])
    out = S.sunshape_sdpa(q[:, :, :300].contiguous(), cache, 0.088, mask="causal")
    assert codec.last_score_backend == "hip_prefill_mfma"
    cents = codec.centroids.cpu().numpy()
    perm = codec.permutation.cpu().numpy()
    ref = O.sdpa(q[:, :, :300].cpu().numpy(), cache.key_indices.cpu().numpy(),
                 v[:, :, :300].cpu().numpy(), cents, perm, 0.088, mask="causal")
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    cache.update_and_fetch(k[:, :, 300:], v[:, :, 300:])
    out2 = S.sunshape_sdpa(q[:, :, 300:].contiguous(), cache, 0.088, mask="causal")
    assert codec.last_score_backend == "hip_prefill_mfma"
    ref2 = O.sdpa(q[:, :, 300:].cpu().numpy(), cache.key_indices.cpu().numpy(), v.cpu().numpy(),
                  cents, perm, 0.088, mask="causal")
    assert rel_err16(out2.float().cpu().numpy(), ref2) <= REL_TOL


def test_prepared_decode_follows_the_cache_and_matches_direct_launch():
    """``sunshape_sdpa`` launches the matrix-core decode through a plan kept
    on the cache.  It must give the same bits as the checked one-shot
    launcher, be rebuilt when the cache's buffers are replaced (capacity
    growth) or the query dtype changes, follow the current stream, and grow
    a workspace too small for the split plan before it launches."""
    codec = make_codec(31)
    b, hq, hkv, d, scale = 2, 8, 2, 128, 0.09
    cache = S.create_kv_cache(codec, n_kv_heads=hkv)
    k, v = kv(32, b, hkv, 700, d)
    cache.update_and_fetch(k[:, :, :200], v[:, :, :200])
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)

    def direct(qq, t_kv):
        ops = cache.fused_operands()
        return S._hip.decode_attn_il8(qq, scale, codec.permutation, codec.centroids, ops["idx"],
                                      ops["values"], t_kv, codebook=codec.kernel_codebook())

    out1 = S.sunshape_sdpa(q, cache, scale)
    plan1 = cache._decode_prepared[2]
    assert torch.equal(out1, direct(q, 200))
    assert S.sunshape_sdpa(q, cache, scale) is not out1 and cache._decode_prepared[2] is plan1
    idx_before = cache.fused_operands()["idx"]
    cache.update_and_fetch(k[:, :, 200:700], v[:, :, 200:700])  # capacity grows
    assert cache.fused_operands()["idx"] is not idx_before
    out2 = S.sunshape_sdpa(q, cache, scale)
    assert cache._decode_prepared[2] is not plan1
    assert torch.equal(out2, direct(q, 700))
    ref = O.sdpa(q.cpu().numpy(), cache.key_indices.cpu().numpy(), v.cpu().numpy(),
                 codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), scale)
    assert rel_err16(out2.float().cpu().numpy(), ref) <= REL_TOL
    qb = q.to(torch.bfloat16)
    out3 = S.sunshape_sdpa(qb, cache, scale)
    assert out3.dtype == torch.bfloat16 and torch.equal(out3, direct(qb, 700))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out4 = S.sunshape_sdpa(q, cache, scale)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(out4, out2)


def test_prepared_decode_grows_a_small_workspace():
    """A split plan that needs more than the per-stream workspace holds: the
    prepared launch sees the library's workspace error (raised before any
    launch), grows the workspace and launches once."""
    codec = make_codec(33)
    b, hq, hkv, d, t_kv = 8, 32, 8, 128, 4096
    splits, need = S._hip.decode_plan(S._hip.KIND_IL8, b, hq, hkv, 1, d, t_kv)
    assert splits > 1 and need > (256 << 10)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, max_tokens=t_kv)
    k, v = kv(34, b, hkv, t_kv, d)
    cache.update_and_fetch(k, v)
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    key = (0, S._hip.stream_handle(DEV))
    S._hip._ws_cache[key] = torch.zeros(256 << 10, dtype=torch.uint8, device=DEV)
    disp = S.get_kernel_stats().get("sunshape_fused_attention_mfma_hip", 0)
    out = S.sunshape_sdpa(q, cache, 0.05)
    assert S.get_kernel_stats().get("sunshape_fused_attention_mfma_hip", 0) == disp + 1
    assert S._hip._ws_cache[key].numel() >= need
    ops = cache.fused_operands()
    ref = S._hip.decode_attn_il8(q, 0.05, codec.permutation, codec.centroids, ops["idx"],
                                 ops["values"], t_kv, codebook=codec.kernel_codebook())
    assert torch.equal(out, ref)


def test_mask_array_takes_two_pass_and_matches():
    codec = make_codec(5)
    b, hq, hkv, d, t_kv, tq = 1, 4, 1, 128, 96, 3
    cache = S.create_kv_cache(codec, n_kv_heads=hkv)
    k, v = kv(6, b, hkv, t_kv, d)
    cache.update_and_fetch(k, v)
    q = torch.randn((b, hq, tq, d), device=DEV).to(torch.float16)
    rng = np.random.default_rng(7)
    m_add = rng.standard_normal((tq, t_kv)).astype(np.float32)
    out = S.sunshape_sdpa(q, cache, 0.09, mask=torch.from_numpy(m_add))
    assert codec.last_score_backend == "hip"
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.09, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), cache.key_indices.cpu().numpy(), None,
                          v.cpu().numpy(), mask=m_add)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    m_bool = rng.random((tq, t_kv)) > 0.3
    m_bool[1] = False  # every key masked: the reference averages the values
    out = S.sunshape_sdpa(q, cache, 0.09, mask=torch.from_numpy(m_bool))
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.09, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), cache.key_indices.cpu().numpy(), None,
                          v.cpu().numpy(), mask=m_bool)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    mean = v[0, 0].double().mean(dim=0).cpu().numpy()
    assert np.abs(ref[0, :, 1] - mean).max() < 1e-12
    assert rel_err16(out[0, :, 1].float().cpu().numpy(), np.broadcast_to(mean, (hq, d))) <= REL_TOL


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.float16])
def test_hybrid_grouped_fused_and_buffered(scale_dtype):
    codec = make_codec(8)
    b, hq, hkv, d = 1, 8, 2, 128
    k, v = kv(9, b, hkv, 300, d)
    # buffer_size 0: every token is compressed, the fused dequant path runs
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="grouped", value_bits=2,
                              buffer_size=0, value_scale_dtype=scale_dtype)
    cache.update_and_fetch(k, v)
    assert cache.buffer_offset == 0 and cache.compressed_offset == 300
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.088)
    assert codec.last_score_backend == "hip_fused_mfma_dequant"
    packed = cache.values_packed_raw.cpu().numpy()
    sc = cache.value_scales_raw.float().cpu().numpy()
    zr = cache.value_zeros_raw.float().cpu().numpy()
    vals = O.dequantize_values(packed.reshape(-1, packed.shape[-1]), sc.reshape(-1, sc.shape[-1]),
                               zr.reshape(-1, zr.shape[-1]), d, 2, 64).reshape(b, hkv, 300, d)
    ref = O.sdpa(q.cpu().numpy(), cache.key_indices.cpu().numpy(), vals,
                 codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), 0.088)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    # default buffer: 128 recent tokens stay fp16, the two-pass path runs
    cache2 = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="grouped", value_bits=2,
                               value_scale_dtype=scale_dtype)
    cache2.update_and_fetch(k, v)
    assert cache2.buffer_offset == 128 and cache2.compressed_offset == 172
    out2 = S.sunshape_sdpa(q, cache2, 0.088)
    assert codec.last_score_backend == "hip_fused_mfma_dequant_buffer"
    vals_all = np.concatenate([vals[:, :, :172], v[:, :, 172:].float().cpu().numpy()], axis=2)
    ref2 = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                           codec.centroids.cpu().numpy(), cache2.key_indices.cpu().numpy(),
                           cache2.buffer_keys.float().cpu().numpy(), vals_all)
    assert rel_err16(out2.float().cpu().numpy(), ref2) <= REL_TOL
    # trim removes buffered tokens first (reference cache.py:954-963)
    cache2.trim(130)
    assert cache2.buffer_offset == 0 and cache2.compressed_offset == 170


@pytest.mark.parametrize("bits,group", [(2, 64), (4, 128), (4, 64), (2, 128)])
def test_hybrid_grouped_interleaved_appends_and_trim(bits, group):
    """Grouped codes kept token-interleaved: appends of ragged sizes (flushes
    that start and end inside a code word), a trim into compressed storage
    and a re-append read back as the oracle's quantisation bit for bit, and
    the fused decode over them matches the oracle."""
    codec = make_codec(21)
    b, hq, hkv, d = 2, 8, 2, 128
    k, v = kv(22 + bits, b, hkv, 420, d)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="grouped", value_bits=bits,
                              value_group_size=group, buffer_size=0)
    pos = 0
    for n in (37, 1, 90, 200):
        cache.update_and_fetch(k[:, :, pos:pos + n], v[:, :, pos:pos + n])
        pos += n
    cache.trim(50)
    pos -= 50
    cache.update_and_fetch(k[:, :, pos:pos + 92], v[:, :, pos:pos + 92])
    pos += 92
    assert cache.compressed_offset == pos == 370 and cache.buffer_offset == 0
    vf = v[:, :, :pos].float().cpu().numpy().reshape(-1, d)
    packed_ref, sc_ref, zr_ref, _ = O.quantize_values(vf, bits, group)
    got = cache.values_packed_raw.cpu().numpy().reshape(-1, packed_ref.shape[-1])
    assert np.array_equal(got.view(np.uint32), packed_ref.view(np.uint32))
    assert np.array_equal(cache.value_scales_raw.cpu().numpy().reshape(-1, d // group), sc_ref)
    assert np.array_equal(cache.value_zeros_raw.cpu().numpy().reshape(-1, d // group), zr_ref)
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.088)
    assert codec.last_score_backend == "hip_fused_mfma_dequant"
    vals = O.dequantize_values(packed_ref, sc_ref, zr_ref, d, bits, group).reshape(b, hkv, pos, d)
    ref = O.sdpa(q.cpu().numpy(), cache.key_indices.cpu().numpy(), vals,
                 codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), 0.088)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    # the dequantised values the two-pass path reads agree with the oracle's
    assert rel_err(cache.values.float().cpu().numpy(), vals) <= 1e-3


@pytest.mark.parametrize("buf,t_total,tq,causal,dtype", [
    (128, 700, 1, False, torch.float16),    # decode step, default buffer
    (200, 1000, 1, False, torch.float16),   # buffer shares longer than one 64-token chunk
    (64, 300, 5, True, torch.float16),      # prefill rows, causal across the buffer
    (128, 450, 1, False, torch.bfloat16),   # bf16 buffer
    (128, 140, 1, False, torch.float32),    # mostly buffer, f32
])
def test_hybrid_buffer_joins_fused_decode(buf, t_total, tq, causal, dtype):
    """Hybrid grouped caches with buffered tokens stay on the fused kernel;
    the result equals the reference's two-pass path over the same cache.
    bf16 caches keep the two passes: the reference rounds the dequantised
    values to bf16 there, which the fused kernel (float32 values) would
    not reproduce to 1e-3."""
    codec = make_codec(31)
    b, hq, hkv, d = 2, 8, 2, 128
    k, v = kv(32 + buf, b, hkv, t_total, d, dtype=dtype)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="grouped", value_bits=2,
                              buffer_size=buf, dtype=dtype)
    pos = 0
    for n in (t_total - 37, 30, 7):
        cache.update_and_fetch(k[:, :, pos:pos + n], v[:, :, pos:pos + n])
        pos += n
    assert cache.buffer_offset > 0 and cache.compressed_offset > 0
    q = torch.randn((b, hq, tq, d), device=DEV).to(torch.float16)
    mask = "causal" if causal else None
    out = S.sunshape_sdpa(q, cache, 0.088, mask=mask)
    assert codec.last_score_backend == ("hip" if dtype == torch.bfloat16
                                        else "hip_fused_mfma_dequant_buffer")
    tc = cache.compressed_offset
    vals = cache.values.float().cpu().numpy()  # compressed values dequantised, then buffer
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), cache.key_indices.cpu().numpy(),
                          cache.buffer_keys.float().cpu().numpy(), vals, mask=mask)
    assert vals.shape[2] == tc + cache.buffer_offset
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("backend,bits,dtype,buf,t_total,tq,causal", [
    ("grouped", 3, torch.float16, 128, 700, 1, False),   # 3-bit codes: reference packed rows
    ("grouped", 3, torch.float16, 64, 300, 5, True),     # prefill rows, causal across the buffer
    ("grouped", 3, torch.float32, 200, 1000, 1, False),  # buffer past one 256-token chunk
    ("fp16", None, torch.bfloat16, 120, 450, 1, False),  # bf16 values: token-major storage
    ("fp16", None, torch.float32, 96, 300, 5, True),
])
def test_hybrid_buffer_joins_fused_valu_decode(backend, bits, dtype, buf, t_total, tq, causal):
    """Hybrid caches whose values take the vector-ALU decodes (3-bit grouped
    codes in the reference's packed rows, token-major bf16 / f32 values) keep
    their buffered tokens in the fused launch (one more split partial), equal
    to the reference's two-pass path over the same cache."""
    codec = make_codec(33)
    b, hq, hkv, d = 2, 8, 2, 128
    k, v = kv(34 + buf, b, hkv, t_total, d, dtype=dtype)
    kw = {"value_bits": bits} if bits else {}
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend=backend, buffer_size=buf,
                              dtype=dtype, **kw)
    assert isinstance(cache, S.HybridSunShapeKVCache)
    pos = 0
    for n in (t_total - 37, 30, 7):
        cache.update_and_fetch(k[:, :, pos:pos + n], v[:, :, pos:pos + n])
        pos += n
    assert cache.buffer_offset > 0 and cache.compressed_offset > 0
    assert cache.fused_operands()["kind"] == ("grouped" if backend == "grouped" else "dense")
    q = torch.randn((b, hq, tq, d), device=DEV).to(torch.float16)
    mask = "causal" if causal else None
    out = S.sunshape_sdpa(q, cache, 0.088, mask=mask)
    assert codec.last_score_backend == ("hip_fused_dequant_buffer" if backend == "grouped"
                                        else "hip_fused_buffer")
    vals = cache.values.float().cpu().numpy()  # compressed values dequantised, then buffer
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), cache.key_indices.cpu().numpy(),
                          cache.buffer_keys.float().cpu().numpy(), vals, mask=mask)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("buf,t_total,tq,causal", [
    (96, 700, 1, False),     # decode step (a 128-token buffer makes a SunShapeKVCache)
    (64, 300, 5, True),      # prefill rows, causal across the buffer
    (120, 140, 1, False),    # mostly buffer
])
def test_hybrid_fp16_buffer_joins_fused_decode(buf, t_total, tq, causal):
    """Hybrid fp16-value caches keep compressed values 8-token interleaved;
    with buffered tokens they stay on the matrix-core kernel, equal to the
    reference's two-pass path over the same cache, and a trim into
    compressed storage followed by appends keeps the values exact."""
    codec = make_codec(41)
    b, hq, hkv, d = 2, 8, 2, 128
    k, v = kv(42 + buf, b, hkv, t_total + 40, d)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="fp16", buffer_size=buf)
    assert isinstance(cache, S.HybridSunShapeKVCache)
    pos = 0
    for n in (t_total - 37, 30, 7):
        cache.update_and_fetch(k[:, :, pos:pos + n], v[:, :, pos:pos + n])
        pos += n
    assert cache.buffer_offset > 0 and cache.compressed_offset > 0
    assert torch.equal(cache.values, v[:, :, :pos])
    q = torch.randn((b, hq, tq, d), device=DEV).to(torch.float16)
    mask = "causal" if causal else None

    def check():
        out = S.sunshape_sdpa(q, cache, 0.088, mask=mask)
        assert codec.last_score_backend == "hip_fused_mfma_buffer"
        vals = cache.values.float().cpu().numpy()
        ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                              codec.centroids.cpu().numpy(), cache.key_indices.cpu().numpy(),
                              cache.buffer_keys.float().cpu().numpy(), vals, mask=mask)
        assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL

    check()
    cache.trim(buf + 5)  # all of the buffer and 5 compressed tokens
    pos -= buf + 5
    cache.update_and_fetch(k[:, :, pos:pos + 40], v[:, :, pos:pos + 40])
    pos += 40
    assert torch.equal(cache.values, v[:, :, :pos])
    if cache.buffer_offset and cache.compressed_offset:
        check()


@pytest.mark.parametrize("backend", ["grouped", "turboquant"])
def test_hybrid_buffer_with_rotated_codec_fused(backend):
    """A rotated codec's buffered tokens join the fused softmax too: their
    keys are rotated like the query, (q R^T) . (k R^T) = q . k, and the
    result equals the two-pass path with the rotated query."""
    codec = make_codec(33, mode="rotated")
    b, hq, hkv, d = 2, 8, 2, 128
    k, v = kv(34, b, hkv, 300, d)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend=backend, value_bits=2)
    cache.update_and_fetch(k, v)
    assert cache.buffer_offset > 0 and cache.compressed_offset > 0
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.088)
    assert codec.last_score_backend.endswith("_buffer")
    vals = cache.values.float().cpu().numpy()
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, None, codec.centroids.cpu().numpy(),
                          cache.key_indices.cpu().numpy(), cache.buffer_keys.float().cpu().numpy(),
                          vals, rotation=codec.rotation.cpu().numpy())
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL


def test_hybrid_fp16_and_sunshape_value_backends():
    codec = make_codec(10)
    b, hq, hkv, d = 1, 4, 1, 128
    k, v = kv(11, b, hkv, 200, d)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="fp16", buffer_size=0)
    assert isinstance(cache, S.HybridSunShapeKVCache)
    cache.update_and_fetch(k, v)
    assert torch.equal(cache.values, v)  # fp16 values kept 8-token interleaved
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.088)
    assert codec.last_score_backend == "hip_fused_mfma"
    ref = O.sdpa(q.cpu().numpy(), cache.key_indices.cpu().numpy(), v.cpu().numpy(),
                 codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), 0.088)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    # SunShape-coded values: the fused decode over gathered value centroids
    vcodec = make_codec(12)
    cache3 = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="sunshape", value_bits=8,
                               value_codec=vcodec, buffer_size=0)
    cache3.update_and_fetch(k, v)
    out3 = S.sunshape_sdpa(q, cache3, 0.088)
    assert codec.last_score_backend == "hip_fused_sunshape_v"
    vals = cache3.values.float().cpu().numpy()
    ref3 = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                           codec.centroids.cpu().numpy(), cache3.key_indices.cpu().numpy(), None,
                           vals)
    assert rel_err16(out3.float().cpu().numpy(), ref3) <= REL_TOL


def test_rotated_codec_fused_decode():
    codec = make_codec(13, mode="rotated")
    b, hq, hkv, d = 1, 8, 2, 128
    cache = S.create_kv_cache(codec, n_kv_heads=hkv)
    k, v = kv(14, b, hkv, 150, d)
    cache.update_and_fetch(k, v)
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.088)
    r = codec.rotation.cpu().numpy().astype(np.float64)
    qs = O.scale_query(q.cpu().numpy(), 0.088).astype(np.float64)
    qt = (qs @ r.T).astype(np.float32).reshape(b, hkv, hq // hkv, 1, d)
    idx = cache.key_indices.cpu().numpy()
    cents = codec.centroids.cpu().numpy()
    vv = v.cpu().numpy()
    ref = np.zeros((b, hq, 1, d))
    for h in range(hkv):
        for rr in range(hq // hkv):
            ref[0, h * (hq // hkv) + rr] = O.fused_attention(qt[0, h, rr], cents, idx[0, h], vv[0, h])
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_turboquant_value_codec_matches_oracle(bits):
    """TurboQuantValueCodec.quantize (value_codecs.py:159-171) against the
    oracle with the oracle's own copy of the reference's Lloyd-Max tables:
    codes bit-exact except coordinates within 1e-5 of a boundary (the
    rotation runs in float32 on the GPU), zero rows included (zero norm,
    every coordinate at the lower-middle code)."""
    d = 128
    tq = S.TurboQuantValueCodec(head_dim=d, bits=bits, seed=43, device=DEV)
    cents, bounds = O.turboquant_tables(bits, d)
    # R is data (the reference draws it from MLX's generator, which is
    # unavailable): the codec's own, checked orthogonal
    rot = tq.rotation.cpu().numpy()
    assert np.abs(rot.astype(np.float64) @ rot.T - np.eye(d)).max() < 1e-5
    g = torch.Generator(device=DEV).manual_seed(15 + bits)
    vals = torch.randn((64, d), generator=g, device=DEV)
    vals[[0, 17, 63]] = 0.0
    packed, norms = tq.quantize(vals)
    v64 = vals.cpu().numpy().astype(np.float64)
    ref_packed, ref_norms, _ = O.turboquant_encode(v64, rot, bounds, bits)
    u = v64 / np.maximum(np.linalg.norm(v64, axis=-1, keepdims=True), 1e-8)
    r = u @ rot.astype(np.float64).T
    near = (np.abs(r[..., None] - bounds.astype(np.float64)) < 1e-5).any(-1)
    near[[0, 17, 63]] = False  # zero rows: exact zeros on both sides
    got_idx = O.unpack_indices(packed.cpu().numpy(), d, bits)
    ref_idx = O.unpack_indices(ref_packed, d, bits)
    assert np.array_equal(got_idx[~near], ref_idx[~near])
    assert near.mean() < 0.01
    assert (got_idx[[0, 17, 63]] == (1 << (bits - 1)) - 1).all()
    assert np.allclose(norms.cpu().numpy(), ref_norms, rtol=1e-6)
    assert (norms.cpu().numpy()[[0, 17, 63]] == 0).all()
    rec = tq.dequantize(packed, norms).cpu().numpy()
    ref_rec = O.turboquant_decode(packed.cpu().numpy(), norms.cpu().numpy(), rot, cents, d, bits)
    assert rel_err(rec, ref_rec) <= 1e-5


def _tq_rows(cache, n):
    """The cache's TurboQuant codes of its first n compressed tokens as
    reference packed rows (uint32), whichever layout it keeps."""
    if cache._values_il is not None:
        return S._hip.grouped_il_to_packed(cache._values_il, 2, n).cpu().numpy().view(np.uint32)
    return cache._values_packed[:, :, :n].cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("bits,t_q", [(2, 1), (3, 1), (4, 3), (2, 3)])
def test_hybrid_turboquant_fused_decode(bits, t_q):
    """A hybrid cache with TurboQuant values and no buffered tokens decodes in
    one fused launch (plus the row rotation) instead of dequantising the
    whole cache; the result equals the oracle SDPA over the oracle's
    dequantisation of the cache's own codes and norms."""
    codec = make_codec(30 + bits)
    b, hq, hkv, d, n = 2, 8, 2, 128, 333
    k, v = kv(31 + bits, b, hkv, n, d)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="turboquant",
                              value_bits=bits, buffer_size=0)
    cache.update_and_fetch(k, v)
    assert cache.buffer_offset == 0 and cache.compressed_offset == n
    q = torch.randn((b, hq, t_q, d), device=DEV).to(torch.float16)
    mask = "causal" if t_q > 1 else None
    out = S.sunshape_sdpa(q, cache, 0.088, mask=mask)
    # 2-bit codes: token-interleaved, matrix-core P.V
    mfma = "mfma_" if bits == 2 else ""
    assert (cache._values_il is not None) == (bits == 2)
    assert codec.last_score_backend == f"hip_fused_{mfma}turboquant"
    tc = cache._value_codec_impl
    vals = O.turboquant_decode(_tq_rows(cache, n),
                               cache._value_norms[:, :, :n].cpu().numpy(),
                               tc.rotation.cpu().numpy(), tc.centroids.cpu().numpy(), d, bits)
    ref = O.sdpa(q.cpu().numpy(), cache.key_indices.cpu().numpy(), vals,
                 codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), 0.088,
                 mask=mask)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    # the default buffer: recent fp16 tokens join the same fused softmax
    cache2 = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="turboquant",
                               value_bits=bits)
    cache2.update_and_fetch(k, v)
    nc, nb = cache2.compressed_offset, cache2.buffer_offset
    assert nb == 128 and nc == n - 128
    out2 = S.sunshape_sdpa(q, cache2, 0.088, mask=mask)
    assert codec.last_score_backend == f"hip_fused_{mfma}turboquant_buffer"
    vals2 = O.turboquant_decode(_tq_rows(cache2, nc),
                                cache2._value_norms[:, :, :nc].cpu().numpy(),
                                tc.rotation.cpu().numpy(), tc.centroids.cpu().numpy(), d, bits)
    vals_all = np.concatenate([vals2, v[:, :, nc:].float().cpu().numpy()], axis=2)
    ref2 = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                           codec.centroids.cpu().numpy(), cache2.key_indices.cpu().numpy(),
                           cache2.buffer_keys.float().cpu().numpy(), vals_all, mask=mask)
    assert rel_err16(out2.float().cpu().numpy(), ref2) <= REL_TOL
    # the value codec's own dequantisation gives the same cache contents
    rows = torch.from_numpy(_tq_rows(cache, n).view(np.int32)).to(DEV)
    rec = tc.dequantize(rows.reshape(-1, tc.packed_dim),
                        cache._value_norms[:, :, :n].reshape(-1)).cpu().numpy()
    assert rel_err(rec.reshape(vals.shape), vals) <= 1e-5


@pytest.mark.parametrize("vbd,buffer_size", [(4, 0), (8, 128)])
def test_hybrid_sunshape_values_fused_decode(vbd, buffer_size):
    """A hybrid cache with SunShape (block-VQ) values decodes in the fused
    kernel, with or without buffered tokens, and equals the oracle SDPA over
    the oracle's dequantisation of the cache's own value indices."""
    codec = make_codec(40 + vbd)
    rng = np.random.default_rng(vbd)
    d = 128
    vcodec = S.SunShapeBlockCodec(d, block_dim=vbd, n_centroids=256, device=DEV)
    vcodec.load_state_dict({"centroids": rng.standard_normal((d // vbd, 256, vbd)).astype(np.float32),
                            "permutation": rng.permutation(d).astype(np.int32)})
    b, hq, hkv, n = 2, 8, 2, 400
    k, v = kv(41 + vbd, b, hkv, n, d)
    cache = S.create_kv_cache(codec, n_kv_heads=hkv, value_backend="sunshape", value_bits=8,
                              value_codec=vcodec, buffer_size=buffer_size)
    cache.update_and_fetch(k, v)
    nc, nbuf = cache.compressed_offset, cache.buffer_offset
    assert nbuf == buffer_size and nc == n - buffer_size
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.088)
    assert codec.last_score_backend == ("hip_fused_sunshape_v_buffer" if buffer_size
                                        else "hip_fused_sunshape_v")
    vi = cache._value_indices[:, :, :nc].cpu().numpy()
    inv = vcodec.inv_permutation.cpu().numpy()
    vals = np.stack([np.stack([O.dequantize_blockvq(vi[bi, hi], vcodec.centroids.cpu().numpy(), inv)
                               for hi in range(hkv)]) for bi in range(b)])
    vals_all = np.concatenate([vals, v[:, :, nc:].float().cpu().numpy()], axis=2)
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), cache.key_indices.cpu().numpy(),
                          cache.buffer_keys.float().cpu().numpy() if nbuf else None, vals_all)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    # the cache's own (two-pass) value read-back agrees with the oracle
    assert rel_err(cache.values[:, :, :nc].float().cpu().numpy(), vals) <= 1e-3


@pytest.mark.parametrize("mode", ["profileperm_baseline", "profileperm_mixed_precision"])
def test_codec_fit_on_gpu_matches_cpu_fit(mode):
    """SunShapeBlockCodec.fit with the k-means on the GPU (every block in one
    launch).  Baseline mode against the oracle's fit (codec.py:299-418):
    the same permutation and a codebook of the same quality (reconstruction
    error within 1 %).  Mixed-precision mode (whose heavy-block selection
    the oracle does not restate) against the package's own NumPy k-means
    from the same initial rows: same permutation and heavy blocks, same
    quality."""
    rng = np.random.default_rng(42)
    s = rng.uniform(0.5, 4.0, 128).astype(np.float32)
    q_cal = (rng.standard_normal((1024, 128)) * s).astype(np.float32)
    k_cal = (rng.standard_normal((2048, 128)) * s).astype(np.float32)
    gpu = S.SunShapeBlockCodec(128, device=DEV, mode=mode, n_refine_dsq=0).fit(
        q_cal, k_cal, kmeans_iters=15, seed=42)
    kt = torch.from_numpy(k_cal).to(DEV)
    err_gpu = float(((gpu.dequantize(gpu.quantize(kt)).float() - kt) ** 2).mean())
    if mode == "profileperm_baseline":
        perm, cents = O.fit_profileperm_baseline(q_cal, k_cal, block_dim=8, n_centroids=256,
                                                 kmeans_iters=15, seed=42)
        assert np.array_equal(gpu.permutation.cpu().numpy(), perm)
        idx, _ = O.encode_blockvq(k_cal, cents, perm)
        rec = O.dequantize_blockvq(idx, cents, O.invert_permutation(perm)).astype(np.float64)
        err_ref = float(((rec - k_cal.astype(np.float64)) ** 2).mean())
    else:
        cpu = S.SunShapeBlockCodec(128, device=DEV, mode=mode, n_refine_dsq=0).fit(
            q_cal, k_cal, kmeans_iters=15, seed=42, kmeans_device="cpu")
        assert torch.equal(gpu.permutation.cpu(), cpu.permutation.cpu())
        assert torch.equal(gpu.mixed_high_precision_blocks.cpu(),
                           cpu.mixed_high_precision_blocks.cpu())
        err_ref = float(((cpu.dequantize(cpu.quantize(kt)).float() - kt) ** 2).mean())
    assert abs(err_gpu / err_ref - 1.0) <= 0.01


@pytest.mark.parametrize("value_backend,value_bits,buffer_size", [
    ("sunshape", 8, 0), ("sunshape", 8, 64), ("fp16", 16, 0), ("fp16", 16, 32),
    ("grouped", 2, 0), ("grouped", 4, 32), ("turboquant", 2, 0), ("turboquant", 2, 32),
    ("turboquant", 3, 0), ("turboquant", 4, 32)])
def test_mixed_precision_heavy_blocks_in_fp16(value_backend, value_bits, buffer_size):
    """A mixed-precision codec with ``heavy_fp16``: the hybrid cache keeps the
    heavy blocks' key dims in fp16, returns them in ``keys``, and every fused
    kernel of the hybrid layouts scores them exactly (matrix-core decodes for
    fp16, grouped and 2-bit TurboQuant values, the vector-ALU kernels for
    SunShape and 3/4-bit TurboQuant values), matching the oracle with heavy
    keys."""
    rng = np.random.default_rng(50)
    d, nb = 128, 16
    heavy = np.zeros(nb, bool)
    heavy[[3, 7, 8, 12]] = True
    # nonzero heavy-block centroids (as after a fit with DSQ refinement): the
    # exact heavy dot products replace them
    cents = rng.standard_normal((nb, 256, 8)).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    codec = S.SunShapeBlockCodec(d, device=DEV, mode="profileperm_mixed_precision",
                                 heavy_fp16=True)
    codec.load_state_dict({"centroids": cents, "permutation": perm,
                           "mixed_high_precision_blocks": heavy})
    hd = codec.heavy_dims().cpu().numpy()
    assert hd.size == 32
    b, hq, hkv, n = 2, 8, 2, 300
    k, v = kv(51, b, hkv, n, d)
    kw = dict(n_kv_heads=hkv, buffer_size=buffer_size)
    if value_backend == "sunshape":
        vcodec = S.SunShapeBlockCodec(d, block_dim=4, n_centroids=256, device=DEV)
        vcodec.load_state_dict({"centroids": rng.standard_normal((32, 256, 4)).astype(np.float32),
                                "permutation": rng.permutation(d).astype(np.int32)})
        cache = S.create_kv_cache(codec, value_backend="sunshape", value_bits=8,
                                  value_codec=vcodec, **kw)
    elif value_backend == "fp16":
        cache = S.create_kv_cache(codec, value_backend="fp16", **kw)
    else:
        cache = S.create_kv_cache(codec, value_backend=value_backend, value_bits=value_bits,
                                  **kw)
    cache.update_and_fetch(k, v)
    nc = cache.compressed_offset
    # returned keys carry the fp16 heavy dims in the original basis
    od = perm[hd]
    assert torch.equal(cache.keys[:, :, :nc][..., od].half().cpu(), k[:, :, :nc][..., od].cpu())
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, cache, 0.088)
    sfx = "_buffer" if buffer_size else ""
    expect = {"sunshape": "hip_fused_sunshape_v" + sfx,
              "fp16": "hip_fused_mfma" + (sfx or "_heavy"),
              # 4-bit grouped codes at head_dim 128 keep the loader-wave
              # kernel shape, which takes no heavy dims: the two-pass path
              "grouped": "hip" if value_bits == 4 else "hip_fused_mfma_dequant" + sfx,
              "turboquant": ("hip_fused_mfma_turboquant" if value_bits == 2
                             else "hip_fused_turboquant") + sfx}[value_backend]
    assert codec.last_score_backend == expect
    kh = k[:, :, :nc].cpu().numpy()[..., perm][..., hd]
    vals = cache.values.float().cpu().numpy()
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, perm, cents, cache.key_indices.cpu().numpy(),
                          cache.buffer_keys.float().cpu().numpy() if cache.buffer_offset else None,
                          vals, heavy_keys=kh, heavy_dims=hd)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    # the reference's semantics (heavy blocks contribute nothing) differ
    ref0 = O.sdpa_two_pass(q.cpu().numpy(), 0.088, perm, cents, cache.key_indices.cpu().numpy(),
                           cache.buffer_keys.float().cpu().numpy() if cache.buffer_offset else None,
                           vals)
    assert rel_err(ref0, ref) > 1e-2


@pytest.mark.parametrize("value_backend", ["sunshape", "fp16"])
def test_fitted_mixed_codec_heavy_fp16_with_buffer(value_backend):
    """A profileperm_mixed_precision codec fitted with DSQ refinement (which
    moves the heavy blocks' centroid 0 away from zero, reference
    codec.py:400-410) and heavy_fp16: a hybrid cache with buffered tokens
    scores the heavy blocks from their fp16 keys only, matching the oracle's
    attention over keys rebuilt from the light-block centroids and the fp16
    heavy dims."""
    rng = np.random.default_rng(60)
    d = 128
    s = rng.uniform(0.5, 4.0, d).astype(np.float32)
    q_cal = (rng.standard_normal((1024, d)) * s).astype(np.float32)
    k_cal = (rng.standard_normal((2048, d)) * s).astype(np.float32)
    codec = S.SunShapeBlockCodec(d, device=DEV, mode="profileperm_mixed_precision",
                                 n_refine_dsq=3, heavy_fp16=True).fit(
        q_cal, k_cal, kmeans_iters=5, seed=42)
    heavy = codec.mixed_high_precision_blocks.cpu().numpy().astype(bool)
    cents = codec.centroids.cpu().numpy()
    assert heavy.any() and np.abs(cents[heavy]).max() > 0.0  # the case the fix is for
    hd = codec.heavy_dims().cpu().numpy()
    perm = codec.permutation.cpu().numpy()
    b, hq, hkv, n = 2, 8, 2, 300
    k = torch.from_numpy((rng.standard_normal((b, hkv, n, d)) * s).astype(np.float16)).to(DEV)
    v = torch.from_numpy(rng.standard_normal((b, hkv, n, d)).astype(np.float16)).to(DEV)
    kw = dict(n_kv_heads=hkv, buffer_size=64)
    if value_backend == "sunshape":
        vcodec = S.SunShapeBlockCodec(d, block_dim=4, n_centroids=256, device=DEV)
        vcodec.load_state_dict({"centroids": rng.standard_normal((32, 256, 4)).astype(np.float32),
                                "permutation": rng.permutation(d).astype(np.int32)})
        cache = S.create_kv_cache(codec, value_backend="sunshape", value_bits=8,
                                  value_codec=vcodec, **kw)
    else:
        cache = S.create_kv_cache(codec, value_backend="fp16", **kw)
    cache.update_and_fetch(k, v)
    assert cache.buffer_offset > 0 and cache.compressed_offset > 0
    nc = cache.compressed_offset
    q = torch.from_numpy((rng.standard_normal((b, hq, 1, d)) * s).astype(np.float16)).to(DEV)
    out = S.sunshape_sdpa(q, cache, 0.088)
    # the matrix-core fp16 decode takes at most 32 heavy dims (more: two-pass)
    assert codec.last_score_backend == {
        "sunshape": "hip_fused_sunshape_v_buffer",
        "fp16": "hip_fused_mfma_buffer" if hd.size <= 32 else "hip"}[value_backend]
    kh = k[:, :, :nc].cpu().numpy()[..., perm][..., hd]
    vals = cache.values.float().cpu().numpy()
    idx = cache.key_indices.cpu().numpy()
    kb = cache.buffer_keys.float().cpu().numpy()
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, perm, cents, idx, kb, vals,
                          heavy_keys=kh, heavy_dims=hd)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
    # the same attention written out over rebuilt keys (codec basis: light
    # blocks from their centroids, heavy dims from the fp16 keys)
    qs = O.scale_query(q.cpu().numpy(), 0.088).astype(np.float64)
    inv = O.invert_permutation(perm)
    for bi in range(b):
        for h in range(hkv):
            kc = O.dequantize_blockvq(idx[bi, h], cents).astype(np.float64)
            kc[:, hd] = kh[bi, h].astype(np.float64)
            keys = np.concatenate([kc[:, inv], kb[bi, h].astype(np.float64)], axis=0)
            for r in range(hq // hkv):
                sc = qs[bi, h * (hq // hkv) + r, 0] @ keys.T
                w = np.exp(sc - sc.max())
                o = (w / w.sum()) @ vals[bi, h].astype(np.float64)
                got = out[bi, h * (hq // hkv) + r, 0].float().cpu().numpy()
                assert np.abs(got - o.astype(np.float16)).max() <= REL_TOL * np.abs(o).max()


def test_router_sends_sunshape_caches_to_sunshape_sdpa():
    codec = make_codec(16)
    cache = S.create_kv_cache(codec, n_kv_heads=1)
    k, v = kv(17, 1, 1, 40, 128)
    cache.update_and_fetch(k, v)
    q = torch.randn((1, 2, 1, 128), device=DEV).to(torch.float16)
    calls = []
    mod = types.ModuleType("ss_test_models_base")

    def original(queries, keys, values, cache, scale, mask, sinks=None):
        calls.append("original")
        return torch.zeros_like(queries)

    mod.scaled_dot_product_attention = original
    sys.modules["ss_test_models_base"] = mod
    try:
        S.patch.register_target("ss_test_models_base")
        S.patch.apply()
        assert S.patch.is_patched()
        out = mod.scaled_dot_product_attention(q, None, None, cache, 0.088, None)
        assert torch.equal(out, S.sunshape_sdpa(q, cache, 0.088))
        mod.scaled_dot_product_attention(q, k, v, object(), 0.088, None)
        assert calls == ["original"]
        S.patch.revert()
        assert mod.scaled_dot_product_attention is original and not S.patch.is_patched()
    finally:
        S.patch.revert()
        S.patch._extra_targets.clear()
        sys.modules.pop("ss_test_models_base", None)


def test_decode_step_append_is_one_fused_launch_and_returns_deferred():
    """SunShapeKVCache.update_and_fetch on decode steps: one
    ss_append_kv_il8 launch per step writes the same indices and values as
    the separate encoder and value append (bit for bit, against the oracle's
    encode and the stored fp16 values), and the returned keys / values are
    DeferredTensors: built only when read, equal to the reference's eager
    return, refused once the cache has changed."""
    codec = make_codec(70)
    b, hkv, d = 2, 4, 128
    k, v = kv(71, b, hkv, 300, d)
    lazy = S.create_kv_cache(codec, n_kv_heads=hkv)
    lazy.fuse_steps = False  # every step's append launches at once (the fused step: below)
    eager = S.create_kv_cache(codec, n_kv_heads=hkv, lazy_fetch=False)
    ko, vo = lazy.update_and_fetch(k[:, :, :290], v[:, :, :290])  # prompt: bulk encoders
    eager.update_and_fetch(k[:, :, :290], v[:, :, :290])
    assert isinstance(ko, S.cache.DeferredTensor) and ko.shape == (b, hkv, 290, d)
    for i in range(290, 300):  # decode steps: the fused append
        before = dict(S.kernels.get_kernel_stats())
        ko, vo = lazy.update_and_fetch(k[:, :, i:i + 1], v[:, :, i:i + 1])
        after = S.kernels.get_kernel_stats()
        assert sum(after.values()) - sum(before.values()) == 1  # one launch, one count
        eko, evo = eager.update_and_fetch(k[:, :, i:i + 1], v[:, :, i:i + 1])
    assert ko.shape == eko.shape and vo.dtype == evo.dtype
    assert torch.equal(ko + 0, eko) and torch.equal(vo.float(), evo.float())
    assert torch.equal(lazy.key_indices, eager.key_indices)
    assert torch.equal(lazy.values, v)
    idx, near = oracle_indices(codec, k)
    got = lazy.key_indices.cpu().numpy()
    assert np.array_equal(got[~near], idx[~near])
    ko2, _ = lazy.update_and_fetch(k[:, :, :1], v[:, :, :1])
    ko3, _ = lazy.update_and_fetch(k[:, :, 1:2], v[:, :, 1:2])
    with pytest.raises(RuntimeError):
        ko2.cpu()  # not built before the cache moved on
    assert ko.cpu().shape == (b, hkv, 300, d)  # built earlier: a snapshot, still valid
    assert ko3.cpu().shape == (b, hkv, 302, d)


@pytest.mark.parametrize("hq,hkv,n_new,causal", [(16, 4, 1, False), (16, 2, 3, True)])
def test_decode_steps_fuse_append_into_attention(hq, hkv, n_new, causal):
    """With fuse_steps (the default) a decode step's new tokens wait in the
    cache and the next sunshape_sdpa encodes, attends and stores them in one
    launch: the cache ends bit-identical to the separate appends, the
    outputs match them (the new tokens attended in float32: within 2e-5)
    and the oracle, update_and_fetch itself launches nothing, and a read of
    the cache, a trim, a save or the next update stores held tokens first.
    A held tensor changed in place is refused."""
    codec = make_codec(74)
    b, d = 2, 128
    t0, steps = 300, 6
    k, v = kv(75, b, hkv, t0 + steps * n_new, d)
    fused = S.create_kv_cache(codec, n_kv_heads=hkv, max_tokens=512)
    plain = S.create_kv_cache(codec, n_kv_heads=hkv, max_tokens=512)
    plain.fuse_steps = False
    fused.update_and_fetch(k[:, :, :t0], v[:, :, :t0])
    plain.update_and_fetch(k[:, :, :t0], v[:, :, :t0])
    g = torch.Generator(device=DEV).manual_seed(76)
    mask = "causal" if causal else None
    for i in range(steps):
        sl = slice(t0 + i * n_new, t0 + (i + 1) * n_new)
        q = torch.randn((b, hq, n_new, d), generator=g, device=DEV).half()
        before = sum(S.kernels.get_kernel_stats().values())
        fused.update_and_fetch(k[:, :, sl], v[:, :, sl])
        assert sum(S.kernels.get_kernel_stats().values()) == before  # held, nothing launched
        out_f = S.sunshape_sdpa(q, fused, 0.088, mask=mask, out_dtype=torch.float32)
        assert codec.last_score_backend == "hip_fused_mfma_step"
        assert sum(S.kernels.get_kernel_stats().values()) == before + 1
        plain.update_and_fetch(k[:, :, sl], v[:, :, sl])
        out_p = S.sunshape_sdpa(q, plain, 0.088, mask=mask, out_dtype=torch.float32)
        assert rel_err(out_f.cpu().numpy(), out_p.cpu().numpy()) <= 2e-5
    assert torch.equal(fused.key_indices, plain.key_indices)
    assert torch.equal(fused.values, plain.values)
    ref = O.sdpa(q.cpu().numpy(), plain.key_indices.cpu().numpy(), plain.values.cpu().numpy(),
                 codec.centroids.cpu().numpy(), codec.permutation.cpu().numpy(), 0.088, mask=mask)
    assert rel_err(out_f.cpu().numpy(), ref) <= REL_TOL
    # held tokens are stored before anything reads or moves the cache
    t_end = fused.offset
    k1, v1 = kv(77, b, hkv, 1, d)
    ko, vo = fused.update_and_fetch(k1, v1)
    assert fused._pending is not None
    assert torch.equal(vo[:, :, -1:], v1)  # building the deferred values stores them
    assert fused._pending is None and fused.offset == t_end + 1
    fused.update_and_fetch(k1 + 1, v1)
    fused.trim(1)
    assert fused._pending is None and fused.offset == t_end + 1
    k2, v2 = kv(78, b, hkv, 1, d)
    fused.update_and_fetch(k2, v2)
    k2.add_(1.0)  # changed in place while held
    with pytest.raises(RuntimeError):
        S.sunshape_sdpa(q[:, :, :1], fused, 0.088)


@pytest.mark.parametrize("bits,buf", [(2, 128), (4, 16)])
def test_hybrid_grouped_decode_steps_fused_equal_separate_appends(bits, buf):
    """HybridSunShapeKVCache decode steps with grouped interleaved values: the
    one-launch step (new tokens stored into the buffer window, the oldest
    encoded and quantised) leaves exactly the state the separate appends
    leave (indices, code words, scale/zero, buffer window), across window
    slides and capacity growth, and the fused decode over it matches the
    oracle's two-pass path."""
    codec = make_codec(72)
    b, hq, hkv, d = 2, 8, 2, 128
    t_all = 700
    k, v = kv(73, b, hkv, t_all, d)
    kw = dict(n_kv_heads=hkv, value_backend="grouped", value_bits=bits, buffer_size=buf,
              value_scale_dtype=torch.float16)
    fused = S.create_kv_cache(codec, **kw)
    fused.fuse_steps = False  # the append launch itself (held steps: below)
    plain = S.create_kv_cache(codec, **kw)
    plain._grouped_step_plan = lambda: None  # the separate appends
    fused.update_and_fetch(k[:, :, :300], v[:, :, :300])
    plain.update_and_fetch(k[:, :, :300], v[:, :, :300])
    n_fused = 0
    for i in range(300, t_all):
        before = sum(S.kernels.get_kernel_stats().values())
        fused.update_and_fetch(k[:, :, i:i + 1], v[:, :, i:i + 1])
        n_fused += sum(S.kernels.get_kernel_stats().values()) - before == 1
        plain.update_and_fetch(k[:, :, i:i + 1], v[:, :, i:i + 1])
    assert n_fused == t_all - 300  # every decode step was one launch
    assert fused.compressed_offset == plain.compressed_offset == t_all - buf
    assert torch.equal(fused.key_indices, plain.key_indices)
    assert torch.equal(fused.values_packed_raw, plain.values_packed_raw)
    assert torch.equal(fused.value_scales_raw, plain.value_scales_raw)
    assert torch.equal(fused.value_zeros_raw, plain.value_zeros_raw)
    assert torch.equal(fused.buffer_keys, plain.buffer_keys)
    assert torch.equal(fused.buffer_values, v[:, :, t_all - buf:])
    q = torch.randn((b, hq, 1, d), device=DEV).to(torch.float16)
    out = S.sunshape_sdpa(q, fused, 0.088)
    assert codec.last_score_backend == "hip_fused_mfma_dequant_buffer"
    assert torch.equal(out, S.sunshape_sdpa(q, plain, 0.088))
    vals = fused.values.float().cpu().numpy()
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), fused.key_indices.cpu().numpy(),
                          fused.buffer_keys.float().cpu().numpy(), vals)
    assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("d,bits,group,szdt,n_new,buf,causal,trim", [
    (128, 2, 64, torch.float16, 1, 128, False, 0),   # config 4's cache, one token a step
    (128, 2, 64, torch.float16, 1, 128, False, 5),   # the buffer not full: steps flush nothing
    (128, 2, 128, torch.float32, 3, 64, True, 0),
    (64, 2, 32, torch.float16, 2, 32, True, 0),
    (64, 2, 64, torch.float32, 4, 16, False, 0),
    (128, 4, 64, torch.float16, 1, 64, False, 0),    # 4-bit codes: the loader-wave shape
    (64, 4, 32, torch.float32, 3, 32, True, 0),
])
def test_hybrid_grouped_steps_fuse_into_attention(d, bits, group, szdt, n_new, buf, causal, trim):
    """With fuse_steps (the default) a decode step of a 2/4-bit grouped-value
    hybrid cache waits in the cache, and the next sunshape_sdpa does the
    buffer flush, the buffer store and the attention in one launch
    (ss_decode_step_grouped_il_hybrid): update_and_fetch launches nothing,
    the cache ends bit-identical to the separate step launches (indices,
    codes, scales, zeros, buffer), the outputs match those over the
    separately stepped cache (the flushed tokens attended in float32: within
    2e-5) and the oracle's two-pass path, and a read of the cache or the next
    update stores a held step first."""
    codec = make_codec(90 + d, d=d)
    b, hq, hkv = 2, 8, 2
    t0, steps = 300, 7
    k, v = kv(91, b, hkv, t0 + steps * n_new + 1, d)
    kw = dict(n_kv_heads=hkv, value_backend="grouped", value_bits=bits, value_group_size=group,
              buffer_size=buf, value_scale_dtype=szdt)
    fused = S.create_kv_cache(codec, **kw)
    plain = S.create_kv_cache(codec, **kw)
    plain.fuse_steps = False
    for c in (fused, plain):
        c.update_and_fetch(k[:, :, :t0], v[:, :, :t0])
        if trim:
            c.trim(trim)
    t_at = t0 - trim
    g = torch.Generator(device=DEV).manual_seed(92)
    mask = "causal" if causal else None
    for i in range(steps):
        sl = slice(t_at + i * n_new, t_at + (i + 1) * n_new)
        q = torch.randn((b, hq, n_new, d), generator=g, device=DEV).half()
        before = sum(S.kernels.get_kernel_stats().values())
        fused.update_and_fetch(k[:, :, sl], v[:, :, sl])
        assert fused._pending is not None
        assert sum(S.kernels.get_kernel_stats().values()) == before  # held, nothing launched
        out_f = S.sunshape_sdpa(q, fused, 0.088, mask=mask, out_dtype=torch.float32)
        assert codec.last_score_backend == "hip_fused_mfma_dequant_step"
        assert sum(S.kernels.get_kernel_stats().values()) == before + 1
        assert fused._pending is None
        plain.update_and_fetch(k[:, :, sl], v[:, :, sl])
        out_p = S.sunshape_sdpa(q, plain, 0.088, mask=mask, out_dtype=torch.float32)
        assert codec.last_score_backend == "hip_fused_mfma_dequant_buffer"
        assert rel_err(out_f.cpu().numpy(), out_p.cpu().numpy()) <= 2e-5
    assert fused.compressed_offset == plain.compressed_offset
    assert fused.buffer_offset == plain.buffer_offset
    assert torch.equal(fused.key_indices, plain.key_indices)
    assert torch.equal(fused.values_packed_raw, plain.values_packed_raw)
    assert torch.equal(fused.value_scales_raw, plain.value_scales_raw)
    assert torch.equal(fused.value_zeros_raw, plain.value_zeros_raw)
    assert torch.equal(fused.buffer_keys, plain.buffer_keys)
    assert torch.equal(fused.buffer_values, plain.buffer_values)
    vals = fused.values.float().cpu().numpy()
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), fused.key_indices.cpu().numpy(),
                          fused.buffer_keys.float().cpu().numpy(), vals,
                          mask="causal" if causal else None)
    assert rel_err(out_f.cpu().numpy(), ref) <= REL_TOL
    # a held step is done before anything reads the cache
    k1, v1 = k[:, :, -1:].contiguous(), v[:, :, -1:].contiguous()
    _, vo = fused.update_and_fetch(k1, v1)
    assert fused._pending is not None
    assert torch.equal(vo[:, :, -1:], v1)  # building the deferred values stores the step
    assert fused._pending is None
    plain.update_and_fetch(k1, v1)
    assert torch.equal(fused.key_indices, plain.key_indices)
    assert torch.equal(fused.values_packed_raw, plain.values_packed_raw)


@pytest.mark.parametrize("d,n_new,buf,causal", [(128, 1, 64, False), (64, 3, 32, True)])
def test_hybrid_fp16_steps_fuse_into_attention(d, n_new, buf, causal):
    """A hybrid cache with fp16 values (a non-default buffer size) holds its
    decode steps too: one ss_decode_step_il8_hybrid launch per step encodes
    the keys leaving the buffer, stores their values interleaved and the new
    tokens in the buffer, and attends every token.  The cache ends
    bit-identical to the unheld steps (buffer copies, then the flush), the
    outputs match the decode over that cache within 2e-5 and the oracle's
    two-pass path within 1e-3."""
    codec = make_codec(95 + d, d=d)
    b, hq, hkv = 2, 8, 2
    t0, steps = 300, 6
    k, v = kv(96, b, hkv, t0 + steps * n_new, d)
    kw = dict(n_kv_heads=hkv, value_backend="fp16", buffer_size=buf)
    fused = S.create_kv_cache(codec, **kw)
    plain = S.create_kv_cache(codec, **kw)
    plain.fuse_steps = False
    assert isinstance(fused, S.HybridSunShapeKVCache) and fused._fp16_il8
    for c in (fused, plain):
        c.update_and_fetch(k[:, :, :t0], v[:, :, :t0])
    g = torch.Generator(device=DEV).manual_seed(97)
    mask = "causal" if causal else None
    for i in range(steps):
        sl = slice(t0 + i * n_new, t0 + (i + 1) * n_new)
        q = torch.randn((b, hq, n_new, d), generator=g, device=DEV).half()
        before = sum(S.kernels.get_kernel_stats().values())
        fused.update_and_fetch(k[:, :, sl], v[:, :, sl])
        assert sum(S.kernels.get_kernel_stats().values()) == before  # held, nothing launched
        out_f = S.sunshape_sdpa(q, fused, 0.088, mask=mask, out_dtype=torch.float32)
        assert codec.last_score_backend == "hip_fused_mfma_step"
        assert sum(S.kernels.get_kernel_stats().values()) == before + 1
        plain.update_and_fetch(k[:, :, sl], v[:, :, sl])
        out_p = S.sunshape_sdpa(q, plain, 0.088, mask=mask, out_dtype=torch.float32)
        assert codec.last_score_backend == "hip_fused_mfma_buffer"
        assert rel_err(out_f.cpu().numpy(), out_p.cpu().numpy()) <= 2e-5
    assert fused.compressed_offset == plain.compressed_offset
    assert torch.equal(fused.key_indices, plain.key_indices)
    assert torch.equal(fused.values, plain.values)
    assert torch.equal(fused.buffer_keys, plain.buffer_keys)
    vals = fused.values.float().cpu().numpy()
    ref = O.sdpa_two_pass(q.cpu().numpy(), 0.088, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), fused.key_indices.cpu().numpy(),
                          fused.buffer_keys.float().cpu().numpy(), vals, mask=mask)
    assert rel_err(out_f.cpu().numpy(), ref) <= REL_TOL
    # a held step is stored before the cache is read
    k1, v1 = k[:, :, -1:].contiguous(), v[:, :, -1:].contiguous()
    fused.update_and_fetch(k1, v1)
    plain.update_and_fetch(k1, v1)
    assert fused._pending is not None
    assert torch.equal(fused.values, plain.values) and fused._pending is None
    assert torch.equal(fused.key_indices, plain.key_indices)


@pytest.mark.parametrize("backend,b,hq,hkv,t0,buf,n_new,qdt", [
    ("grouped", 1, 4, 4, 20, 8, 1, torch.float16),      # a dozen compressed tokens: one split, fewer units than waves
    ("grouped", 3, 32, 8, 5000, 8, 4, torch.float16),   # every step flushes four tokens; two splits
    ("grouped", 3, 32, 8, 5000, 8, 1, torch.float16),   # ten splits (the last hands over whole units only)
    ("grouped", 1, 32, 8, 5000, 8, 4, torch.bfloat16),  # eight splits; bf16 queries
    ("grouped", 2, 16, 2, 1100, 128, 2, torch.float32),  # eight query heads a KV head: two row groups
    ("fp16", 1, 4, 4, 20, 8, 1, torch.float16),
    ("fp16", 3, 32, 8, 5000, 16, 4, torch.bfloat16),
])
def test_hybrid_steps_fuse_at_edge_shapes(backend, b, hq, hkv, t0, buf, n_new, qdt):
    """One-launch hybrid steps at shapes the other tests do not reach: a
    single split holding fewer 64-token units than waves, steps that flush
    the most tokens, up to ten splits, several row groups a KV head.  The
    cache ends bit-identical to the unheld steps; the outputs match the
    oracle's two-pass path over that cache within 1e-3 and the decode over
    it within 5e-4 (fp16 values: 2e-5).  The grouped kernels' sums carry the
    codes' bf16 bias (128 + code) and lose about 7 bits to its subtraction,
    so two split layouts of 5000 tokens differ by up to 1.2e-4 of the largest
    output, each within 1.2e-4 of the exact float32-value result."""
    codec = make_codec(98)
    d = 128
    steps = 3
    k, v = kv(99, b, hkv, t0 + steps * n_new, d)
    kw = dict(n_kv_heads=hkv, value_backend=backend, buffer_size=buf)
    if backend == "grouped":
        kw.update(value_bits=2, value_scale_dtype=torch.float16)
    fused = S.create_kv_cache(codec, **kw)
    plain = S.create_kv_cache(codec, **kw)
    plain.fuse_steps = False
    for c in (fused, plain):
        c.update_and_fetch(k[:, :, :t0], v[:, :, :t0])
    g = torch.Generator(device=DEV).manual_seed(100)
    for i in range(steps):
        sl = slice(t0 + i * n_new, t0 + (i + 1) * n_new)
        q = torch.randn((b, hq, n_new, d), generator=g, device=DEV).to(qdt)
        fused.update_and_fetch(k[:, :, sl], v[:, :, sl])
        assert fused._pending is not None
        out_f = S.sunshape_sdpa(q, fused, 0.088, mask="causal", out_dtype=torch.float32)
        assert codec.last_score_backend in ("hip_fused_mfma_dequant_step", "hip_fused_mfma_step")
        plain.update_and_fetch(k[:, :, sl], v[:, :, sl])
        out_p = S.sunshape_sdpa(q, plain, 0.088, mask="causal", out_dtype=torch.float32)
        tol = 5e-4 if backend == "grouped" else 2e-5
        assert rel_err(out_f.cpu().numpy(), out_p.cpu().numpy()) <= tol
    assert fused.compressed_offset == plain.compressed_offset
    assert torch.equal(fused.key_indices, plain.key_indices)
    assert torch.equal(fused.values, plain.values)
    assert torch.equal(fused.buffer_keys, plain.buffer_keys)
    vals = fused.values.float().cpu().numpy()
    if qdt == torch.bfloat16:  # q * scale rounded to bf16, as the kernels form it
        qref, sc = (q.float() * 0.088).to(torch.bfloat16).float().cpu().numpy(), 1.0
    else:
        qref, sc = q.cpu().numpy(), 0.088
    ref = O.sdpa_two_pass(qref, sc, codec.permutation.cpu().numpy(),
                          codec.centroids.cpu().numpy(), fused.key_indices.cpu().numpy(),
                          fused.buffer_keys.float().cpu().numpy(), vals, mask="causal")
    assert rel_err(out_f.cpu().numpy(), ref) <= REL_TOL
    assert rel_err(out_p.cpu().numpy(), ref) <= REL_TOL  # the buffered decode, same splits as ever


def test_hybrid_grouped_step_ties_take_the_exact_ranking():
    """A flushed key exactly halfway between two centroids of every block
    (an exact tie, which no float error bound clears) and one a hair nearer
    the second: the one-launch hybrid step's encode ranks the tie exactly
    (the lower index) and stores the indices the separate step launch
    stores."""
    rng = np.random.default_rng(93)
    d, nb, b, hq, hkv, buf, t0 = 128, 16, 1, 8, 2, 16, 100
    c = rng.standard_normal((nb, 256, 8)).astype(np.float32) * 0.5
    c[:, 3, :] = 1.0   # the two centroids the keys sit between
    c[:, 7, :] = 3.0
    perm = rng.permutation(d).astype(np.int32)
    codec = S.SunShapeBlockCodec(d, n_centroids=256, device=DEV)
    codec.load_state_dict({"centroids": c, "permutation": perm})
    k, v = kv(94, b, hkv, t0 + 2, d)
    # the buffer's two oldest tokens, which the next two steps flush
    k[:, :, t0 - buf] = 2.0                                        # tie: index 3
    near = np.full(d, 2.0, np.float32)
    near[perm[0::8]] = np.float16(2.0 + 2.0 ** -9)                 # block dim 0 nearer 7
    k[:, :, t0 - buf + 1] = torch.tensor(near.astype(np.float16), device=DEV)
    kw = dict(n_kv_heads=hkv, value_backend="grouped", value_bits=2, buffer_size=buf,
              value_scale_dtype=torch.float16)
    fused = S.create_kv_cache(codec, **kw)
    plain = S.create_kv_cache(codec, **kw)
    plain.fuse_steps = False
    for cc in (fused, plain):
        cc.update_and_fetch(k[:, :, :t0], v[:, :, :t0])
    q = torch.randn((b, hq, 1, d), device=DEV).half()
    for i in range(2):
        sl = slice(t0 + i, t0 + i + 1)
        fused.update_and_fetch(k[:, :, sl], v[:, :, sl])
        out_f = S.sunshape_sdpa(q, fused, 0.088, out_dtype=torch.float32)
        assert codec.last_score_backend == "hip_fused_mfma_dequant_step"
        plain.update_and_fetch(k[:, :, sl], v[:, :, sl])
        out_p = S.sunshape_sdpa(q, plain, 0.088, out_dtype=torch.float32)
        assert rel_err(out_f.cpu().numpy(), out_p.cpu().numpy()) <= 2e-5
    assert torch.equal(fused.key_indices, plain.key_indices)
    got = fused.key_indices[:, :, t0 - buf:t0 - buf + 2].cpu().numpy()
    assert (got[:, :, 0] == 3).all() and (got[:, :, 1] == 7).all()


@pytest.mark.parametrize("backend,bits,buf,qdt", [
    ("grouped", 2, 128, torch.float16),     # config 4's cache: 2-bit grouped, default buffer
    ("grouped", 4, 64, torch.bfloat16),
    ("turboquant", 2, 128, torch.float16),
    ("fp16", None, 96, torch.float16),      # fp16 values, a buffer
    ("grouped", 2, 0, torch.float16),       # no buffer
])
def test_hybrid_prompt_takes_the_prefill_kernel(backend, bits, buf, qdt):
    """A prompt (mask "causal") against a hybrid cache runs on the
    matrix-core prefill kernel: compressed keys from the codebook, the
    buffered keys whole, every value in one interleaved fp16 copy.  It
    matches the reference's two-pass path (the oracle) over the same cache,
    for the first prompt and for a second chunk after it (rows offset by the
    cached tokens)."""
    codec = make_codec(80)
    b, hq, hkv, d = 1, 32, 8, 128
    kw = dict(n_kv_heads=hkv, value_backend=backend, buffer_size=buf)
    if bits:
        kw.update(value_bits=bits, value_scale_dtype=torch.float16)
    cache = S.create_kv_cache(codec, **kw)
    assert isinstance(cache, S.HybridSunShapeKVCache)
    k, v = kv(81, b, hkv, 700, d)
    q = torch.randn((b, hq, 700, d), device=DEV).to(qdt)
    cents = codec.centroids.cpu().numpy()
    perm = codec.permutation.cpu().numpy()
    for lo, hi in ((0, 500), (500, 700)):
        cache.update_and_fetch(k[:, :, lo:hi], v[:, :, lo:hi])
        qq = q[:, :, lo:hi].contiguous()
        out = S.sunshape_sdpa(qq, cache, 0.088, mask="causal")
        assert codec.last_score_backend == "hip_prefill_mfma_hybrid"
        out32 = S.sunshape_sdpa(qq, cache, 0.088, mask="causal", out_dtype=torch.float32)
        vals = cache.values.float().cpu().numpy()  # compressed values dequantised, then buffer
        if qdt == torch.bfloat16:  # q * scale rounded to bf16, as the kernels form it
            qref, sc = (qq.float() * 0.088).to(torch.bfloat16).float().cpu().numpy(), 1.0
        else:
            qref, sc = qq.cpu().numpy(), 0.088
        ref = O.sdpa_two_pass(qref, sc, perm, cents, cache.key_indices.cpu().numpy(),
                              cache.buffer_keys.float().cpu().numpy() if cache.buffer_offset
                              else None, vals, mask="causal")
        # values enter the prompt kernel rounded to fp16 (dequantised codes
        # take more bits): within 2^-12 of each, a few 1e-4 of the output
        assert rel_err(out32.cpu().numpy(), ref) <= REL_TOL
        if qdt == torch.float16:
            assert rel_err16(out.float().cpu().numpy(), ref) <= REL_TOL
