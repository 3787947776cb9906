"""Pins the oracle's LUT, score gather and fused attention (CPU only).

The reference's known-answer tests [6], [7], [11], [12], [14]
(reference test_kernels.py:163-482) are restated with their np.random.seed
streams: the expected output is the textbook ``softmax(q k_hat^T) V`` with
k_hat reconstructed from the codebook -- a different route from the oracle's
LUT + gather.  Tolerances are the reference's own (1e-3 scores; 5e-3 / 1e-2
outputs) and, where the oracle is float64, much tighter ones too.
"""

import math

import numpy as np
import pytest

from oracle import sunshape_oracle as O


def k_hat_of(cents, idx):
    return O.dequantize_blockvq(idx, cents)


def explicit_attention(q, k_hat, v, causal=False, q_offset=0, masked=-1e30):
    s = q.astype(np.float64) @ k_hat.astype(np.float64).T
    if causal:
        qp = np.arange(q_offset, q_offset + q.shape[0])
        s = np.where(qp[:, None] >= np.arange(k_hat.shape[0])[None, :], s, masked)
    w = np.exp(s - s.max(axis=-1, keepdims=True))
    w = w / w.sum(axis=-1, keepdims=True)
    return w @ v.astype(np.float64)


def test_known_answer_6_score_gather():
    np.random.seed(55)
    qdots = np.random.randn(4, 16, 256).astype(np.float32)
    idx = np.random.randint(0, 256, size=(32, 16), dtype=np.uint8)
    ref = np.take_along_axis(qdots[:, None, :, :], idx[None, :, :, None].astype(np.int64),
                             axis=-1)[..., 0].sum(axis=2)
    assert np.abs(O.gather_scores(qdots, idx) - ref).max() < 1e-5


def test_scores_equal_q_dot_reconstructed_keys_in_original_basis():
    """attention_scores == q @ dequantize(k).T (reference
    test_sunshape_mlx.py:172-182): the permutation cancels in the dot."""
    rng = np.random.default_rng(3)
    cents = rng.standard_normal((16, 256, 8)).astype(np.float32)
    perm = rng.permutation(128).astype(np.int32)
    idx = rng.integers(0, 256, (100, 16)).astype(np.uint8)
    q = rng.standard_normal((8, 128)).astype(np.float32)
    k_orig = O.dequantize_blockvq(idx, cents, O.invert_permutation(perm))
    s = O.attention_scores(q, idx, cents, perm)
    ref = q.astype(np.float64) @ k_orig.astype(np.float64).T
    assert np.abs(s - ref).max() < 1e-9 * np.abs(ref).max()
    # planted mistake: forgetting the query permutation breaks it
    bad = O.gather_scores(O.query_centroid_dots(q, cents), idx)
    assert np.abs(bad - ref).max() > 1e-2


def test_known_answer_7_materialized_causal():
    np.random.seed(42)
    t_q, t_kv, nb, nc, bd = 4, 32, 16, 256, 8
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.int32)
    v = np.random.randn(t_kv, nb * bd).astype(np.float32)
    q = np.random.randn(t_q, nb * bd).astype(np.float32)
    ref = explicit_attention(q, k_hat_of(cents, idx), v, True, t_kv - t_q, -1e9)
    qd = O.query_centroid_dots(q, cents)
    out = O.materialized_block_vq_attention(qd, idx, v, t_q, t_kv)
    assert np.abs(out - ref).max() < 5e-3
    assert np.abs(out - ref).max() < 1e-9


@pytest.mark.parametrize("seed,t_q,t_kv,causal,vscale,tol", [
    (111, 1, 64, False, 1.0, 5e-3),   # [11]
    (222, 4, 32, True, 1.0, 5e-3),    # [12]
    (444, 1, 512, False, 0.1, 1e-2),  # [14]
])
def test_known_answers_fused(seed, t_q, t_kv, causal, vscale, tol):
    np.random.seed(seed)
    nb, nc, bd = 16, 256, 8
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.uint8)
    v = (np.random.randn(t_kv, nb * bd).astype(np.float32) * vscale).astype(np.float32)
    q = (np.random.randn(t_q, nb * bd).astype(np.float32) * vscale).astype(np.float32)
    q_off = t_kv - t_q if causal else 0
    ref = explicit_attention(q, k_hat_of(cents, idx), v, causal, q_off)
    out = O.fused_attention(q, cents, idx, v, causal, q_off)
    assert np.abs(out - ref).max() < tol
    assert np.abs(out - ref).max() < 1e-9


def test_online_literal_equals_two_pass():
    rng = np.random.default_rng(9)
    cents = rng.standard_normal((8, 64, 8)).astype(np.float32)
    idx = rng.integers(0, 64, (150, 8)).astype(np.uint8)
    v = rng.standard_normal((150, 64)).astype(np.float32)
    q = rng.standard_normal((5, 64)).astype(np.float32) * 0.5
    for causal, off in ((False, 0), (True, 145), (True, 2)):
        a = O.fused_attention(q, cents, idx, v, causal, off)
        b = O.fused_attention_online_literal(q, cents, idx, v, causal, off)
        assert np.abs(a - b).max() < 1e-10


def test_fully_masked_rows_output_zero():
    rng = np.random.default_rng(1)
    cents = rng.standard_normal((8, 16, 8)).astype(np.float32)
    idx = rng.integers(0, 16, (10, 8)).astype(np.uint8)
    v = rng.standard_normal((10, 64)).astype(np.float32)
    q = rng.standard_normal((3, 64)).astype(np.float32)
    # q_offset -5: row 0 admits t <= -5 (none), row 2 admits t <= -3 (none)
    out = O.fused_attention(q, cents, idx, v, True, -5)
    assert not out.any()
    assert not O.fused_attention_online_literal(q, cents, idx, v, True, -5).any()


def test_split_lse_merge_equals_whole():
    """The split-T decomposition used on the GPU: partials (m, l, acc) of
    token chunks merged by log-sum-exp give the same output."""
    rng = np.random.default_rng(12)
    s = rng.standard_normal(1000) * 3
    v = rng.standard_normal((1000, 16))
    whole = (np.exp(s - s.max()) @ v) / np.exp(s - s.max()).sum()
    parts = []
    for lo in range(0, 1000, 137):
        ss = s[lo:lo + 137]
        m = ss.max()
        p = np.exp(ss - m)
        parts.append((m, p.sum(), p @ v[lo:lo + 137]))
    parts.append((-1e30, 0.0, np.zeros(16)))  # an empty split
    assert np.abs(O.lse_merge(parts) - whole).max() < 1e-12


def test_sdpa_gqa_head_mapping_and_scale():
    """q head h*rep + r reads KV head h (attention.py:220); scale is applied in
    the query dtype before the permutation (attention.py:208, 228)."""
    rng = np.random.default_rng(21)
    b_, hq, hkv, d, t = 1, 6, 2, 64, 40
    cents = rng.standard_normal((8, 32, 8)).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    idx = rng.integers(0, 32, (b_, hkv, t, 8)).astype(np.uint8)
    vals = rng.standard_normal((b_, hkv, t, d)).astype(np.float16)
    q = rng.standard_normal((b_, hq, 1, d)).astype(np.float16)
    scale = 0.125
    out = O.sdpa(q, idx, vals, cents, perm, scale)
    inv = O.invert_permutation(perm)
    for hh in range(hq):
        kv = hh // (hq // hkv)
        qs = (q[0, hh].astype(np.float32) * np.float32(scale)).astype(np.float16)
        ref = explicit_attention(qs.astype(np.float32),
                                 O.dequantize_blockvq(idx[0, kv], cents, inv), vals[0, kv])
        assert np.abs(out[0, hh] - ref).max() < 1e-9
    # planted mistake: interleaved GQA mapping (kv = hh % hkv) must differ
    kv_wrong = 1 % hkv
    qs = (q[0, 1].astype(np.float32) * np.float32(scale)).astype(np.float16)
    wrong = explicit_attention(qs.astype(np.float32),
                               O.dequantize_blockvq(idx[0, kv_wrong], cents, inv),
                               vals[0, kv_wrong])
    assert np.abs(out[0, 1] - wrong).max() > 1e-3


def test_sdpa_two_pass_equals_fused_without_buffer():
    rng = np.random.default_rng(30)
    b_, hq, hkv, d, t = 1, 4, 2, 64, 33
    cents = rng.standard_normal((8, 64, 8)).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    idx = rng.integers(0, 64, (b_, hkv, t, 8)).astype(np.uint8)
    vals = rng.standard_normal((b_, hkv, t, d)).astype(np.float16)
    q = rng.standard_normal((b_, hq, 3, d)).astype(np.float16)
    a = O.sdpa(q, idx, vals, cents, perm, 0.2, mask="causal")
    b = O.sdpa_two_pass(q, 0.2, perm, cents, idx, None, vals, mask="causal")
    assert np.abs(a - b).max() < 1e-10


def test_sdpa_two_pass_buffer_scores_use_original_basis():
    """Buffered fp16 keys are scored against the *unpermuted* scaled query
    (attention.py:318-321)."""
    rng = np.random.default_rng(31)
    d = 64
    perm = rng.permutation(d).astype(np.int32)
    cents = rng.standard_normal((8, 16, 8)).astype(np.float32)
    kb = rng.standard_normal((1, 1, 5, d)).astype(np.float16)
    vals = rng.standard_normal((1, 1, 5, d)).astype(np.float16)
    q = rng.standard_normal((1, 1, 1, d)).astype(np.float16)
    out = O.sdpa_two_pass(q, 0.3, perm, cents, np.zeros((1, 1, 0, 8), np.uint8), kb, vals)
    qs = O.scale_query(q, 0.3)[0, 0].astype(np.float64)
    ref = explicit_attention(qs, kb[0, 0], vals[0, 0])
    assert np.abs(out[0, 0] - ref).max() < 1e-12


def test_sdpa_two_pass_rotation_scores_as_reconstructed_keys():
    """Rotated codecs: codec-space queries are q_scaled @ R^T
    (attention.py:229-230), so a compressed score is q . (C[idx] R), the
    query against the key reconstructed in the original basis (pinned
    against attention over those keys written out, so R in place of R^T
    fails for a non-symmetric rotation); buffered keys stay in the original
    basis.  A permutation matrix as R gives the permutation path."""
    rng = np.random.default_rng(33)
    b_, hq, hkv, d, t, tb = 1, 2, 1, 64, 30, 6
    rot, _ = np.linalg.qr(rng.standard_normal((d, d)))
    rot = rot.astype(np.float32)
    cents = rng.standard_normal((8, 32, 8)).astype(np.float32)
    idx = rng.integers(0, 32, (b_, hkv, t, 8)).astype(np.uint8)
    kb = rng.standard_normal((b_, hkv, tb, d)).astype(np.float16)
    vals = rng.standard_normal((b_, hkv, t + tb, d)).astype(np.float16)
    q = rng.standard_normal((b_, hq, 1, d)).astype(np.float16)
    out = O.sdpa_two_pass(q, 0.2, None, cents, idx, kb, vals, rotation=rot)
    k_orig = O.dequantize_blockvq(idx[0, 0], cents).astype(np.float64) @ rot.astype(np.float64)
    keys = np.concatenate([k_orig, kb[0, 0].astype(np.float64)])
    qs = O.scale_query(q, 0.2)[0].astype(np.float64)
    for h in range(hq):
        ref = explicit_attention(qs[h], keys, vals[0, 0])
        assert np.abs(out[0, h] - ref).max() < 1e-5
    perm = rng.permutation(d).astype(np.int32)
    pmat = np.zeros((d, d), np.float32)
    pmat[np.arange(d), perm] = 1.0  # (q @ P^T)[j] = q[perm[j]]
    a = O.sdpa_two_pass(q, 0.2, perm, cents, idx, kb, vals)
    b = O.sdpa_two_pass(q, 0.2, None, cents, idx, kb, vals, rotation=pmat)
    assert np.abs(a - b).max() < 1e-12


def test_sdpa_heavy_blocks_score_as_exact_key_dots():
    """Mixed-precision extension: with the heavy blocks' key dims kept in
    fp16, each compressed score is q . k_hat where k_hat takes the centroids
    on light blocks and the fp16 dims on heavy ones, all in the original
    basis (pinned against attention written out over the reconstructed keys,
    not the LUT).  The heavy blocks' centroids are nonzero (as after a fit
    with DSQ refinement) and must not add to the scores."""
    rng = np.random.default_rng(32)
    b_, hq, hkv, d, t, bd = 1, 2, 1, 64, 40, 8
    nb = d // bd
    perm = rng.permutation(d).astype(np.int32)
    cents = rng.standard_normal((nb, 32, bd)).astype(np.float32)
    heavy = np.array([1, 6])
    hd = np.concatenate([np.arange(b * bd, (b + 1) * bd) for b in heavy]).astype(np.int32)
    keys = rng.standard_normal((b_, hkv, t, d)).astype(np.float32)
    idx = np.stack([O.encode_blockvq(keys[0, 0], cents, perm)[0]])[None]
    kh = O.apply_permutation(keys[0, 0], perm)[:, hd].astype(np.float16)[None, None]
    vals = rng.standard_normal((b_, hkv, t, d)).astype(np.float16)
    q = rng.standard_normal((b_, hq, 1, d)).astype(np.float16)
    out = O.sdpa_two_pass(q, 0.25, perm, cents, idx, None, vals, heavy_keys=kh, heavy_dims=hd)
    # k_hat in codec space: centroids of light blocks, fp16 dims of heavy ones
    kc = O.dequantize_blockvq(idx[0, 0], cents).astype(np.float64)
    kc[:, hd] = kh[0, 0].astype(np.float64)
    k_orig = kc[:, O.invert_permutation(perm)]
    qs = O.scale_query(q, 0.25)[0].astype(np.float64)
    for h in range(hq):
        ref = explicit_attention(qs[h], k_orig, vals[0, 0])
        assert np.abs(out[0, h] - ref).max() < 1e-9


def test_cpu_baseline_forms_agree_with_oracle():
    rng = np.random.default_rng(40)
    b_, hq, hkv, d, t = 1, 8, 2, 128, 500
    cents = rng.standard_normal((16, 256, 8)).astype(np.float32)
    perm = rng.permutation(d).astype(np.int32)
    idx = rng.integers(0, 256, (b_, hkv, t, 16)).astype(np.uint8)
    vals = rng.standard_normal((b_, hkv, t, d)).astype(np.float16)
    q = rng.standard_normal((b_, hq, 1, d)).astype(np.float16)
    ref = O.sdpa(q, idx, vals, cents, perm, 1 / math.sqrt(d))[:, :, 0]
    qt = O.apply_permutation(O.scale_query(q, 1 / math.sqrt(d)), perm).astype(np.float32)
    qt = qt.reshape(b_, hkv, hq // hkv, d)
    for f in (O.decode_cpu_vectorised, O.decode_cpu_reference_shaped,
              lambda *a: O.decode_cpu_parallel(*a, n_threads=4, chunk=128)):
        out = f(qt, cents, idx, vals)
        assert np.abs(out - ref).max() / np.abs(ref).max() < 1e-4


def _mask_case(seed=34):
    """A hybrid-shaped two-pass case: compressed keys plus buffered fp16
    keys, GQA 2:1, three query rows, and the same keys written out in the
    original basis."""
    rng = np.random.default_rng(seed)
    b_, hq, hkv, d, tc, tb, tq = 1, 4, 2, 32, 20, 5, 3
    perm = rng.permutation(d).astype(np.int32)
    cents = rng.standard_normal((4, 16, 8)).astype(np.float32)
    idx = rng.integers(0, 16, (b_, hkv, tc, 4)).astype(np.uint8)
    kb = rng.standard_normal((b_, hkv, tb, d)).astype(np.float16)
    vals = rng.standard_normal((b_, hkv, tc + tb, d)).astype(np.float16)
    q = rng.standard_normal((b_, hq, tq, d)).astype(np.float16)
    inv = O.invert_permutation(perm)
    keys = np.stack([np.concatenate([O.dequantize_blockvq(idx[0, h], cents, inv).astype(np.float64),
                                     kb[0, h].astype(np.float64)]) for h in range(hkv)])
    return q, perm, cents, idx, kb, vals, keys, rng


def _check_bool_mask_pins(two_pass):
    """The reference's boolean-mask semantics (attention.py:339-346, masked
    scores filled with float32's lowest value before the softmax), written
    out over the reconstructed keys: a row that keeps some keys is the
    softmax over exactly those keys; a row that keeps none is the mean of
    all the values.  Returns the largest deviation."""
    q, perm, cents, idx, kb, vals, keys, rng = _mask_case()
    t_kv = keys.shape[1]
    m = rng.random((3, t_kv)) > 0.4
    m[1, :] = False               # every key masked
    m[2, :] = False
    m[2, [0, 7, 21]] = True       # compressed and buffered keys kept
    out = two_pass(q, 0.3, perm, cents, idx, kb, vals, mask=m)
    qs = O.scale_query(q, 0.3)[0].astype(np.float64)
    worst = 0.0
    for hh in range(4):
        h = hh // 2
        v = vals[0, h].astype(np.float64)
        for r in range(3):
            keep = m[r]
            if keep.any():
                ref = explicit_attention(qs[hh, r][None], keys[h][keep], v[keep])[0]
            else:
                ref = v.mean(axis=0)
            worst = max(worst, float(np.abs(out[0, hh, r] - ref).max()))
    return worst


def test_sdpa_two_pass_bool_mask_semantics():
    assert _check_bool_mask_pins(O.sdpa_two_pass) < 1e-12


def test_sdpa_two_pass_bool_mask_pins_catch_planted_mistakes(monkeypatch):
    """Mistakes planted in the oracle fail the pins: the fused kernel's
    zero output for an empty row (the reference's two-pass path averages the
    values), and a mask read the wrong way round."""
    fill = O._softmax_rows_min_fill
    monkeypatch.setattr(O, "_softmax_rows_min_fill", O._softmax_rows)
    assert _check_bool_mask_pins(O.sdpa_two_pass) > 1e-2
    monkeypatch.setattr(O, "_softmax_rows_min_fill", lambda s, valid, v: fill(s, ~valid, v))
    assert _check_bool_mask_pins(O.sdpa_two_pass) > 1e-2


def test_sdpa_two_pass_additive_mask_semantics():
    """Float masks are added to the scores (attention.py:342-343): the
    output is softmax(q k^T + m) V over the reconstructed keys, so a large
    negative entry all but removes a key.  Planted in the oracle: a mask
    subtracted instead fails the pin."""
    q, perm, cents, idx, kb, vals, keys, rng = _mask_case(35)
    t_kv = keys.shape[1]
    m = (rng.standard_normal((3, t_kv)) * 2.0).astype(np.float32)
    m[0, 3] = -1e4
    qs = O.scale_query(q, 0.3)[0].astype(np.float64)

    def worst_of(out):
        w = 0.0
        for hh in range(4):
            h = hh // 2
            s = qs[hh] @ keys[h].T + m
            p = np.exp(s - s.max(axis=1, keepdims=True))
            ref = (p / p.sum(axis=1, keepdims=True)) @ vals[0, h].astype(np.float64)
            w = max(w, float(np.abs(out[0, hh] - ref).max()))
        return w

    assert worst_of(O.sdpa_two_pass(q, 0.3, perm, cents, idx, kb, vals, mask=m)) < 1e-12
    assert worst_of(O.sdpa_two_pass(q, 0.3, perm, cents, idx, kb, vals, mask=-m)) > 1e-2


def test_sdpa_two_pass_causal_rows_before_the_cache_average_values():
    """A causal mask with more query rows than keys (offset T_kv - T_q < 0)
    masks every key of the first rows; the two-pass path, like the
    reference's (attention.py:329-336), averages the values there, while
    the fused kernel's literal loop gives 0 (kernels.py:218-222)."""
    q, perm, cents, idx, kb, vals, keys, rng = _mask_case(36)
    idx2 = idx[:, :, :2]
    vals2 = vals[:, :, :2]
    # two keys, three query rows (offset -1): row 0 sees no key, row 1 key 0,
    # row 2 both
    out = O.sdpa_two_pass(q, 0.3, perm, cents, idx2, None, vals2, mask="causal")
    qs = O.scale_query(q, 0.3)[0].astype(np.float64)
    for hh in range(4):
        h = hh // 2
        v = vals2[0, h].astype(np.float64)
        assert np.abs(out[0, hh, 0] - v.mean(axis=0)).max() < 1e-12
        assert np.abs(out[0, hh, 1] - v[0]).max() < 1e-12
        ref = explicit_attention(qs[hh, 2][None], keys[h][:2], v)[0]
        assert np.abs(out[0, hh, 2] - ref).max() < 1e-12
