"""Pins the oracle's value codecs, packing and scalar quantisation (CPU only).

Restates the reference's known-answer tests [1]-[5], [9], [15]-[17]
(reference test_kernels.py:49-160, 265-284, 485-651) with their np.random.seed
streams, plus closed forms of the bit layout and of the Lloyd-Max tables.
"""

import math

import numpy as np
import pytest

from oracle import sunshape_oracle as O
import sunshape_mlx_amd as S


@pytest.mark.parametrize("bits,d", [(2, 128), (3, 100), (4, 128)])
def test_known_answer_1_pack_roundtrip(bits, d):
    np.random.seed(42)
    x = np.random.randint(0, 1 << bits, size=(32, d), dtype=np.uint8)
    assert np.array_equal(O.unpack_indices(O.pack_indices(x, bits), d, bits), x.astype(np.uint32))


def test_known_answer_2_3bit_unaligned():
    np.random.seed(99)
    x = np.random.randint(0, 8, size=(5, 27), dtype=np.uint8)
    p = O.pack_indices(x, 3)
    assert p.shape == (5, 3)
    assert np.array_equal(O.unpack_indices(p, 27, 3), x.astype(np.uint32))


@pytest.mark.parametrize("bits,maxv,d", [(2, 3, 32), (3, 7, 30), (4, 15, 32)])
def test_known_answer_3_boundaries(bits, maxv, d):
    z = O.unpack_indices(O.pack_indices(np.zeros((1, d), np.uint8), bits), d, bits)
    m = O.unpack_indices(O.pack_indices(np.full((1, d), maxv, np.uint8), bits), d, bits)
    assert not z.any() and (m == maxv).all()


def test_known_answer_9_3bit_no_stray_bits():
    p = O.pack_indices(np.full((1, 30), 7, np.uint8), 3)
    assert int(p[0, 0]) >> 30 == 0
    assert int(p[0, 0]) == (1 << 30) - 1


def test_pack_bit_layout_closed_form():
    """Element i of a word sits at bits [b*i, b*i + b); values are masked."""
    x = np.zeros((1, 16), np.uint8)
    x[0, 3] = 2
    x[0, 15] = 7  # masked to 3 at 2 bits
    p = O.pack_indices(x, 2)
    assert int(p[0, 0]) == (2 << 6) | (3 << 30)


@pytest.mark.parametrize("bits,thresh", [(4, 0.15), (2, 0.55)])
def test_known_answer_4_grouped_rmse(bits, thresh):
    np.random.seed(123)
    v = np.random.randn(64, 128).astype(np.float32)
    p, s, z, g = O.quantize_values(v, bits, 64)
    deq = O.dequantize_values(p, s, z, 128, bits, 64)
    rel = np.sqrt(np.mean((v - deq) ** 2)) / (np.std(v) + 1e-8)
    assert g == 2 and rel < thresh


def test_grouped_quant_closed_form():
    v = np.array([[0.0, 1.0, 2.0, 3.0, 10.0, 10.0, 10.0, 10.0]], np.float32)
    p, s, z, _ = O.quantize_values(np.tile(v, (1, 2)), 2, 8)
    assert np.allclose(s[0], [10 / 3, 10 / 3]) and np.allclose(z[0], [0, 0])
    codes = O.unpack_indices(p, 16, 2)[0]
    # (v - 0) / (10/3) = 0, .3, .6, .9, 3, ... -> rint -> 0, 0, 1, 1, 3, 3, 3, 3
    assert list(codes[:8]) == [0, 0, 1, 1, 3, 3, 3, 3]
    # constant group: scale clamps to 1e-8, codes 0, dequant exact
    p, s, z, _ = O.quantize_values(np.full((1, 16), 2.5, np.float32), 4, 16)
    assert s[0, 0] == np.float32(1e-8) and not O.unpack_indices(p, 16, 4).any()
    assert (O.dequantize_values(p, s, z, 16, 4, 16) == 2.5).all()


def test_known_answer_5_scalar_quantize():
    np.random.seed(77)
    bnd = np.array([-1.0, -0.5, 0.0, 0.5, 1.0], np.float32)
    v = np.random.randn(100, 64).astype(np.float32)
    assert np.array_equal(O.scalar_quantize(v, bnd),
                          np.searchsorted(bnd, v, side="left").astype(np.uint8))


@pytest.mark.parametrize("seed,bits,t_q,t_kv,causal", [
    (555, 4, 1, 64, False),  # [15]
    (666, 4, 4, 32, True),   # [16]
    (777, 2, 1, 64, False),  # [17]
])
def test_known_answers_fused_dequant(seed, bits, t_q, t_kv, causal):
    np.random.seed(seed)
    nb, nc, bd, d = 16, 256, 8, 128
    cents = np.random.randn(nb, nc, bd).astype(np.float32)
    idx = np.random.randint(0, nc, size=(t_kv, nb), dtype=np.uint8)
    q = np.random.randn(t_q, d).astype(np.float32)
    v = np.random.randn(t_kv, d).astype(np.float32)
    p, s, z, _ = O.quantize_values(v, bits, 64)
    deq = O.dequantize_values(p, s, z, d, bits, 64)
    k_hat = O.dequantize_blockvq(idx, cents).astype(np.float64)
    sc = q.astype(np.float64) @ k_hat.T
    if causal:
        qp = np.arange(t_kv - t_q, t_kv)
        sc = np.where(qp[:, None] >= np.arange(t_kv)[None, :], sc, -1e30)
    w = np.exp(sc - sc.max(axis=-1, keepdims=True))
    ref = (w / w.sum(axis=-1, keepdims=True)) @ deq
    out = O.fused_attention_grouped(q, cents, idx, p, s, z, d, bits, 64, causal,
                                    t_kv - t_q if causal else 0)
    assert np.abs(out - ref).max() < 5e-3
    assert np.abs(out - ref).max() < 1e-9


def test_lloyd_max_tables():
    """The reference's literal tables (value_codecs.py:20-87), pinned by what
    the Lloyd-Max conditions fix: 1 bit is +-sqrt(2/pi) (closed form); every
    table is symmetric with boundaries at the midpoints of adjacent levels
    (middle boundary exactly 0, so a zero coordinate gets the upper-middle
    code); the levels are the fixed point of the conditions computed here
    independently, to 1e-9 at 2 and 3 bits and 4e-4 at 4 bits, where the
    literals are measurably off it (so they must be kept as data)."""
    l1, b1 = O.lloyd_max_gaussian(1)
    assert np.allclose(l1, [-math.sqrt(2 / math.pi), math.sqrt(2 / math.pi)], atol=1e-15)
    assert b1.tolist() == [0.0]
    for bits, tol in ((2, 1e-9), (3, 1e-9), (4, 4e-4)):
        lv, bd = O.lloyd_max_gaussian(bits)
        assert lv.size == 1 << bits and bd.size == lv.size - 1
        assert np.array_equal(lv, -lv[::-1])
        assert np.array_equal(bd, 0.5 * (lv[1:] + lv[:-1]))
        assert bd[bd.size // 2] == 0.0
        fl, fb = O.lloyd_max_fixed_point(bits)
        assert np.abs(lv - fl).max() < tol and np.abs(bd - fb).max() < tol
    l4, _ = O.lloyd_max_gaussian(4)
    assert np.abs(l4 - O.lloyd_max_fixed_point(4)[0]).max() > 1e-4
    # Max (1960), table I, to its printed precision
    l2, b2 = O.lloyd_max_gaussian(2)
    assert np.allclose(l2, [-1.510, -0.4528, 0.4528, 1.510], atol=5e-4)
    assert np.allclose(b2, [-0.9816, 0.0, 0.9816], atol=5e-4)
    l3, _ = O.lloyd_max_gaussian(3)
    assert np.allclose(l3[4:], [0.2451, 0.7560, 1.344, 2.152], atol=5e-4)


def test_scalar_quantize_zero_coordinate_takes_lower_middle_code():
    """With the exact-zero middle boundary, ``#(0 > boundaries)`` counts only
    the negative boundaries: a zero value row (zero norm, zero rotated
    coordinates) gets code 2^(bits-1) - 1 at every bit width (code 1 at 2
    bits, as in the reference)."""
    for bits in (2, 3, 4):
        _, b = O.turboquant_tables(bits, 128)
        assert O.scalar_quantize(np.zeros(5, np.float32), b).tolist() == [(1 << (bits - 1)) - 1] * 5


def test_turboquant_codec_tables_equal_reference_literals():
    """The product's TurboQuant tables (built from its own copy of the
    positive levels) equal the reference's literal tables scaled by
    1/sqrt(D) and rounded to float32 (value_codecs.py:148-151), bit for bit,
    at every bit width and D = 64, 128."""
    for bits in (2, 3, 4):
        for d in (64, 128):
            tq = S.TurboQuantValueCodec(head_dim=d, bits=bits, device="cpu")
            c, b = O.turboquant_tables(bits, d)
            assert np.array_equal(tq.centroids.numpy(), c)
            assert np.array_equal(tq.boundaries.numpy(), b)
    for bits in (1, 2, 3, 4):
        lv, bd = S.value_codecs.lloyd_max_gaussian(bits)
        rl, rb = O.lloyd_max_gaussian(bits)
        assert list(lv) == rl.tolist() and list(bd) == rb.tolist()


def test_rotation_orthogonal_and_turboquant_roundtrip():
    r = O.rotation_matrix(64, 43)
    assert np.abs(r @ r.T - np.eye(64)).max() < 1e-5
    lv, bd = O.lloyd_max_gaussian(2)
    cents = (lv / math.sqrt(64)).astype(np.float32)
    bnds = (bd / math.sqrt(64)).astype(np.float32)
    rng = np.random.default_rng(0)
    v = rng.standard_normal((64, 64)).astype(np.float32)
    p, n, _ = O.turboquant_encode(v, r, bnds, 2)
    vh = O.turboquant_decode(p, n, r, cents, 64, 2)
    assert np.mean((v - vh) ** 2) < 1.5  # reference test_sunshape_mlx.py:495-504 bound
    assert np.mean((v - vh) ** 2) < 0.15  # 2-bit Lloyd-Max distortion ~0.1175 per unit var
