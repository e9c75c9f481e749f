"""Pins for oracle.qmv: closed forms, round trips and an independent route."""

import numpy as np

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.qmv import (dequantize_affine4, make_affine4_weights, pack_affine4, qmm_affine4,
                        qmm_affine4_groupwise, unpack_affine4)


def test_pack_roundtrip_and_nibble_order():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(5, 64), dtype=np.uint8)
    w = pack_affine4(q)
    assert w.dtype == np.uint32 and w.shape == (5, 8)
    assert np.array_equal(unpack_affine4(w), q)
    # little-endian nibbles: q[n, 8j+i] sits in bits 4i..4i+3 of word j
    q1 = np.zeros((1, 8), np.uint8); q1[0, 1] = 0xA; q1[0, 7] = 0x3
    assert int(pack_affine4(q1)[0, 0]) == (0xA << 4) | (0x3 << 28)


def test_bf16_rounding_is_nearest_even():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0], np.float32)
    bits = f32_to_bf16_bits(vals)
    back = bf16_bits_to_f32(bits)
    assert back[0] == 1.0 and back[1] == 1.0            # tie -> even
    assert back[2] == np.float32(1.0 + 4 * 2 ** -8)     # tie -> even (up)
    assert back[3] == -2.5 and back[4] == 0.0


def test_closed_form_zero_nibbles_is_bias_times_group_sums():
    rng = np.random.default_rng(1)
    n, k, gs = 6, 256, 64
    w = pack_affine4(np.zeros((n, k), np.uint8))
    s = rng.random((n, k // gs)); b = rng.normal(size=(n, k // gs))
    x = rng.normal(size=(3, k))
    want = x.reshape(3, -1, gs).sum(axis=2) @ b.T
    assert np.allclose(qmm_affine4(x, w, s, b, gs), want, rtol=1e-12, atol=1e-12)


def test_closed_form_all_fifteen_unit_scale():
    rng = np.random.default_rng(2)
    n, k, gs = 4, 128, 64
    w = pack_affine4(np.full((n, k), 15, np.uint8))
    x = rng.normal(size=(2, k))
    y = qmm_affine4(x, w, np.ones((n, k // gs)), np.zeros((n, k // gs)), gs)
    assert np.allclose(y, 15 * x.sum(axis=1)[:, None], rtol=1e-12)


def test_single_nonzero_group():
    n, k, gs = 2, 192, 64
    q = np.zeros((n, k), np.uint8); q[1, 64:128] = 7
    s = np.zeros((n, 3)); s[1, 1] = 0.5
    x = np.arange(k, dtype=np.float64)[None, :]
    y = qmm_affine4(x, pack_affine4(q), s, np.zeros((n, 3)), gs)
    assert y[0, 0] == 0.0 and y[0, 1] == 7 * 0.5 * x[0, 64:128].sum()


def test_groupwise_route_matches_dense_route():
    rng = np.random.default_rng(3)
    w, s, b = make_affine4_weights(rng, 40, 512, 64)
    x = f32_to_bf16_bits(rng.normal(size=(4, 512)).astype(np.float32))
    a = qmm_affine4(x, w, s, b, 64)
    c = qmm_affine4_groupwise(x, w, s, b, 64)
    assert np.allclose(a, c, rtol=1e-11, atol=1e-11)
    deq = dequantize_affine4(w, s, b, 64)
    assert deq.shape == (40, 512)
    assert np.allclose(a, bf16_bits_to_f32(x).astype(np.float64) @ deq.T, rtol=1e-12, atol=1e-12)


# ---- any-width packs (8-bit, group 32) -------------------------------------

def test_pack_affine_byte_order_and_roundtrip():
    from oracle.qmv import pack_affine, unpack_affine
    # 8-bit: value i of a word in bits 8i..8i+7
    assert int(pack_affine(np.array([[1, 2, 3, 4]], np.uint8), 8)[0, 0]) == 0x04030201
    assert int(pack_affine(np.array([[255, 0, 0, 128]], np.uint8), 8)[0, 0]) == 0x800000FF
    # 2-bit: sixteen values per word
    q2 = np.zeros((1, 16), np.uint8); q2[0, 15] = 3; q2[0, 1] = 1
    assert int(pack_affine(q2, 2)[0, 0]) == (3 << 30) | (1 << 2)
    rng = np.random.default_rng(10)
    for bits in (2, 4, 8):
        q = rng.integers(0, 1 << bits, size=(3, 64), dtype=np.uint8)
        assert np.array_equal(unpack_affine(pack_affine(q, bits), bits), q)
    q = rng.integers(0, 16, size=(3, 64), dtype=np.uint8)
    assert np.array_equal(pack_affine(q, 4), pack_affine4(q))


def test_qmm_affine_closed_forms_8bit_group32():
    from oracle.qmv import pack_affine, qmm_affine
    rng = np.random.default_rng(11)
    n, k, gs = 5, 128, 32
    x = rng.normal(size=(3, k))
    s = rng.random((n, k // gs)); b = rng.normal(size=(n, k // gs))
    zero = pack_affine(np.zeros((n, k), np.uint8), 8)
    assert np.allclose(qmm_affine(x, zero, s, b, gs, 8), x.reshape(3, -1, gs).sum(axis=2) @ b.T, rtol=1e-12,
                       atol=1e-12)
    full = pack_affine(np.full((n, k), 255, np.uint8), 8)
    y = qmm_affine(x, full, np.ones((n, k // gs)), np.zeros((n, k // gs)), gs, 8)
    assert np.allclose(y, 255 * x.sum(axis=1)[:, None], rtol=1e-12)
    # one non-zero 32-group
    q = np.zeros((n, k), np.uint8); q[2, 32:64] = 200
    s1 = np.zeros((n, k // gs)); s1[2, 1] = 0.25
    y = qmm_affine(x, pack_affine(q, 8), s1, np.zeros((n, k // gs)), gs, 8)
    assert np.allclose(y[:, 2], 200 * 0.25 * x[:, 32:64].sum(axis=1), rtol=1e-12) and np.all(y[:, [0, 1, 3, 4]] == 0)


def test_qmm_affine_matches_scalar_loops_and_the_4bit_route():
    """Brute force from the packed words by explicit shifts (tiny case), and
    the 4-bit route of the general function against qmm_affine4."""
    from oracle.qmv import make_affine_weights, qmm_affine
    rng = np.random.default_rng(12)
    for bits, gs in ((8, 32), (8, 64), (4, 32), (2, 32)):
        w, s, b = make_affine_weights(rng, 3, 64, gs, bits)
        x = rng.normal(size=(2, 64))
        sf, bf = bf16_bits_to_f32(s).astype(np.float64), bf16_bits_to_f32(b).astype(np.float64)
        want = np.zeros((2, 3))
        vpw = 32 // bits
        for m in range(2):
            for nn in range(3):
                acc = 0.0
                for kk in range(64):
                    word = int(w[nn, kk // vpw])
                    q = (word >> (bits * (kk % vpw))) & ((1 << bits) - 1)
                    acc += x[m, kk] * (q * sf[nn, kk // gs] + bf[nn, kk // gs])
                want[m, nn] = acc
        assert np.allclose(qmm_affine(x, w, s, b, gs, bits), want, rtol=1e-12, atol=1e-12), (bits, gs)
    w, s, b = make_affine4_weights(rng, 16, 256, 64)
    x = rng.normal(size=(3, 256))
    assert np.allclose(qmm_affine(x, w, s, b, 64, 4), qmm_affine4(x, w, s, b, 64), rtol=1e-12, atol=1e-12)
