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
