"""Pins for oracle.model (CPU)."""

import numpy as np

from oracle.model import rmsnorm, rope_rotate_half, route_topk


def test_rope_position_zero_is_identity_and_preserves_norm():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(3, 128))
    assert np.allclose(rope_rotate_half(x, np.zeros(3), 1e6), x)
    y = rope_rotate_half(x, np.array([5, 77, 4000]), 1e6)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1))
    # rotate-half pairing: dims j and j+64 rotate together by pos * base^(-2j/128)
    e = np.zeros(128); e[0] = 1.0
    r = rope_rotate_half(e[None], np.array([2.0]), 1e6)[0]
    assert np.isclose(r[0], np.cos(2.0)) and np.isclose(r[64], np.sin(2.0))


def test_rmsnorm_closed_form():
    x = np.array([[3.0, 4.0]])
    assert np.allclose(rmsnorm(x, np.array([1.0, 2.0]), 0.0), [[3 / np.sqrt(12.5), 8 / np.sqrt(12.5)]])


def test_route_topk_ties_and_weights():
    ids, w = route_topk(np.array([[1.0, 3.0, 3.0, 0.0]]), 2)
    assert ids.tolist() == [[1, 2]] and np.allclose(w, [[0.5, 0.5]])
