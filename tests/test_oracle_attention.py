"""Pins for oracle.attention."""

import numpy as np

from oracle import attention as A


def test_mask_semantics_and_shape_invariance():
    # tests/test_ragged_kv_cache.py:108-138
    m1 = A.ragged_causal_mask([0, 3], 2, 6)
    m2 = A.ragged_causal_mask([4, 1], 2, 6)
    assert m1.shape == m2.shape == (2, 1, 2, 6) and m1.dtype == bool
    assert m1[1, 0, 0].tolist() == [True] * 4 + [False] * 2
    assert m1[1, 0, 1].tolist() == [True] * 5 + [False]
    add = A.ragged_additive_mask([1], 1, 3)
    assert add[0, 0, 0].tolist() == [0.0, 0.0, -np.inf]


def test_attention_matches_bruteforce():
    rng = np.random.default_rng(0)
    B, Hq, Hkv, L, D, cap = 2, 4, 2, 3, 8, 12
    q = rng.normal(size=(B, Hq, L, D)); k = rng.normal(size=(B, Hkv, cap, D)); v = rng.normal(size=(B, Hkv, cap, D))
    qs = [5, 9]
    assert np.allclose(A.ragged_gqa_attention(q, k, v, qs), A.ragged_gqa_attention_bruteforce(q, k, v, qs), atol=1e-12)


def test_single_key_returns_value_and_rows_independent():
    rng = np.random.default_rng(1)
    q = rng.normal(size=(2, 2, 1, 4)); k = rng.normal(size=(2, 1, 5, 4)); v = rng.normal(size=(2, 1, 5, 4))
    out = A.ragged_gqa_attention(q, k, v, [0, 3])
    assert np.allclose(out[0, :, 0], v[0, 0, 0][None, :], atol=1e-14)
    # row 1 alone gives the same answer as in the batch (per-row independence)
    solo = A.ragged_gqa_attention(q[1:], k[1:], v[1:], [3])
    assert np.array_equal(solo[0], out[1])


def test_uniform_offset_equals_plain_causal_prefix():
    rng = np.random.default_rng(2)
    q = rng.normal(size=(1, 2, 3, 4)); k = rng.normal(size=(1, 2, 10, 4)); v = rng.normal(size=(1, 2, 10, 4))
    out = A.ragged_gqa_attention(q, k, v, [4])
    trunc = A.ragged_gqa_attention(q, k[:, :, :7], v[:, :, :7], [4])
    assert np.allclose(out, trunc, atol=1e-14)

