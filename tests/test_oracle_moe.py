"""Pins for oracle.moe."""

import numpy as np

from oracle import moe as M
from oracle.qmv import make_affine4_weights


def test_sort_rows_closed_form_and_counting_sort():
    rng = np.random.default_rng(4)
    idx = rng.integers(0, 16, size=(9, 4))
    row_map, sorted_ids, inv, order = M.sort_rows(idx)
    flat = idx.reshape(-1)
    # counting sort (stable) reproduces the order
    cs = [i for e in range(16) for i in range(flat.size) if flat[i] == e]
    assert order.tolist() == cs
    assert np.array_equal(order[inv], np.arange(flat.size))
    assert np.array_equal(row_map, order // 4) and np.array_equal(sorted_ids, flat[order])
    off = M.expert_offsets(sorted_ids, 16)
    assert off[-1] == flat.size and np.all(np.diff(off) >= 0)


def test_moe_sorted_chain_equals_per_expert_loop():
    rng = np.random.default_rng(5)
    E, H, F, T, k = 6, 128, 64, 5, 3
    gu = make_affine4_weights(rng, E * 2 * F, H)
    gu = tuple(a.reshape(E, 2 * F, -1) for a in gu)
    dn = make_affine4_weights(rng, E * H, F)
    dn = tuple(a.reshape(E, H, -1) for a in dn)
    x = rng.normal(size=(T, H))
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    sc = rng.random((T, k))
    assert np.allclose(M.moe_forward(x, idx, sc, gu, dn, 64), M.moe_forward_loop(x, idx, sc, gu, dn, 64), atol=1e-10)
    assert np.allclose(M.silu(np.array([0.0, 1.0])), [0.0, 1.0 / (1.0 + np.exp(-1.0))])

