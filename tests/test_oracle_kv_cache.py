"""Pins for oracle.kv_cache (the ragged cache gates)."""

import numpy as np

from oracle import kv_cache as KV


def test_kv_scatter_replay_and_restore():
    rng = np.random.default_rng(3)
    cache = np.zeros((2, 2, 8, 4), np.uint16)
    new = rng.integers(1, 1 << 15, size=(2, 2, 3, 4)).astype(np.uint16)
    c1 = KV.scatter(cache, new, [0, 4])
    assert np.array_equal(c1[1, :, 4:7], new[1]) and not c1[1, :, :4].any()
    # REPLAY rewrite at offset-1 overwrites in place, leaves the rest
    new2 = rng.integers(1, 1 << 15, size=(2, 2, 3, 4)).astype(np.uint16)
    c2 = KV.scatter(c1, new2, [2, 3])
    assert np.array_equal(c2[0, :, 0:2], c1[0, :, 0:2]) and np.array_equal(c2[1, :, 3:6], new2[1])
    r = KV.restore_masked(c2, c1, [True, False])
    assert np.array_equal(r[0], c1[0]) and np.array_equal(r[1], c2[1])
    assert KV.grow_capacity(300, 256, 256) == 512 and KV.grow_capacity(10, 0, 256) == 256
    off, n = KV.trim([5, 2, 7], 4)
    assert n == 2 and off.tolist() == [3, 0, 5]

