"""GPU tests of the RaggedBatchKVCache protocol: the reference's mechanics
tests (``tests/test_ragged_kv_cache.py:524-759``: per-row scatter and advance,
grow, filter/extend, snapshot round trip, trim, from_scalar_cache, the host
capacity bound, reserve and frozen capacity) plus copy on write: a buffer the
cache adopted or handed out is never changed by a later in-place write."""

from types import SimpleNamespace

import pytest
import torch

pytestmark = pytest.mark.gpu


def _rand(*shape, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(shape, device="cuda", generator=g).to(torch.bfloat16)


def _cache(**kw):
    from mtplx_amd.ragged_kv_cache import RaggedBatchKVCache
    return RaggedBatchKVCache(**kw)


def _offs(rg):
    return rg.offsets.cpu().tolist()


def test_update_appends_at_per_row_offsets(gpu):
    B, H, D = 4, 2, 8
    rg = _cache(step=8)
    rg.offsets = torch.tensor([1, 3, 0, 5], dtype=torch.int32, device="cuda")
    rg.keys = torch.zeros((B, H, 8, D), dtype=torch.bfloat16, device="cuda")
    rg.values = torch.zeros_like(rg.keys)
    nk, nv = _rand(B, H, 2, D, seed=1), _rand(B, H, 2, D, seed=2)
    k, v = rg.update_and_fetch(nk, nv)
    for r, s in enumerate([1, 3, 0, 5]):
        assert torch.equal(k[r, :, s:s + 2], nk[r]) and torch.equal(v[r, :, s:s + 2], nv[r])
    assert _offs(rg) == [3, 5, 2, 7]
    assert not rg.write_fault()


def test_per_row_advance_via_new_offsets(gpu):
    B, H, D = 3, 2, 8
    rg = _cache(step=8, keys=torch.zeros((B, H, 8, D), dtype=torch.bfloat16, device="cuda"),
                values=torch.zeros((B, H, 8, D), dtype=torch.bfloat16, device="cuda"), offsets=[2, 2, 2])
    nk, nv = _rand(B, H, 2, D, seed=3), _rand(B, H, 2, D, seed=4)
    k, _ = rg.update_and_fetch(nk, nv, write_start=[2, 1, 0], new_offsets=[4, 3, 2])
    assert _offs(rg) == [4, 3, 2]
    assert torch.equal(k[1, :, 1:3], nk[1]) and torch.equal(k[2, :, 0:2], nk[2])


def test_grow_preserves_existing_content(gpu):
    B, H, D = 2, 2, 8
    seed_k = _rand(B, H, 3, D, seed=5)
    keys = torch.zeros((B, H, 4, D), dtype=torch.bfloat16, device="cuda")
    keys[:, :, :3] = seed_k
    rg = _cache(step=4, keys=keys, values=torch.zeros_like(keys), offsets=[3, 2])
    k, _ = rg.update_and_fetch(_rand(B, H, 2, D, seed=6), _rand(B, H, 2, D, seed=7), write_start=[3, 4])
    assert int(k.shape[2]) >= 6
    assert torch.equal(k[:, :, :3], seed_k)


def test_filter_and_extend(gpu):
    H, D = 2, 8
    keys, vals = _rand(4, H, 8, D, seed=8), _rand(4, H, 8, D, seed=9)
    rg = _cache(step=8, keys=keys, values=vals, offsets=[2, 4, 1, 5])
    rg.filter([0, 2])
    assert _offs(rg) == [2, 1]
    assert torch.equal(rg.keys[0], keys[0]) and torch.equal(rg.keys[1], keys[2])
    a = _cache(step=4, keys=_rand(2, H, 4, D, seed=10), values=_rand(2, H, 4, D, seed=11), offsets=[2, 3])
    b = _cache(step=8, keys=_rand(1, H, 8, D, seed=12), values=_rand(1, H, 8, D, seed=13), offsets=[5])
    a_k = a.keys.clone()
    a.extend(b)
    assert _offs(a) == [2, 3, 5] and int(a.keys.shape[0]) == 3 and int(a.keys.shape[2]) == 8
    assert torch.equal(a.keys[:2, :, :4], a_k) and torch.equal(a.keys[2], b.keys[0])
    assert not a.keys[:2, :, 4:].any()      # zero pad to the larger capacity


def test_extend_into_empty_then_write_leaves_source(gpu):
    H, D = 2, 8
    b = _cache(step=8, keys=_rand(2, H, 8, D, seed=14), values=_rand(2, H, 8, D, seed=15), offsets=[1, 2])
    b_k, b_v = b.keys.clone(), b.values.clone()
    a = _cache(step=8)
    a.extend(b)
    a.update_and_fetch(_rand(2, H, 2, D, seed=16), _rand(2, H, 2, D, seed=17))
    assert torch.equal(b.keys, b_k) and torch.equal(b.values, b_v)
    assert _offs(b) == [1, 2] and _offs(a) == [3, 4]


def test_state_snapshot_round_trip(gpu):
    """cache_state.snapshot_cache keeps ``state``/``meta_state``; a later write
    must not change the captured tensors (reference: immutable arrays)."""
    B, H, D = 3, 2, 8
    keys, vals = _rand(B, H, 8, D, seed=18), _rand(B, H, 8, D, seed=19)
    rg = _cache(step=8, keys=keys.clone(), values=vals.clone(), offsets=[2, 4, 1])
    snap, meta = rg.state, rg.meta_state
    rg.update_and_fetch(_rand(B, H, 2, D, seed=20), _rand(B, H, 2, D, seed=21))
    assert _offs(rg) == [4, 6, 3]
    assert torch.equal(snap[0], keys) and torch.equal(snap[1], vals)   # captured state untouched
    assert snap[2].cpu().tolist() == [2, 4, 1]
    rg.state = snap
    rg.meta_state = meta
    assert _offs(rg) == [2, 4, 1] and torch.equal(rg.keys, keys) and meta == ("ragged_batch_kv", "8")
    # writing after the restore copies again: snap stays as captured
    rg.update_and_fetch(_rand(B, H, 1, D, seed=22), _rand(B, H, 1, D, seed=23))
    assert torch.equal(snap[0], keys)


def test_snapshot_restore_and_masked_restore(gpu):
    B, H, D = 3, 2, 8
    rg = _cache(step=8, keys=_rand(B, H, 8, D, seed=24), values=_rand(B, H, 8, D, seed=25), offsets=[2, 3, 4])
    snap = rg.snapshot()
    rg.update_and_fetch(_rand(B, H, 2, D, seed=26), _rand(B, H, 2, D, seed=27))
    after = rg.keys.clone()
    rg.restore_masked(snap, [True, False, True], positions=(0, 8))
    assert _offs(rg) == [2, 5, 4]
    assert torch.equal(rg.keys[0], snap.keys[0]) and torch.equal(rg.keys[2], snap.keys[2])
    assert torch.equal(rg.keys[1], after[1])
    rg.restore(snap)
    assert _offs(rg) == [2, 3, 4] and torch.equal(rg.keys, snap.keys)
    rg.update_and_fetch(_rand(B, H, 1, D, seed=28), _rand(B, H, 1, D, seed=29))
    assert not torch.equal(rg.keys, snap.keys)          # the snapshot itself is never written


def test_trim_whole_batch(gpu):
    rg = _cache(step=8, keys=torch.zeros((3, 2, 8, 8), dtype=torch.bfloat16, device="cuda"),
                values=torch.zeros((3, 2, 8, 8), dtype=torch.bfloat16, device="cuda"), offsets=[5, 8, 6])
    assert rg.trim(3) == 3 and _offs(rg) == [2, 5, 3]
    assert rg.trim(10) == 2 and _offs(rg) == [0, 3, 1]


def test_from_scalar_cache_seed_and_copy_on_write(gpu):
    from mtplx_amd.ragged_kv_cache import RaggedBatchKVCache
    sc = SimpleNamespace(keys=_rand(4, 2, 5, 8, seed=30), values=_rand(4, 2, 5, 8, seed=31), offset=5, step=64)
    src_k = sc.keys.clone()
    rg = RaggedBatchKVCache.from_scalar_cache(sc)
    assert _offs(rg) == [5] * 4 and torch.equal(rg.keys, sc.keys)
    assert rg._capacity_bound == 5 and rg.step == 64
    rg.update_and_fetch(_rand(4, 2, 2, 8, seed=32), _rand(4, 2, 2, 8, seed=33))
    assert rg._capacity_bound == 7
    assert torch.equal(sc.keys, src_k)                   # the scalar cache is not written
    with pytest.raises(ValueError):
        RaggedBatchKVCache.from_scalar_cache(SimpleNamespace(offset=0))


def test_capacity_bound_monotone_and_reserve(gpu):
    from mtplx_amd.ragged_kv_cache import RaggedBatchKVCache
    B, H, D = 2, 2, 8
    rg = RaggedBatchKVCache.from_scalar_cache(SimpleNamespace(keys=None, values=None, offset=0, step=4),
                                              batch_size=B)
    assert rg._capacity_bound == 0
    for cycle in range(6):
        rg.update_and_fetch(_rand(B, H, 2, D, seed=40 + cycle), _rand(B, H, 2, D, seed=50 + cycle))
        assert rg._capacity_bound == 2 * (cycle + 1)
        assert int(rg.keys.shape[2]) >= rg._capacity_bound
    # reserve pre-grows so no grow happens inside update_and_fetch
    rg = _cache(step=16, keys=torch.zeros((4, H, 16, D), dtype=torch.bfloat16, device="cuda"),
                values=torch.zeros((4, H, 16, D), dtype=torch.bfloat16, device="cuda"), offsets=[14] * 4)
    rg._capacity_bound = 14
    rg.reserve(2)
    assert int(rg.keys.shape[2]) == 16
    key_len = int(rg.make_mask(2).shape[-1])
    keys, _ = rg.update_and_fetch(_rand(4, H, 2, D, seed=60), _rand(4, H, 2, D, seed=61))
    assert int(keys.shape[2]) == 16 == key_len
    rg.reserve(2)
    assert int(rg.keys.shape[2]) == 32 and int(rg.make_mask(2).shape[-1]) == 32


def test_freeze_capacity_pins_the_buffer(gpu):
    B, H, D = 2, 2, 8
    rg = _cache(step=16, keys=torch.zeros((B, H, 16, D), dtype=torch.bfloat16, device="cuda"),
                values=torch.zeros((B, H, 16, D), dtype=torch.bfloat16, device="cuda"), offsets=[3, 7])
    rg.freeze_capacity(40)
    assert int(rg.keys.shape[2]) == 48                   # step-rounded once
    for i in range(3):
        rg.update_and_fetch(_rand(B, H, 2, D, seed=70 + i), _rand(B, H, 2, D, seed=80 + i))
        assert int(rg.keys.shape[2]) == 48
    rg.reserve(100)
    assert int(rg.keys.shape[2]) == 48
    empty = _cache(step=16, batch_size=B)
    empty.freeze_capacity(20)
    empty.update_and_fetch(_rand(B, H, 1, D, seed=90), _rand(B, H, 1, D, seed=91))
    assert int(empty.keys.shape[2]) == 32


def test_batch_size_mismatch_raises(gpu):
    rg = _cache(step=8, batch_size=3)
    with pytest.raises(ValueError):
        rg.update_and_fetch(_rand(2, 2, 1, 8), _rand(2, 2, 1, 8))
    with pytest.raises(ValueError):
        _cache(batch_size=3, offsets=[1, 2])
