"""Ragged KV cache mechanics, bit-exact.

Restates ``RaggedBatchKVCache`` (``mtplx/ragged_kv_cache.py:71-496``):
per-row scatter of a ``[B, Hkv, q, D]`` block at ``write_start[b]``
(``update_and_fetch`` :201-277), capacity growth in ``step`` units
(``_grow_to`` :183-199), whole-batch trim clamped at the smallest offset
(:366-379), per-row masked restore (:473-496), filter/extend (:418-455).

Parity pins (tests/test_oracle_kv_cache.py): the reference's gates — uniform
offsets equal the scalar tail cache, per-row independence, REPLAY rewrite in
place, masked restore bitwise, grow preserves content (``tests/test_ragged_kv_cache.py``).
"""

from __future__ import annotations

import numpy as np


def grow_capacity(required: int, current: int, step: int) -> int:
    """``_grow_to``: new capacity = max(ceil(required/step)*step, step) when it must grow."""
    if required <= current and current > 0:
        return current
    n = (int(required) + step - 1) // step
    return max(n * step, step)


def scatter(cache: np.ndarray, new: np.ndarray, write_start) -> np.ndarray:
    """``cache[b, :, ws[b]+i, :] = new[b, :, i, :]`` (returns a copy)."""
    out = np.array(cache, copy=True)
    ws = np.asarray(write_start, dtype=np.int64).reshape(-1)
    q = new.shape[2]
    for b in range(cache.shape[0]):
        out[b, :, ws[b]:ws[b] + q, :] = new[b]
    return out


def restore_masked(current: np.ndarray, snap: np.ndarray, row_mask) -> np.ndarray:
    """Rows with ``row_mask`` take the snapshot (zero-padded to the larger capacity)."""
    cap = max(current.shape[2], snap.shape[2])
    def pad(a):
        if a.shape[2] == cap:
            return a
        z = np.zeros(a.shape[:2] + (cap - a.shape[2],) + a.shape[3:], dtype=a.dtype)
        return np.concatenate([a, z], axis=2)
    m = np.asarray(row_mask, dtype=bool).reshape(-1)[:, None, None, None]
    return np.where(m, pad(snap), pad(current))


def trim(offsets, n: int):
    """Whole-batch trim: subtract ``min(n, max(min(offsets), 0))``, clamp at 0."""
    off = np.asarray(offsets, dtype=np.int32)
    n = min(int(n), max(int(off.min()), 0))
    return np.maximum(off - n, 0).astype(np.int32), n
