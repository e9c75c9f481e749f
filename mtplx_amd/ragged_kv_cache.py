"""Ragged-batch KV cache (``mtplx/ragged_kv_cache.py``) on gfx950.

Same protocol as the reference's ``RaggedBatchKVCache`` (:71-496): physical
buffers ``[B, Hkv, cap, D]``, per-row logical lengths ``offsets`` int32 ``[B]``
kept on the GPU, per-row scatter at ``write_start`` (``update_and_fetch``
:201-277), a host capacity bound so no write forces a device read (:103-113),
frozen capacity (:340), ragged mask (:279), whole-batch trim (:366), masked
per-row restore (:473), filter/extend (:418-455), snapshots (:457-471).

Differences, on purpose: writes are in place (a HIP scatter into the
preallocated buffer) rather than a functional copy, so a snapshot is an owned
copy taken before the write; ``restore_masked`` can be limited to a position
range (the rows' speculative window) instead of rewriting whole buffers.
The reference's arrays are immutable, so every buffer this cache did not
allocate itself — given to the constructor, adopted by ``extend`` or
``from_scalar_cache``, set through ``state`` — or handed out through
``state`` is copied before the next in-place write (copy on write): a write
never changes another cache, the source scalar cache or a captured state.
The bookkeeping bodies (capacity bound and frozen capacity in
``update_and_fetch``, ``reserve``, ``freeze_capacity``, ``trim``, ``filter``,
``extend``, ``state``/``meta_state``) restate the reference's methods step
by step; they are the protocol a drop-in must keep.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from . import _lib
from .ragged_attention import ragged_causal_mask

__all__ = ["RaggedBatchKVCache", "RaggedKVSnapshot", "snapshot_ragged_caches", "restore_ragged_caches",
           "restore_ragged_caches_masked"]


def _as_int32_vector(value: Any, *, batch_size: int | None = None, device=None) -> torch.Tensor:
    t = value if isinstance(value, torch.Tensor) else torch.as_tensor(value)
    t = t.to(dtype=torch.int32, device=device if device is not None else (t.device if t.is_cuda else "cuda"))
    t = t.reshape(-1).contiguous()
    if batch_size is not None and t.numel() != int(batch_size):
        raise ValueError(f"expected a length-{batch_size} per-row vector, got size {t.numel()}")
    return t


@dataclass(frozen=True)
class RaggedKVSnapshot:
    keys: Any
    values: Any
    offsets: Any
    step: int


class RaggedBatchKVCache:
    def __init__(self, *, batch_size: int | None = None, step: int = 256, keys: torch.Tensor | None = None,
                 values: torch.Tensor | None = None, offsets: Any | None = None) -> None:
        self._keys = keys
        self._values = values
        self.step = int(step)
        if offsets is not None:
            self.offsets = _as_int32_vector(offsets, batch_size=batch_size)
        elif batch_size is not None:
            self.offsets = torch.zeros((int(batch_size),), dtype=torch.int32, device="cuda")
        elif keys is not None:
            self.offsets = torch.zeros((int(keys.shape[0]),), dtype=torch.int32, device=keys.device)
        else:
            self.offsets = None
        self._capacity_bound: int | None = None
        self._frozen_capacity: int | None = None
        self._status = None
        # True while keys/values may be referenced outside this cache.
        self._shared = keys is not None

    # Buffers assigned from outside (``cache.keys = t``, as the reference's
    # own tests do) may be referenced elsewhere: they are marked shared.
    @property
    def keys(self):
        return self._keys

    @keys.setter
    def keys(self, value) -> None:
        self._keys = value
        self._shared = value is not None

    @property
    def values(self):
        return self._values

    @values.setter
    def values(self, value) -> None:
        self._values = value
        self._shared = value is not None

    def _set_buffers(self, k, v, *, shared: bool) -> None:
        self._keys, self._values = k, v
        self._shared = shared and k is not None

    def _own_buffers(self) -> None:
        """Copy buffers that may be referenced elsewhere before writing in place."""
        if self._shared and self._keys is not None:
            self._keys = self._keys.clone()
            self._values = self._values.clone()
        self._shared = False

    # -- construction ---------------------------------------------------------
    @classmethod
    def from_scalar_cache(cls, entry: Any, *, batch_size: int | None = None,
                          step: int | None = None) -> "RaggedBatchKVCache":
        keys = getattr(entry, "keys", None)
        values = getattr(entry, "values", None)
        scalar_offset = int(getattr(entry, "offset", 0))
        if batch_size is None and keys is not None:
            batch_size = int(keys.shape[0])
        if batch_size is None:
            raise ValueError("batch_size is required when the source cache has no keys")
        dev = keys.device if keys is not None else "cuda"
        out = cls(batch_size=int(batch_size), step=int(step or getattr(entry, "step", 256)), keys=keys,
                  values=values, offsets=torch.full((int(batch_size),), scalar_offset, dtype=torch.int32, device=dev))
        out._capacity_bound = scalar_offset
        return out

    # -- core contract ---------------------------------------------------------
    @property
    def offset(self) -> torch.Tensor:
        return self.offsets

    def _ensure_offsets(self, batch_size: int, device) -> None:
        if self.offsets is None:
            self.offsets = torch.zeros((int(batch_size),), dtype=torch.int32, device=device)
        elif self.offsets.numel() != int(batch_size):
            raise ValueError(f"batch size mismatch: cache has {self.offsets.numel()} rows, write has {int(batch_size)}")

    def _grow_to(self, required: int, tk: torch.Tensor, tv: torch.Tensor) -> None:
        B, H, _, kd = tk.shape
        vd = tv.shape[3]
        cur = 0 if self.keys is None else int(self.keys.shape[2])
        if required <= cur and self.keys is not None:
            return
        n = (int(required) + self.step - 1) // self.step
        new_cap = max(n * self.step, self.step)
        nk = torch.zeros((B, H, new_cap, kd), dtype=tk.dtype, device=tk.device)
        nv = torch.zeros((B, H, new_cap, vd), dtype=tv.dtype, device=tv.device)
        if self.keys is not None:
            nk[:, :, :cur].copy_(self.keys)
            nv[:, :, :cur].copy_(self.values)
        self._set_buffers(nk, nv, shared=False)

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor, *, write_start: Any | None = None,
                         new_offsets: Any | None = None):
        B, H, q, D = (int(s) for s in keys.shape)
        self._ensure_offsets(B, keys.device)
        start = self.offsets if write_start is None else _as_int32_vector(write_start, batch_size=B,
                                                                          device=keys.device)
        resulting = (start + q) if new_offsets is None else _as_int32_vector(new_offsets, batch_size=B,
                                                                             device=keys.device)
        if self._frozen_capacity is not None:
            required = self._frozen_capacity
        elif self._capacity_bound is not None:
            self._capacity_bound += q
            required = self._capacity_bound
        else:
            required = int(start.max().item()) + q   # legacy single device read, as the reference
        self._grow_to(required, keys, values)
        self._own_buffers()
        if self._status is None or self._status.device != keys.device:
            self._status = torch.zeros(1, dtype=torch.int32, device=keys.device)
        kc, vc = keys.contiguous(), values.contiguous()   # named: both must stay allocated
        _lib.call("mtp_kv_scatter", self.keys.data_ptr(), self.values.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                  start.data_ptr(), B, H, int(self.keys.shape[2]), q, D,
                  self._status.data_ptr(), _lib.stream_handle(keys.device))
        self.offsets = resulting.to(torch.int32)
        return self.keys, self.values

    def write_fault(self) -> bool:
        """True if any scatter hit a position outside the buffer (device flag, reads it)."""
        return bool(self._status is not None and int(self._status.item()) != 0)

    def make_mask(self, q_len: int, *, return_array: bool = False, window_size: int | None = None,
                  key_len: int | None = None) -> torch.Tensor:
        del return_array, window_size
        if key_len is None:
            key_len = 0 if self.keys is None else int(self.keys.shape[2])
        return ragged_causal_mask(self.offsets, int(q_len), int(key_len))

    def reserve(self, additional_positions: int) -> None:
        if self.keys is None or self.values is None:
            return
        if self._frozen_capacity is not None:
            self._grow_to(self._frozen_capacity, self.keys, self.values)
            return
        if self._capacity_bound is None:
            return
        self._grow_to(self._capacity_bound + int(additional_positions), self.keys, self.values)

    def freeze_capacity(self, capacity: int) -> None:
        cap = int(capacity)
        if self.keys is not None and self.values is not None:
            self._grow_to(cap, self.keys, self.values)
        self._frozen_capacity = cap

    def size(self) -> int:
        return 0 if self.offsets is None else int(self.offsets.max().item())

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        if self.offsets is None:
            return 0
        n = min(int(n), max(int(self.offsets.min().item()), 0))
        self.offsets = torch.clamp(self.offsets - n, min=0).to(torch.int32)
        return n

    def empty(self) -> bool:
        return self.keys is None

    @property
    def nbytes(self) -> int:
        if self.keys is None or self.values is None:
            return 0
        return self.keys.numel() * self.keys.element_size() + self.values.numel() * self.values.element_size()

    @property
    def state(self):
        """``(keys, values, offsets)``. The tensors are handed out as they are;
        the cache copies its buffers before its next in-place write, so what
        the caller holds keeps this moment's contents (the reference's
        immutable-array semantics)."""
        if self.keys is not None:
            self._shared = True
        return (self.keys, self.values, self.offsets)

    @state.setter
    def state(self, value) -> None:
        if value is None:
            self._set_buffers(None, None, shared=False)
            self.offsets = None
            return
        k, v, off = value
        self._set_buffers(k, v, shared=True)
        self.offsets = None if off is None else _as_int32_vector(off)

    @property
    def meta_state(self) -> tuple:
        return ("ragged_batch_kv", str(self.step))

    @meta_state.setter
    def meta_state(self, value) -> None:
        if value and len(value) > 1:
            self.step = int(value[1])

    def filter(self, batch_indices: Any) -> None:
        idx = _as_int32_vector(batch_indices, device=self.keys.device if self.keys is not None else None).long()
        if self.keys is not None:
            # advanced indexing: new buffers
            self._set_buffers(self.keys[idx].contiguous(), self.values[idx].contiguous(), shared=False)
        if self.offsets is not None:
            self.offsets = self.offsets[idx].to(torch.int32).contiguous()

    def extend(self, other: "RaggedBatchKVCache") -> None:
        if other.keys is None:
            return
        if self.keys is None:
            self._set_buffers(other.keys, other.values, shared=True)
            self.offsets = None if other.offsets is None else other.offsets.to(torch.int32).clone()
            other._shared = True
            return
        cap = max(int(self.keys.shape[2]), int(other.keys.shape[2]))
        ak, av = _pad_seq_to(self.keys, cap), _pad_seq_to(self.values, cap)
        bk, bv = _pad_seq_to(other.keys, cap), _pad_seq_to(other.values, cap)
        self._set_buffers(torch.cat([ak, bk], dim=0), torch.cat([av, bv], dim=0), shared=False)
        self.offsets = torch.cat([self.offsets, other.offsets]).to(torch.int32)

    def snapshot(self) -> RaggedKVSnapshot:
        return RaggedKVSnapshot(None if self.keys is None else self.keys.clone(),
                                None if self.values is None else self.values.clone(),
                                None if self.offsets is None else self.offsets.clone(), int(self.step))

    def restore(self, snap: RaggedKVSnapshot) -> None:
        self._set_buffers(None if snap.keys is None else snap.keys.clone(),
                          None if snap.values is None else snap.values.clone(), shared=False)
        self.offsets = None if snap.offsets is None else snap.offsets.clone()
        self.step = int(snap.step)

    def restore_masked(self, snap: RaggedKVSnapshot, row_mask: Any, *, positions: tuple[int, int] | None = None):
        """Rows where ``row_mask`` is true revert offsets and buffer to ``snap``
        (zero past the snapshot's capacity); other rows keep their state.
        ``positions=(lo, hi)`` limits the buffer copy to that range."""
        dev = self.offsets.device if self.offsets is not None else "cuda"
        mask = (row_mask if isinstance(row_mask, torch.Tensor) else torch.as_tensor(row_mask)).to(
            device=dev, dtype=torch.bool).reshape(-1)
        if snap.offsets is not None and self.offsets is not None:
            self.offsets = torch.where(mask, snap.offsets, self.offsets).to(torch.int32)
        if snap.keys is None or self.keys is None:
            return
        cap = int(self.keys.shape[2])
        if int(snap.keys.shape[2]) > cap:
            self._grow_to(int(snap.keys.shape[2]), self.keys, self.values)
            cap = int(self.keys.shape[2])
        lo, hi = (0, cap) if positions is None else (max(0, int(positions[0])), min(cap, int(positions[1])))
        self._own_buffers()
        m8 = mask.to(torch.uint8).contiguous()
        B, H, _, D = (int(s) for s in self.keys.shape)
        st = _lib.stream_handle(self.keys.device)
        for cur, sn in ((self.keys, snap.keys), (self.values, snap.values)):
            sn = sn.contiguous()
            _lib.call("mtp_kv_restore_masked", cur.data_ptr(), sn.data_ptr(), m8.data_ptr(), B, H, cap,
                      int(sn.shape[2]), D, lo, hi, st)


def _pad_seq_to(buf: torch.Tensor, cap: int) -> torch.Tensor:
    seq = int(buf.shape[2])
    if seq >= cap:
        return buf
    pad = torch.zeros((buf.shape[0], buf.shape[1], cap - seq, buf.shape[3]), dtype=buf.dtype, device=buf.device)
    return torch.cat([buf, pad], dim=2)


def snapshot_ragged_caches(cache: list) -> tuple:
    return tuple(e.snapshot() if isinstance(e, RaggedBatchKVCache) else None for e in cache)


def restore_ragged_caches(cache: list, snapshots: tuple) -> None:
    for e, s in zip(cache, snapshots):
        if isinstance(e, RaggedBatchKVCache) and s is not None:
            e.restore(s)


def restore_ragged_caches_masked(cache: list, snapshots: tuple, row_mask: Any) -> None:
    for e, s in zip(cache, snapshots):
        if isinstance(e, RaggedBatchKVCache) and s is not None:
            e.restore_masked(s, row_mask)
