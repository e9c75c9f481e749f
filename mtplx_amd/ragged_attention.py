"""Ragged per-row causal attention (``mtplx/ragged_attention.py``) on gfx950.

``ragged_causal_mask`` / ``ragged_additive_mask`` keep the reference's fixed
``[B, 1, q_len, key_len]`` contract (:42-105). ``ragged_sdpa`` is the
attention those masks feed in the reference (stock SDPA over the padded
buffer, ``mtplx/attention_split.py:347``): here one kernel applies the same
rule ``j <= q_start[b] + i`` implicitly, reading offsets on the GPU.
"""

from __future__ import annotations

import math
from typing import Any

import torch

from . import _lib

__all__ = ["ragged_causal_mask", "ragged_additive_mask", "ragged_sdpa"]


def _q_start_vector(q_start: Any, device=None) -> torch.Tensor:
    if isinstance(q_start, torch.Tensor):
        t = q_start
    else:
        t = torch.as_tensor(q_start)
    return t.to(device=device or ("cuda" if not t.is_cuda else t.device), dtype=torch.int32).reshape(-1).contiguous()


def ragged_causal_mask(q_start: Any, q_len: int, key_len: int) -> torch.Tensor:
    """bool ``[B, 1, q_len, key_len]``: ``mask[b, 0, i, j] = j <= q_start[b] + i``."""
    qs = _q_start_vector(q_start)
    B = qs.numel()
    out = torch.empty((B, 1, int(q_len), int(key_len)), dtype=torch.uint8, device=qs.device)
    _lib.call("mtp_ragged_causal_mask", out.data_ptr(), qs.data_ptr(), B, int(q_len), int(key_len),
              _lib.stream_handle(qs.device))
    return out.view(torch.bool)


def ragged_additive_mask(q_start: Any, q_len: int, key_len: int, *, dtype=torch.float32) -> torch.Tensor:
    """``0`` where allowed, ``-inf`` elsewhere (same shape)."""
    allow = ragged_causal_mask(q_start, q_len, key_len)
    neg = torch.full((), float("-inf"), dtype=dtype, device=allow.device)
    return torch.where(allow, torch.zeros((), dtype=dtype, device=allow.device), neg)


_WS: dict = {}


def ragged_sdpa(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, q_start: Any, *,
                scale: float | None = None, q_lens: Any | None = None, split_keys: int = 0,
                out: torch.Tensor | None = None, rows_layout: bool = False) -> torch.Tensor:
    """``softmax(q k^T * scale + ragged mask) v`` with GQA.

    ``queries`` ``[B, Hq, L, 128]``, ``keys``/``values`` ``[B, Hkv, cap, 128]``
    bf16; ``q_start`` int32 ``[B]`` (may stay on the GPU). ``rows_layout``
    writes ``[B, L, Hq, 128]`` (the o-projection input rows).
    """
    B, Hq, L, D = (int(s) for s in queries.shape)
    Hkv, cap = int(keys.shape[1]), int(keys.shape[2])
    if not (queries.is_cuda and keys.is_cuda and values.is_cuda):
        raise RuntimeError("ragged_sdpa runs on the GPU only")
    for t in (queries, keys, values):
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise TypeError("queries/keys/values must be contiguous bfloat16")
    qs = _q_start_vector(q_start, queries.device)
    ql = None if q_lens is None else _q_start_vector(q_lens, queries.device)
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if out is None:
        shape = (B, L, Hq, D) if rows_layout else (B, Hq, L, D)
        out = torch.empty(shape, dtype=torch.bfloat16, device=queries.device)
    nb = _lib.query("mtp_attn_workspace_bytes", B, Hkv, cap, split_keys)
    ws = _lib.WORKSPACES.get(nb, "attn", queries.device)
    fn = "mtp_ragged_gqa_attn_rows" if rows_layout else "mtp_ragged_gqa_attn"
    _lib.call(fn, queries.data_ptr(), keys.data_ptr(), values.data_ptr(), qs.data_ptr(),
              None if ql is None else ql.data_ptr(), out.data_ptr(), B, Hq, Hkv, L, D, cap, scale, split_keys,
              ws.data_ptr(), ws.numel(), _lib.stream_handle(queries.device))
    return out
