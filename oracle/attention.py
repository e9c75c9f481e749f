"""Ragged-batch GQA verify attention, float64.

Mask rule (``mtplx/ragged_attention.py:42-85``): query ``i`` of row ``b`` sits
at absolute position ``q_start[b] + i`` and may attend key ``j`` iff
``j <= q_start[b] + i``; shape ``[B, 1, q_len, key_len]`` regardless of the
values. The consumer is MLX's SDPA (``mtplx/attention_split.py:347``) with GQA
head grouping ``q_head // (Hq / Hkv)`` and softmax in float.

Parity pins (tests/test_oracle_attention.py): mask semantics and shape
invariance (``tests/test_ragged_kv_cache.py:108-138``); a single-key row
returns that key's value exactly; uniform offsets equal plain causal attention
over the valid prefix; per-row independence (``tests/test_ragged_kv_cache.py:318-385``);
brute-force per-(b,h,i) loop on tiny inputs.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32


def _f64(a):
    a = np.asarray(a)
    return bf16_bits_to_f32(a).astype(np.float64) if a.dtype == np.uint16 else a.astype(np.float64)


def ragged_causal_mask(q_start, q_len: int, key_len: int) -> np.ndarray:
    """bool ``[B, 1, q_len, key_len]``, ``mask[b,0,i,j] = j <= q_start[b] + i``."""
    starts = np.asarray(q_start, dtype=np.int32).reshape(-1)
    qpos = starts[:, None] + np.arange(int(q_len), dtype=np.int32)[None, :]
    kpos = np.arange(int(key_len), dtype=np.int32)
    return kpos[None, None, None, :] <= qpos[:, None, :, None]


def ragged_additive_mask(q_start, q_len: int, key_len: int) -> np.ndarray:
    """float64 form: 0 where allowed, -inf elsewhere (``mtplx/ragged_attention.py:88-105``)."""
    return np.where(ragged_causal_mask(q_start, q_len, key_len), 0.0, -np.inf)


def ragged_gqa_attention(q, k, v, q_start, scale: float | None = None) -> np.ndarray:
    """``q`` [B, Hq, L, D]; ``k``/``v`` [B, Hkv, cap, D] (padded cache);
    ``q_start`` int32 [B]. Returns float64 [B, Hq, L, D]."""
    qf, kf, vf = _f64(q), _f64(k), _f64(v)
    B, Hq, L, D = qf.shape
    Hkv, cap = kf.shape[1], kf.shape[2]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    rep = Hq // Hkv
    scale = (1.0 / np.sqrt(D)) if scale is None else float(scale)
    mask = ragged_causal_mask(q_start, L, cap)  # [B,1,L,cap]
    out = np.zeros((B, Hq, L, D), dtype=np.float64)
    for b in range(B):
        for h in range(Hq):
            kv = h // rep
            s = (qf[b, h] @ kf[b, kv].T) * scale          # [L, cap]
            s = np.where(mask[b, 0], s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            p /= p.sum(axis=1, keepdims=True)
            out[b, h] = p @ vf[b, kv]
    return out


def ragged_gqa_attention_bruteforce(q, k, v, q_start, scale: float | None = None) -> np.ndarray:
    """Scalar-loop restatement used to pin :func:`ragged_gqa_attention`."""
    qf, kf, vf = _f64(q), _f64(k), _f64(v)
    B, Hq, L, D = qf.shape
    Hkv = kf.shape[1]
    rep = Hq // Hkv
    scale = (1.0 / np.sqrt(D)) if scale is None else float(scale)
    out = np.zeros((B, Hq, L, D))
    for b in range(B):
        for h in range(Hq):
            for i in range(L):
                last = int(q_start[b]) + i
                keys = range(0, min(last + 1, kf.shape[2]))
                logits = [sum(qf[b, h, i, d] * kf[b, h // rep, j, d] for d in range(D)) * scale for j in keys]
                mx = max(logits)
                w = [np.exp(t - mx) for t in logits]
                tot = sum(w)
                for d in range(D):
                    out[b, h, i, d] = sum(w[t] * vf[b, h // rep, j, d] for t, j in enumerate(keys)) / tot
    return out
