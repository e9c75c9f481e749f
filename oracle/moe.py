"""Expert-sorted MoE dispatch, bit-exact indices and float64 arithmetic.

Restates ``mtplx/moe_sorted_gather.py``: ``sort_rows`` (:221-238 — ``order =
argsort(flat)``, ``inv_order = argsort(order)``, ``row_map = order // top_k``,
``sorted = flat[order]``), ``gather_qmm_rows`` (:241-285 — row ``i`` is token
``row_map[i]`` times expert ``sorted[i]``'s dequantised weights),
``swiglu_rows`` (:288-328 — ``silu(gate) * up`` of the fused ``[gate | up]``
output), and the caller's unsort + weighted combine
(``mtplx/models/qwen4_exp.py:1544-1577``).

The sort is stable (ties keep flat order). MLX's GPU argsort stability could
not be checked here (MLX is absent) — the final unsorted output does not
depend on the within-expert order.

Parity pins (tests/test_oracle_moe.py): per-expert loop oracle
(``tests/test_moe_sorted_gather.py:57-65``), the stable-argsort closed form
against a counting sort, ``inv_order`` inverts ``order``, SwiGLU closed form.
"""

from __future__ import annotations

import numpy as np

from .qmv import dequantize_affine4, _as_f64


def sort_rows(indices: np.ndarray):
    """Returns ``(row_map, sorted_ids, inv_order, order)`` for ``indices`` [T, top_k]."""
    indices = np.asarray(indices)
    top_k = indices.shape[-1]
    flat = indices.reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable")
    inv_order = np.argsort(order, kind="stable")
    row_map = (order // top_k).astype(np.uint32)
    return row_map, flat[order].astype(np.uint32), inv_order.astype(np.uint32), order.astype(np.uint32)


def expert_offsets(sorted_ids: np.ndarray, n_experts: int) -> np.ndarray:
    """int32 [E+1]: rows of expert e are ``sorted[off[e]:off[e+1]]``."""
    counts = np.bincount(np.asarray(sorted_ids, dtype=np.int64), minlength=n_experts)
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def gather_qmm_rows(x, row_map, sorted_ids, w, scales, biases, group_size: int) -> np.ndarray:
    """``y[i] = x[row_map[i]] @ deq(W[sorted_ids[i]]).T``; ``w`` is [E, N, K/8]."""
    xf = _as_f64(x).reshape(-1, np.asarray(w).shape[2] * 8)
    rows = len(row_map)
    n = np.asarray(w).shape[1]
    y = np.zeros((rows, n))
    cache: dict[int, np.ndarray] = {}
    for i in range(rows):
        e = int(sorted_ids[i])
        if e not in cache:
            cache[e] = dequantize_affine4(w[e], scales[e], biases[e], group_size)
        y[i] = xf[int(row_map[i])] @ cache[e].T
    return y


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def swiglu_rows(x, row_map, sorted_ids, w, scales, biases, group_size: int, bf16_storage: bool = False) -> np.ndarray:
    """``silu(gate) * up`` of the fused ``[gate | up]`` gathered product, [rows, N/2].

    ``bf16_storage`` rounds where the reference chain stores bf16 tensors
    (the gathered product, ``silu(gate)`` and the product itself,
    ``mtplx/moe_sorted_gather.py:322-328``)."""
    gu = gather_qmm_rows(x, row_map, sorted_ids, w, scales, biases, group_size)
    half = gu.shape[1] // 2
    if not bf16_storage:
        return silu(gu[:, :half]) * gu[:, half:]
    from .bf16 import round_to_bf16
    gu = round_to_bf16(gu)
    return round_to_bf16(round_to_bf16(silu(gu[:, :half])) * gu[:, half:])


def moe_forward(x, indices, route_weights, gate_up, down, group_size: int, bf16_storage: bool = False) -> np.ndarray:
    """Routed experts of one token block: sort -> SwiGLU rows -> down rows ->
    unsort -> score-weighted sum over top_k. ``gate_up``/``down`` are
    ``(w, scales, biases)`` triples with a leading expert axis.

    ``bf16_storage`` rounds where the reference's sorted chain stores bf16
    tensors: the gathered gate|up product, ``silu(gate)`` and the SwiGLU rows
    (``swiglu_rows``, ``mtplx/moe_sorted_gather.py:322-328``) and each
    expert's down-projection rows, which the block then weights and sums
    (``mtplx/models/qwen4_exp.py:1565-1577``, ``:1438-1441``)."""
    xf = _as_f64(x)
    T, top_k = np.asarray(indices).shape
    row_map, sorted_ids, inv_order, _ = sort_rows(indices)
    h = swiglu_rows(xf, row_map, sorted_ids, *gate_up, group_size, bf16_storage=bf16_storage)
    y_sorted = gather_qmm_rows(h, np.arange(len(row_map)), sorted_ids, *down, group_size)
    if bf16_storage:
        from .bf16 import round_to_bf16
        y_sorted = round_to_bf16(y_sorted)
    y = y_sorted[inv_order.astype(np.int64)].reshape(T, top_k, -1)
    return (y * np.asarray(route_weights, dtype=np.float64)[:, :, None]).sum(axis=1)


def moe_forward_loop(x, indices, route_weights, gate_up, down, group_size: int) -> np.ndarray:
    """Per-token, per-expert loop (no sorting) — the pin for :func:`moe_forward`."""
    xf = _as_f64(x)
    T, top_k = np.asarray(indices).shape
    out = np.zeros((T, np.asarray(down[0]).shape[1]))
    for t in range(T):
        for j in range(top_k):
            e = int(indices[t, j])
            wgu = dequantize_affine4(gate_up[0][e], gate_up[1][e], gate_up[2][e], group_size)
            gu = wgu @ xf[t]
            half = gu.shape[0] // 2
            h = silu(gu[:half]) * gu[half:]
            wd = dequantize_affine4(down[0][e], down[1][e], down[2][e], group_size)
            out[t] += float(route_weights[t, j]) * (wd @ h)
    return out
