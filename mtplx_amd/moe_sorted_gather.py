"""Expert-sorted MoE gather (``mtplx/moe_sorted_gather.py``) on gfx950.

Keeps the reference's entry points and constants: ``gather_qmm`` with the
``mx.gather_qmm`` signature (:170), ``sort_rows`` (:221), ``gather_qmm_rows``
(:241), ``swiglu_rows`` (:288), ``switch_linear`` (:339), and the row-pad rule
(:66-113). The pad guard exists for an Apple MLX kernel's 16-bit row count; the
gfx950 kernels count rows in 32 bits, so ``guard_active()`` is False and
``pad_rows`` returns 0 — the rule's arithmetic is kept for callers that ask.

GPU work: ``mtp_moe_sort`` (stable counting sort + expert offsets + active
list) and ``mtp_gather_qmv_affine4`` (rows read in place through the row map,
one column of workgroups per active expert, optional fused SwiGLU).
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib

INT16_ROW_BOUND = 32767
ROW_ALIGN = 64
FIXED_MLX_RELEASE = (0, 32, 3)
_PRE_RELEASE = re.compile(r"^[.\-_]?(dev|a|b|c|rc|alpha|beta|pre|preview)\d*", re.I)
_STATS = {"padded_calls": 0, "padded_rows": 0}


def mlx_release_affected(version: str) -> bool:
    """``mtplx/moe_sorted_gather.py:80``: the MLX release test, kept verbatim in behaviour."""
    m = re.match(r"^\s*v?(\d+)\.(\d+)\.(\d+)(.*)$", str(version))
    if m is None:
        return True
    rel = tuple(int(p) for p in m.groups()[:3])
    if rel < FIXED_MLX_RELEASE:
        return True
    return rel == FIXED_MLX_RELEASE and bool(_PRE_RELEASE.match(m.group(4) or ""))


def guard_active() -> bool:
    return False


def pad_rows(rows: int) -> int:
    rows = int(rows)
    if rows <= INT16_ROW_BOUND or rows % ROW_ALIGN == 0 or not guard_active():
        return 0
    return ROW_ALIGN - rows % ROW_ALIGN


def stats() -> dict:
    return dict(_STATS)


@dataclass
class ExpertSort:
    """Device outputs of one expert sort."""

    row_map: torch.Tensor      # uint32-as-int32 [R]: token row of sorted row i
    sorted_ids: torch.Tensor   # [R] expert of sorted row i (ascending)
    inv_order: torch.Tensor    # [R] sorted position of flat row j
    expert_off: torch.Tensor   # int32 [E+1]
    active: torch.Tensor       # int32 [1+E]: count, then active experts
    top_k: int
    n_experts: int


def expert_sort(indices: torch.Tensor, n_experts: int) -> ExpertSort:
    """Stable counting sort of ``indices`` ``[..., top_k]`` on the GPU."""
    top_k = int(indices.shape[-1])
    flat = indices.reshape(-1, top_k).to(torch.int32).contiguous()
    T = flat.shape[0]
    R = T * top_k
    dev = indices.device
    row_map = torch.empty(R, dtype=torch.int32, device=dev)
    sorted_ids = torch.empty(R, dtype=torch.int32, device=dev)
    inv = torch.empty(R, dtype=torch.int32, device=dev)
    off = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    active = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    _lib.call("mtp_moe_sort", flat.data_ptr(), T, top_k, n_experts, row_map.data_ptr(), sorted_ids.data_ptr(),
              inv.data_ptr(), off.data_ptr(), active.data_ptr(), None, 0, _lib.stream_handle(dev))
    return ExpertSort(row_map, sorted_ids, inv, off, active, top_k, n_experts)


def sort_rows(x: torch.Tensor, indices: torch.Tensor, n_experts: int | None = None):
    """``(tokens [n,1,K], row_map, sorted_indices, inv_order)`` exactly as
    ``mtplx/moe_sorted_gather.py:221-238`` (stable sort of the flattened ids)."""
    E = int(n_experts) if n_experts is not None else int(indices.max().item()) + 1
    es = expert_sort(indices, E)
    tokens = x.reshape(-1, 1, x.shape[-1])
    return tokens, es.row_map, es.sorted_ids, es.inv_order


def _gather(x, x2, es: ExpertSort, rowmap, w, scales, biases, w1, s1, b1, n_out, xmode, emode, rows_per_expert,
            group_size, max_rows):
    R = int(es.row_map.numel())
    K = int(x.shape[-1])
    y = torch.empty((R, n_out), dtype=torch.bfloat16, device=x.device)
    ptr = _lib.ptr
    _lib.call("mtp_gather_qmv_affine4", x.data_ptr(), ptr(x2), ptr(rowmap), es.expert_off.data_ptr(),
              es.active.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(), ptr(w1), ptr(s1), ptr(b1),
              y.data_ptr(), max_rows, es.n_experts, n_out, K, group_size, xmode, emode, rows_per_expert, None, 0,
              _lib.stream_handle(x.device))
    return y


def gather_qmm_rows(tokens: torch.Tensor, es: ExpertSort, w: torch.Tensor, scales: torch.Tensor,
                    biases: torch.Tensor, *, group_size: int, bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """``gather_qmm(tokens[row_map], w, ..., sorted_indices=True)`` with rows read
    in place through the map (``mtplx/moe_sorted_gather.py:241``). ``w`` is
    ``[E, N, K/8]``; returns ``[R, 1, N]`` in sorted order."""
    if bits != 4 or mode != "affine":
        raise NotImplementedError("gfx950 gather path is 4-bit affine")
    x = tokens.reshape(-1, tokens.shape[-1]).contiguous()
    N = int(w.shape[-2])
    T = x.shape[0]
    y = _gather(x, None, es, es.row_map, w, scales, biases, None, None, None, N, 0, 0, N, group_size, T)
    return y.reshape(-1, 1, N)


def swiglu_rows(tokens: torch.Tensor, es: ExpertSort, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                *, group_size: int, bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """``silu(gate) * up`` of the fused ``[gate | up]`` sorted gather
    (``mtplx/moe_sorted_gather.py:288``); ``w`` is ``[E, 2F, K/8]``. Returns ``[R, 1, F]``."""
    if bits != 4 or mode != "affine":
        raise NotImplementedError("gfx950 gather path is 4-bit affine")
    x = tokens.reshape(-1, tokens.shape[-1]).contiguous()
    F = int(w.shape[-2]) // 2
    kw = int(w.shape[-1])
    gs_k = int(scales.shape[-1])
    w_up = w.reshape(-1, kw)[F:]            # up rows start F rows into expert 0; same per-expert stride
    s_up = scales.reshape(-1, gs_k)[F:]
    b_up = biases.reshape(-1, gs_k)[F:]
    y = _gather(x, None, es, es.row_map, w, scales, biases, w_up, s_up, b_up, F, 0, 3, 2 * F, group_size, x.shape[0])
    return y.reshape(-1, 1, F)


def switch_linear(module: Any, x: torch.Tensor, es: ExpertSort, *, sorted_indices: bool = True,
                  swiglu_up: torch.Tensor | None = None) -> torch.Tensor:
    """Expert linear over rows already in sorted order (``mtplx/moe_sorted_gather.py:339``):
    ``y[i] = x[i] @ W[e_i]^T``; with ``swiglu_up`` the input is ``silu(x) * up``."""
    if not sorted_indices:
        raise NotImplementedError("unsorted switch_linear: sort with expert_sort first")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    N = int(module.weight.shape[-2])
    up = None if swiglu_up is None else swiglu_up.reshape(x2.shape).contiguous()
    T = max(1, x2.shape[0] // max(es.top_k, 1))
    y = _gather(x2, up, es, None, module.weight, module.scales, module.biases, None, None, None, N,
                1 if up is not None else 0, 0, N, module.group_size, T)
    return y.reshape(*x.shape[:-1], N)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None = None,
               lhs_indices: torch.Tensor | None = None, rhs_indices: torch.Tensor | None = None,
               transpose: bool = True, group_size: int | None = None, bits: int | None = None,
               mode: str = "affine", *, sorted_indices: bool = False) -> torch.Tensor:
    """``y[i] = x[lhs_indices[i]] @ dequant(w[rhs_indices[i]]).T`` (the
    ``mx.gather_qmm`` contract, ``mtplx/moe_sorted_gather.py:170``), 2-D rows."""
    if not transpose or biases is None:
        raise NotImplementedError("gfx950 gather_qmm supports transpose=True affine weights")
    E = int(w.shape[0])
    rhs = rhs_indices.reshape(-1, 1).to(torch.int32)
    es = expert_sort(rhs, E)
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    lhs = torch.arange(rhs.shape[0], device=x.device, dtype=torch.int32) if lhs_indices is None \
        else lhs_indices.reshape(-1).to(torch.int32)
    rowmap = lhs[es.row_map.long()].contiguous()     # x row of sorted row i
    N = int(w.shape[-2])
    y_sorted = _gather(x2, None, es, rowmap, w, scales, biases, None, None, None, N, 0, 0, N,
                       int(group_size or 64), int(rhs.shape[0]))
    return y_sorted[es.inv_order.long()]


def moe_combine(y_sorted: torch.Tensor, es: ExpertSort, route_weights: torch.Tensor,
                shared: torch.Tensor | None = None) -> torch.Tensor:
    """Unsort + route-weighted sum over top_k (+ shared expert)
    (``mtplx/models/qwen4_exp.py:1544-1577``)."""
    H = int(y_sorted.shape[-1])
    R = int(es.inv_order.numel())
    T = R // es.top_k
    out = torch.empty((T, H), dtype=torch.bfloat16, device=y_sorted.device)
    w = route_weights.to(torch.float32).contiguous()
    _lib.call("mtp_moe_combine", y_sorted.contiguous().data_ptr(), es.inv_order.data_ptr(), w.data_ptr(),
              _lib.ptr(shared), out.data_ptr(), T, es.top_k, H, _lib.stream_handle(y_sorted.device))
    return out


def route(router_logits: torch.Tensor, top_k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k experts per token (value desc, id asc) and renormalised softmax weights."""
    T, E = (int(s) for s in router_logits.shape)
    lg = router_logits.to(torch.float32).contiguous()
    ids = torch.empty((T, top_k), dtype=torch.int32, device=lg.device)
    wts = torch.empty((T, top_k), dtype=torch.float32, device=lg.device)
    _lib.call("mtp_moe_route", lg.data_ptr(), T, E, top_k, ids.data_ptr(), wts.data_ptr(), _lib.stream_handle(lg.device))
    return ids, wts
