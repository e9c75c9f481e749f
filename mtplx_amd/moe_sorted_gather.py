"""Expert-sorted MoE gather (``mtplx/moe_sorted_gather.py``) on gfx950.

Keeps the reference's entry points and constants: ``gather_qmm`` with the
``mx.gather_qmm`` signature (:170), ``sort_rows`` (:221), ``gather_qmm_rows``
(:241), ``swiglu_rows`` (:288), ``switch_linear`` (:339), and the row-pad rule
(:66-113). The pad guard exists for an Apple MLX kernel's 16-bit row count; the
gfx950 kernels count rows in 32 bits, so ``guard_active()`` is False and
``pad_rows`` returns 0 — the rule's arithmetic is kept for callers that ask.

GPU work: ``mtp_moe_sort`` (stable counting sort + expert offsets + active
list) and ``mtp_gather_qmv_affine4`` (rows read in place through the row map,
one column of workgroups per active expert, optional fused SwiGLU); expert
stacks packed once (``QuantizedLinear.pack``) run
``mtp_gather_qmv_affine4_packed_rows`` (layout 1) or
``mtp_gather_qmv_affine4_packed_mf16`` (layout 2) instead.
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
    active: torch.Tensor       # int32 [1+E]: count, then active experts; count -1: invalid ids
    top_k: int
    n_experts: int

    def check(self) -> None:
        """Raise ``ValueError`` if the sort flagged its ids (an id outside
        ``[0, n_experts)``, or a descent where ascending ids were promised).
        Synchronises with the device; the sort itself never does."""
        if int(self.active[0].item()) < 0:
            raise ValueError(f"expert ids outside [0, {self.n_experts}) or not ascending")


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


_expert_sort = expert_sort   # for functions whose ``expert_sort`` keyword shadows the name


def segments(sorted_ids: torch.Tensor, n_experts: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(expert_off int32 [E+1], active int32 [1+E])`` from ids already in
    ascending order (``mtp_moe_segments``)."""
    ids = sorted_ids.reshape(-1).to(torch.int32).contiguous()
    dev = ids.device
    off = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    active = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    _lib.call("mtp_moe_segments", ids.data_ptr(), int(ids.numel()), int(n_experts), off.data_ptr(), active.data_ptr(),
              _lib.stream_handle(dev))
    return off, active


def _sorted_rows(rhs_indices: torch.Tensor, n_experts: int, top_k: int = 1) -> ExpertSort:
    """An :class:`ExpertSort` view of rows whose expert ids are already sorted
    (the ``sorted_indices=True`` contract). No host synchronisation: ids that
    do not ascend inside ``[0, n_experts)`` are flagged on the device
    (``ExpertSort.check``) and the gathered matmul then runs no expert, so its
    (zero-filled) output stays zero."""
    ids = rhs_indices.reshape(-1).to(torch.int32).contiguous()
    off, active = segments(ids, n_experts)
    R = int(ids.numel())
    ar = torch.arange(R, dtype=torch.int32, device=ids.device)
    return ExpertSort(ar, ids, ar, off, active, top_k, n_experts)


SORT_MAX_EXPERTS = 4096   # the single-workgroup counting sort's bound (mtp_moe_sort)


def sort_rows(x: torch.Tensor, indices: torch.Tensor, n_experts: int | None = None):
    """``(tokens [n,1,K], row_map, sorted_indices, inv_order)`` exactly as
    ``mtplx/moe_sorted_gather.py:221-238`` (stable sort of the flattened ids).
    Without ``n_experts`` the sort counts over ``SORT_MAX_EXPERTS`` bins, so
    the call never waits on the device; an id outside that range is flagged
    on the device and leaves the identity order."""
    E = int(n_experts) if n_experts is not None else SORT_MAX_EXPERTS
    es = expert_sort(indices, E)
    tokens = x.reshape(-1, 1, x.shape[-1])
    return tokens, es.row_map, es.sorted_ids, es.inv_order


def _stack_pack(module) -> tuple[torch.Tensor, str] | None:
    """An expert stack's tile-major pack and the packed-expert entry point
    that reads it: layout 1 (``QuantizedLinear.pack()``) or layout 2
    (``pack(layout=2)``, what the verify step keeps), or None."""
    if getattr(module, "packed", None) is not None:
        return module.packed, "mtp_gather_qmv_affine4_packed_rows"
    if getattr(module, "packed_mf16", None) is not None:
        return module.packed_mf16, "mtp_gather_qmv_affine4_packed_mf16"
    return None


def _gather_packed(x, es: ExpertSort, rowmap, module, n_out, group_size, max_rows):
    """The sorted rows through an expert stack's tile-major pack, on the
    verify step's packed-expert kernels (both row classes)."""
    pack, fn = _stack_pack(module)
    R = int(es.row_map.numel())
    K = int(x.shape[-1])
    y = torch.zeros((R, n_out), dtype=torch.bfloat16, device=x.device)   # flagged sort: zeros
    _lib.call(fn, x.data_ptr(), _lib.ptr(rowmap), es.expert_off.data_ptr(), es.active.data_ptr(), pack.data_ptr(),
              y.data_ptr(), max_rows, es.n_experts, n_out, K, group_size, 0, n_out, 0, _lib.stream_handle(x.device))
    return y


def _packable(module, N: int, K: int) -> bool:
    return (_stack_pack(module) is not None and N % 32 == 0 and K % 256 == 0
            and int(module.group_size) in (64, 128))


def _gather(x, x2, es: ExpertSort, rowmap, w, scales, biases, w1, s1, b1, n_out, xmode, emode, rows_per_expert,
            group_size, max_rows):
    R = int(es.row_map.numel())
    K = int(x.shape[-1])
    # zero-filled: rows of a flagged sort (no expert runs) read as zeros
    y = torch.zeros((R, n_out), dtype=torch.bfloat16, device=x.device)
    ptr = _lib.ptr
    _lib.call("mtp_gather_qmv_affine4", x.data_ptr(), ptr(x2), ptr(rowmap), es.expert_off.data_ptr(),
              es.active.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(), ptr(w1), ptr(s1), ptr(b1),
              y.data_ptr(), max_rows, es.n_experts, n_out, K, group_size, xmode, emode, rows_per_expert, None, 0,
              _lib.stream_handle(x.device))
    return y


def _check_quant(bits, mode):
    if int(bits) != 4 or mode != "affine":
        raise NotImplementedError(f"gfx950 gather path is 4-bit affine (got bits={bits}, mode={mode!r})")


def gather_qmm_rows(tokens: torch.Tensor, row_map: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                    biases: torch.Tensor, rhs_indices: torch.Tensor, *, group_size: int, bits: int,
                    mode: str = "affine", expert_sort: ExpertSort | None = None) -> torch.Tensor:
    """``gather_qmm(tokens[row_map], w, ..., rhs_indices, sorted_indices=True)``
    with each token row read in place through ``row_map``
    (``mtplx/moe_sorted_gather.py:241``). ``w`` is ``[E, N, K/8]``,
    ``rhs_indices`` ascending; returns ``[R, 1, N]`` in sorted order.
    ``expert_sort``: the :func:`expert_sort` that produced the rows, which
    saves the segment pass."""
    _check_quant(bits, mode)
    x = tokens.reshape(-1, tokens.shape[-1]).contiguous()
    E, N = int(w.shape[0]), int(w.shape[-2])
    es = expert_sort if expert_sort is not None else _sorted_rows(rhs_indices, E)
    rm = row_map.reshape(-1).to(torch.int32).contiguous()
    R = int(rm.numel())
    y = _gather(x, None, es, rm, w, scales, biases, None, None, None, N, 0, 0, N, int(group_size), R)
    return y.reshape(R, 1, N)


def swiglu_rows(tokens: torch.Tensor, row_map: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                biases: torch.Tensor, rhs_indices: torch.Tensor, *, group_size: int, bits: int,
                mode: str = "affine", expert_sort: ExpertSort | None = None) -> torch.Tensor:
    """``nn.silu(gate) * up`` of the fused ``[gate | up]`` sorted gather
    (``mtplx/moe_sorted_gather.py:288``); ``w`` is ``[E, 2F, K/8]``. One kernel:
    the gate and up halves of a column tile are computed together and only
    the product is stored. Returns ``[R, 1, F]``."""
    _check_quant(bits, mode)
    x = tokens.reshape(-1, tokens.shape[-1]).contiguous()
    E = int(w.shape[0])
    F = int(w.shape[-2]) // 2
    kw = int(w.shape[-1])
    gs_k = int(scales.shape[-1])
    es = expert_sort if expert_sort is not None else _sorted_rows(rhs_indices, E)
    rm = row_map.reshape(-1).to(torch.int32).contiguous()
    R = int(rm.numel())
    w_up = w.reshape(-1, kw)[F:]            # up rows start F rows into expert 0; same per-expert stride
    s_up = scales.reshape(-1, gs_k)[F:]
    b_up = biases.reshape(-1, gs_k)[F:]
    y = _gather(x, None, es, rm, w, scales, biases, w_up, s_up, b_up, F, 0, 3, 2 * F, int(group_size), R)
    return y.reshape(R, 1, F)


def switch_linear(module: Any, x: torch.Tensor, indices: torch.Tensor, *, sorted_indices: bool,
                  expert_sort: ExpertSort | None = None) -> torch.Tensor:
    """``module(x, indices, sorted_indices=...)`` for a quantized switch linear
    (``mtplx/moe_sorted_gather.py:339``): row ``i`` of ``x`` times expert
    ``indices[i]``'s weights; ``module`` exposes ``weight [E, N, K/8]``,
    ``scales``, ``biases``, ``group_size``, ``bits``, ``mode``. Unsorted indices
    are sorted on the GPU and the result returned in the caller's order."""
    _check_quant(getattr(module, "bits", 4), getattr(module, "mode", "affine"))
    shape = getattr(module, "_shape", None) or tuple(module.weight.shape)
    E, N = int(shape[0]), int(shape[-2])
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    K = int(x2.shape[-1])
    ids = indices.reshape(-1)
    if int(ids.numel()) != int(x2.shape[0]):
        raise ValueError(f"switch_linear: {x2.shape[0]} rows but {ids.numel()} expert indices")
    # An expert stack packed once (QuantizedLinear.pack()) streams its
    # tile-major copy, also after its MLX triple is released.
    packed = _packable(module, N, K) and x2.dtype == torch.bfloat16

    def run(es, rowmap):
        if packed:
            return _gather_packed(x2, es, rowmap, module, N, int(module.group_size), int(x2.shape[0]))
        return _gather(x2, None, es, rowmap, module.weight, module.scales, module.biases, None, None, None, N, 0, 0,
                       N, int(module.group_size), int(x2.shape[0]))

    if sorted_indices:
        es = expert_sort if expert_sort is not None else _sorted_rows(ids, E)
        return run(es, None).reshape(*lead, N)
    es = _expert_sort(ids.reshape(-1, 1), E)
    y = run(es, es.row_map)
    return y[es.inv_order.long()].reshape(*lead, N)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None = None,
               lhs_indices: torch.Tensor | None = None, rhs_indices: torch.Tensor | None = None,
               transpose: bool = True, group_size: int | None = None, bits: int | None = None,
               mode: str = "affine", *, sorted_indices: bool = False) -> torch.Tensor:
    """``y[b] = x[lhs[b]] @ dequant(w[rhs[b]]).T`` (the ``mx.gather_qmm``
    contract, ``mtplx/moe_sorted_gather.py:170``) for single-row operands:
    ``x`` is ``[..., 1, K]`` (or ``[n, K]`` rows); without ``lhs_indices`` the
    batch axes of ``x`` broadcast against ``rhs_indices`` (mlx-lm's SwitchGLU
    call, ``x [T,1,1,K]`` with ``indices [T,k]`` gives ``[T,k,1,N]``)."""
    if not transpose or biases is None:
        raise NotImplementedError("gfx950 gather_qmm supports transpose=True affine weights")
    _check_quant(4 if bits is None else bits, mode)
    E, N, K = int(w.shape[0]), int(w.shape[-2]), int(x.shape[-1])
    if rhs_indices is None:
        raise ValueError("gather_qmm needs rhs_indices")
    if x.dim() >= 2 and x.shape[-2] == 1:
        xb = x.reshape(*x.shape[:-2], K)          # batch of single rows
        out_tail = (1, N)
    else:
        xb = x.reshape(-1, K)
        out_tail = (N,)
    rows = xb.reshape(-1, K).contiguous()
    if lhs_indices is None:
        batch = torch.broadcast_shapes(tuple(xb.shape[:-1]), tuple(rhs_indices.shape))
        lhs = torch.arange(rows.shape[0], device=x.device, dtype=torch.int32).reshape(xb.shape[:-1])
        lhs = lhs.broadcast_to(batch).reshape(-1)
        rhs = rhs_indices.broadcast_to(batch).reshape(-1)
    else:
        batch = tuple(torch.broadcast_shapes(tuple(lhs_indices.shape), tuple(rhs_indices.shape)))
        lhs = lhs_indices.broadcast_to(batch).reshape(-1)
        rhs = rhs_indices.broadcast_to(batch).reshape(-1)
    lhs = lhs.to(torch.int32).contiguous()
    rhs = rhs.to(torch.int32).contiguous()
    R = int(rhs.numel())
    gs = int(group_size or 64)
    if sorted_indices:
        es = _sorted_rows(rhs, E)
        y = _gather(rows, None, es, lhs, w, scales, biases, None, None, None, N, 0, 0, N, gs, R)
    else:
        es = expert_sort(rhs.reshape(-1, 1), E)
        rowmap = lhs[es.row_map.long()].contiguous()     # x row of sorted row i
        y = _gather(rows, None, es, rowmap, w, scales, biases, None, None, None, N, 0, 0, N, gs, R)
        y = y[es.inv_order.long()]
    return y.reshape(*batch, *out_tail)


def moe_combine(y_sorted: torch.Tensor, inv_order, route_weights: torch.Tensor, shared: torch.Tensor | None = None,
                *, shared_gate: torch.Tensor | None = None, resid: torch.Tensor | None = None,
                out: torch.Tensor | None = None, ss_out: torch.Tensor | None = None) -> torch.Tensor:
    """The sparse block's tail (``mtplx/models/qwen4_exp.py:1438-1445``, the
    unsort of ``:1544-1577``): ``bf16(sum_j w[t,j] * y_sorted[inv_order[t*k+j]])``
    plus ``sigmoid(shared_gate[t]) * shared[t]`` (``shared_gate``: fp32 ``[T]``
    or a strided column), plus ``resid`` when given. ``inv_order`` is the
    tensor or an :class:`ExpertSort`. ``ss_out`` (fp32, ``H`` entries, T <= 32):
    each 32-column block's sums of squares of the output rows, ``[H/32][32]``."""
    if isinstance(inv_order, ExpertSort):
        inv, top_k = inv_order.inv_order, inv_order.top_k
    else:
        inv, top_k = inv_order, int(route_weights.shape[-1])
    H = int(y_sorted.shape[-1])
    R = int(inv.numel())
    T = R // top_k
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=y_sorted.device)
    w = route_weights.to(torch.float32).contiguous()
    gate_ld = 1
    if shared_gate is not None:
        gate_ld = int(shared_gate.stride(0)) if shared_gate.dim() > 0 else 1
    # Converted copies are bound to names so that each stays allocated until
    # the call has been queued (a freed temporary's block can be handed to the
    # next temporary in the same argument list).
    ys = y_sorted.contiguous()
    inv32 = inv.to(torch.int32).contiguous()
    if ss_out is not None:
        if ss_out.dtype != torch.float32 or ss_out.numel() < H or not ss_out.is_contiguous():
            raise ValueError(f"ss_out must be a contiguous fp32 tensor of at least {H} entries")
        _lib.call("mtp_moe_combine_ss", ys.data_ptr(), inv32.data_ptr(), w.data_ptr(), _lib.ptr(shared),
                  _lib.ptr(shared_gate), gate_ld, _lib.ptr(resid), out.data_ptr(), ss_out.data_ptr(), T, top_k, H,
                  _lib.stream_handle(y_sorted.device))
        return out
    _lib.call("mtp_moe_combine", ys.data_ptr(), inv32.data_ptr(), w.data_ptr(), _lib.ptr(shared),
              _lib.ptr(shared_gate), gate_ld, _lib.ptr(resid), out.data_ptr(), T, top_k, H,
              _lib.stream_handle(y_sorted.device))
    return out


def route(router_logits: torch.Tensor, top_k: int, skew: torch.Tensor | None = None,
          n_experts: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k experts per token of ``router_logits[:, :E]`` (+ ``skew``) in
    (value desc, id asc) order and the renormalised softmax weights."""
    T = int(router_logits.shape[0])
    E = int(n_experts) if n_experts is not None else int(router_logits.shape[1])
    lg = router_logits if router_logits.dtype == torch.float32 and router_logits.stride(1) == 1 else \
        router_logits.to(torch.float32).contiguous()
    ids = torch.empty((T, top_k), dtype=torch.int32, device=lg.device)
    wts = torch.empty((T, top_k), dtype=torch.float32, device=lg.device)
    sk = None if skew is None else skew.to(torch.float32).contiguous()
    _lib.call("mtp_moe_route", lg.data_ptr(), int(lg.stride(0)), _lib.ptr(sk), T, E, top_k, ids.data_ptr(),
              wts.data_ptr(), _lib.stream_handle(lg.device))
    return ids, wts


# ---------------------------------------------------------------------------
# The mlx-lm switch layers the reference patches (``mlx_lm.models.switch_layers``
# ``QuantizedSwitchLinear`` / ``SwitchGLU`` / ``SwiGLU``), restated on torch
# tensors with their call contracts, and the reference's idempotent patches
# of them (``mtplx/moe_sorted_gather.py:359-481``).

_GUARD_MARK = "_mtplx_switch_linear_guard"
_GLU_MARK = "_mtplx_switch_glu_rows"
# Routed rows from which the sorted chain runs on the row-map kernel (the
# caller regime's threshold, ``mtplx/models/qwen4_exp.py:1548``; the
# reference's Apple kernel needs 4096+, ``kernels/moe_sorted_gather_nax.py:86``).
SWITCH_GLU_MIN_ROWS = 64


def _silu(x: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.silu(x)


class SwiGLU:
    """``activation(x, gate) = silu(gate) * x`` (mlx-lm's SwiGLU)."""

    def __call__(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        return _silu(gate) * x


class QuantizedSwitchLinear:
    """Expert-stacked 4-bit affine projection: ``weight`` ``[E, N, K/8]``,
    ``scales`` / ``biases`` ``[E, N, K/gs]``. ``module(x, indices,
    sorted_indices=False)`` is ``gather_qmm(x, w, s, b, rhs_indices=indices,
    transpose=True)`` (+ the expert's bias row), mlx-lm's contract."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = 64,
                 bits: int = 4, mode: str = "affine", bias: torch.Tensor | None = None):
        self.weight = weight.view(torch.int32) if weight.dtype == torch.uint32 else weight
        self.scales = scales
        self.biases = biases
        self.group_size = int(group_size)
        self.bits = int(bits)
        self.mode = mode
        self.bias = bias
        self.packed = None
        self._shape = tuple(int(d) for d in self.weight.shape)
        self.training = False

    def __contains__(self, name: str) -> bool:
        return getattr(self, name, None) is not None

    def __call__(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        y = gather_qmm(x, self.weight, self.scales, self.biases, rhs_indices=indices, transpose=True,
                       group_size=self.group_size, bits=self.bits, mode=self.mode, sorted_indices=sorted_indices)
        if self.bias is not None:
            y = y + self.bias[indices.long()].unsqueeze(-2)
        return y


class SwitchGLU:
    """mlx-lm's ``SwitchGLU``: ``down(activation(up(x), gate(x)))`` per routed
    expert; from 64 routed rows the rows are expert-sorted first and the
    result unsorted (``_gather_sort`` / ``_scatter_unsort``)."""

    def __init__(self, gate_proj: QuantizedSwitchLinear, up_proj: QuantizedSwitchLinear,
                 down_proj: QuantizedSwitchLinear, activation=None):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj
        self.activation = activation if activation is not None else SwiGLU()
        self.training = False

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        x = x.unsqueeze(-2).unsqueeze(-2)                     # [..., 1, 1, D]
        do_sort = int(indices.numel()) >= 64
        idx, inv = indices, None
        if do_sort:
            top_k = int(indices.shape[-1])
            flat = indices.reshape(-1)
            es = expert_sort(flat.reshape(-1, 1), int(self.gate_proj._shape[0]))
            rows = x.reshape(-1, 1, int(x.shape[-1]))
            # sorting [R, 1] ids: row_map is the flat position, whose token row is position // top_k
            x = rows[es.row_map.long() // top_k]
            idx, inv = es.sorted_ids, es.inv_order
        x_up = self.up_proj(x, idx, sorted_indices=do_sort)
        x_gate = self.gate_proj(x, idx, sorted_indices=do_sort)
        y = self.down_proj(self.activation(x_up, x_gate), idx, sorted_indices=do_sort)
        if do_sort:
            y = y[inv.long()].reshape(*indices.shape, *y.shape[-2:])
        return y.squeeze(-2)


def install_switch_linear_guard(cls=None) -> bool:
    """The reference's row-pad guard around the quantized switch linear's
    ``__call__`` (``mtplx/moe_sorted_gather.py:359-397``). It is a no-op
    wherever :func:`guard_active` is false, which is everywhere here (the
    gfx950 gathers count rows in 32 bits), so nothing is installed and False
    is returned, as the reference does off its affected MLX releases. Where
    the guard were active it wraps ``cls.__call__`` once (marker attribute)."""
    if not guard_active():
        return False
    cls = QuantizedSwitchLinear if cls is None else cls
    current = cls.__call__
    if getattr(current, _GUARD_MARK, False):
        return True

    def guarded_call(self, x, indices, sorted_indices=False):
        if sorted_indices:
            pad = pad_rows(int(indices.shape[0]))
            if pad:
                rows = int(indices.shape[0])
                xp = torch.cat([x, x[-1:].expand(pad, *x.shape[1:])], 0)
                ip = torch.cat([indices, indices[-1:].expand(pad)], 0)
                _STATS["padded_calls"] += 1
                _STATS["padded_rows"] += pad
                return current(self, xp, ip, sorted_indices=True)[:rows]
        return current(self, x, indices, sorted_indices=sorted_indices)

    setattr(guarded_call, _GUARD_MARK, True)
    cls.__call__ = guarded_call
    return True


def _glu_projections(module: Any):
    """The gate and up projections of a quantized ``SwitchGLU`` with the
    SwiGLU activation and no bias (same group size and bits), else None."""
    if type(getattr(module, "activation", None)) is not SwiGLU:
        return None
    gate, up = getattr(module, "gate_proj", None), getattr(module, "up_proj", None)
    for proj in (gate, up):
        if not isinstance(proj, QuantizedSwitchLinear) or proj.bias is not None or proj.mode != "affine" or \
                proj.weight is None:
            return None
    if gate.group_size != up.group_size or gate.bits != up.bits or gate.bits != 4 or gate._shape != up._shape:
        return None
    return gate, up


def switch_glu_rows(module: Any, x: torch.Tensor, indices: torch.Tensor, original) -> torch.Tensor:
    """``SwitchGLU.__call__`` with its sorted regime on the row-map kernel
    (``mtplx/moe_sorted_gather.py:420``): the rows are sorted as the stock
    call sorts them, the gate and up gathers and ``silu(gate) * up`` run as
    one kernel reading each token row in place through the sort's row map
    (``mtp_gather_qmv_affine4`` emode 3 over the separate gate and up
    stacks), then the down projection with sorted indices and the unsort.
    Training, fewer than ``SWITCH_GLU_MIN_ROWS`` routed rows, another
    activation or layout run ``original``."""
    if getattr(module, "training", False) or int(indices.numel()) < SWITCH_GLU_MIN_ROWS:
        return original(module, x, indices)
    projections = _glu_projections(module)
    if projections is None or x.dtype != torch.bfloat16 or not x.is_cuda:
        return original(module, x, indices)
    gate, up = projections
    E, F = int(gate._shape[0]), int(gate._shape[1])
    K = int(x.shape[-1])
    if K % 256 or int(gate.group_size) not in (64, 128):
        return original(module, x, indices)
    top_k = int(indices.shape[-1])
    es = expert_sort(indices.reshape(-1, top_k), E)
    rows = x.reshape(-1, K).contiguous()
    R = int(es.row_map.numel())
    h = _gather(rows, None, es, es.row_map, gate.weight, gate.scales, gate.biases, up.weight, up.scales, up.biases,
                F, 0, 3, F, int(gate.group_size), R)
    y = module.down_proj(h.reshape(R, 1, F), es.sorted_ids, sorted_indices=True)
    y = y[es.inv_order.long()]
    return y.reshape(*indices.shape, *y.shape[-2:]).squeeze(-2)


def install_switch_glu_rows(cls=None) -> bool:
    """Route ``SwitchGLU.__call__`` through :func:`switch_glu_rows`
    (``mtplx/moe_sorted_gather.py:458-481``): wraps the class's current call
    once (marker attribute ``_mtplx_switch_glu_rows``), so a second install
    is a no-op. Returns whether it is installed."""
    from . import _lib

    _lib.load()   # the row-map kernel lives in the HIP library; raises when it is missing
    cls = SwitchGLU if cls is None else cls
    current = cls.__call__
    if getattr(current, _GLU_MARK, False):
        return True

    def rows_call(self, x, indices):
        return switch_glu_rows(self, x, indices, current)

    setattr(rows_call, _GLU_MARK, True)
    rows_call.__wrapped__ = current
    cls.__call__ = rows_call
    return True
