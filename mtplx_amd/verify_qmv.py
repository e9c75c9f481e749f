"""Verify-row quantized GEMV call surface (``mtplx/verify_qmv.py``) on gfx950.

Same function names, arguments and fallback convention as the reference:
an ineligible call returns ``module(x)`` — here the general gfx950 matmul of
:class:`~mtplx_amd.quant.QuantizedLinear` — and never raises on shape. The
reference's fixed-M probes (M=3 "multi3", M=4 pair) are generalised to every
verify-row count M = sum_b (K_b + 1): up to 32 rows on the streaming kernel,
more on the 9..64-row MFMA kernel over the module's layout-1 pack (packed on
first use and kept on the module; 64-row launches past 64 rows).
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib
from .quant import QuantizedLinear
from .verify_kernels import STREAM_ROWS, _pack_cache_enabled, fast_path, quantized_matmul, rows_matmul


def _affine4(module: Any) -> bool:
    return (isinstance(module, QuantizedLinear) and module.bits == 4 and module.group_size in (64, 128)
            and module.mode == "affine"
            and (module.biases is not None or module.packed is not None or module.packed_mf16 is not None))


def _packed(module: QuantizedLinear, m: int) -> tuple[torch.Tensor, int] | None:
    """The module's tile-major pack for ``m`` rows: layout 2 (the 16x16x32
    MFMA form) at up to 16 rows, else layout 1, or None. A pack reads the
    weights as 1 KB contiguous runs per wave load (cfg1 shape: 15.7 us
    against 25.5 us on the MLX layout, whose per-lane row reads scatter), so
    a module that still holds its MLX triple is packed for the layout on its
    first call and keeps it (unless ``MTPLX_AMD_PACK_CACHE=0``); a released
    module serves the layout it has."""
    if m <= 16 and module.packed_mf16 is not None:
        return module.packed_mf16, 2
    can_pack = module.weight is not None and fast_path(module.bits, module.group_size, module.in_features) and \
        _pack_cache_enabled()
    if m <= 16 and can_pack:
        return module.pack(layout=2), 2
    if module.packed is not None:
        return module.packed, 1
    if can_pack:
        return module.pack(), 1
    return None


def _qmv_packed(stream, m: int, n: int, k: int, **kw) -> None:
    """mtp_qmv_affine4_ex on packed weights with this stream's split-K workspace."""
    dev = kw["x"].device
    ws = _lib.WORKSPACES.get(max(256, _lib.query("mtp_qmv_workspace_bytes", m, n, k, 1)), "verify_qmv", dev)
    _lib.qmv_ex(stream, M=m, N=n, K=k, ws=ws, ws_bytes=ws.numel(), **kw)


def is_multi3_qmv4_eligible(module: Any) -> bool:
    """``mtplx/verify_qmv.py:19``: 4-bit affine, K % 512 == 0, N % 8 == 0 (group 64/128 here)."""
    if not _affine4(module):
        return False
    k = module.in_features
    n = module.out_features
    return k % 512 == 0 and n % 8 == 0


def is_smalln_pair_qmv4_eligible(left: Any, right: Any) -> bool:
    """``mtplx/verify_qmv.py:36``: two equal-shape tiny-N (48) affine int4 linears."""
    if not (_affine4(left) and _affine4(right)):
        return False
    if left.group_size != right.group_size or left._shape != right._shape:
        return False
    return left.in_features % 512 == 0 and left.out_features == 48


def _rows(x: torch.Tensor, module: QuantizedLinear) -> tuple[torch.Tensor, tuple] | None:
    if x.dim() < 2 or x.dtype != torch.bfloat16 or not x.is_cuda:
        return None
    if module.scales is not None and (module.scales.dtype != x.dtype or module.biases.dtype != x.dtype):
        return None
    k = int(x.shape[-1])
    if k != module.in_features:
        return None
    lead = x.shape[:-1]
    m = 1
    for d in lead:
        m *= int(d)
    if m < 1:
        return None
    return x.reshape(m, k).contiguous(), lead


def _add_bias(y: torch.Tensor, module: QuantizedLinear) -> torch.Tensor:
    return y + module.bias if module.bias is not None else y


def packed_matmul(x: torch.Tensor, module: QuantizedLinear, *, exact: bool = False) -> torch.Tensor | None:
    """``x @ module.weight.T`` on the module's cached pack (bf16 rows on the
    GPU), or None when there is no suitable pack or x does not qualify. Up to
    32 rows stream the pack on ``mtp_qmv_affine4_ex``; more rows (or
    ``exact``: every M, the row-invariant greedy lane) run
    ``mtp_qmm_affine4_mfma`` on the layout-1 pack. A module with an MLX
    triple but no layout-1 pack gets one here when the MFMA kernel needs it.
    Never falls back to ``module(x)``, so a patched ``__call__`` may use it."""
    if len(module._shape) != 2:   # expert stacks go through switch_linear
        return None
    r = _rows(x, module)
    if r is None:
        return None
    x2, lead = r
    m, k = (int(d) for d in x2.shape)
    n = module.out_features
    if m > STREAM_ROWS or exact:
        if module.packed is None:
            if module.weight is None or not fast_path(module.bits, module.group_size, k):
                return None
            module.pack()
        y = rows_matmul(x2, module.packed, n, module.group_size)
        return _add_bias(y, module).reshape(*lead, n)
    pk = _packed(module, m)
    if pk is None:
        return None
    y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    _qmv_packed(_lib.stream_handle(x.device), m, n, k, x=x2, w0=pk[0], y0=y, group_size=module.group_size,
                xmode=0, emode=0, packed=pk[1])
    return _add_bias(y, module).reshape(*lead, n)


def multi3_qmv4_matmul(x: torch.Tensor, module: QuantizedLinear) -> torch.Tensor:
    """``x @ module.weight.T`` on the verify kernel (``mtplx/verify_qmv.py:194``)."""
    if not is_multi3_qmv4_eligible(module):
        return module(x)
    y = packed_matmul(x, module)
    if y is not None:
        return y
    r = _rows(x, module)
    if r is None or module.weight is None:
        return module(x)
    x2, lead = r
    n = module.out_features
    y = quantized_matmul(x2, module.weight, module.scales, module.biases, group_size=module.group_size, bits=4)
    return _add_bias(y, module).reshape(*lead, n)


stocklike_qmv4_matmul = multi3_qmv4_matmul  # ``mtplx/verify_qmv.py:1217``: same contract, any M


def smalln_pair_qmv4_matmul(x: torch.Tensor, left_module: QuantizedLinear,
                            right_module: QuantizedLinear) -> tuple[torch.Tensor, torch.Tensor]:
    """Pair of tiny-N projections sharing one read of ``x`` (``mtplx/verify_qmv.py:377``)."""
    if not is_smalln_pair_qmv4_eligible(left_module, right_module):
        return left_module(x), right_module(x)
    return multi3_dual_qmv4_matmul(x, left_module, right_module, _pair_checked=True)


def multi3_dual_qmv4_matmul(x: torch.Tensor, gate_module: QuantizedLinear, up_module: QuantizedLinear,
                            _pair_checked: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Gate/up projections in one launch (``mtplx/verify_qmv.py:614``)."""
    ok = _pair_checked or (is_multi3_qmv4_eligible(gate_module) and is_multi3_qmv4_eligible(up_module)
                           and gate_module._shape == up_module._shape
                           and gate_module.group_size == up_module.group_size)
    r = _rows(x, gate_module) if ok else None
    if r is None or int(r[0].shape[0]) > STREAM_ROWS:
        # past 32 rows: one MFMA launch per projection (no two-output form there)
        return gate_module(x), up_module(x)
    x2, lead = r
    n = gate_module.out_features
    m, k = (int(d) for d in x2.shape)
    y0 = torch.empty((m, n), dtype=x.dtype, device=x.device)
    y1 = torch.empty_like(y0)
    pg, pu = _packed(gate_module, m), _packed(up_module, m)
    if pg is not None and pu is not None and pg[1] == pu[1]:
        _qmv_packed(_lib.stream_handle(x.device), m, n, k, x=x2, w0=pg[0], w1=pu[0], y0=y0, y1=y1,
                    group_size=gate_module.group_size, xmode=0, emode=2, packed=pg[1])
    elif gate_module.weight is None or up_module.weight is None:
        return gate_module(x), up_module(x)
    else:
        _lib.call("mtp_qmv_affine4_dual", x2.data_ptr(), gate_module.weight.data_ptr(),
                  gate_module.scales.data_ptr(), gate_module.biases.data_ptr(), up_module.weight.data_ptr(),
                  up_module.scales.data_ptr(), up_module.biases.data_ptr(), y0.data_ptr(), y1.data_ptr(), m, n, k,
                  gate_module.group_size, 0, None, 0, _lib.stream_handle(x.device))
    return _add_bias(y0, gate_module).reshape(*lead, n), _add_bias(y1, up_module).reshape(*lead, n)


multi3_parallel_dual_qmv4_matmul = multi3_dual_qmv4_matmul  # ``mtplx/verify_qmv.py:833``


def multi3_swiglu_down_qmv4_matmul(gate: torch.Tensor, up: torch.Tensor, module: QuantizedLinear) -> torch.Tensor:
    """``module(silu(gate) * up)`` with the activation fused into the matmul's
    input staging (``mtplx/verify_qmv.py:1063``)."""
    def fallback():
        return module(torch.nn.functional.silu(gate) * up)

    if gate.shape != up.shape or not is_multi3_qmv4_eligible(module):
        return fallback()
    r = _rows(gate, module)
    if r is None or up.dtype != gate.dtype or int(r[0].shape[0]) > STREAM_ROWS:
        return fallback()
    g2, lead = r
    u2 = up.reshape(g2.shape).contiguous()
    n = module.out_features
    m, k = (int(d) for d in g2.shape)
    y = torch.empty((m, n), dtype=gate.dtype, device=gate.device)
    pk = _packed(module, m)
    if pk is not None:
        _qmv_packed(_lib.stream_handle(gate.device), m, n, k, x=g2, x2=u2, w0=pk[0], y0=y,
                    group_size=module.group_size, xmode=1, emode=0, packed=pk[1])
    elif module.weight is None:
        return fallback()
    else:
        _lib.call("mtp_qmv_affine4_swiglu_in", g2.data_ptr(), u2.data_ptr(), module.weight.data_ptr(),
                  module.scales.data_ptr(), module.biases.data_ptr(), None, y.data_ptr(), m, n, k,
                  module.group_size, None, 0, _lib.stream_handle(gate.device))
    return _add_bias(y, module).reshape(*lead, n)


def is_stocklike_qmv8_eligible(module: Any) -> bool:
    """``mtplx/verify_qmv.py:1256``: an 8-bit affine QuantizedLinear with
    biases, group 32/64/128, K % 256 == 0 and N % 8 == 0."""
    if not isinstance(module, QuantizedLinear):
        return False
    if module.bits != 8 or module.group_size not in (32, 64, 128) or module.mode != "affine":
        return False
    if module.biases is None or module.weight.dim() != 2:
        return False
    k = int(module.weight.shape[1]) * 4
    n = int(module.weight.shape[0])
    return k % 256 == 0 and n % 8 == 0


def stocklike_qmv8_matmul(x: torch.Tensor, module: Any) -> torch.Tensor:
    """``mtplx/verify_qmv.py:1377``: 8-bit verify rows on ``mtp_qmv_affine``
    (one batch of rows, bf16 x/scales/biases); anything else -> ``module(x)``
    as in the reference."""
    if not is_stocklike_qmv8_eligible(module):
        return module(x)
    if x.dim() < 2 or x.dtype != torch.bfloat16 or module.scales.dtype != x.dtype or \
            module.biases.dtype != x.dtype:
        return module(x)
    k = int(x.shape[-1])
    if k != int(module.weight.shape[1]) * 4:
        return module(x)
    lead = x.shape[:-2]
    count = 1
    for d in lead:
        count *= int(d)
    if count != 1:
        return module(x)
    m, n = int(x.shape[-2]), module.out_features
    x2 = x.reshape(m, k).contiguous()
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _lib.call("mtp_qmv_affine", x2.data_ptr(), module.weight.data_ptr(), module.scales.data_ptr(),
              module.biases.data_ptr(), y.data_ptr(), None, m, n, k, module.group_size, 8,
              _lib.stream_handle(x.device))
    return _add_bias(y, module).reshape(*lead, m, n)
