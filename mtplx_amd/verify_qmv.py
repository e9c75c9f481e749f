"""Verify-row quantized GEMV call surface (``mtplx/verify_qmv.py``) on gfx950.

Same function names, arguments and fallback convention as the reference:
an ineligible call returns ``module(x)`` — here the general gfx950 matmul of
:class:`~mtplx_amd.quant.QuantizedLinear` — and never raises on shape. The
reference's fixed-M probes (M=3 "multi3", M=4 pair) are generalised to any
M <= 32 rows, which is what the verify forward produces (M = B*(K+1)).
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib
from .quant import QuantizedLinear


def _affine4(module: Any) -> bool:
    return (isinstance(module, QuantizedLinear) and module.bits == 4 and module.group_size in (64, 128)
            and module.mode == "affine" and module.biases is not None)


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
    if left.group_size != right.group_size or left.weight.shape != right.weight.shape:
        return False
    return left.in_features % 512 == 0 and left.out_features == 48


def _rows(x: torch.Tensor, module: QuantizedLinear) -> tuple[torch.Tensor, tuple] | None:
    if x.dim() < 2 or x.dtype != torch.bfloat16 or not x.is_cuda:
        return None
    if module.scales.dtype != x.dtype or module.biases.dtype != x.dtype:
        return None
    k = int(x.shape[-1])
    if k != module.in_features:
        return None
    lead = x.shape[:-1]
    m = 1
    for d in lead:
        m *= int(d)
    if m > 32:
        return None
    return x.reshape(m, k).contiguous(), lead


def _add_bias(y: torch.Tensor, module: QuantizedLinear) -> torch.Tensor:
    return y + module.bias if module.bias is not None else y


def multi3_qmv4_matmul(x: torch.Tensor, module: QuantizedLinear) -> torch.Tensor:
    """``x @ module.weight.T`` on the verify kernel (``mtplx/verify_qmv.py:194``)."""
    if not is_multi3_qmv4_eligible(module):
        return module(x)
    r = _rows(x, module)
    if r is None:
        return module(x)
    x2, lead = r
    n = module.out_features
    y = torch.empty((x2.shape[0], n), dtype=x.dtype, device=x.device)
    _lib.call("mtp_qmv_affine4", x2.data_ptr(), module.weight.data_ptr(), module.scales.data_ptr(),
              module.biases.data_ptr(), y.data_ptr(), x2.shape[0], n, x2.shape[1], module.group_size, None, 0,
              _lib.stream_handle(x.device))
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
                           and gate_module.weight.shape == up_module.weight.shape
                           and gate_module.group_size == up_module.group_size)
    r = _rows(x, gate_module) if ok else None
    if r is None:
        return gate_module(x), up_module(x)
    x2, lead = r
    n = gate_module.out_features
    y0 = torch.empty((x2.shape[0], n), dtype=x.dtype, device=x.device)
    y1 = torch.empty_like(y0)
    _lib.call("mtp_qmv_affine4_dual", x2.data_ptr(), gate_module.weight.data_ptr(), gate_module.scales.data_ptr(),
              gate_module.biases.data_ptr(), up_module.weight.data_ptr(), up_module.scales.data_ptr(),
              up_module.biases.data_ptr(), y0.data_ptr(), y1.data_ptr(), x2.shape[0], n, x2.shape[1],
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
    if r is None or up.dtype != gate.dtype:
        return fallback()
    g2, lead = r
    u2 = up.reshape(g2.shape).contiguous()
    n = module.out_features
    y = torch.empty((g2.shape[0], n), dtype=gate.dtype, device=gate.device)
    _lib.call("mtp_qmv_affine4_swiglu_in", g2.data_ptr(), u2.data_ptr(), module.weight.data_ptr(),
              module.scales.data_ptr(), module.biases.data_ptr(), None, y.data_ptr(), g2.shape[0], n, g2.shape[1],
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
