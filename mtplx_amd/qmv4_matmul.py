"""The qmv4 core's call surface (``mtplx/kernels/qmv4_matmul.py:158-215``):
``qmv4_eligible(x, module)`` and ``qmv4_matmul(x, module)`` with the
reference's eligibility (bf16 x, 4-bit affine, groups 32/64/128, no bias,
M <= 6, K % 512 == 0) and its fall back to the stock quantized matmul on
other shapes, so callers can route unconditionally.

Eligible calls run ``mtp_qmv_affine4`` (groups 64/128) or ``mtp_qmv_affine``
(group 32) through :func:`mtplx_amd.verify_kernels.quantized_matmul`; the
fallback is ``module(x)``, the same kernels. There is no CPU path.
"""

from __future__ import annotations

from typing import Any

import torch

from .verify_kernels import quantized_matmul


def qmv4_eligible(x: torch.Tensor, module: Any) -> bool:
    """``module`` needs .weight/.scales/.biases/.group_size/.bits (a
    QuantizedLinear or any pack carrying the same attributes)."""
    if x.dtype != torch.bfloat16:
        return False
    if getattr(module, "bits", None) != 4:
        return False
    if getattr(module, "mode", "affine") not in (None, "affine"):
        return False
    gs = int(getattr(module, "group_size", 0) or 0)
    if gs not in (32, 64, 128):
        return False
    w = getattr(module, "weight", None)
    scales = getattr(module, "scales", None)
    if w is None or scales is None or getattr(module, "biases", None) is None:
        return False
    if w.dtype not in (torch.int32, torch.uint32) or scales.dtype != x.dtype:
        return False
    if getattr(module, "bias", None) is not None:
        return False
    m = int(x.shape[-2]) if x.dim() >= 2 else 1
    k = int(x.shape[-1])
    if m > 6 or k % 512 != 0:
        return False
    return int(w.shape[1]) * 8 == k


def qmv4_matmul(x: torch.Tensor, module: Any) -> torch.Tensor:
    """``x @ module.weight.T`` (transpose convention) via the qmv4 core; x is
    ``[..., M, K]`` with M <= 6. Ineligible shapes take the stock quantized
    matmul (``module(x)``)."""
    if not qmv4_eligible(x, module):
        return module(x)
    lead = x.shape[:-2]
    m, k = int(x.shape[-2]), int(x.shape[-1])
    y = quantized_matmul(x.reshape(m, k), module.weight, module.scales, module.biases,
                         group_size=int(module.group_size), bits=4)
    return y.reshape(*lead, m, int(module.weight.shape[0]))
