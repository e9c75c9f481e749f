"""Verify-shape quantized matmul dispatch onto the gfx950 kernels.

Replaces the reference's verify qmm family (``mtplx/verify_kernels.py``:
``vk_eligible_ksplit`` :567, ``_run_ksplit`` :531, ``vk_qmm_m4_impl`` :580) and
is what a :class:`~mtplx_amd.quant.QuantizedLinear` call runs
(the ``mx.quantized_matmul(x, w, s, b, transpose=True)`` contract).

Kernels: ``mtp_qmv_affine4`` for 4-bit groups of 64/128 with K % 256 == 0 —
MFMA 32x32x16 bf16 with exact nibble operands, fp32 accumulation, one
workgroup per 32 output columns (``csrc/qmv.hip``; rows beyond 32 in 32-row
launches) — and ``mtp_qmv_affine`` for the other MLX affine packs (4- or
8-bit, groups 32/64/128, K % 32 == 0; ``csrc/qmv_generic.hip``). There is no
CPU path.
"""

from __future__ import annotations

import torch

from . import _lib

MAX_ROWS = 32


def _check(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int,
           bits: int, mode: str) -> tuple[int, int]:
    if mode != "affine" or bits not in (4, 8):
        raise NotImplementedError(f"only 4- and 8-bit affine are on the gfx950 path (got {bits}-bit {mode})")
    if group_size not in (32, 64, 128):
        raise NotImplementedError(f"group_size {group_size} not on the gfx950 path (32, 64, 128)")
    if not x.is_cuda:
        raise RuntimeError("verify matmul needs a GPU tensor; there is no CPU path")
    if x.dtype != torch.bfloat16 or scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        raise TypeError("x, scales and biases must be bfloat16")
    n, kw = int(w.shape[-2]), int(w.shape[-1])
    k = kw * 32 // bits
    if int(x.shape[-1]) != k:
        raise ValueError(f"x has K={int(x.shape[-1])}, weight packs K={k}")
    if k % 32 or k % group_size:
        raise NotImplementedError(f"K={k} must be a multiple of 32 and of the group size on the gfx950 path")
    return n, k


def fast_path(bits: int, group_size: int, k: int) -> bool:
    """Whether the MFMA streaming kernel takes this pack (else the general one)."""
    return int(bits) == 4 and int(group_size) in (64, 128) and int(k) % 256 == 0


def vk_eligible_ksplit(m: int, K: int, N: int, bits: int, group_size: int, dtype) -> bool:
    """Eligibility of the verify kernel (``mtplx/verify_kernels.py:567``), for this build's kernel."""
    return int(bits) == 4 and int(group_size) in (64, 128) and dtype == torch.bfloat16 and 1 <= int(m) \
        and int(K) % 256 == 0 and int(N) >= 1


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
                     group_size: int = 64, bits: int = 4, mode: str = "affine",
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ dequantize(w, scales, biases).T`` for ``x`` of shape ``[..., K]``."""
    n, k = _check(x, w, scales, biases, group_size, bits, mode)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k).contiguous()
    m = x2.shape[0]
    y = out if out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    st = _lib.stream_handle(x.device)
    if not fast_path(bits, group_size, k):
        _lib.call("mtp_qmv_affine", x2.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(), y.data_ptr(),
                  None, m, n, k, group_size, bits, st)
        return y.reshape(*lead, n)
    for r0 in range(0, m, MAX_ROWS):
        r = min(MAX_ROWS, m - r0)
        _lib.call("mtp_qmv_affine4", x2[r0:].data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                  y[r0:].data_ptr(), r, n, k, group_size, None, 0, st)
    return y.reshape(*lead, n)


def vk_qmm_m4_impl(impl: str, x2: torch.Tensor, w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
                   bits: int = 4, group_size: int = 64) -> torch.Tensor:
    """Named-implementation entry (``mtplx/verify_kernels.py:580``). Every name
    maps to the one gfx950 kernel; the names are kept for callers that pass them."""
    if impl not in ("vk", "vk_u2", "vk_k", "vk_hybrid", "oct", "twin"):
        raise ValueError(f"unknown verify implementation {impl!r}")
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)
