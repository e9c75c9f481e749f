"""The cross-row M-row qmv lane's call surface (``mtplx/verify_crossrow.py``):
``crossrow_enabled`` (:48), ``crossrow_eligible`` (:57), ``make_chunk_sums``
(:111) and ``crossrow_qmm`` (:249), with the reference's eligibility
(2 <= m <= 5, 4-bit, groups 32/64, K % 512 == 0, N % 8 == 0, bf16).

``make_chunk_sums`` fills the reference's table layout on the GPU
(``mtp_chunk_sums``: per 512-k block and lane, the 16-value slice sum of
each row, stride 8). ``crossrow_qmm`` checks a given table's size and then
runs the verify matmul, which forms its group sums while staging x: the
result is the same with or without the table, as in the reference, where
the table reproduces the kernel's own accumulation order.
"""

from __future__ import annotations

import os

import torch

from . import _lib
from .verify_kernels import quantized_matmul

_SUMS_STRIDE = 8
_BLOCK = 512


def crossrow_enabled() -> bool:
    return str(os.environ.get("MTPLX_VK_CROSSROW", "")).strip().lower() in {"1", "true", "on", "yes"}


def crossrow_eligible(m: int, k: int, n: int, bits: int, group_size: int, dtype) -> bool:
    return (2 <= int(m) <= 5 and int(bits) == 4 and int(group_size) in (32, 64) and int(k) % _BLOCK == 0
            and int(n) % 8 == 0 and dtype == torch.bfloat16)


def make_chunk_sums(x: torch.Tensor) -> torch.Tensor:
    """Per-lane activation slice sums for ``crossrow_qmm(..., xsums=...)``:
    fp32 ``[(K/512) * 32 * 8]``, entry ``(kb*32 + lane)*8 + m`` = the sum of
    row m's 16 values at ``kb*512 + lane*16``."""
    m, k = int(x.shape[-2]), int(x.shape[-1])
    if x.dtype != torch.bfloat16 or not x.is_cuda:
        raise TypeError("make_chunk_sums takes a bfloat16 GPU tensor")
    x2 = x.reshape(m, k).contiguous()
    out = torch.empty(((k // _BLOCK) * 32 * _SUMS_STRIDE,), dtype=torch.float32, device=x.device)
    _lib.call("mtp_chunk_sums", x2.data_ptr(), m, k, out.data_ptr(), _lib.stream_handle(x.device))
    return out


def crossrow_qmm(x: torch.Tensor, w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
                 group_size: int, xsums: torch.Tensor | None = None) -> torch.Tensor:
    """M-row affine-4 matmul ``[m, n]`` (bf16), optional chunk-sum table."""
    m, k = int(x.shape[-2]), int(x.shape[-1])
    if xsums is not None and int(xsums.numel()) != (k // _BLOCK) * 32 * _SUMS_STRIDE:
        raise ValueError(f"xsums has {int(xsums.numel())} entries, K={k} needs {(k // _BLOCK) * 32 * _SUMS_STRIDE}")
    return quantized_matmul(x.reshape(m, k), w_q, scales, biases, group_size=int(group_size), bits=4)
