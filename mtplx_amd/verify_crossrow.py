"""The cross-row M-row qmv lane's call surface (``mtplx/verify_crossrow.py``):
``crossrow_enabled`` (:48), ``crossrow_eligible`` (:57), ``make_chunk_sums``
(:111) and ``crossrow_qmm`` (:249), with the reference's eligibility
(2 <= m <= 5, 4-bit, groups 32/64, K % 512 == 0, N % 8 == 0, bf16).

``make_chunk_sums`` fills the reference's table layout on the GPU
(``mtp_chunk_sums``: per 512-k block and lane, the 16-value slice sum of
each row, stride 8). ``crossrow_qmm`` with a table runs ``mtp_crossrow_qmm``,
whose 32-k block finishes read their activation sums from the table (two
slices per block) instead of re-summing the staged x; without one it runs
the verify matmul, which forms the sums while staging x. Both meet the same
oracle bar; the two sum orders differ only in fp32 rounding.
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
    if xsums is None:
        return quantized_matmul(x.reshape(m, k), w_q, scales, biases, group_size=int(group_size), bits=4)
    if int(xsums.numel()) != (k // _BLOCK) * 32 * _SUMS_STRIDE:
        raise ValueError(f"xsums has {int(xsums.numel())} entries, K={k} needs {(k // _BLOCK) * 32 * _SUMS_STRIDE}")
    if xsums.dtype != torch.float32 or not xsums.is_cuda or m > _SUMS_STRIDE:
        raise ValueError("xsums must be the fp32 GPU table of make_chunk_sums (at most 8 rows)")
    if x.dtype != torch.bfloat16 or scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        raise TypeError("x, scales and biases must be bfloat16")
    n = int(w_q.shape[-2])
    if int(w_q.shape[-1]) * 8 != k:
        raise ValueError(f"x has K={k}, the 4-bit weight packs K={int(w_q.shape[-1]) * 8}")
    x2 = x.reshape(m, k).contiguous()
    xs = xsums.contiguous()
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _lib.call("mtp_crossrow_qmm", x2.data_ptr(), xs.data_ptr(), w_q.data_ptr(), scales.data_ptr(), biases.data_ptr(),
              y.data_ptr(), m, n, k, int(group_size), _lib.stream_handle(x.device))
    return y
