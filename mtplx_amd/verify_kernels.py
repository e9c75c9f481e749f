"""Verify-shape quantized matmul dispatch onto the gfx950 kernels.

Replaces the reference's verify qmm family (``mtplx/verify_kernels.py``:
the fixed-M entry points ``vk_eligible_m4`` / ``vk_eligible_m6`` :222-228,
``vk_qmm_m4`` / ``vk_qmm_m6`` :253-260 and their split-K forms
``vk_qmm_m4_ksplit`` / ``vk_qmm_m6_ksplit`` :263-270, ``vk_eligible_ksplit``
:567, ``_run_ksplit`` :531, ``vk_qmm_m4_impl`` :580) and is what a
:class:`~mtplx_amd.quant.QuantizedLinear` call runs (the
``mx.quantized_matmul(x, w, s, b, transpose=True)`` contract).

Kernels, by rows M (4-bit groups of 64/128 with K % 256 == 0):

* M <= 32: ``mtp_qmv_affine4_ex`` (the streaming kernel: 1 KB contiguous
  weight loads per wave, the leftover tiles split by K over all CUs) on a
  tile-major pack of the triple, layout 2 (the 16x16x32 MFMA form) up to 16
  rows and layout 1 beyond, packed once and kept like the M > 32 pack
  (cfg1 shape: 15.7 against 25.5 us for ``mtp_qmv_affine4`` on the MLX
  layout, which runs when ``MTPLX_AMD_PACK_CACHE=0``);
* M > 32: ``mtp_qmm_affine4_mfma`` (each weight quad read once for 64 rows)
  on the layout-1 tile-major pack, in 64-row launches. A raw MLX triple is
  packed once and the pack kept, keyed by the weight tensor (a verify
  forward calls every projection again each step); ``MTPLX_AMD_PACK_CACHE=0``
  packs into a temporary instead.

Other MLX affine packs (4- or 8-bit, groups 32/64/128, K % 32 == 0) take
``mtp_qmv_affine`` (``csrc/qmv_generic.hip``). There is no CPU path.

The fixed-M names keep the reference's signatures and eligibility ranges
(4 rows; 5..6 rows), widened to the formats these kernels take; every
``_ksplit`` / implementation name runs the same kernels, which choose their
own K split.
"""

from __future__ import annotations

import os
import weakref

import torch

from . import _lib

STREAM_ROWS = 32     # the streaming kernel's row bound
MFMA_ROWS = 64       # the 9..64-row MFMA kernel's row bound


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
    """Whether the MFMA kernels take this pack (else the general one)."""
    return int(bits) == 4 and int(group_size) in (64, 128) and int(k) % 256 == 0


def vk_eligible_ksplit(m: int, K: int, N: int, bits: int, group_size: int, dtype) -> bool:
    """Eligibility of the verify kernels (``mtplx/verify_kernels.py:567``) for
    this build's kernels: 4-bit affine groups 64/128, K % 256 == 0, bf16, any
    M >= 1 (the reference's split-K form takes 4..6 rows; these kernels take
    every verify-row count)."""
    return int(bits) == 4 and int(group_size) in (64, 128) and dtype == torch.bfloat16 and 1 <= int(m) \
        and int(K) % 256 == 0 and int(N) >= 1


def _formats_ok(K: int, bits: int, group_size: int, dtype) -> bool:
    return int(bits) in (4, 8) and int(group_size) in (32, 64, 128) and dtype == torch.bfloat16 and \
        int(K) % 32 == 0 and int(K) % int(group_size) == 0


def vk_eligible_m4(m: int, K: int, N: int, bits: int, group_size: int, dtype) -> bool:
    """``mtplx/verify_kernels.py:222``: exactly 4 rows, a format these kernels take."""
    return int(m) == 4 and int(N) >= 1 and _formats_ok(K, bits, group_size, dtype)


def vk_eligible_m6(m: int, K: int, N: int, bits: int, group_size: int, dtype) -> bool:
    """``mtplx/verify_kernels.py:226``: 5 or 6 rows, a format these kernels take."""
    return 5 <= int(m) <= 6 and int(N) >= 1 and _formats_ok(K, bits, group_size, dtype)


# -- tile-major packs of raw MLX triples --------------------------------------

# (id(weight tensor), layout) -> (weakref to it, version, scales ptr, biases ptr, group size, pack).
# Keyed by identity (a tensor's == is elementwise); entries go when their weight tensor is collected.
_PACKS: dict = {}


def _pack_cache_enabled() -> bool:
    return (os.environ.get("MTPLX_AMD_PACK_CACHE") or "1").strip() not in {"0", "false", "off", "no"}


def _cached_pack(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int,
                 layout: int) -> torch.Tensor:
    key_ok = _pack_cache_enabled()
    key = (id(w), layout)
    if key_ok:
        hit = _PACKS.get(key)
        if hit is not None:
            ref, ver, sp, bp, gs, pack = hit
            if ref() is w and ver == w._version and sp == scales.data_ptr() and bp == biases.data_ptr() and \
                    gs == group_size:
                return pack
    n, k = int(w.shape[-2]), int(w.shape[-1]) * 8
    nbytes = _lib.query("mtp_pack_affine4_bytes", n, k)
    if nbytes == 0:
        raise NotImplementedError(f"cannot pack N={n} K={k} (K must be a multiple of 256)")
    wc, sc, bc = w.contiguous(), scales.contiguous(), biases.contiguous()
    out = torch.empty(nbytes // 4, dtype=torch.int32, device=w.device)
    _lib.call("mtp_pack_affine4" if layout == 1 else "mtp_pack_affine4_mf16", wc.data_ptr(), sc.data_ptr(),
              bc.data_ptr(), out.data_ptr(), n, k, int(group_size), _lib.stream_handle(w.device))
    if key_ok:
        if key not in _PACKS:
            weakref.finalize(w, _PACKS.pop, key, None)
        _PACKS[key] = (weakref.ref(w), w._version, scales.data_ptr(), biases.data_ptr(), int(group_size), out)
    return out


def layout1_pack(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int) -> torch.Tensor:
    """The layout-1 tile-major copy (``mtp_pack_affine4``) of a 4-bit MLX
    triple ``[N, K/8]``. Kept per weight tensor while the tensor lives and its
    version counter, scales and biases are unchanged (unless
    ``MTPLX_AMD_PACK_CACHE=0``, which packs into a temporary every call)."""
    return _cached_pack(w, scales, biases, group_size, 1)


def layout2_pack(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int) -> torch.Tensor:
    """The layout-2 copy (``mtp_pack_affine4_mf16``, the 16x16x32 MFMA order
    for up to 16 rows) of a 4-bit MLX triple, kept as :func:`layout1_pack`
    keeps its own."""
    return _cached_pack(w, scales, biases, group_size, 2)


def rows_matmul(x2: torch.Tensor, pack: torch.Tensor, n: int, group_size: int,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """``x2 [M, K] @ W.T`` on a layout-1 pack with ``mtp_qmm_affine4_mfma``,
    in launches of up to 64 rows. Each row's sums run in an order fixed by
    (N, K) alone, so a row's output does not depend on M or on the other
    rows (the exact lane's matmul)."""
    m, k = (int(d) for d in x2.shape)
    y = out if out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x2.device)
    st = _lib.stream_handle(x2.device)
    ws = _lib.WORKSPACES.get(max(256, _lib.query("mtp_qmm_workspace_bytes", min(m, MFMA_ROWS), n, k, 0)), "qmm",
                             x2.device)
    for r0 in range(0, m, MFMA_ROWS):
        r = min(MFMA_ROWS, m - r0)
        _lib.qmm_mfma(st, x=x2[r0:].data_ptr(), w0=pack, y=y[r0:].data_ptr(), M=r, N=n, K=k,
                      group_size=int(group_size), emode=0, ws=ws, ws_bytes=ws.numel())
    return y


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
                     group_size: int = 64, bits: int = 4, mode: str = "affine",
                     out: torch.Tensor | None = None, exact: bool = False) -> torch.Tensor:
    """``x @ dequantize(w, scales, biases).T`` for ``x`` of shape ``[..., K]``.
    ``exact``: every M on the row-invariant MFMA kernel (the greedy lane)."""
    n, k = _check(x, w, scales, biases, group_size, bits, mode)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k).contiguous()
    m = x2.shape[0]
    if not fast_path(bits, group_size, k):
        y = out if out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
        _lib.call("mtp_qmv_affine", x2.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(), y.data_ptr(),
                  None, m, n, k, group_size, bits, _lib.stream_handle(x.device))
        return y.reshape(*lead, n)
    if m > STREAM_ROWS or exact:
        y = rows_matmul(x2, layout1_pack(w, scales, biases, group_size), n, group_size, out)
        return y.reshape(*lead, n)
    y = out if out is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    st = _lib.stream_handle(x.device)
    if not _pack_cache_enabled():   # no copy kept: the MLX layout in place
        _lib.call("mtp_qmv_affine4", x2.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(), y.data_ptr(),
                  m, n, k, group_size, None, 0, st)
        return y.reshape(*lead, n)
    lay = 2 if m <= 16 else 1
    pack = layout2_pack(w, scales, biases, group_size) if lay == 2 else layout1_pack(w, scales, biases, group_size)
    ws = _lib.WORKSPACES.get(max(256, _lib.query("mtp_qmv_workspace_bytes", m, n, k, 1)), "verify_qmv", x.device)
    _lib.qmv_ex(st, x=x2, w0=pack, y0=y, M=m, N=n, K=k, group_size=int(group_size), xmode=0, emode=0, packed=lay,
                ws=ws, ws_bytes=ws.numel())
    return y.reshape(*lead, n)


def vk_qmm_m4(x2, w_q, scales, biases, *, bits: int = 4, group_size: int = 64):
    """4-row verify matmul (``mtplx/verify_kernels.py:253``)."""
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)


def vk_qmm_m6(x2, w_q, scales, biases, *, bits: int = 4, group_size: int = 64):
    """5..6-row verify matmul (``mtplx/verify_kernels.py:258``); no padding
    rows are needed here, the output has the caller's M rows."""
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)


def vk_qmm_m4_ksplit(x2, w_q, scales, biases, *, bits: int = 4, group_size: int = 64):
    """``mtplx/verify_kernels.py:263``: the same kernels (they split K themselves)."""
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)


def vk_qmm_m6_ksplit(x2, w_q, scales, biases, *, bits: int = 4, group_size: int = 64):
    """``mtplx/verify_kernels.py:268``: the same kernels (they split K themselves)."""
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)


def vk_qmm_m4_impl(impl: str, x2: torch.Tensor, w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
                   bits: int = 4, group_size: int = 64) -> torch.Tensor:
    """Named-implementation entry (``mtplx/verify_kernels.py:580``). Every name
    maps to the same gfx950 kernels; the names are kept for callers that pass them."""
    if impl not in ("vk", "vk_u2", "vk_k", "vk_hybrid", "oct", "twin"):
        raise ValueError(f"unknown verify implementation {impl!r}")
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)
