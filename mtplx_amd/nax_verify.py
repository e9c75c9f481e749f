"""Operator boundary for verify-shaped quantized linears (``mtplx/nax_verify.py``).

The reference monkeypatches ``nn.QuantizedLinear.__call__`` so verify-shaped
calls (M in 4..16, not prefill) reach its verify kernels
(``install_nax_qlinear_patch`` :738, ``patched`` :754, 4-bit branch :882-930)
and counts every fallback (:730-736). Here the patch installs the same routing
on :class:`~mtplx_amd.quant.QuantizedLinear`: M <= 32 rows go to the gfx950
verify kernel, larger M to 32-row launches of the same kernel; ineligible
layers (8-bit, group 32) fall back to the original call and are counted.
"""

from __future__ import annotations

from collections import Counter

import torch

from .quant import QuantizedLinear
from .verify_kernels import quantized_matmul, vk_eligible_ksplit

_ORIGINAL_CALL = None
_FALLBACKS: Counter = Counter()


def nax_env_enabled() -> bool:
    """The reference gates on Apple's tensor units; the gfx950 route is always available."""
    return True


def _count_qlinear_fallback(bits: int, m: int) -> None:
    _FALLBACKS[(int(bits), int(m))] += 1


def fallback_counts() -> dict:
    return dict(_FALLBACKS)


def m4_ksplit_eligible(M: int, K: int, N: int, bits: int, group_size: int, dtype) -> bool:
    return 1 <= int(M) <= 32 and vk_eligible_ksplit(M, K, N, bits, group_size, dtype)


m6_ksplit_eligible = m4_ksplit_eligible
m16_nax_eligible = m4_ksplit_eligible


def nax_qmm_m4(x2: torch.Tensor, w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
               group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """M=4 verify qmm (``mtplx/nax_verify.py:977``)."""
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)


nax_qmm_m6 = nax_qmm_m4    # ``mtplx/nax_verify.py:628``
nax_qmm_m16 = nax_qmm_m4   # ``mtplx/nax_verify.py:690``


def install_nax_qlinear_patch() -> dict:
    """Route QuantizedLinear calls through the verify kernels; idempotent."""
    global _ORIGINAL_CALL
    if _ORIGINAL_CALL is None:
        _ORIGINAL_CALL = QuantizedLinear.__call__

        def patched(self, x):
            k = int(x.shape[-1])
            m = x.numel() // max(k, 1)
            if vk_eligible_ksplit(m, k, self.out_features, self.bits, self.group_size, x.dtype):
                from .verify_qmv import packed_matmul
                y = packed_matmul(x, self)   # a module packed once streams its tile-major copy
                if y is not None:
                    return y
                y = quantized_matmul(x, self.weight, self.scales, self.biases, group_size=self.group_size,
                                     bits=self.bits)
                return y + self.bias if self.bias is not None else y
            _count_qlinear_fallback(self.bits, m)
            return _ORIGINAL_CALL(self, x)

        patched._mtplx_amd_patch = True
        QuantizedLinear.__call__ = patched
    return {"installed": True, "route": "gfx950-mfma-qmv"}


def uninstall_nax_qlinear_patch() -> None:
    global _ORIGINAL_CALL
    if _ORIGINAL_CALL is not None:
        QuantizedLinear.__call__ = _ORIGINAL_CALL
        _ORIGINAL_CALL = None
