"""Operator boundary for verify-shaped quantized linears (``mtplx/nax_verify.py``).

The reference monkeypatches ``nn.QuantizedLinear.__call__`` so verify-shaped
calls reach its verify kernels (``install_nax_qlinear_patch`` :738,
``patched`` :754, 8-bit branch :766-880, 4-bit branch :882-930), and counts
every fallback (:730-736). Here the patch installs the same routing on
:class:`~mtplx_amd.quant.QuantizedLinear`:

* a forward inside ``exact_verify(True)`` (the greedy lane,
  :mod:`mtplx_amd.attention_context`) runs every eligible 4-bit call on the
  row-invariant MFMA kernel over the layer's layout-1 pack, whatever M, and
  counts it under ``"exact_t0"`` as the reference counts its stock-matmul
  drop (:755-763);
* other eligible 4-bit calls (groups 64/128, K % 256 == 0): up to 32 rows on
  the streaming verify kernel, 33..64 rows on the 9..64-row MFMA kernel over
  the layout-1 pack, more rows in 64-row launches of it; also after the
  layer's MLX triple has been released;
* 8-bit layers (and 4-bit group 32) run the general affine kernel, the
  ``vk_qmm_m4`` / ``vk_qmm_m6`` lane of the reference's 8-bit branch;
* anything else falls through to the original call and is counted.
"""

from __future__ import annotations

from collections import Counter

import torch

from .attention_context import exact_lane_counts, exact_verify_required
from .quant import QuantizedLinear
from .verify_kernels import quantized_matmul, vk_eligible_ksplit

_ORIGINAL_CALL = None
_FALLBACKS: Counter = Counter()
# The reference's name for the fallback counter (``mtplx/nax_verify.py:730``):
# keys "b<bits>_m<M>" for calls that fell through, "exact_t0" for greedy-lane calls.
nax_qlinear_fallback_counts: Counter = Counter()


def nax_env_enabled() -> bool:
    """The reference gates on Apple's tensor units; the gfx950 route is always available."""
    return True


def _count_qlinear_fallback(bits: int, m: int) -> None:
    _FALLBACKS[(int(bits), int(m))] += 1
    nax_qlinear_fallback_counts[f"b{int(bits)}_m{int(m)}"] += 1


def fallback_counts() -> dict:
    return dict(_FALLBACKS)


def m4_ksplit_eligible(M: int, K: int, N: int, bits: int, group_size: int, dtype) -> bool:
    return 1 <= int(M) and vk_eligible_ksplit(M, K, N, bits, group_size, dtype)


m6_ksplit_eligible = m4_ksplit_eligible
m16_nax_eligible = m4_ksplit_eligible


def nax_qmm_m4(x2: torch.Tensor, w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
               group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """M=4 verify qmm (``mtplx/nax_verify.py:977``)."""
    return quantized_matmul(x2, w_q, scales, biases, group_size=group_size, bits=bits)


nax_qmm_m6 = nax_qmm_m4    # ``mtplx/nax_verify.py:628``
nax_qmm_m16 = nax_qmm_m4   # ``mtplx/nax_verify.py:690``


def _general_eligible(module: QuantizedLinear, k: int, x: torch.Tensor) -> bool:
    """Formats of the general affine kernel (the 8-bit and group-32 lanes)."""
    return (module.weight is not None and module.mode == "affine" and module.bits in (4, 8)
            and module.group_size in (32, 64, 128) and k % 32 == 0 and k % module.group_size == 0
            and x.dtype == torch.bfloat16 and x.is_cuda and len(module._shape) == 2
            and module.scales.dtype == torch.bfloat16)


def install_nax_qlinear_patch() -> dict:
    """Route QuantizedLinear calls through the verify kernels; idempotent."""
    global _ORIGINAL_CALL
    if _ORIGINAL_CALL is not None:
        return {"installed": True, "already": True, "route": "gfx950-mfma-qmv"}
    _ORIGINAL_CALL = QuantizedLinear.__call__

    def patched(self, x):
        from .verify_qmv import packed_matmul

        k = int(x.shape[-1])
        m = x.numel() // max(k, 1)
        if vk_eligible_ksplit(m, k, self.out_features, self.bits, self.group_size, x.dtype):
            exact = exact_verify_required()
            y = packed_matmul(x, self, exact=exact)   # a packed module streams its tile-major copy
            if y is not None:
                if exact:
                    nax_qlinear_fallback_counts["exact_t0"] += 1
                    exact_lane_counts[f"qlinear_m{m}"] += 1
                return y
            if self.weight is not None:
                y = quantized_matmul(x, self.weight, self.scales, self.biases, group_size=self.group_size,
                                     bits=self.bits, exact=exact)
                if exact:
                    nax_qlinear_fallback_counts["exact_t0"] += 1
                    exact_lane_counts[f"qlinear_m{m}"] += 1
                return y + self.bias if self.bias is not None else y
        elif _general_eligible(self, k, x):
            y = quantized_matmul(x, self.weight, self.scales, self.biases, group_size=self.group_size, bits=self.bits)
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
