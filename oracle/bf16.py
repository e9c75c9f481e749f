"""bfloat16 <-> float conversions on uint16 bit patterns (NumPy has no bf16).

Round-to-nearest-even, NaN preserved — the IEEE rule every bf16 producer in
the path uses (torch's ``.to(torch.bfloat16)`` and the HIP kernels'
``__float2bfloat16``).
"""

from __future__ import annotations

import numpy as np


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    b = np.asarray(bits).astype(np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns, round to nearest even."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    r = np.where(nan, np.uint16(0x7FC0), r)
    return r.astype(np.uint16)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """Value of ``x`` after a round trip through bf16, as float64."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32))).astype(np.float64)
