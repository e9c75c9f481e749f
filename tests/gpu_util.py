"""Helpers shared by the GPU parity tests (torch <-> oracle conversions)."""

import numpy as np
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 torch tensor -> uint16 bit patterns (numpy)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def from_bits(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_values(t: torch.Tensor) -> np.ndarray:
    return bf16_bits_to_f32(bits(t)).astype(np.float64)


def randn_bf16(rng: np.random.Generator, shape, scale=1.0, device="cuda") -> torch.Tensor:
    return from_bits(f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32)), device)


def u32(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(device)


def assert_close(got: np.ndarray, want: np.ndarray, rtol=1e-2, atol=1e-2, what=""):
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside rtol={rtol} atol={atol}; "
                             f"first {idx.tolist()} got {got[tuple(idx[0])]} want {want[tuple(idx[0])]}")
