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


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """One bf16 ulp at |v| (8 significant bits)."""
    return np.exp2(np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126))) - 7)


def assert_resid_close(got: np.ndarray, prod: np.ndarray, want: np.ndarray, what=""):
    """bf16(bf16(x @ W) + resid) outputs: the north-star bar (rtol = atol =
    1e-2) plus one bf16 ulp of the rounded product. Both sides round the
    product to bf16 from sums that differ in their last fp32 bits, so it may
    land one ulp apart; where the residual cancels much of the product, that
    ulp is several ulps of the result (product -8.25, result -4.25: 0.0625)."""
    bad = np.abs(got - want) > 1e-2 + 1e-2 * np.abs(want) + bf16_ulp(prod)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside the bar; first {idx.tolist()} "
                             f"got {got[tuple(idx[0])]} want {want[tuple(idx[0])]} product {prod[tuple(idx[0])]}")


def assert_swiglu_close(got: np.ndarray, gate: np.ndarray, up: np.ndarray, want: np.ndarray, what=""):
    """bf16(bf16(silu(bf16(gate))) * bf16(up)) outputs
    (rtol = atol = 1e-2) plus one bf16 ulp of each rounded factor carried
    through the product. Both sides round gate, silu and up to bf16 from
    sums that differ in their last fp32 bits, so a value on a rounding
    boundary may land one ulp apart; where silu is steep relative to its
    value (its tail, gate < -4) and |up| is large, one ulp of gate moves the
    product by several output ulps (gate -6, up -63: 0.023)."""
    sig = 1.0 / (1.0 + np.exp(-gate))
    s = gate * sig
    ds = np.abs(sig * (1.0 + gate * (1.0 - sig)))
    carry = np.abs(up) * (ds * bf16_ulp(gate) + bf16_ulp(s)) + np.abs(s) * bf16_ulp(up)
    bad = np.abs(got - want) > 1e-2 + 1e-2 * np.abs(want) + carry
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside the bar; first {idx.tolist()} got "
                             f"{got[tuple(idx[0])]} want {want[tuple(idx[0])]}")
