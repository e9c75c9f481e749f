"""4-bit affine group-wise quantized matmul, float64.

Format (restated from the reference's kernels, ``mtplx/verify_kernels.py:69-88``
and the dequant line ``:372``; crossrow twin ``mtplx/verify_crossrow.py:203-209``):

* ``weight`` uint32 ``[N, K/8]``; nibble ``i`` (bits ``4i..4i+3``) of word ``j``
  of row ``n`` is the quantized value ``q[n, 8j+i]`` (little-endian nibbles);
* ``scales``/``biases`` ``[N, K/group_size]`` (bf16 in the path);
* ``w[n, k] = q[n, k] * scales[n, k // gs] + biases[n, k // gs]``;
* ``y[m, n] = sum_k x[m, k] * w[n, k]`` (``x @ w.T``), accumulated in fp32 by
  the reference kernels and in float64 here.

Parity pins (tests/test_oracle_qmv.py): pack/unpack round trip, closed forms
q≡0 -> y = sum_g b_g*sum(x_g); s=1,b=0,q≡15 -> 15*sum(x); a single non-zero
group; agreement with a dense float matmul of the dequantized matrix.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32


def pack_affine4(q: np.ndarray) -> np.ndarray:
    """uint8 ``[N, K]`` nibbles (0..15) -> uint32 ``[N, K/8]`` words."""
    q = np.asarray(q)
    if q.ndim != 2 or q.shape[1] % 8:
        raise ValueError("pack_affine4 expects [N, K] with K % 8 == 0")
    if q.min(initial=0) < 0 or q.max(initial=0) > 15:
        raise ValueError("nibbles must lie in 0..15")
    q = q.astype(np.uint32).reshape(q.shape[0], -1, 8)
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))[None, None, :]
    return np.bitwise_or.reduce(q << shifts, axis=2).astype(np.uint32)


def unpack_affine4(w: np.ndarray) -> np.ndarray:
    """uint32 ``[N, K/8]`` -> uint8 ``[N, K]``."""
    w = np.asarray(w, dtype=np.uint32)
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))[None, None, :]
    q = (w[:, :, None] >> shifts) & np.uint32(0xF)
    return q.reshape(w.shape[0], -1).astype(np.uint8)


def _as_f64(a: np.ndarray) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.uint16:  # bf16 bit patterns
        return bf16_bits_to_f32(a).astype(np.float64)
    return a.astype(np.float64)


def dequantize_affine4(w: np.ndarray, scales: np.ndarray, biases: np.ndarray, group_size: int) -> np.ndarray:
    """Dense float64 ``[N, K]`` weights, ``q*s + b`` per group."""
    q = unpack_affine4(w).astype(np.float64)
    s = np.repeat(_as_f64(scales), group_size, axis=1)
    b = np.repeat(_as_f64(biases), group_size, axis=1)
    if s.shape != q.shape:
        raise ValueError(f"scales {s.shape} do not match weights {q.shape} at group {group_size}")
    return q * s + b


def qmm_affine4(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray, group_size: int) -> np.ndarray:
    """``x @ dequant(W).T`` in float64; ``x`` is ``[..., K]`` (bf16 bits or float)."""
    xf = _as_f64(x)
    lead = xf.shape[:-1]
    x2 = xf.reshape(-1, xf.shape[-1])
    n, kw = np.asarray(w).shape
    if x2.shape[1] != kw * 8:
        raise ValueError(f"x has K={x2.shape[1]}, weight packs K={kw * 8}")
    y = np.zeros((x2.shape[0], n), dtype=np.float64)
    # Row blocks keep the float64 dequant of a large matrix inside a few MB.
    step = max(1, (1 << 22) // max(1, kw * 8))
    for n0 in range(0, n, step):
        sl = slice(n0, min(n, n0 + step))
        deq = dequantize_affine4(np.asarray(w)[sl], np.asarray(scales)[sl], np.asarray(biases)[sl], group_size)
        y[:, sl] = x2 @ deq.T
    return y.reshape(*lead, n)


def qmm_affine4_groupwise(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray, group_size: int) -> np.ndarray:
    """Same contraction through the reference dot-core's regrouping
    ``y = sum_g s_g * sum_k x_k q_k + b_g * sum_k x_k`` (``mtplx/verify_qmv.py:58-191``:
    ``scale*Σxq + bias*Σx`` per group). Independent route used to pin
    :func:`qmm_affine4`."""
    xf = _as_f64(x).reshape(-1, np.asarray(w).shape[1] * 8)
    q = unpack_affine4(w).astype(np.float64)
    n, k = q.shape
    g = k // group_size
    s = _as_f64(scales)
    b = _as_f64(biases)
    xg = xf.reshape(xf.shape[0], g, group_size)
    qg = q.reshape(n, g, group_size)
    dots = np.einsum("mgk,ngk->mng", xg, qg)
    xsum = xg.sum(axis=2)  # [M, G]
    return (dots * s[None]).sum(axis=2) + xsum @ b.T


def make_affine4_weights(rng: np.random.Generator, n: int, k: int, group_size: int = 64,
                         scale_std: float = 0.02, bias_std: float = 0.01):
    """Synthetic layer in the BASELINE recipe: nibbles U{0..15}, scales
    |N(0, scale_std)|, biases N(0, bias_std), both rounded to bf16.

    Returns ``(w uint32 [n,k/8], scales bf16-bits [n,k/gs], biases bf16-bits)``.
    """
    from .bf16 import f32_to_bf16_bits

    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = np.abs(rng.normal(0.0, scale_std, size=(n, k // group_size))).astype(np.float32)
    b = rng.normal(0.0, bias_std, size=(n, k // group_size)).astype(np.float32)
    return pack_affine4(q), f32_to_bf16_bits(s), f32_to_bf16_bits(b)


# ---------------------------------------------------------------------------
# Any power-of-two width (MLX affine quantization, mlx==0.32.2 as the
# reference's pyproject.toml:36 pins; its verify lanes read 8-bit packs at
# mtplx/verify_qmv.py:1256-1377 and group-32 packs at
# mtplx/kernels/qmv4_matmul.py:158-176): a uint32 word holds 32/bits values,
# value i in bits bits*i .. bits*i + bits - 1 (little-endian fields).

def pack_affine(q: np.ndarray, bits: int) -> np.ndarray:
    """uint ``[N, K]`` values in 0..2^bits-1 -> uint32 ``[N, K*bits/32]``."""
    if bits not in (2, 4, 8):
        raise ValueError("bits must be 2, 4 or 8")
    vpw = 32 // bits
    q = np.asarray(q)
    if q.ndim != 2 or q.shape[1] % vpw:
        raise ValueError(f"pack_affine expects [N, K] with K % {vpw} == 0")
    if q.min(initial=0) < 0 or q.max(initial=0) > (1 << bits) - 1:
        raise ValueError(f"values must lie in 0..{(1 << bits) - 1}")
    q = q.astype(np.uint32).reshape(q.shape[0], -1, vpw)
    shifts = (np.arange(vpw, dtype=np.uint32) * np.uint32(bits))[None, None, :]
    return np.bitwise_or.reduce(q << shifts, axis=2).astype(np.uint32)


def unpack_affine(w: np.ndarray, bits: int) -> np.ndarray:
    """uint32 ``[N, K*bits/32]`` -> ``[N, K]`` values."""
    vpw = 32 // bits
    w = np.asarray(w, dtype=np.uint32)
    shifts = (np.arange(vpw, dtype=np.uint32) * np.uint32(bits))[None, None, :]
    q = (w[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(w.shape[0], -1).astype(np.uint16 if bits > 8 else np.uint8)


def qmm_affine(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray, group_size: int,
               bits: int) -> np.ndarray:
    """``x @ dequant(W).T`` in float64 for ``bits``-wide affine weights."""
    xf = _as_f64(x)
    lead = xf.shape[:-1]
    x2 = xf.reshape(-1, xf.shape[-1])
    n = np.asarray(w).shape[0]
    k = np.asarray(w).shape[1] * (32 // bits)
    if x2.shape[1] != k:
        raise ValueError(f"x has K={x2.shape[1]}, weight packs K={k}")
    y = np.zeros((x2.shape[0], n), dtype=np.float64)
    step = max(1, (1 << 22) // max(1, k))
    for n0 in range(0, n, step):
        sl = slice(n0, min(n, n0 + step))
        q = unpack_affine(np.asarray(w)[sl], bits).astype(np.float64)
        s = np.repeat(_as_f64(np.asarray(scales)[sl]), group_size, axis=1)
        b = np.repeat(_as_f64(np.asarray(biases)[sl]), group_size, axis=1)
        if s.shape != q.shape:
            raise ValueError(f"scales {s.shape} do not match weights {q.shape} at group {group_size}")
        y[:, sl] = x2 @ (q * s + b).T
    return y.reshape(*lead, n)


def make_affine_weights(rng: np.random.Generator, n: int, k: int, group_size: int, bits: int,
                        scale_std: float = 0.02, bias_std: float = 0.01):
    """Synthetic ``bits``-wide layer: values U{0..2^bits-1}, scales |N(0,
    scale_std)|, biases N(0, bias_std), bf16. Returns ``(w, scales, biases)``."""
    from .bf16 import f32_to_bf16_bits

    q = rng.integers(0, 1 << bits, size=(n, k), dtype=np.uint16)
    s = np.abs(rng.normal(0.0, scale_std, size=(n, k // group_size))).astype(np.float32)
    b = rng.normal(0.0, bias_std, size=(n, k // group_size)).astype(np.float32)
    return pack_affine(q, bits), f32_to_bf16_bits(s), f32_to_bf16_bits(b)
