"""Quantized linear layer in the reference's 4-bit affine format, on the GPU.

Mirrors the attributes the reference's verify kernels read from MLX's
``nn.QuantizedLinear`` (``mtplx/verify_qmv.py:19-34``, ``mtplx/nax_verify.py:754``):
``weight`` uint32 ``[N, K/8]`` (held as int32), ``scales``/``biases`` bf16
``[N, K/group_size]``, ``group_size``, ``bits``, ``mode`` and an optional
``bias``. Calling the layer runs the HIP verify matmul; nothing runs on the CPU.
"""

from __future__ import annotations

import torch


class QuantizedLinear:
    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int = 64, bits: int = 4, mode: str = "affine", bias: torch.Tensor | None = None):
        if weight.dtype not in (torch.int32, torch.uint32):
            raise TypeError("weight must be int32/uint32 packed words")
        self.weight = weight.view(torch.int32) if weight.dtype == torch.uint32 else weight
        self.scales = scales
        self.biases = biases
        self.group_size = int(group_size)
        self.bits = int(bits)
        self.mode = mode
        self.bias = bias
        self.packed: torch.Tensor | None = None         # layout 1 (any M)
        self.packed_mf16: torch.Tensor | None = None    # layout 2 (M <= 16)
        self._shape = tuple(int(d) for d in self.weight.shape)   # kept when the source is released

    def pack(self, row_order: torch.Tensor | None = None, layout: int = 1) -> torch.Tensor:
        """Tile-major copy of the weights for the streaming kernel. ``layout``
        1 serves any M (``packed=1``); 2 is the 16x16x32-MFMA order for M <= 16
        (``packed=2``). Without ``row_order`` each layout is made once and
        cached; with it, packed row i is original row ``row_order[i]`` (e.g.
        :func:`rope_row_order`)."""
        if row_order is None and layout == 1 and self.packed is not None:
            return self.packed
        if row_order is None and layout == 2 and self.packed_mf16 is not None:
            return self.packed_mf16
        if layout not in (1, 2):
            raise ValueError(f"layout {layout} (1 or 2)")
        from . import _lib

        if self.weight is None:
            raise RuntimeError("the layer's source weights were released; only its cached packs remain")
        experts = self.weight.dim() == 3
        if self.weight.dim() not in (2, 3) or self.bits != 4 or self.mode != "affine":
            raise NotImplementedError("packing covers 2-D (or expert-stacked 3-D) 4-bit affine layers")
        if experts and (row_order is not None or self.out_features % 32):
            raise NotImplementedError("expert stacks pack without a row order, with N a multiple of 32")
        # An expert stack [E, N, K/8] packs as the [E*N, K] matrix: with N a
        # multiple of 32 no tile straddles two experts, so expert e's tiles
        # start at tile e * N / 32.
        n, k = self.out_features * (self._shape[0] if experts else 1), self.in_features
        nbytes = _lib.query("mtp_pack_affine4_bytes", n, k)
        if nbytes == 0:
            raise NotImplementedError(f"cannot pack N={n} K={k} (K must be a multiple of 256)")
        w, s, b = self.weight, self.scales, self.biases
        if experts:
            w, s, b = w.reshape(n, -1), s.reshape(n, -1), b.reshape(n, -1)
        if row_order is not None:
            idx = row_order.to(device=w.device, dtype=torch.long)
            if idx.numel() != n:
                raise ValueError(f"row_order has {idx.numel()} entries, layer has {n} rows")
            w, s, b = w[idx].contiguous(), s[idx].contiguous(), b[idx].contiguous()
        out = torch.empty(nbytes // 4, dtype=torch.int32, device=w.device)
        _lib.call("mtp_pack_affine4" if layout == 1 else "mtp_pack_affine4_mf16", w.data_ptr(), s.data_ptr(),
                  b.data_ptr(), out.data_ptr(), n, k, self.group_size, _lib.stream_handle(w.device))
        if row_order is None:
            if layout == 1:
                self.packed = out
            else:
                self.packed_mf16 = out
        return out

    def release_source(self) -> None:
        """Free the MLX-layout triple once the packs the caller needs are
        cached (an expert stack of a large MoE is held only in its packed
        copy). Calls that need the triple raise afterwards."""
        if self.packed is None and self.packed_mf16 is None:
            raise RuntimeError("pack the layer before releasing its source weights")
        self.weight = self.scales = self.biases = None

    @property
    def in_features(self) -> int:
        return self._shape[-1] * 32 // self.bits

    @property
    def out_features(self) -> int:
        return self._shape[-2]

    def __contains__(self, name: str) -> bool:   # MLX-style `"bias" in module`
        return getattr(self, name, None) is not None

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """``x @ W.T (+ bias)``: on the layer's tile-major packs when it has
        them (past 32 rows the layout-1 pack, made here on first use), else
        on the MLX triple."""
        from .verify_kernels import quantized_matmul
        from .verify_qmv import packed_matmul

        y = packed_matmul(x, self)
        if y is not None:
            return y
        if self.weight is None:
            raise RuntimeError("the layer's source weights were released and its packs do not serve this call "
                               "(bf16 rows on the GPU with K equal to the layer's in_features)")
        y = quantized_matmul(x, self.weight, self.scales, self.biases, group_size=self.group_size, bits=self.bits,
                             mode=self.mode)
        if self.bias is not None:
            y = y + self.bias
        return y

    @classmethod
    def random(cls, out_features: int, in_features: int, group_size: int = 64, *, generator=None,
               device="cuda", scale_std: float = 0.02, bias_std: float = 0.01, experts: int | None = None,
               centered: bool = False, bits: int = 4):
        """Synthetic layer (random init): nibbles U{0..15}, scales |N(0,scale_std)|,
        biases N(0,bias_std), bf16 — the BASELINE weight recipe. ``experts``
        adds a leading expert axis (MoE switch layers). ``centered`` sets each
        group's bias to -7.5 x its scale instead, so the weights have zero
        mean (no per-row offset in the outputs). ``bits`` 4 or 8 (uniform
        fields, 32/bits per word)."""
        if bits not in (4, 8):
            raise ValueError("bits must be 4 or 8")
        lead = () if experts is None else (experts,)
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, lead + (out_features, in_features * bits // 32), dtype=torch.int32,
                          device=device, generator=generator)
        g = in_features // group_size
        s = (torch.randn(lead + (out_features, g), device=device, generator=generator) * scale_std).abs()
        b = torch.randn(lead + (out_features, g), device=device, generator=generator) * bias_std
        s = s.to(torch.bfloat16)
        if centered:
            b = -0.5 * ((1 << bits) - 1) * s.float()
        return cls(w, s, b.to(torch.bfloat16), group_size=group_size, bits=bits)


def rope_row_order(n_heads: int, head_dim: int) -> torch.Tensor:
    """Row order of a q|k|v projection for the fused RoPE epilogue (emode 4 of
    ``mtp_qmv_affine4_ex``): packed tile t = head t // (D/32), sub-block
    sb = t % (D/32); its column c is dimension 16 sb + c % 16 + (c // 16) * D/2,
    so the rotate-half pairs (d, d + D/2) of a head share one 32-column tile."""
    if head_dim % 32:
        raise ValueError("head_dim must be a multiple of 32")
    tph = head_dim // 32
    t = torch.arange(n_heads * tph).repeat_interleave(32)
    c = torch.arange(32).repeat(n_heads * tph)
    head, sb = t // tph, t % tph
    return head * head_dim + 16 * sb + c % 16 + (c // 16) * (head_dim // 2)
