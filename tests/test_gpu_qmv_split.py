"""GPU parity: the full K split of the per-tile kernel, which packed weights
use when all of x does not fit in LDS (M >= 16 at large K): each workgroup
stages one K part of x and streams that part of a group of tiles; the part
that arrives last at a tile adds the fp32 parts in part order. Bars: one bf16
ulp against the reference-layout kernel (which stages x in chunks instead),
bitwise repeat determinism, arrival counters left at zero, the north-star
rtol/atol 1e-2 against the float64 oracle, and a clear error without a
workspace."""

import numpy as np
import pytest
import torch

from oracle.bf16 import round_to_bf16
from oracle.moe import silu
from oracle.qmv import qmm_affine4
from tests.gpu_util import assert_close, bf16_values, bits

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


CASES = [  # m, n, k, xmode, emode
    (32, 17408, 5120, 0, 0),     # cfg4-sized 32-row launch
    (16, 5120, 17408, 0, 1),     # down-shaped, residual
    (32, 2048, 5120, 2, 3),      # fused norm + gate/up + SwiGLU
    (24, 1000, 8192, 0, 0),
]


@pytest.mark.parametrize("m,n,k,xmode,emode", CASES)
def test_full_split_matches_reference_layout_and_oracle(gpu, m, n, k, xmode, emode):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(m + n + k + emode)
    q0 = QuantizedLinear.random(n, k, 64, generator=g)
    q1 = QuantizedLinear.random(n, k, 64, generator=g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
    nb = _lib.query("mtp_qmv_workspace_bytes", m, n, k, 1)
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")

    def run(packed):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        kw = dict(x=x, M=m, N=n, K=k, group_size=64, xmode=xmode, emode=emode, packed=packed, y0=y)
        if packed:
            kw.update(w0=q0.pack(), ws=ws, ws_bytes=ws.numel())
            if emode == 3:
                kw["w1"] = q1.pack()
        else:
            kw.update(w0=q0.weight, s0=q0.scales, b0=q0.biases)
            if emode == 3:
                kw.update(w1=q1.weight, s1=q1.scales, b1=q1.biases)
        if xmode == 2:
            kw.update(x2=nw, eps=1e-6)
        if emode == 1:
            kw.update(resid=r, ss_out=torch.zeros(((n + 31) // 32) * 32, dtype=torch.float32, device="cuda"))
        _lib.qmv_ex(_st(), **kw)
        torch.cuda.synchronize()
        return y

    y1, y2 = run(1), run(1)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), "full split not deterministic"
    nblk = (n + 31) // 32
    cnt = ws[: 4 * nblk]   # the counter area opens the workspace
    assert int(cnt.view(torch.int32).abs().sum().item()) == 0, "arrival counters not reset"
    a, b = bf16_values(y1), bf16_values(run(0))
    assert not np.isnan(a).any(), "unwritten outputs"
    # One ulp of the rounded matmul value (the parts reassociate its fp32
    # sum); with a residual, that value is rounded again after the add, so
    # the bound is an ulp of each: 2^-7 of the larger of the matmul term and
    # the result.
    scale = np.maximum(np.abs(a), np.abs(b))
    if emode == 1:
        scale = np.maximum(scale, 2.0 * np.abs(b - bf16_values(r)))
    tol = scale * 2.0 ** -7 + 1e-4 * np.abs(b).max()
    assert (np.abs(a - b) <= tol).all(), f"full split vs reference layout: max diff {np.abs(a - b).max()}"
    if n * k <= 12_000_000:
        xb = bits(x)
        if xmode == 2:
            xv = bf16_values(x)
            inv = 1.0 / np.sqrt((xv * xv).mean(axis=1, keepdims=True) + 1e-6)
            xb = round_to_bf16(xv * inv * bf16_values(nw)[None, :])

        def qnp(q):
            return q.weight.cpu().numpy().view(np.uint32), bits(q.scales), bits(q.biases)
        g0 = qmm_affine4(xb, *qnp(q0), 64)
        if emode == 3:
            want = round_to_bf16(round_to_bf16(silu(round_to_bf16(g0))) * round_to_bf16(qmm_affine4(xb, *qnp(q1), 64)))
        elif emode == 1:
            want = round_to_bf16(round_to_bf16(g0) + bf16_values(r))
        else:
            want = g0
        assert_close(a, want, what=f"full split M={m} N={n} K={k} x{xmode} e{emode}")


def test_full_split_needs_workspace(gpu):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    m, n, k = 32, 1024, 5120
    q = QuantizedLinear.random(n, k, 64)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.MtpError) as e:
        _lib.qmv_ex(_st(), x=x, w0=q.pack(), y0=y, M=m, N=n, K=k, group_size=64, packed=1)
    assert e.value.code == -2 and b"workspace" in str(e.value).encode()


def test_one_workspace_serves_split_shapes_in_turn(gpu):
    """Full-split and tail-split calls of different shapes alternate on one
    workspace (as a verify forward's projections do, layer after layer):
    every result repeats bitwise and the counter area ends at zero."""
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(31)
    shapes = [(16, 5120, 17408, 0), (16, 17408, 5120, 3), (16, 7168, 5120, 0), (4, 17408, 5120, 3),
              (4, 5120, 17408, 0)]
    nb = max(_lib.query("mtp_qmv_workspace_bytes", m, n, k, 1) for m, n, k, _ in shapes)
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    runs = []
    for m, n, k, e in shapes:
        q0 = QuantizedLinear.random(n, k, 64, generator=g)
        q1 = QuantizedLinear.random(n, k, 64, generator=g) if e == 3 else None
        runs.append((m, n, k, e, q0, q1, torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)))

    def call(m, n, k, e, q0, q1, x):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        kw = dict(x=x, w0=q0.pack(), y0=y, M=m, N=n, K=k, group_size=64, xmode=0, emode=e, packed=1, ws=ws,
                  ws_bytes=ws.numel())
        if q1 is not None:
            kw["w1"] = q1.pack()
        _lib.qmv_ex(_st(), **kw)
        return y

    first = [call(*a) for a in runs]
    second = [call(*a) for a in runs]
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert not torch.isnan(a.float()).any()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert int(torch.count_nonzero(ws[:65536])) == 0
