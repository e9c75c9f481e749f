"""GPU parity: the per-tile verify matmul with a workspace (schedule 0), which
splits the leftover tiles of its last round by K over all CUs and adds the
parts in a fixed order. Bars: one bf16 ulp against the unsplit kernel (the
parts reassociate the fp32 sums of the leftover tiles only), bitwise repeat
determinism, arrival counters left at zero, and the north-star rtol/atol 1e-2
against the float64 oracle."""

import numpy as np
import pytest
import torch

from oracle.bf16 import round_to_bf16
from oracle.moe import silu
from oracle.qmv import qmm_affine4
from tests.gpu_util import assert_close, bf16_values, bits

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _run(q0, q1, x, nw, ssin, r, xmode, emode, M, N, K, ws):
    from mtplx_amd import _lib
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ss = torch.zeros(((N + 31) // 32) * 32, dtype=torch.float32, device="cuda")
    kw = dict(x=x, M=M, N=N, K=K, group_size=64, xmode=xmode, emode=emode, packed=1, y0=y, w0=q0.pack())
    if xmode == 2:
        kw.update(x2=nw, eps=1e-6, ss_in=ssin)
    if emode == 1:
        kw.update(resid=r, ss_out=ss)
    if emode == 3:
        kw.update(w1=q1.pack())
    if ws is not None:
        kw.update(ws=ws, ws_bytes=ws.numel(), schedule=0)
    _lib.qmv_ex(_stream(), **kw)
    torch.cuda.synchronize()
    return y, ss


CASES = [  # (M, N, K, xmode, emode): N/32 tiles = 512 + E, E | 256 on a 256-CU part
    (4, 17408, 5120, 2, 3),    # fused RMSNorm + gate/up + SwiGLU: 544 tiles, 32 split 8 ways
    (4, 17408, 5120, 0, 0),
    (4, 18432, 2048, 0, 1),    # 576 tiles: 64 split 4 ways, residual + ss
    (2, 20480, 1024, 2, 0),    # 640 tiles: 128 split 2 ways
    (3, 17408, 2048, 0, 3),
    # fewer tiles than CUs, every tile split floor(256 / T) ways (at most one part per quad):
    (16, 257, 4096, 0, 0),     # router | shared gate of the MoE block: 9 tiles, 16 parts each
    (16, 1536, 4096, 2, 3),    # shared expert gate/up + SwiGLU, fused norm: 48 tiles, 5 parts
    (16, 4096, 1536, 0, 1),    # shared expert down + residual: 128 tiles, 2 parts
    (4, 1024, 4096, 2, 0),     # 32 tiles, 8 parts
]


@pytest.mark.parametrize("m,n,k,xmode,emode", CASES)
def test_tail_split_matches_unsplit_and_oracle(gpu, m, n, k, xmode, emode):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(m * 31 + n + k + emode)
    q0 = QuantizedLinear.random(n, k, 64, generator=g)
    q1 = QuantizedLinear.random(n, k, 64, generator=g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
    xf = x.float()
    ssin = torch.zeros(((k + 31) // 32) * 32, dtype=torch.float32, device="cuda")
    ssin.view(-1, 32)[:, :m] = (xf * xf).view(m, -1, 32).sum(dim=2).t()
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
    nb = _lib.query("mtp_qmv_workspace_bytes", m, n, k, 1)
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    y1, ss1 = _run(q0, q1, x, nw, ssin, r, xmode, emode, m, n, k, ws)
    y2, ss2 = _run(q0, q1, x, nw, ssin, r, xmode, emode, m, n, k, ws)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), "tail split not deterministic"
    assert torch.equal(ss1, ss2)
    assert not torch.isnan(y1.float()).any(), "unwritten outputs"
    nblk = (n + 31) // 32
    cnt = ws[: 4 * nblk]   # the counter area opens the workspace
    assert int(cnt.view(torch.int32).abs().sum().item()) == 0, "arrival counters not reset"
    y0, _ = _run(q0, q1, x, nw, ssin, r, xmode, emode, m, n, k, None)
    a, b = bf16_values(y1), bf16_values(y0)
    tol = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + 1e-4 * np.abs(b).max()
    assert (np.abs(a - b) <= tol).all(), f"tail split vs unsplit: max diff {np.abs(a - b).max()}"
    # only the leftover tiles may differ at all (256-CU part)
    lead = n // 32 - (n // 32) % 256
    assert torch.equal(y1[:, : lead * 32].view(torch.int16), y0[:, : lead * 32].view(torch.int16))
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
        assert_close(a, want, what=f"tail split M={m} N={n} K={k} x{xmode} e{emode}")
