"""GPU parity: stream-K verify matmul (packed weights + workspace) vs the oracle.

The stream-K kernel splits column tiles between workgroups and fixes them up
through a workspace. Its sums run in a different order from the per-tile
kernel, so the bar against the per-tile result is one bf16 ulp, and against
the float64 oracle it is the north-star rtol/atol 1e-2. Repeated launches must
be bitwise identical (the fix-up order is fixed). Successive launches share
one workspace, whose arrival counters each launch must leave at zero.
"""

import numpy as np
import pytest
import torch

from oracle.moe import silu
from oracle.bf16 import round_to_bf16
from oracle.qmv import qmm_affine4
from tests.gpu_util import assert_close, bf16_values, bits

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _np(q):
    return q.weight.cpu().numpy().view(np.uint32), bits(q.scales), bits(q.biases)


def _run(q0, q1, x, nw, r, xmode, emode, M, N, K, ws):
    from mtplx_amd import _lib
    y0 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ss = torch.zeros(((N + 31) // 32) * 32, dtype=torch.float32, device="cuda")
    kw = dict(x=x, x2=nw if xmode == 2 else None, eps=1e-6, M=M, N=N, K=K, group_size=64, xmode=xmode, emode=emode,
              packed=1, y0=y0, resid=r if emode == 1 else None, ss_out=ss if emode == 1 else None,
              w0=q0.pack(), w1=q1.pack() if emode >= 2 else None)
    if ws is not None:
        kw.update(ws=ws, ws_bytes=ws.numel(), schedule=1)
    _lib.qmv_ex(_stream(), **kw)
    torch.cuda.synchronize()
    return y0, ss


CASES = [  # (M, N, K, xmode, emode)
    (4, 17408, 5120, 0, 0),     # cfg1
    (4, 17408, 5120, 2, 3),     # fused norm + gate/up + SwiGLU
    (4, 5120, 17408, 0, 1),     # down + residual (+ss)
    (4, 5120, 5120, 0, 1),      # o_proj + residual
    (4, 7168, 5120, 2, 0),      # fused norm + q|k|v
    (1, 1000, 1024, 0, 0), (3, 300, 768, 2, 0), (8, 2048, 2560, 0, 1), (6, 640, 512, 0, 3),
    (2, 96, 256, 0, 0),         # fewer items than CUs
]


@pytest.mark.parametrize("m,n,k,xmode,emode", CASES)
def test_stream_k_matches_per_tile_and_oracle(gpu, m, n, k, xmode, emode):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(m * 7919 + n + k)
    q0 = QuantizedLinear.random(n, k, 64, generator=g)
    q1 = QuantizedLinear.random(n, k, 64, generator=g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
    nb = _lib.query("mtp_qmv_workspace_bytes", m, n, k, 1 if emode >= 2 else 0)
    assert nb > 0
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    y_sk, ss_sk = _run(q0, q1, x, nw, r, xmode, emode, m, n, k, ws)
    y_sk2, ss_sk2 = _run(q0, q1, x, nw, r, xmode, emode, m, n, k, ws)
    assert torch.equal(y_sk.view(torch.int16), y_sk2.view(torch.int16)), "stream-K not deterministic"
    assert torch.equal(ss_sk, ss_sk2)
    assert not torch.isnan(y_sk.float()).any(), "unwritten outputs"
    # counters (after the partials) left at zero for the next launch
    nblk = (n + 31) // 32
    cnt = ws[ws.numel() - (nblk * 4 + 255) // 256 * 256:][: 4 * nblk]
    assert int(cnt.view(torch.int32).abs().sum().item()) == 0
    y_pt, ss_pt = _run(q0, q1, x, nw, r, xmode, emode, m, n, k, None)
    a, b = bf16_values(y_sk), bf16_values(y_pt)
    # one bf16 ulp, plus a floor for values that cancel to near zero
    tol = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + 1e-4 * np.abs(b).max()
    assert (np.abs(a - b) <= tol).all(), f"stream-K vs per-tile: max diff {np.abs(a - b).max()}"
    if emode == 1:   # per 32-column block, per row: sum of squares of the stored y
        nblk = (n + 31) // 32
        ypad = np.zeros((m, nblk * 32))
        ypad[:, :n] = a
        want_ss = (ypad.reshape(m, nblk, 32) ** 2).sum(axis=2).T
        got_ss = ss_sk.cpu().numpy().reshape(-1, 32)[:nblk, :m]
        assert np.allclose(got_ss, want_ss, rtol=1e-5, atol=1e-5)
    if n * k <= 4_000_000:
        xb = bits(x)
        if xmode == 2:
            xf = bf16_values(x)
            inv = 1.0 / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + 1e-6)
            xb = round_to_bf16(xf * inv * bf16_values(nw)[None, :])
        g0 = qmm_affine4(xb, *_np(q0), 64)
        if emode == 3:
            want = round_to_bf16(round_to_bf16(silu(round_to_bf16(g0))) * round_to_bf16(qmm_affine4(xb, *_np(q1), 64)))
        elif emode == 1:
            want = round_to_bf16(round_to_bf16(g0) + bf16_values(r))
        else:
            want = g0
        assert_close(a, want, what=f"stream-K M={m} N={n} K={k} x{xmode} e{emode}")


def test_stream_k_workspace_shared_across_shapes(gpu):
    """Back-to-back launches of different shapes on one workspace (the verify
    step's pattern) each match their own fresh-workspace result."""
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(11)
    shapes = [(4, 5120, 17408, 0, 1), (4, 7168, 5120, 2, 0), (4, 5120, 5120, 0, 1), (4, 17408, 5120, 2, 3)]
    nb = max(_lib.query("mtp_qmv_workspace_bytes", m, n, k, 1) for m, n, k, _, _ in shapes)
    shared = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    for m, n, k, xm, em in shapes * 2:
        q0 = QuantizedLinear.random(n, k, 64, generator=g)
        q1 = QuantizedLinear.random(n, k, 64, generator=g)
        x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
        nw = torch.ones(k, dtype=torch.bfloat16, device="cuda")
        r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
        fresh = torch.zeros(nb, dtype=torch.uint8, device="cuda")
        y1, _ = _run(q0, q1, x, nw, r, xm, em, m, n, k, shared)
        y2, _ = _run(q0, q1, x, nw, r, xm, em, m, n, k, fresh)
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), (m, n, k, xm, em)


def test_stream_k_rejects_small_workspace(gpu):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    q = QuantizedLinear.random(1024, 1024, 64)
    x = torch.randn((4, 1024), device="cuda").to(torch.bfloat16)
    y = torch.empty((4, 1024), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(256, dtype=torch.uint8, device="cuda")
    with pytest.raises(_lib.MtpError) as e:
        _lib.qmv_ex(_stream(), x=x, w0=q.pack(), y0=y, M=4, N=1024, K=1024, group_size=64, packed=1, ws=ws,
                    ws_bytes=ws.numel(), schedule=1)
    assert e.value.code == -3
