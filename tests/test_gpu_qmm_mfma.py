"""GPU parity of the 9..64-row quantized matmul (mtp_qmm_affine4_mfma), the
continuous-batched ragged verify's projections: each weight quad is read
once for all rows, x streams through LDS by quads, leftover column groups
are split by K with the last arriving part adding the parts in order.

Bars: the north-star rtol/atol 1e-2 against the float64 oracle for every
epilogue (store, fp32 store, residual, SwiGLU pair; the pair's bar also
carries one bf16 ulp of each rounded factor through the product, see
``assert_swiglu_close``), group sizes 64 and 128,
shapes that take the K split and shapes that do not; bitwise repeat
determinism; arrival counters back at zero; one bf16 ulp (plus 1e-4 of the
row's scale where a sum cancels) against the skinny kernel
(mtp_qmv_affine4_ex) where both run (M <= 32); a clear error without a
workspace."""

import numpy as np
import pytest
import torch

from oracle.bf16 import round_to_bf16
from oracle.moe import silu
from oracle.qmv import qmm_affine4
from tests.gpu_util import assert_resid_close, assert_swiglu_close, assert_close, bf16_values, bits

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _layer(n, k, gs, g):
    from mtplx_amd.quant import QuantizedLinear
    return QuantizedLinear.random(n, k, gs, generator=g)


def _triple(q):
    return (q.weight.cpu().numpy().view(np.uint32), bits(q.scales), bits(q.biases))


def _run(m, n, k, emode, gs, x, q0, q1=None, resid=None, fp32=False):
    from mtplx_amd import _lib
    nb = _lib.query("mtp_qmm_workspace_bytes", m, n, k, 1 if emode == 3 else 0)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device="cuda")
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    yf = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda") if fp32 else None
    kw = dict(x=x, w0=q0.pack(), M=m, N=n, K=k, group_size=gs, emode=emode, ws=ws, ws_bytes=ws.numel())
    if fp32:
        kw["yf"] = yf
    else:
        kw["y"] = y
    if q1 is not None:
        kw["w1"] = q1.pack()
    if resid is not None:
        kw["resid"] = resid
    _lib.qmm_mfma(_st(), **kw)
    torch.cuda.synchronize()
    return (yf if fp32 else y), ws, nb


CASES = [  # m, n, k, emode, gs
    (64, 17408, 5120, 0, 64),    # cfg4 gate-sized, 64 rows
    (48, 5120, 17408, 1, 64),    # down-shaped + residual (K split)
    (64, 2048, 5120, 3, 64),     # SwiGLU pair
    (33, 7168, 5120, 0, 64),     # q|k|v-shaped, odd rows
    (45, 2048, 5120, 3, 64),     # SwiGLU pair at cfg4's 45 rows (rows 48..63 not finished)
    (49, 5120, 5120, 1, 64),     # just past 48 rows: every row group finished
    (16, 5120, 5120, 1, 128),    # o-shaped, group 128
    (9, 1000, 2048, 0, 64),      # N not a multiple of 32
    (64, 151936 // 8, 5120, 2, 64),   # lm_head slice, fp32 out
]


@pytest.mark.parametrize("m,n,k,emode,gs", CASES)
def test_rows_kernel_matches_oracle(gpu, m, n, k, emode, gs):
    g = torch.Generator(device="cuda").manual_seed(m * 7 + n + k + emode)
    q0 = _layer(n, k, gs, g)
    q1 = _layer(n, k, gs, g) if emode == 3 else None
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16) if emode == 1 else None
    fp32 = emode == 2
    y, ws, nb = _run(m, n, k, 0 if fp32 else emode, gs, x, q0, q1, r, fp32)
    got = y.cpu().numpy().astype(np.float64) if fp32 else bf16_values(y)
    xb = bits(x)
    a = round_to_bf16(qmm_affine4(xb, *_triple(q0), gs))
    if emode == 0 or emode == 2:
        want = a
    elif emode == 1:
        want = round_to_bf16(a + bf16_values(r))
    else:
        up = round_to_bf16(qmm_affine4(xb, *_triple(q1), gs))
        want = round_to_bf16(round_to_bf16(silu(a)) * up)
    if emode == 3:
        assert_swiglu_close(got, a, up, want, what=f"rows kernel m={m} n={n} k={k} SwiGLU")
    elif emode == 1:
        assert_resid_close(got, a, want, what=f"rows kernel m={m} n={n} k={k} + residual")
    else:
        assert_close(got, want, what=f"rows kernel m={m} n={n} k={k} e={emode}")
    # deterministic, counters returned to zero
    y2, ws2, _ = _run(m, n, k, 0 if fp32 else emode, gs, x, q0, q1, r, fp32)
    assert torch.equal(y.view(torch.int32) if fp32 else y.view(torch.int16),
                       y2.view(torch.int32) if fp32 else y2.view(torch.int16))
    if nb:
        # the arrival counters sit in the workspace's first 64 KiB
        assert int(torch.count_nonzero(ws2[:65536])) == 0


@pytest.mark.parametrize("m", [16, 32])
def test_rows_kernel_within_one_ulp_of_skinny_kernel(gpu, m):
    from mtplx_amd import _lib
    n, k = 4096, 5120
    g = torch.Generator(device="cuda").manual_seed(100 + m)
    q0 = _layer(n, k, 64, g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    y, _, _ = _run(m, n, k, 0, 64, x, q0)
    nb = _lib.query("mtp_qmv_workspace_bytes", m, n, k, 0)
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    y_sk = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    _lib.qmv_ex(_st(), x=x, w0=q0.pack(), y0=y_sk, M=m, N=n, K=k, group_size=64, xmode=0, emode=0, packed=1, ws=ws,
                ws_bytes=ws.numel())
    torch.cuda.synchronize()
    # Same arithmetic in another fp32 summation order: one bf16 ulp, except
    # where the sum cancels (there a few ulps of a small value, far below
    # the row's scale).
    a, b = bf16_values(y), bf16_values(y_sk)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(b), 1e-30))) - 7)
    assert (np.abs(a - b) <= ulp + 1e-4 * np.abs(b).max(axis=1, keepdims=True)).all()


def test_rows_kernel_needs_workspace_when_splitting(gpu):
    from mtplx_amd import _lib
    m, n, k = 64, 5120, 17408
    nb = _lib.query("mtp_qmm_workspace_bytes", m, n, k, 0)
    assert nb > 0
    g = torch.Generator(device="cuda").manual_seed(5)
    q0 = _layer(n, k, 64, g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.MtpError) as e:
        _lib.qmm_mfma(_st(), x=x, w0=q0.pack(), y=y, M=m, N=n, K=k, group_size=64, emode=0)
    assert e.value.code == -3
    with pytest.raises(_lib.MtpError):
        _lib.qmm_mfma(_st(), x=x, w0=q0.pack(), y=y, M=65, N=n, K=k, group_size=64, emode=0)


def test_one_workspace_serves_shapes_in_turn(gpu):
    """Calls of different shapes alternate on one workspace (as the ragged
    verify's projections do, layer after layer): every result repeats
    bitwise, so no shape's partials land on another shape's counters."""
    from mtplx_amd import _lib
    g = torch.Generator(device="cuda").manual_seed(21)
    shapes = [(45, 5120, 17408, 1), (45, 17408, 5120, 3), (45, 7168, 5120, 0), (45, 5120, 5120, 1)]
    nb = max(_lib.query("mtp_qmm_workspace_bytes", m, n, k, 1 if e == 3 else 0) for m, n, k, e in shapes)
    assert nb > 0
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    runs = []
    for m, n, k, e in shapes:
        q0 = _layer(n, k, 64, g)
        q1 = _layer(n, k, 64, g) if e == 3 else None
        x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
        r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16) if e == 1 else None
        runs.append((m, n, k, e, q0, q1, x, r))

    def call(m, n, k, e, q0, q1, x, r):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        kw = dict(x=x, w0=q0.pack(), y=y, M=m, N=n, K=k, group_size=64, emode=e, ws=ws, ws_bytes=ws.numel())
        if q1 is not None:
            kw["w1"] = q1.pack()
        if r is not None:
            kw["resid"] = r
        _lib.qmm_mfma(_st(), **kw)
        return y

    first = [call(*a) for a in runs]
    second = [call(*a) for a in runs]
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert not torch.isnan(a.float()).any()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert int(torch.count_nonzero(ws[:65536])) == 0
