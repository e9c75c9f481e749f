"""GPU parity: matmul input sums handed over by the producer (xmode 3).

An epilogue with y_sums writes the per-32-column row sums of its stored
outputs; those are bit-exact against the kernel's own stored y summed on the
host in fp32, in column order. A matmul with xmode 3 reads x together with
those sums (its staging is then the copy alone): one bf16 ulp from the plain
path, which sums x itself, and within the north-star rtol/atol 1e-2 of the
float64 oracle.
"""

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


def _block_sums(v: np.ndarray) -> np.ndarray:
    """[M, N] values -> [N/32, 32] fp32 row sums per 32-column block,
    accumulated in column order in fp32 (rows past M zero)."""
    m, n = v.shape
    out = np.zeros((n // 32, 32), dtype=np.float32)
    for b in range(n // 32):
        acc = np.zeros(m, dtype=np.float32)
        for c in range(32):
            acc = (acc + v[:, 32 * b + c].astype(np.float32)).astype(np.float32)
        out[b, :m] = acc
    return out


def _ws(m, n, k):
    from mtplx_amd import _lib
    nb = _lib.query("mtp_qmv_workspace_bytes", m, n, k, 1)
    return torch.zeros(nb, dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("m,n,k,emode,use_ws", [
    (4, 17408, 1024, 3, True),    # SwiGLU output (gate/up shape), tail split
    (4, 5120, 17408, 1, True),    # residual (down shape)
    (3, 2048, 1024, 0, False),
    (7, 640, 512, 3, False),
])
def test_epilogue_writes_row_sums(gpu, m, n, k, emode, use_ws):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(n + k + m + emode)
    q0 = QuantizedLinear.random(n, k, 64, generator=g)
    q1 = QuantizedLinear.random(n, k, 64, generator=g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    sums = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    kw = {}
    if use_ws:
        wsb = _ws(m, n, k)
        kw.update(ws=wsb, ws_bytes=wsb.numel())
    if emode == 3:
        kw["w1"] = q1.pack()
    if emode == 1:
        kw.update(resid=r, ss_out=torch.zeros(n, dtype=torch.float32, device="cuda"))
    _lib.qmv_ex(_st(), x=x, w0=q0.pack(), y0=y, y_sums=sums, M=m, N=n, K=k, group_size=64, xmode=0, emode=emode,
                packed=1, **kw)
    torch.cuda.synchronize()
    got = sums.cpu().numpy().reshape(-1, 32)
    assert np.array_equal(got[:, :m], _block_sums(bf16_values(y))[:, :m])


@pytest.mark.parametrize("m,n,k,emode,use_ws", [
    (4, 5120, 17408, 1, True),    # down_proj with the SwiGLU output's sums
    (4, 17408, 5120, 3, True),
    (2, 1000, 1024, 0, False),
    (7, 640, 512, 3, False),
])
def test_handed_over_sums_match_plain_and_oracle(gpu, m, n, k, emode, use_ws):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(m + n + k + emode)
    q0 = QuantizedLinear.random(n, k, 64, generator=g)
    q1 = QuantizedLinear.random(n, k, 64, generator=g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
    sums = torch.from_numpy(_block_sums(bf16_values(x)).reshape(-1)).cuda()
    wsb = _ws(m, n, k) if use_ws else None

    def run(**kw):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        extra = dict(ws=wsb, ws_bytes=wsb.numel()) if use_ws else {}
        if emode == 3:
            extra["w1"] = q1.pack()
        if emode == 1:
            extra.update(resid=r, ss_out=torch.zeros(n, dtype=torch.float32, device="cuda"))
        _lib.qmv_ex(_st(), x=x, w0=q0.pack(), y0=y, M=m, N=n, K=k, group_size=64, emode=emode, packed=1,
                    **extra, **kw)
        torch.cuda.synchronize()
        return bf16_values(y)

    pre = run(x_sums=sums, xmode=3)
    plain = run(xmode=0)
    tol = np.maximum(np.abs(plain), np.abs(pre)) * 2.0 ** -7 + 1e-4 * np.abs(plain).max()
    assert (np.abs(plain - pre) <= tol).all(), np.abs(plain - pre).max()
    if n * k <= 40_000_000:
        def qnp(q):
            return q.weight.cpu().numpy().view(np.uint32), bits(q.scales), bits(q.biases)
        xb = bits(x)
        g0 = qmm_affine4(xb, *qnp(q0), 64)
        if emode == 3:
            want = round_to_bf16(round_to_bf16(silu(round_to_bf16(g0))) * round_to_bf16(qmm_affine4(xb, *qnp(q1), 64)))
        elif emode == 1:
            want = round_to_bf16(round_to_bf16(g0) + bf16_values(r))
        else:
            want = g0
        assert_close(pre, want, what=f"xmode 3 vs oracle M={m} N={n} K={k} e{emode}")


def test_handed_over_sums_required(gpu):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    q = QuantizedLinear.random(256, 256, 64)
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((4, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.MtpError) as e:
        _lib.qmv_ex(_st(), x=x, w0=q.pack(), y0=y, M=4, N=256, K=256, group_size=64, xmode=3, packed=1)
    assert e.value.code == -1
