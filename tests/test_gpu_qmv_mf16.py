"""GPU parity: packed layout 2 and its 16x16x32-MFMA quads (M <= 4, and up
to 16 rows with x row m at A row m).

The layout is pinned bit-for-bit by a NumPy restatement. The matmul computes
the same per-group sums as layout 1, with the MFMA summing each 32-k step in
another grouping, so outputs agree with layout 1 to one bf16 ulp. They also
meet the north-star rtol/atol 1e-2 against the float64 oracle, through every
producer and epilogue the verify step uses: the tail split, the RoPE epilogue
(bit-exact against the same weights' layout-1 result) and handed-over sums.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import round_to_bf16
from oracle.moe import silu
from oracle.qmv import make_affine4_weights, qmm_affine4
from tests.gpu_util import assert_close, bf16_values, bits, from_bits, u32
from tests.test_gpu_qmv import _nibbles_natural, _pack_reference

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _pack2_reference(w, s, b, gs):
    """NumPy restatement of layout 2 (include/mtplx_amd.h)."""
    N, kw = w.shape
    Q = kw * 8 // 256
    T = -(-N // 32)
    out = _pack_reference(w, s, b, gs).reshape(T, Q, 1152)   # scale/bias words are shared
    out[:, :, :1024] = 0
    for nb in range(T):
        for q in range(Q):
            for u in range(4):
                for l in range(64):
                    for jj in range(4):
                        row = nb * 32 + 16 * (jj & 1) + (l & 15)
                        if row < N:
                            word = w[row, 32 * q + 8 * u + 4 * (jj >> 1) + (l >> 4)]
                            out[nb, q, 256 * u + 4 * l + jj] = _nibbles_natural([word])[0]
    return out.reshape(-1)


@pytest.mark.parametrize("n,k,gs", [(70, 512, 64), (64, 768, 128)])
def test_pack_layout2_bit_exact(gpu, n, k, gs):
    from mtplx_amd.quant import QuantizedLinear
    rng = np.random.default_rng(n * 3 + k)
    w, s, b = make_affine4_weights(rng, n, k, gs)
    q = QuantizedLinear(u32(w), from_bits(s), from_bits(b), group_size=gs)
    got = q.pack(layout=2).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, _pack2_reference(w, s, b, gs))


CASES = [  # m, n, k, xmode, emode, use_ws
    (4, 17408, 5120, 2, 3, True),     # fused norm + gate/up + SwiGLU, tail split
    (4, 5120, 17408, 0, 1, False),    # down + residual
    (4, 5120, 5120, 0, 1, True),      # o_proj + residual
    (1, 1000, 1024, 0, 0, False),
    (3, 300, 768, 2, 0, False),
    (2, 640, 512, 0, 3, False),
    (4, 151936 // 8, 5120, 2, 0, True),
    # 5..16 rows: every A row a row of x, four output rows per lane
    (16, 4096, 4096, 2, 3, True),     # cfg5-width fused norm + gate/up + SwiGLU, tail split
    (16, 4096, 4096, 0, 1, True),     # cfg5-width o_proj + residual
    (9, 4096, 1536, 0, 1, False),     # down width of an expert, 9 rows
    (5, 300, 768, 2, 0, False),
    (12, 640, 512, 0, 3, False),
    (16, 1000, 1024, 0, 0, False),
    (8, 5120, 17408, 0, 0, True),     # x beyond LDS: full K split
]


@pytest.mark.parametrize("m,n,k,xmode,emode,use_ws", CASES)
def test_layout2_matches_layout1_and_oracle(gpu, m, n, k, xmode, emode, use_ws):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(m * 13 + n + k + emode)
    q0 = QuantizedLinear.random(n, k, 64, generator=g)
    q1 = QuantizedLinear.random(n, k, 64, generator=g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
    nb = _lib.query("mtp_qmv_workspace_bytes", m, n, k, 1)
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")

    def run(layout):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        kw = dict(x=x, M=m, N=n, K=k, group_size=64, xmode=xmode, emode=emode, packed=layout, y0=y,
                  w0=q0.pack(layout=layout))
        if xmode == 2:
            kw.update(x2=nw, eps=1e-6)
        if emode == 1:
            kw.update(resid=r, ss_out=torch.zeros(n, dtype=torch.float32, device="cuda"))
        if emode == 3:
            kw.update(w1=q1.pack(layout=layout))
        if use_ws:
            kw.update(ws=ws, ws_bytes=ws.numel())
        _lib.qmv_ex(_st(), **kw)
        torch.cuda.synchronize()
        return bf16_values(y)

    a, b = run(2), run(1)
    assert not np.isnan(a).any(), "unwritten outputs"
    tol = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + 1e-4 * np.abs(b).max()
    assert (np.abs(a - b) <= tol).all(), f"layout 2 vs 1: max diff {np.abs(a - b).max()}"
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
        assert_close(a, want, what=f"layout 2 M={m} N={n} K={k} x{xmode} e{emode}")


@pytest.mark.parametrize("B", [1, 4])
def test_layout2_rope_epilogue_and_limits(gpu, B):
    """The RoPE epilogue on layout 2 equals the layout-2 q|k|v matmul plus the
    RoPE writer, bit for bit, at 4 rows and at 16 (4 requests); M > 16 is
    refused."""
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear, rope_row_order
    L, Hq, Hkv, D, K, cap = 4, 8, 2, 128, 1024, 256
    M, N = B * L, (Hq + 2 * Hkv) * D
    g = torch.Generator(device="cuda").manual_seed(3)
    q = QuantizedLinear.random(N, K, 64, generator=g)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(K, device="cuda", generator=g)).to(torch.bfloat16)
    qs = torch.tensor([100 + 7 * b for b in range(B)], dtype=torch.int32, device="cuda")

    def bufs():
        return (torch.zeros((B, Hq, L, D), dtype=torch.bfloat16, device="cuda"),
                torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device="cuda"),
                torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device="cuda"),
                torch.zeros(B, dtype=torch.int32, device="cuda"))
    qo0, kc0, vc0, st0 = bufs()
    qkv = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    _lib.qmv_ex(_st(), x=x, x2=nw, eps=1e-6, w0=q.pack(layout=2), y0=qkv, M=M, N=N, K=K, group_size=64, xmode=2,
                emode=0, packed=2)
    _lib.call("mtp_rope_qkv_to_cache_vt", qkv.data_ptr(), qs.data_ptr(), None, qo0.data_ptr(), kc0.data_ptr(),
              vc0.data_ptr(), B, L, Hq, Hkv, D, cap, 1e6, st0.data_ptr(), _st())
    qo1, kc1, vc1, st1 = bufs()
    rope = dict(q_start=qs, q_out=qo1, k_cache=kc1, v_cache=vc1, status=st1, L=L, Hq=Hq, Hkv=Hkv, D=D, cap=cap,
                blocked=1, rope_base=1e6)
    _lib.qmv_ex(_st(), rope=rope, x=x, x2=nw, eps=1e-6, w0=q.pack(rope_row_order(Hq + 2 * Hkv, D), layout=2), M=M,
                N=N, K=K, group_size=64, xmode=2, emode=4, packed=2)
    torch.cuda.synchronize()
    assert torch.equal(qo0.view(torch.int16), qo1.view(torch.int16))
    assert torch.equal(kc0.view(torch.int16), kc1.view(torch.int16))
    assert torch.equal(vc0.view(torch.int16), vc1.view(torch.int16))
    x17 = torch.zeros((17, K), dtype=torch.bfloat16, device="cuda")
    y17 = torch.empty((17, N), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.MtpError) as e:
        _lib.qmv_ex(_st(), x=x17, w0=q.pack(layout=2), y0=y17, M=17, N=N, K=K, group_size=64, packed=2)
    assert e.value.code == -2
