"""GPU parity: the q|k|v matmul with the RoPE epilogue (emode 4) against the
unfused pair (q|k|v matmul, then mtp_rope_qkv_to_cache / _vt) - bit-exact on
q, the K and V caches and the status flag. The weights are packed in RoPE tile
order for the fused call and in natural order for the unfused one, so the test
also pins the row order of ``rope_row_order``. The unfused pair itself is held
to the oracle by tests/test_gpu_qmv.py and tests/test_gpu_attention.py."""

import numpy as np
import pytest
import torch

from mtplx_amd import _lib
from mtplx_amd.quant import QuantizedLinear, rope_row_order
from tests.gpu_util import randn_bf16


def _st():
    return torch.cuda.current_stream().cuda_stream


CASES = [  # B, L, Hq, Hkv, D, K, xmode, blocked, cap, starts, lens
    (1, 4, 40, 8, 128, 5120, 2, 1, 4096, [4000], None),     # the verify step's shape
    (2, 4, 8, 2, 128, 512, 2, 1, 256, [254, 30], [4, 2]),   # ragged rows, two past the cache end
    (2, 3, 4, 1, 128, 256, 0, 0, 256, [7, 0], None),
    (1, 6, 6, 2, 64, 768, 2, 0, 256, [100], [5]),           # D = 64
    (8, 1, 4, 2, 128, 1024, 0, 1, 256, [0, 1, 2, 31, 32, 63, 200, 255], None),
    (4, 4, 32, 4, 128, 4096, 2, 1, 8192, [8000, 100, 5000, 3], None),   # 16 rows: the cfg5 step's shape
    (2, 8, 8, 2, 128, 512, 2, 1, 256, [200, 10], [8, 5]),              # 16 rows, ragged
]


@pytest.mark.gpu
def test_rope_fusable_query(gpu):
    """The fused form takes up to 16 rows with all of x in LDS: the cfg5
    width (K = 4096) at 16 rows, not the 27B width (K = 5120)."""
    from mtplx_amd import _lib
    assert _lib.query("mtp_qmv_rope_fusable", 4, 7168, 5120) == 1
    assert _lib.query("mtp_qmv_rope_fusable", 16, 5120, 4096) == 1
    assert _lib.query("mtp_qmv_rope_fusable", 16, 7168, 5120) == 0
    assert _lib.query("mtp_qmv_rope_fusable", 17, 5120, 4096) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("B,L,Hq,Hkv,D,K,xmode,blocked,cap,starts,lens", CASES)
def test_rope_epilogue_matches_unfused(gpu, B, L, Hq, Hkv, D, K, xmode, blocked, cap, starts, lens):
    rng = np.random.default_rng(B * 1000 + L * 100 + D + K)
    g = torch.Generator(device="cuda").manual_seed(K + D)
    M, N = B * L, (Hq + 2 * Hkv) * D
    q = QuantizedLinear.random(N, K, 64, generator=g)
    x = randn_bf16(rng, (M, K))
    nw = (1 + 0.1 * torch.randn(K, device="cuda", generator=g)).to(torch.bfloat16)
    qs = torch.tensor(starts, dtype=torch.int32, device="cuda")
    ql = None if lens is None else torch.tensor(lens, dtype=torch.int32, device="cuda")
    common = dict(x=x, x2=nw if xmode == 2 else None, eps=1e-6, M=M, N=N, K=K, group_size=64, xmode=xmode,
                  packed=1)

    def caches():
        return (torch.full((B, Hq, L, D), float("nan"), dtype=torch.bfloat16, device="cuda"),
                torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device="cuda"),
                torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device="cuda"),
                torch.zeros(1, dtype=torch.int32, device="cuda"))

    # unfused: natural-order packed weights, stored q|k|v rows, then the RoPE writer
    qo0, kc0, vc0, st0 = caches()
    qkv = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    _lib.qmv_ex(_st(), w0=q.pack(), y0=qkv, emode=0, **common)
    fn = "mtp_rope_qkv_to_cache_vt" if blocked else "mtp_rope_qkv_to_cache"
    _lib.call(fn, qkv.data_ptr(), qs.data_ptr(), _lib.ptr(ql), qo0.data_ptr(), kc0.data_ptr(), vc0.data_ptr(), B, L,
              Hq, Hkv, D, cap, 1e6, st0.data_ptr(), _st())

    # fused: RoPE-order packed weights, emode 4
    qo1, kc1, vc1, st1 = caches()
    rope = dict(q_start=qs, q_lens=ql, q_out=qo1, k_cache=kc1, v_cache=vc1, status=st1, L=L, Hq=Hq, Hkv=Hkv, D=D,
                cap=cap, blocked=blocked, rope_base=1e6)
    _lib.qmv_ex(_st(), rope=rope, w0=q.pack(rope_row_order(Hq + 2 * Hkv, D)), emode=4, **common)
    torch.cuda.synchronize()

    assert torch.equal(qo0.view(torch.int16), qo1.view(torch.int16)), "q differs"
    assert torch.equal(kc0.view(torch.int16), kc1.view(torch.int16)), "K cache differs"
    assert torch.equal(vc0.view(torch.int16), vc1.view(torch.int16)), "V cache differs"
    assert int(st0.item()) == int(st1.item())
    past_end = any(s + (L if lens is None else n) > cap for s, n in zip(starts, lens or starts))
    assert int(st1.item()) == (1 if past_end else 0)
    assert int(kc1.view(torch.int16).abs().sum().item()) > 0   # something was written


def test_rope_row_order_pairs():
    """Each packed 32-row tile holds 16 rotate-half pairs (d, d + D/2) of one head."""
    for D in (64, 128):
        order = rope_row_order(3, D).numpy()
        assert sorted(order.tolist()) == list(range(3 * D))
        t = order.reshape(-1, 32)
        assert (t[:, 16:] - t[:, :16] == D // 2).all()
        assert (t // D == t[:, :1] // D).all()


@pytest.mark.gpu
def test_rope_epilogue_rejects_bad_shapes(gpu):
    q = QuantizedLinear.random(12 * 128, 256, 64)
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    o = torch.zeros((1, 8, 4, 128), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((1, 2, 256, 128), dtype=torch.bfloat16, device="cuda")
    qs = torch.zeros(1, dtype=torch.int32, device="cuda")
    rope = dict(q_start=qs, q_out=o, k_cache=kc, v_cache=kc, L=4, Hq=9, Hkv=2, D=128, cap=256, blocked=1,
                rope_base=1e6)   # (9 + 4) * 128 != N
    with pytest.raises(_lib.MtpError) as e:
        _lib.qmv_ex(_st(), rope=rope, x=x, w0=q.pack(), M=4, N=12 * 128, K=256, group_size=64, emode=4, packed=1)
    assert e.value.code == -1
