"""GPU parity of the general affine matmul (``mtp_qmv_affine``: 4- or 8-bit,
groups 32/64/128) and of the call surfaces that route to it: the 8-bit verify
lane (``stocklike_qmv8_matmul``), the qmv4 core (``qmv4_matmul``) and the
cross-row lane (``make_chunk_sums``, ``crossrow_qmm``).

Bars: bf16 outputs within rtol/atol 1e-2 of the float64 oracle
(``oracle.qmv.qmm_affine``); fp32 outputs hold the bf16-rounded values; the
4-bit group-64 result within one bf16 ulp (plus 1e-4 of the row scale where
a sum cancels) of the MFMA kernel's; the chunk-sum table bit-exact against
fp32 sums in index order; eligibility truth tables as the reference's."""

import numpy as np
import pytest
import torch

from oracle.bf16 import round_to_bf16
from oracle.qmv import make_affine_weights, qmm_affine
from tests.gpu_util import assert_close, bf16_values, bits, randn_bf16, u32

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _layer(rng, n, k, gs, b):
    from mtplx_amd.quant import QuantizedLinear
    from tests.gpu_util import from_bits
    w, s, bb = make_affine_weights(rng, n, k, gs, b)
    return QuantizedLinear(u32(w), from_bits(s), from_bits(bb), group_size=gs, bits=b), (w, s, bb)


CASES = [  # bits, gs, m, n, k
    (8, 64, 4, 1000, 5120),
    (8, 32, 1, 512, 512),
    (8, 128, 11, 333, 1024),     # two launches of rows, N not a multiple of 64
    (4, 32, 4, 2048, 5120),
    (4, 32, 6, 96, 96),          # K not a multiple of the 512-k chunk
    (4, 128, 8, 640, 2048),
    (8, 32, 3, 64, 17408),
]


@pytest.mark.parametrize("b,gs,m,n,k", CASES)
def test_general_matmul_matches_oracle(gpu, b, gs, m, n, k):
    from mtplx_amd import _lib
    rng = np.random.default_rng(b * 1000 + gs + m + n + k)
    q, (w, s, bb) = _layer(rng, n, k, gs, b)
    x = randn_bf16(rng, (m, k))
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_qmv_affine", x.data_ptr(), q.weight.data_ptr(), q.scales.data_ptr(), q.biases.data_ptr(),
              y.data_ptr(), None, m, n, k, gs, b, _st())
    torch.cuda.synchronize()
    want = round_to_bf16(qmm_affine(bits(x), w, s, bb, gs, b))
    assert_close(bf16_values(y), want, what=f"{b}-bit g{gs} m={m} n={n} k={k}")
    # fp32 output holds the same bf16-rounded values
    yf = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    _lib.call("mtp_qmv_affine", x.data_ptr(), q.weight.data_ptr(), q.scales.data_ptr(), q.biases.data_ptr(), None,
              yf.data_ptr(), m, n, k, gs, b, _st())
    torch.cuda.synchronize()
    assert torch.equal(yf, y.float())
    # the module call routes here for the packs the MFMA kernel does not take
    from mtplx_amd.verify_kernels import fast_path
    y2 = q(x)
    torch.cuda.synchronize()
    if fast_path(b, gs, k):
        assert_close(bf16_values(y2), want, what="module call (MFMA kernel)")
    else:
        assert torch.equal(y2, y)


def test_general_4bit_within_one_ulp_of_mfma_kernel(gpu):
    from mtplx_amd import _lib
    rng = np.random.default_rng(7)
    m, n, k = 4, 4096, 5120
    q, _ = _layer(rng, n, k, 64, 4)
    x = randn_bf16(rng, (m, k))
    a = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_qmv_affine", x.data_ptr(), q.weight.data_ptr(), q.scales.data_ptr(), q.biases.data_ptr(),
              a.data_ptr(), None, m, n, k, 64, 4, _st())
    b = q(x)
    torch.cuda.synchronize()
    av, bv = bf16_values(a), bf16_values(b)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(bv), 1e-30))) - 7)
    assert (np.abs(av - bv) <= ulp + 1e-4 * np.abs(bv).max(axis=1, keepdims=True)).all()


def test_general_matmul_rejects_unsupported(gpu):
    from mtplx_amd import _lib
    x = torch.zeros((2, 512), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((64, 512 * 2 // 32), dtype=torch.int32, device="cuda")
    s = torch.zeros((64, 16), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((2, 64), dtype=torch.bfloat16, device="cuda")
    for bits_, gs, code in ((2, 32, -2), (4, 16, -2), (8, 96, -2)):
        with pytest.raises(_lib.MtpError) as e:
            _lib.call("mtp_qmv_affine", x.data_ptr(), w.data_ptr(), s.data_ptr(), s.data_ptr(), y.data_ptr(), None,
                      2, 64, 512, gs, bits_, _st())
        assert e.value.code == code
    with pytest.raises(_lib.MtpError):
        _lib.call("mtp_qmv_affine", x.data_ptr(), w.data_ptr(), s.data_ptr(), s.data_ptr(), y.data_ptr(), None,
                  2, 64, 500, 32, 8, _st())


def test_stocklike_qmv8_lane(gpu):
    from mtplx_amd.verify_qmv import is_stocklike_qmv8_eligible, stocklike_qmv8_matmul
    rng = np.random.default_rng(8)
    q8, (w, s, bb) = _layer(rng, 1024, 2048, 64, 8)
    q4, _ = _layer(rng, 64, 512, 64, 4)
    q8odd, _ = _layer(rng, 1020, 512, 32, 8)       # N % 8 != 0
    assert is_stocklike_qmv8_eligible(q8) and not is_stocklike_qmv8_eligible(q4)
    assert not is_stocklike_qmv8_eligible(q8odd) and not is_stocklike_qmv8_eligible(object())
    x = randn_bf16(rng, (1, 3, 2048))
    y = stocklike_qmv8_matmul(x, q8)
    torch.cuda.synchronize()
    assert y.shape == (1, 3, 1024)
    want = round_to_bf16(qmm_affine(bits(x.reshape(3, 2048)), w, s, bb, 64, 8))
    assert_close(bf16_values(y.reshape(3, 1024)), want, what="stocklike qmv8")
    # batched leading dims take module(x), same values
    xb = randn_bf16(rng, (2, 3, 2048))
    yb = stocklike_qmv8_matmul(xb, q8)
    torch.cuda.synchronize()
    want_b = round_to_bf16(qmm_affine(bits(xb.reshape(6, 2048)), w, s, bb, 64, 8))
    assert_close(bf16_values(yb.reshape(6, 1024)), want_b, what="stocklike qmv8 fallback")


def test_qmv4_core_surface(gpu):
    from mtplx_amd.qmv4_matmul import qmv4_eligible, qmv4_matmul
    rng = np.random.default_rng(9)
    for gs in (32, 64, 128):
        q, (w, s, bb) = _layer(rng, 768, 1024, gs, 4)
        for m in (1, 6, 7):
            x = randn_bf16(rng, (m, 1024))
            assert qmv4_eligible(x, q) == (m <= 6)
            y = qmv4_matmul(x, q)
            torch.cuda.synchronize()
            want = round_to_bf16(qmm_affine(bits(x), w, s, bb, gs, 4))
            assert_close(bf16_values(y), want, what=f"qmv4 g{gs} m={m}")
    q8, _ = _layer(rng, 64, 512, 64, 8)
    assert not qmv4_eligible(randn_bf16(rng, (2, 512)), q8)
    q, _ = _layer(rng, 64, 768, 64, 4)
    assert not qmv4_eligible(randn_bf16(rng, (2, 768)), q)   # K % 512 != 0


def test_crossrow_surface(gpu):
    from mtplx_amd.verify_crossrow import crossrow_eligible, crossrow_qmm, make_chunk_sums
    assert crossrow_eligible(4, 5120, 17408, 4, 64, torch.bfloat16)
    assert crossrow_eligible(2, 512, 8, 4, 32, torch.bfloat16)
    assert not crossrow_eligible(1, 5120, 17408, 4, 64, torch.bfloat16)
    assert not crossrow_eligible(6, 5120, 17408, 4, 64, torch.bfloat16)
    assert not crossrow_eligible(4, 5120, 17408, 4, 128, torch.bfloat16)
    assert not crossrow_eligible(4, 5000, 17408, 4, 64, torch.bfloat16)
    assert not crossrow_eligible(4, 5120, 17404, 4, 64, torch.bfloat16)
    assert not crossrow_eligible(4, 5120, 17408, 8, 64, torch.bfloat16)
    rng = np.random.default_rng(10)
    m, n, k = 4, 1024, 5120
    x = randn_bf16(rng, (m, k))
    t = make_chunk_sums(x)
    torch.cuda.synchronize()
    # fp32 sums of each lane's 16 values, in index order
    xv = bf16_values(x).astype(np.float32).reshape(m, k // 16, 16)
    want = np.zeros((k // 16, 8), np.float32)
    acc = np.zeros((m, k // 16), np.float32)
    for i in range(16):
        acc = (acc + xv[:, :, i]).astype(np.float32)
    want[:, :m] = acc.T
    assert np.array_equal(t.cpu().numpy(), want.reshape(-1))
    for gs in (32, 64):
        q, (w, s, bb) = _layer(rng, n, k, gs, 4)
        y0 = crossrow_qmm(x, q.weight, q.scales, q.biases, group_size=gs)
        y1 = crossrow_qmm(x, q.weight, q.scales, q.biases, group_size=gs, xsums=t)
        # the table is what the bias term reads: an all-zero table drops it
        y2 = crossrow_qmm(x, q.weight, q.scales, q.biases, group_size=gs, xsums=torch.zeros_like(t))
        torch.cuda.synchronize()
        want_y = round_to_bf16(qmm_affine(bits(x), w, s, bb, gs, 4))
        assert_close(bf16_values(y0), want_y, what=f"crossrow g{gs}")
        assert_close(bf16_values(y1), want_y, what=f"crossrow g{gs} with the chunk-sum table")
        want_nb = round_to_bf16(qmm_affine(bits(x), w, s, np.zeros_like(bb), gs, 4))
        assert_close(bf16_values(y2), want_nb, what=f"crossrow g{gs} with a zero table")
    with pytest.raises(ValueError):
        crossrow_qmm(x, q.weight, q.scales, q.biases, group_size=64, xsums=t[:-8])
