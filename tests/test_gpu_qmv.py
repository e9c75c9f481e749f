"""GPU parity: 4-bit affine verify matmul (all entry points) vs the float64 oracle.

Bar (north star): bf16 outputs within rtol 1e-2 / atol 1e-2 of the oracle.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_to_bf16
from oracle.moe import silu
from oracle.qmv import make_affine4_weights, qmm_affine4
from tests.gpu_util import assert_close, bf16_values, bits, from_bits, randn_bf16, u32

pytestmark = pytest.mark.gpu


def _layer(rng, n, k, gs=64):
    w, s, b = make_affine4_weights(rng, n, k, gs)
    return (w, s, b), (u32(w), from_bits(s), from_bits(b))


def _ws(lib, m, n, k, dual=0):
    nb = lib.mtp_qmv_workspace_bytes(m, n, k, dual)
    return torch.zeros(max(nb, 256), dtype=torch.uint8, device="cuda"), nb


def _stream():
    return torch.cuda.current_stream().cuda_stream


def test_mfma_32x32x16_output_layout(gpu):
    out = torch.zeros(64 * 16, dtype=torch.float32, device="cuda")
    from mtplx_amd import _lib
    _lib.call("mtp_probe_mfma_layout", out.data_ptr(), _stream())
    got = out.cpu().numpy().reshape(64, 16)
    for lane in range(64):
        for r in range(16):
            i = 8 * (r // 4) + 4 * (lane // 32) + r % 4
            j = lane % 32
            want = float(i + 1) if i % 16 == j % 16 else 0.0
            assert got[lane, r] == want, (lane, r, got[lane, r], want)


SHAPES = [  # (M, N, K, gs)
    (4, 17408, 5120, 64),     # BASELINE cfg1
    (1, 1032, 2560, 64), (2, 2560, 6144, 64), (4, 1032, 2560, 128),
    (6, 136, 1024, 64), (8, 256, 768, 128), (3, 100, 768, 64),
    (16, 512, 1024, 64), (24, 300, 1280, 64), (32, 1024, 2048, 128), (5, 7168, 5120, 64),
]


@pytest.mark.parametrize("m,n,k,gs", SHAPES)
def test_qmv_matches_oracle(gpu, m, n, k, gs):
    from mtplx_amd import _lib
    rng = np.random.default_rng(1000 + m * 7 + n)
    (w, s, b), (tw, ts, tb) = _layer(rng, n, k, gs)
    x = randn_bf16(rng, (m, k))
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")   # poisoned
    ws, nb = _ws(lib=_lib.load(), m=m, n=n, k=k)
    _lib.call("mtp_qmv_affine4", x.data_ptr(), tw.data_ptr(), ts.data_ptr(), tb.data_ptr(), y.data_ptr(),
              m, n, k, gs, ws.data_ptr(), nb, _stream())
    torch.cuda.synchronize()
    want = qmm_affine4(bits(x), w, s, b, gs)
    got = bf16_values(y)
    assert np.isfinite(got).all(), "unwritten (NaN-poisoned) outputs"
    assert_close(got, want, what=f"qmv M={m} N={n} K={k}")
    rel = np.abs(got - want).max() / (np.abs(want).max() + 1e-9)
    assert rel < 4e-3, rel
    # deterministic: a second launch is bitwise identical
    y2 = torch.empty_like(y)
    _lib.call("mtp_qmv_affine4", x.data_ptr(), tw.data_ptr(), ts.data_ptr(), tb.data_ptr(), y2.data_ptr(),
              m, n, k, gs, ws.data_ptr(), nb, _stream())
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_qmv_closed_form_zero_nibbles(gpu):
    from mtplx_amd import _lib
    rng = np.random.default_rng(5)
    m, n, k = 4, 256, 1024
    w = np.zeros((n, k // 8), np.uint32)
    s = f32_to_bf16_bits(np.abs(rng.normal(0, 0.02, (n, k // 64))).astype(np.float32))
    b = f32_to_bf16_bits(rng.normal(0, 0.01, (n, k // 64)).astype(np.float32))
    x = randn_bf16(rng, (m, k))
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    ws, nb = _ws(_lib.load(), m, n, k)
    tw, ts, tb = u32(w), from_bits(s), from_bits(b)   # keep the buffers alive across the launch
    _lib.call("mtp_qmv_affine4", x.data_ptr(), tw.data_ptr(), ts.data_ptr(), tb.data_ptr(),
              y.data_ptr(), m, n, k, 64, ws.data_ptr(), nb, _stream())
    xv = bf16_values(x)
    want = xv.reshape(m, -1, 64).sum(axis=2) @ bf16_bits_to_f32(b).astype(np.float64).T
    assert_close(bf16_values(y), want, what="q=0 closed form")


def test_residual_dual_swiglu_and_rmsnorm_variants(gpu):
    from mtplx_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(11)
    m, n, k = 4, 1536, 2048
    (w0, s0, b0), (tw0, ts0, tb0) = _layer(rng, n, k)
    (w1, s1, b1), (tw1, ts1, tb1) = _layer(rng, n, k)
    x = randn_bf16(rng, (m, k))
    xb = bits(x)
    st = _stream()
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device="cuda")
    W = ws.numel()
    y0 = qmm_affine4(xb, w0, s0, b0, 64)
    y1 = qmm_affine4(xb, w1, s1, b1, 64)

    # residual
    r = randn_bf16(rng, (m, n))
    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    ss = torch.full(((n // 32 + 1) * 32,), float("nan"), dtype=torch.float32, device="cuda")
    _lib.call("mtp_qmv_affine4_residual", x.data_ptr(), tw0.data_ptr(), ts0.data_ptr(), tb0.data_ptr(), r.data_ptr(),
              out.data_ptr(), ss.data_ptr(), m, n, k, 64, ws.data_ptr(), W, st)
    assert_close(bf16_values(out), round_to_bf16(y0) + bf16_values(r), what="residual")
    ov = bf16_values(out)
    ssn = ss.cpu().numpy()[: (n // 32) * 32].reshape(n // 32, 32)[:, :m]
    assert np.allclose(ssn.sum(axis=0), (ov ** 2).sum(axis=1), rtol=1e-4), "row sums of squares"
    assert np.allclose(ssn, (ov ** 2).reshape(m, n // 32, 32).sum(axis=2).T, rtol=1e-4), "per-block sums"

    # dual (two outputs) and dual swiglu
    o0 = torch.empty((m, n), dtype=torch.bfloat16, device="cuda"); o1 = torch.empty_like(o0)
    _lib.call("mtp_qmv_affine4_dual", x.data_ptr(), tw0.data_ptr(), ts0.data_ptr(), tb0.data_ptr(), tw1.data_ptr(),
              ts1.data_ptr(), tb1.data_ptr(), o0.data_ptr(), o1.data_ptr(), m, n, k, 64, 0, ws.data_ptr(), W, st)
    assert_close(bf16_values(o0), y0, what="dual y0")
    assert_close(bf16_values(o1), y1, what="dual y1")
    h = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_qmv_affine4_dual", x.data_ptr(), tw0.data_ptr(), ts0.data_ptr(), tb0.data_ptr(), tw1.data_ptr(),
              ts1.data_ptr(), tb1.data_ptr(), h.data_ptr(), None, m, n, k, 64, 1, ws.data_ptr(), W, st)
    assert_close(bf16_values(h), silu(y0) * y1, what="dual swiglu")

    # swiglu input -> down projection (+ residual)
    (wd, sd, bd), (twd, tsd, tbd) = _layer(rng, k, n)
    g = randn_bf16(rng, (m, n)); u = randn_bf16(rng, (m, n))
    act = round_to_bf16(round_to_bf16(silu(bf16_values(g))) * bf16_values(u))
    want = qmm_affine4(f32_to_bf16_bits(act.astype(np.float32)), wd, sd, bd, 64)
    yd = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_qmv_affine4_swiglu_in", g.data_ptr(), u.data_ptr(), twd.data_ptr(), tsd.data_ptr(), tbd.data_ptr(),
              None, yd.data_ptr(), m, k, n, 64, ws.data_ptr(), W, st)
    assert_close(bf16_values(yd), want, what="swiglu-in")

    # rmsnorm input (bf16 and fp32 outputs) and rmsnorm + dual swiglu
    nw = randn_bf16(rng, (k,), 0.1)
    xv = bf16_values(x)
    xn = xv / np.sqrt((xv ** 2).mean(axis=1, keepdims=True) + 1e-6) * bf16_values(nw)[None]
    xnb = f32_to_bf16_bits(xn.astype(np.float32))
    yn = qmm_affine4(xnb, w0, s0, b0, 64)
    o = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_qmv_affine4_rmsnorm_in", x.data_ptr(), nw.data_ptr(), None, ctypes.c_float(1e-6), tw0.data_ptr(),
              ts0.data_ptr(), tb0.data_ptr(), o.data_ptr(), m, n, k, 64, ws.data_ptr(), W, st)
    assert_close(bf16_values(o), yn, what="rmsnorm-in")
    of = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _lib.call("mtp_qmv_affine4_rmsnorm_f32", x.data_ptr(), nw.data_ptr(), None, ctypes.c_float(1e-6), tw0.data_ptr(),
              ts0.data_ptr(), tb0.data_ptr(), of.data_ptr(), m, n, k, 64, ws.data_ptr(), W, st)
    ofn = of.cpu().numpy().astype(np.float64)
    assert_close(ofn, yn, what="rmsnorm-f32")
    assert np.array_equal(round_to_bf16(ofn), ofn), "fp32 logits must carry bf16 values"
    hd = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_qmv_affine4_rmsnorm_dual", x.data_ptr(), nw.data_ptr(), None, ctypes.c_float(1e-6), tw0.data_ptr(),
              ts0.data_ptr(), tb0.data_ptr(), tw1.data_ptr(), ts1.data_ptr(), tb1.data_ptr(), hd.data_ptr(),
              m, n, k, 64, ws.data_ptr(), W, st)
    yn1 = qmm_affine4(xnb, w1, s1, b1, 64)
    assert_close(bf16_values(hd), silu(yn) * yn1, what="rmsnorm-dual-swiglu")

    # statistics handed over from a residual producer give the same result
    ssx = torch.empty((k // 32) * 32, dtype=torch.float32, device="cuda")
    xsq = (xv ** 2).reshape(m, k // 32, 32).sum(axis=2).T                     # [k/32, m]
    ssx_np = np.zeros((k // 32, 32), np.float32); ssx_np[:, :m] = xsq
    ssx.copy_(torch.from_numpy(ssx_np.reshape(-1)))
    o2 = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_qmv_affine4_rmsnorm_in", x.data_ptr(), nw.data_ptr(), ssx.data_ptr(), ctypes.c_float(1e-6),
              tw0.data_ptr(), ts0.data_ptr(), tb0.data_ptr(), o2.data_ptr(), m, n, k, 64, ws.data_ptr(), W, st)
    assert_close(bf16_values(o2), yn, what="rmsnorm-in with handed-over statistics")


def test_bad_arguments_raise(gpu):
    from mtplx_amd import _lib
    x = torch.zeros((4, 100), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.MtpError):
        _lib.call("mtp_qmv_affine4", x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(),
                  4, 8, 100, 64, None, 0, _stream())
    with pytest.raises(_lib.MtpError):   # group size 32 is not on the GPU path
        _lib.call("mtp_qmv_affine4", x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(),
                  4, 8, 256, 32, None, 0, _stream())


def _nibbles_natural(words):
    """Nibble k of each word moved to position (k >> 1) + 4 (k & 1)."""
    words = np.asarray(words, dtype=np.uint32)
    out = np.zeros_like(words)
    for k in range(8):
        pos = (k >> 1) + 4 * (k & 1)
        out |= ((words >> np.uint32(4 * k)) & np.uint32(0xF)) << np.uint32(4 * pos)
    return out


def _pack_reference(w, s, b, gs):
    """NumPy restatement of the tile-major layout (include/mtplx_amd.h)."""
    N, kw = w.shape
    K = kw * 8
    Q = K // 256
    T = -(-N // 32)
    out = np.zeros((T, Q, 1152), np.uint32)
    sb = s.view(np.uint16); bb = b.view(np.uint16)
    for nb in range(T):
        for q in range(Q):
            for u in range(4):
                for l in range(64):
                    row = nb * 32 + (l & 31)
                    if row < N:
                        out[nb, q, 256 * u + 4 * l: 256 * u + 4 * l + 4] = \
                            _nibbles_natural(w[row, 32 * q + 8 * u + 4 * (l >> 5):][:4])
            for c in range(32):
                row = nb * 32 + c
                if row < N:
                    e = [sb[row, (4 * q + g) * 64 // gs] for g in range(4)] + [bb[row, (4 * q + g) * 64 // gs] for g in range(4)]
                    e = np.array(e, np.uint16).view(np.uint32)
                    out[nb, q, 1024 + 4 * c: 1024 + 4 * c + 4] = e
    return out.reshape(-1)


@pytest.mark.parametrize("n,k,gs", [(70, 512, 64), (64, 768, 128)])
def test_pack_layout_bit_exact(gpu, n, k, gs):
    from mtplx_amd.quant import QuantizedLinear
    rng = np.random.default_rng(n + k)
    w, s, b = make_affine4_weights(rng, n, k, gs)
    q = QuantizedLinear(u32(w), from_bits(s), from_bits(b), group_size=gs)
    got = q.pack().cpu().numpy().view(np.uint32)
    assert np.array_equal(got, _pack_reference(w, s, b, gs))


@pytest.mark.parametrize("m,n,k,gs,xmode,emode", [
    (4, 17408, 5120, 64, 0, 0), (4, 7168, 5120, 64, 2, 0), (4, 5120, 17408, 64, 0, 1),
    (4, 1536, 2048, 64, 2, 3), (4, 300, 1024, 128, 0, 0), (8, 600, 1024, 64, 2, 3), (16, 256, 512, 64, 0, 1),
    (4, 151936 // 8, 5120, 64, 2, 0), (16, 512, 1024, 64, 0, 2), (12, 640, 1024, 64, 1, 0), (3, 640, 1024, 64, 1, 2)])
def test_packed_path_matches_unpacked(gpu, m, n, k, gs, xmode, emode):
    """The tile-major paths (layout 1, and layout 2 up to 16 rows) compute the
    same sums as the reference-layout path with the k of each MFMA operand in
    another order, so outputs agree to one bf16 ulp (and both meet the oracle
    bar); xmode 1 (silu(x) * x2) and emode 2 (two outputs) included."""
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(m * 1000 + n)
    q0 = QuantizedLinear.random(n, k, gs, generator=g)
    q1 = QuantizedLinear.random(n, k, gs, generator=g)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
    up = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    r = torch.randn((m, n), device="cuda", generator=g).to(torch.bfloat16)
    st = _stream()
    outs = []
    layouts = (0, 1, 2) if m <= 16 else (0, 1)
    for packed in layouts:
        y0 = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        y1 = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        ss = torch.zeros(((n + 31) // 32) * 32, dtype=torch.float32, device="cuda")
        kw = dict(x=x, x2=nw if xmode == 2 else (up if xmode == 1 else None), eps=1e-6, M=m, N=n, K=k,
                  group_size=gs, xmode=xmode,
                  emode=emode, packed=packed, y0=y0, y1=y1 if emode == 2 else None,
                  resid=r if emode == 1 else None, ss_out=ss if emode == 1 else None)
        if packed:
            kw.update(w0=q0.pack(layout=packed), w1=q1.pack(layout=packed) if emode >= 2 else None)
        else:
            kw.update(w0=q0.weight, s0=q0.scales, b0=q0.biases, w1=q1.weight if emode >= 2 else None,
                      s1=q1.scales if emode >= 2 else None, b1=q1.biases if emode >= 2 else None)
        _lib.qmv_ex(st, **kw)
        torch.cuda.synchronize()
        outs.append((y0.clone(), ss.clone(), y1.clone()))
    for i in range(1, len(layouts)):
        for j in ((0, 2) if emode == 2 else (0,)):
            a, b = bf16_values(outs[i][j]), bf16_values(outs[0][j])
            tol = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + 1e-4 * np.abs(b).max()
            assert (np.abs(a - b) <= tol).all(), (layouts[i], j, np.abs(a - b).max())
        if emode == 1:
            assert torch.allclose(outs[0][1], outs[i][1], rtol=1e-3, atol=1e-3)
        assert not torch.isnan(outs[i][0].float()).any()
    if xmode == 0 and emode == 0 and n * k <= 4_000_000:
        want = qmm_affine4(bits(x), *(t.cpu().numpy().view(np.uint32) if i == 0 else bits(t)
                                       for i, t in enumerate((q0.weight, q0.scales, q0.biases))), gs)
        assert_close(bf16_values(outs[1][0]), want, what="packed vs oracle")
