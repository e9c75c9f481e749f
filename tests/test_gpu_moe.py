"""GPU parity: expert sort (bit-exact), routing, gathered quantized matmul and
the sorted SwiGLU chain vs the oracle."""

import numpy as np
import pytest
import torch

from oracle import moe as OM
from oracle.model import route_topk
from oracle.qmv import make_affine4_weights
from tests.gpu_util import assert_close, bf16_values, bits, from_bits, randn_bf16, u32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,k,E", [(16, 8, 256), (4, 2, 8), (64, 8, 128), (1, 1, 4), (200, 10, 300),
                                    (1024, 8, 4096), (333, 2, 2)])
def test_expert_sort_bit_exact(gpu, T, k, E):
    from mtplx_amd.moe_sorted_gather import expert_sort
    rng = np.random.default_rng(T * k + E)
    # Zipf-skewed picks, distinct per token
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    es = expert_sort(torch.from_numpy(idx).cuda(), E)
    torch.cuda.synchronize()
    row_map, sorted_ids, inv, order = OM.sort_rows(idx)
    assert es.row_map.cpu().numpy().astype(np.uint32).tolist() == row_map.tolist()
    assert es.sorted_ids.cpu().numpy().tolist() == sorted_ids.astype(np.int64).tolist()
    assert es.inv_order.cpu().numpy().tolist() == inv.astype(np.int64).tolist()
    assert es.expert_off.cpu().numpy().tolist() == OM.expert_offsets(sorted_ids, E).tolist()
    act = es.active.cpu().numpy()
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert act[0] == (counts > 0).sum() and act[1:1 + act[0]].tolist() == np.nonzero(counts)[0].tolist()


def test_bad_expert_id_flagged(gpu):
    from mtplx_amd.moe_sorted_gather import expert_sort
    es = expert_sort(torch.tensor([[0, 9]], dtype=torch.int32, device="cuda"), 8)
    assert int(es.active[0]) == -1


def test_route_matches_oracle(gpu):
    from mtplx_amd.moe_sorted_gather import route
    rng = np.random.default_rng(2)
    lg = rng.normal(size=(16, 256)).astype(np.float32)
    lg[3, 7] = lg[3, 9] = 40.0
    ids, w = route(torch.from_numpy(lg).cuda(), 8)
    wi, ww = route_topk(lg, 8)
    assert ids.cpu().numpy().tolist() == wi.tolist()
    assert np.allclose(w.cpu().numpy(), ww, atol=1e-6)
    # strided logits ([T, E+1] router output) plus a per-expert skew, added in fp32
    full = rng.normal(size=(16, 257)).astype(np.float32)
    skew = (-1.1 * np.log(1.0 + rng.permutation(256))).astype(np.float32)
    ids, w = route(torch.from_numpy(full).cuda(), 8, skew=torch.from_numpy(skew).cuda(), n_experts=256)
    wi, ww = route_topk((full[:, :256] + skew[None, :]).astype(np.float64), 8)
    assert ids.cpu().numpy().tolist() == wi.tolist()
    assert np.allclose(w.cpu().numpy(), ww, atol=1e-6)
    # ties (repeated values, +0 and -0), the register path's widest row (512)
    # and the LDS path (1000 experts), top_k up to 64
    for E, k in ((512, 8), (300, 64), (1000, 10), (4096, 8)):
        lg = rng.integers(-3, 4, size=(5, E)).astype(np.float32)
        lg[0, ::7] = -0.0
        lg[0, 1::7] = 0.0
        ids, w = route(torch.from_numpy(lg).cuda(), k)
        wi, ww = route_topk(lg, k)
        assert ids.cpu().numpy().tolist() == wi.tolist(), (E, k)
        assert np.allclose(w.cpu().numpy(), ww, atol=1e-6), (E, k)


def test_segments_from_sorted_ids(gpu):
    from mtplx_amd.moe_sorted_gather import segments
    ids = np.array([0, 0, 3, 3, 3, 7, 9, 9], np.int32)
    off, act = segments(torch.from_numpy(ids).cuda(), 10)
    assert off.cpu().numpy().tolist() == OM.expert_offsets(ids, 10).tolist()
    a = act.cpu().numpy()
    assert a[0] == 4 and a[1:5].tolist() == [0, 3, 7, 9]
    _, act = segments(torch.tensor([0, 2, 1], dtype=torch.int32, device="cuda"), 4)
    assert int(act[0]) == -1
    _, act = segments(torch.tensor([0, 4], dtype=torch.int32, device="cuda"), 4)
    assert int(act[0]) == -1


def _experts(rng, E, H, F):
    gu = make_affine4_weights(rng, E * 2 * F, H)
    gu = tuple(a.reshape(E, 2 * F, -1) for a in gu)
    dn = make_affine4_weights(rng, E * H, F)
    dn = tuple(a.reshape(E, H, -1) for a in dn)
    return gu, dn


def test_gathered_swiglu_down_and_combine(gpu):
    """The ExpertSort fast path (what the verify step uses)."""
    from mtplx_amd.moe_sorted_gather import expert_sort, moe_combine, swiglu_rows, switch_linear
    from mtplx_amd.quant import QuantizedLinear
    rng = np.random.default_rng(3)
    E, H, F, T, k = 12, 512, 256, 16, 4
    gu, dn = _experts(rng, E, H, F)
    x = randn_bf16(rng, (T, H))
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = rng.random((T, k)).astype(np.float32)
    es = expert_sort(torch.from_numpy(idx).cuda(), E)
    tgu = (u32(gu[0]), from_bits(gu[1]), from_bits(gu[2]))
    h = swiglu_rows(x.reshape(T, 1, H), es.row_map, *tgu, es.sorted_ids, group_size=64, bits=4, expert_sort=es)
    row_map, sorted_ids, inv, _ = OM.sort_rows(idx)
    want_h = OM.swiglu_rows(bits(x), row_map, sorted_ids, *gu, 64, bf16_storage=True)
    assert_close(bf16_values(h.reshape(-1, F)), want_h, what="swiglu rows")
    down = QuantizedLinear(u32(dn[0]), from_bits(dn[1]), from_bits(dn[2]))
    y = switch_linear(down, h, es.sorted_ids, sorted_indices=True, expert_sort=es).reshape(-1, H)
    want_y = OM.gather_qmm_rows(bits(h.reshape(-1, F)), np.arange(T * k), sorted_ids, *dn, 64)
    assert_close(bf16_values(y), want_y, what="down rows")
    yv = bf16_values(y)     # the combine is checked on the stored (bf16) expert outputs
    routed = (yv[inv.astype(np.int64)].reshape(T, k, H) * sc[:, :, None]).sum(axis=1)
    out = moe_combine(y, es, torch.from_numpy(sc).cuda())
    assert_close(bf16_values(out), routed, what="combine")
    # gated shared expert + residual: h + bf16(bf16(routed) + bf16(sigmoid(g) * shared))
    shared = randn_bf16(rng, (T, H))
    resid = randn_bf16(rng, (T, H))
    gates = rng.normal(size=(T, 3)).astype(np.float32)
    out = moe_combine(y, es, torch.from_numpy(sc).cuda(), shared, shared_gate=torch.from_numpy(gates).cuda()[:, 1],
                      resid=resid)
    sg = 1.0 / (1.0 + np.exp(-gates[:, 1:2].astype(np.float64)))
    from oracle.bf16 import round_to_bf16 as rb
    want = rb(bf16_values(resid) + rb(rb(routed) + rb(sg * bf16_values(shared))))
    assert_close(bf16_values(out), want, what="gated combine")


def test_reference_call_sequence(gpu):
    """The sorted chain exactly as ``mtplx/models/qwen4_exp.py:1565-1577`` calls
    it: sort_rows -> swiglu_rows(tokens, row_map, w, s, b, idx, ...) ->
    switch_linear(down, h, idx, sorted_indices=True) -> unsort (mlx-lm
    _scatter_unsort) -> score-weighted sum, against the oracle's moe_forward."""
    from mtplx_amd.moe_sorted_gather import sort_rows, swiglu_rows, switch_linear
    from mtplx_amd.quant import QuantizedLinear
    rng = np.random.default_rng(6)
    E, H, F, T, k = 10, 256, 256, 12, 4
    gu, dn = _experts(rng, E, H, F)
    x = randn_bf16(rng, (T, H))
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = rng.random((T, k)); sc /= sc.sum(axis=1, keepdims=True)
    tokens, row_map, sidx, inv_order = sort_rows(x, torch.from_numpy(idx).cuda())
    o_row_map, o_sorted, o_inv, _ = OM.sort_rows(idx)
    assert row_map.cpu().numpy().astype(np.uint32).tolist() == o_row_map.tolist()
    assert sidx.cpu().numpy().tolist() == o_sorted.astype(np.int64).tolist()
    assert inv_order.cpu().numpy().tolist() == o_inv.astype(np.int64).tolist()
    h = swiglu_rows(tokens, row_map, u32(gu[0]), from_bits(gu[1]), from_bits(gu[2]), sidx, group_size=64, bits=4,
                    mode="affine")
    assert tuple(h.shape) == (T * k, 1, F)
    # each stored tensor against the oracle on the same (bf16) inputs
    want_h = OM.swiglu_rows(bits(x), o_row_map, o_sorted, *gu, 64, bf16_storage=True)
    assert_close(bf16_values(h.reshape(-1, F)), want_h, what="swiglu_rows")
    down = QuantizedLinear(u32(dn[0]), from_bits(dn[1]), from_bits(dn[2]))
    y = switch_linear(down, h, sidx, sorted_indices=True)
    assert tuple(y.shape) == (T * k, 1, H)
    want_y = OM.gather_qmm_rows(bits(h.reshape(-1, F)), np.arange(T * k), o_sorted, *dn, 64)
    assert_close(bf16_values(y.reshape(-1, H)), want_y, what="switch_linear")
    y_unsorted = y[inv_order.long()].reshape(T, k, 1, H).squeeze(-2)
    # the unsort puts expert (t, j)'s output at flat row t*k + j
    yv = bf16_values(y.reshape(-1, H))
    assert np.array_equal(bf16_values(y_unsorted).reshape(T * k, H), yv[o_inv.astype(np.int64)])
    # unsorted switch_linear returns rows in the caller's order
    hs = h.reshape(-1, F)[inv_order.long()].contiguous()
    y2 = switch_linear(down, hs, torch.from_numpy(idx).cuda().reshape(-1), sorted_indices=False)
    assert torch.equal(y2.reshape(T * k, H), y_unsorted.reshape(T * k, H))
    # the same stack packed once (its MLX triple released) runs on the
    # packed-expert kernel, sorted and unsorted, against the same oracle
    down.pack()
    down.release_source()
    yp = switch_linear(down, h, sidx, sorted_indices=True)
    assert_close(bf16_values(yp.reshape(-1, H)), want_y, what="switch_linear on a pack")
    yp2 = switch_linear(down, hs, torch.from_numpy(idx).cuda().reshape(-1), sorted_indices=False)
    assert torch.equal(yp2.reshape(T * k, H), yp[inv_order.long()].reshape(T * k, H))
    # and a stack held only in layout 2 (as the verify step keeps its experts)
    down2 = QuantizedLinear(u32(dn[0]), from_bits(dn[1]), from_bits(dn[2]))
    down2.pack(layout=2)
    down2.release_source()
    yq = switch_linear(down2, h, sidx, sorted_indices=True)
    assert_close(bf16_values(yq.reshape(-1, H)), want_y, what="switch_linear on a layout-2 pack")


def test_gather_qmm_contract(gpu):
    from mtplx_amd.moe_sorted_gather import gather_qmm
    rng = np.random.default_rng(4)
    E, N, K, R = 6, 256, 512, 20
    w = make_affine4_weights(rng, E * N, K)
    w = tuple(a.reshape(E, N, -1) for a in w)
    x = randn_bf16(rng, (9, K))
    lhs = rng.integers(0, 9, size=R).astype(np.int32)
    rhs = rng.integers(0, E, size=R).astype(np.int32)
    y = gather_qmm(x, u32(w[0]), from_bits(w[1]), from_bits(w[2]), torch.from_numpy(lhs).cuda(),
                   torch.from_numpy(rhs).cuda(), group_size=64, bits=4)
    want = np.stack([OM.gather_qmm_rows(bits(x)[lhs[i]:lhs[i] + 1], [0], [rhs[i]], *w, 64)[0] for i in range(R)])
    assert_close(bf16_values(y), want, what="gather_qmm")
    # mlx-lm SwitchGLU form: x [T,1,1,K] broadcast against indices [T,k] -> [T,k,1,N]
    T, k = 5, 3
    xs = randn_bf16(rng, (T, 1, 1, K))
    ind = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    y = gather_qmm(xs, u32(w[0]), from_bits(w[1]), from_bits(w[2]), rhs_indices=torch.from_numpy(ind).cuda(),
                   group_size=64, bits=4)
    assert tuple(y.shape) == (T, k, 1, N)
    xb = bits(xs.reshape(T, K))
    for t in range(T):
        for j in range(k):
            want = OM.gather_qmm_rows(xb[t:t + 1], [0], [ind[t, j]], *w, 64)[0]
            assert_close(bf16_values(y[t, j, 0]), want, what="switch-glu form")


def _within_one_ulp(a, b, what, ulps=1):
    """|a - b| <= ``ulps`` bf16 ulps of b (plus 1e-4 of the row's scale where
    a sum cancels): the packed path sums the same products with the k of each
    MFMA operand in another order. One ulp for a rounded sum; two through
    SwiGLU, which rounds the gate and the up sum (each one ulp apart at most)
    and then their product."""
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(b), 1e-30))) - 7)
    bad = np.abs(a - b) > ulps * ulp + 1e-4 * np.abs(b).max(axis=1, keepdims=True)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} beyond {ulps} ulp"


@pytest.mark.parametrize("T,k,E,H,F,gs,zipf", [
    (16, 8, 64, 1024, 512, 64, 1.1),   # cfg5-like: hot experts with all 16 rows, a tail of 1..4
    (40, 4, 16, 512, 256, 64, 2.0),    # experts past 16 rows (several 16-row tiles)
    (3, 2, 8, 512, 256, 128, 0.0),     # group 128, one or two rows per expert
    (32, 8, 64, 512, 256, 64, 50.0),   # every token on the same 8 experts (32 rows each), 56 experts idle
])
def test_packed_expert_matmul(gpu, T, k, E, H, F, gs, zipf):
    """mtp_gather_qmv_affine4_packed (the verify step's routed experts) against
    the oracle's sorted chain (bf16 bar) and within one bf16 ulp of the
    MLX-layout gather, for experts of every row class; the layout-2 entry
    (mtp_gather_qmv_affine4_packed_mf16) against the same bar and within one
    ulp of layout 1."""
    from mtplx_amd import _lib
    from mtplx_amd.moe_sorted_gather import expert_sort
    from mtplx_amd.quant import QuantizedLinear
    rng = np.random.default_rng(T * 100 + E)
    gu = make_affine4_weights(rng, E * 2 * F, H, gs)
    gu = tuple(a.reshape(E, 2 * F, -1) for a in gu)
    dn = make_affine4_weights(rng, E * H, F, gs)
    dn = tuple(a.reshape(E, H, -1) for a in dn)
    x = randn_bf16(rng, (T, H))
    p = np.exp(-zipf * np.log(np.arange(1, E + 1)))
    p /= p.sum()
    idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    es = expert_sort(torch.from_numpy(idx).cuda(), E)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    qgu = QuantizedLinear(u32(gu[0]), from_bits(gu[1]), from_bits(gu[2]), group_size=gs)
    qdn = QuantizedLinear(u32(dn[0]), from_bits(dn[1]), from_bits(dn[2]), group_size=gs)
    st = torch.cuda.current_stream().cuda_stream
    R = T * k
    h = torch.full((R, F), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_gather_qmv_affine4_packed", x.data_ptr(), es.row_map.data_ptr(), es.expert_off.data_ptr(),
              es.active.data_ptr(), qgu.pack().data_ptr(), h.data_ptr(), T, E, F, H, gs, 3, 2 * F, st)
    y = torch.full((R, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_gather_qmv_affine4_packed", h.data_ptr(), None, es.expert_off.data_ptr(), es.active.data_ptr(),
              qdn.pack().data_ptr(), y.data_ptr(), T, E, H, F, gs, 0, H, st)
    # the MLX-layout gather on the same inputs
    kw, gk = H // 8, H // gs
    h0 = torch.full((R, F), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_gather_qmv_affine4", x.data_ptr(), None, es.row_map.data_ptr(), es.expert_off.data_ptr(),
              es.active.data_ptr(), qgu.weight.data_ptr(), qgu.scales.data_ptr(), qgu.biases.data_ptr(),
              qgu.weight.reshape(-1, kw)[F:].data_ptr(), qgu.scales.reshape(-1, gk)[F:].data_ptr(),
              qgu.biases.reshape(-1, gk)[F:].data_ptr(), h0.data_ptr(), T, E, F, H, gs, 0, 3, 2 * F, None, 0, st)
    y0 = torch.full((R, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib.call("mtp_gather_qmv_affine4", h.data_ptr(), None, None, es.expert_off.data_ptr(), es.active.data_ptr(),
              qdn.weight.data_ptr(), qdn.scales.data_ptr(), qdn.biases.data_ptr(), None, None, None, y0.data_ptr(),
              T, E, H, F, gs, 0, 0, H, None, 0, st)
    torch.cuda.synchronize()
    assert counts.max() > (16 if T > 16 else 4) or zipf == 0.0   # the case reaches the row class it is for
    row_map, sorted_ids, _, _ = OM.sort_rows(idx)
    want_h = OM.swiglu_rows(bits(x), row_map, sorted_ids, *gu, gs, bf16_storage=True)
    hv = bf16_values(h)
    assert_close(hv, want_h, what=f"packed gate|up + SwiGLU T={T} E={E}")
    _within_one_ulp(hv, bf16_values(h0), "packed vs MLX-layout gate|up")
    want_y = OM.gather_qmm_rows(bits(h), np.arange(R), sorted_ids, *dn, gs)
    yv = bf16_values(y)
    assert_close(yv, want_y, what=f"packed down T={T} E={E}")
    _within_one_ulp(yv, bf16_values(y0), "packed vs MLX-layout down")
    # layout 2 (16x16x32 quads: the 4-row form for 1-4-row experts, the
    # 16-row form for 16-row tiles), each class on its own launch
    h2 = torch.full((R, F), float("nan"), dtype=torch.bfloat16, device="cuda")
    y2 = torch.full((R, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    for row_class in (1, 2):
        _lib.call("mtp_gather_qmv_affine4_packed_mf16", x.data_ptr(), es.row_map.data_ptr(), es.expert_off.data_ptr(),
                  es.active.data_ptr(), qgu.pack(layout=2).data_ptr(), h2.data_ptr(), T, E, F, H, gs, 3, 2 * F,
                  row_class, st)
    for row_class in (1, 2):
        _lib.call("mtp_gather_qmv_affine4_packed_mf16", h.data_ptr(), None, es.expert_off.data_ptr(),
                  es.active.data_ptr(), qdn.pack(layout=2).data_ptr(), y2.data_ptr(), T, E, H, F, gs, 0, H, row_class,
                  st)
    torch.cuda.synchronize()
    h2v, y2v = bf16_values(h2), bf16_values(y2)
    assert_close(h2v, want_h, what=f"layout-2 gate|up + SwiGLU T={T} E={E}")
    _within_one_ulp(h2v, hv, "layout 2 vs layout 1 gate|up + SwiGLU", ulps=2)
    assert_close(y2v, want_y, what=f"layout-2 down T={T} E={E}")
    _within_one_ulp(y2v, yv, "layout 2 vs layout 1 down")


def test_packed_expert_matmul_refuses_bad_shapes(gpu):
    from mtplx_amd import _lib
    z = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for N, K, rpe, em in ((48, 512, 48, 0), (64, 500, 64, 0), (64, 512, 64, 3), (64, 512, 64, 1)):
        with pytest.raises(_lib.MtpError):
            _lib.call("mtp_gather_qmv_affine4_packed", z.data_ptr(), None, z.data_ptr(), z.data_ptr(), z.data_ptr(),
                      z.data_ptr(), 4, 2, N, K, 64, em, rpe, st)


def test_combine_sums_of_squares(gpu):
    """mtp_moe_combine_ss: the same rows as mtp_moe_combine and, per 32-column
    block, the fp32 sum of the squared stored values in column order (the
    residual epilogue's statistics), bit for bit."""
    from mtplx_amd.moe_sorted_gather import expert_sort, moe_combine
    rng = np.random.default_rng(9)
    T, k, E, H = 16, 8, 64, 4096
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    es = expert_sort(torch.from_numpy(idx).cuda(), E)
    y = randn_bf16(rng, (T * k, H))
    sc = torch.from_numpy(rng.random((T, k)).astype(np.float32)).cuda()
    shared = randn_bf16(rng, (T, H))
    resid = randn_bf16(rng, (T, H))
    gate = torch.from_numpy(rng.normal(size=(T, 2)).astype(np.float32)).cuda()[:, 1]
    ss = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    out = moe_combine(y, es, sc, shared, shared_gate=gate, resid=resid, ss_out=ss)
    out0 = moe_combine(y, es, sc, shared, shared_gate=gate, resid=resid)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out0.view(torch.int16))
    v = bf16_values(out).astype(np.float32).reshape(T, H // 32, 32)
    acc = np.zeros((T, H // 32), np.float32)
    for c in range(32):   # sequential fp32 sums; bf16 squares are exact in fp32
        acc = acc + v[:, :, c] * v[:, :, c]
    got = ss.reshape(H // 32, 32).cpu().numpy()
    assert np.array_equal(got[:, :T], acc.T)
    from mtplx_amd import _lib
    with pytest.raises(_lib.MtpError):   # H % 32 != 0: no whole 32-column blocks
        moe_combine(y[:, :3984], es, sc, ss_out=torch.empty(3984, device="cuda"))
