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


@pytest.mark.parametrize("T,k,E", [(16, 8, 256), (4, 2, 8), (64, 8, 128), (1, 1, 4), (200, 10, 300)])
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


def test_gathered_swiglu_down_and_combine(gpu):
    from mtplx_amd.moe_sorted_gather import expert_sort, moe_combine, swiglu_rows, switch_linear
    from mtplx_amd.quant import QuantizedLinear
    rng = np.random.default_rng(3)
    E, H, F, T, k = 12, 512, 256, 16, 4
    gu = make_affine4_weights(rng, E * 2 * F, H)
    gu = tuple(a.reshape(E, 2 * F, -1) for a in gu)
    dn = make_affine4_weights(rng, E * H, F)
    dn = tuple(a.reshape(E, H, -1) for a in dn)
    x = randn_bf16(rng, (T, H))
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = rng.random((T, k)).astype(np.float32)
    es = expert_sort(torch.from_numpy(idx).cuda(), E)
    tgu = (u32(gu[0]), from_bits(gu[1]), from_bits(gu[2]))
    h = swiglu_rows(x.reshape(T, 1, H), es, *tgu, group_size=64)
    row_map, sorted_ids, inv, _ = OM.sort_rows(idx)
    want_h = OM.swiglu_rows(bits(x), row_map, sorted_ids, *gu, 64, bf16_storage=True)
    assert_close(bf16_values(h.reshape(-1, F)), want_h, what="swiglu rows")
    down = QuantizedLinear(u32(dn[0]), from_bits(dn[1]), from_bits(dn[2]))
    y = switch_linear(down, h.reshape(-1, F), es)
    want_y = OM.gather_qmm_rows(bits(h.reshape(-1, F)), np.arange(T * k), sorted_ids, *dn, 64)
    assert_close(bf16_values(y), want_y, what="down rows")
    out = moe_combine(y, es, torch.from_numpy(sc).cuda())
    yv = bf16_values(y)     # the combine is checked on the stored (bf16) expert outputs
    want_out = (yv[inv.astype(np.int64)].reshape(T, k, H) * sc[:, :, None]).sum(axis=1)
    assert_close(bf16_values(out), want_out, what="combine")


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
