"""GPU tests of the drop-in boundary beyond 32 verify rows and of the
reference entry points the facade keeps:

* the ``QuantizedLinear`` patch and ``verify_kernels.quantized_matmul`` at
  33, 45, 64 and 70 rows, on packed, released and plain modules and on raw
  MLX triples, against the float64 oracle (rtol = atol = 1e-2);
* the exact (greedy) lane through the patch: a row's output is bit-identical
  at M = 1, 4 and 45;
* the fixed-M names of ``mtplx/verify_kernels.py:222-268``;
* the SwitchGLU patch (``install_switch_glu_rows``) and the inactive switch
  linear guard, against the per-expert oracle loop;
* the ``fast_sampling`` surface against the oracle law.
"""

import numpy as np
import pytest
import torch

from oracle import moe as OM
from oracle import sampler as S
from oracle.bf16 import f32_to_bf16_bits, round_to_bf16
from oracle.qmv import make_affine4_weights, qmm_affine4
from tests.gpu_util import assert_close, bf16_values, bits, from_bits, randn_bf16, u32

pytestmark = pytest.mark.gpu


def _ql(n, k, seed):
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(seed)
    return QuantizedLinear.random(n, k, 64, generator=g)


def _np(q):
    return (q.weight.cpu().numpy().view(np.uint32), bits(q.scales), bits(q.biases))


@pytest.mark.parametrize("m", [33, 45, 64, 70])
def test_patch_rows_past_32(gpu, m):
    from mtplx_amd import nax_verify
    from mtplx_amd.verify_kernels import quantized_matmul
    rng = np.random.default_rng(m)
    plain, packed, released = _ql(1024, 2048, 1), _ql(1024, 2048, 2), _ql(1024, 2048, 3)
    refs = {id(q): _np(q) for q in (plain, packed, released)}
    packed.pack()
    released.pack()
    released.pack(layout=2)
    released.release_source()
    x = randn_bf16(rng, (m, 2048))
    xb = bits(x)
    nax_verify.install_nax_qlinear_patch()
    try:
        before = dict(nax_verify.fallback_counts())
        for name, q in (("plain", plain), ("packed", packed), ("released", released)):
            y = q(x)
            assert tuple(y.shape) == (m, 1024)
            assert_close(bf16_values(y), qmm_affine4(xb, *refs[id(q)], 64), what=f"patched {name} m={m}")
        assert nax_verify.fallback_counts() == before          # nothing fell through
        assert plain.packed is not None                       # packed on first use past 32 rows
    finally:
        nax_verify.uninstall_nax_qlinear_patch()
    w, s, b = make_affine4_weights(rng, 512, 1024, 64)
    xr = randn_bf16(rng, (m, 1024))
    wt, st_, bt = u32(w), from_bits(s), from_bits(b)
    y1 = quantized_matmul(xr, wt, st_, bt, group_size=64)
    y2 = quantized_matmul(xr, wt, st_, bt, group_size=64)          # the kept pack
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert_close(bf16_values(y1), qmm_affine4(bits(xr), w, s, b, 64), what=f"raw triple m={m}")


def test_exact_lane_rows_are_batch_invariant(gpu):
    """Inside exact_verify(True) a row's output is bit-identical at M = 1, 4
    and 45, and meets the oracle bar; the calls are counted as exact_t0."""
    from mtplx_amd import nax_verify
    from mtplx_amd.attention_context import exact_verify
    rng = np.random.default_rng(5)
    q = _ql(5120, 5120, 9)
    ref = _np(q)
    x = randn_bf16(rng, (45, 5120))
    nax_verify.install_nax_qlinear_patch()
    try:
        n0 = nax_verify.nax_qlinear_fallback_counts["exact_t0"]
        with exact_verify(True):
            y45 = q(x)
            y4 = q(x[12:16])
            y1 = q(x[13:14])
        torch.cuda.synchronize()
        assert nax_verify.nax_qlinear_fallback_counts["exact_t0"] == n0 + 3
        assert torch.equal(y45[12:16].view(torch.int16), y4.view(torch.int16))
        assert torch.equal(y45[13:14].view(torch.int16), y1.view(torch.int16))
        assert_close(bf16_values(y45), qmm_affine4(bits(x), *ref, 64), what="exact lane")
        y4s = q(x[12:16])                                           # outside the context: the streaming kernel
        assert_close(bf16_values(y4s), qmm_affine4(bits(x[12:16]), *ref, 64), what="streaming lane")
    finally:
        nax_verify.uninstall_nax_qlinear_patch()


def test_fixed_m_entry_points(gpu):
    from mtplx_amd import verify_kernels as VK
    rng = np.random.default_rng(6)
    w, s, b = make_affine4_weights(rng, 1024, 2048, 64)
    wt, st_, bt = u32(w), from_bits(s), from_bits(b)
    assert VK.vk_eligible_m4(4, 2048, 1024, 4, 64, torch.bfloat16)
    assert not VK.vk_eligible_m4(5, 2048, 1024, 4, 64, torch.bfloat16)
    assert VK.vk_eligible_m6(5, 2048, 1024, 8, 32, torch.bfloat16) and VK.vk_eligible_m6(6, 2048, 1024, 4, 64,
                                                                                          torch.bfloat16)
    assert not VK.vk_eligible_m6(4, 2048, 1024, 4, 64, torch.bfloat16)
    assert not VK.vk_eligible_m4(4, 2048, 1024, 4, 64, torch.float32)
    for m, fns in ((4, (VK.vk_qmm_m4, VK.vk_qmm_m4_ksplit)), (5, (VK.vk_qmm_m6, VK.vk_qmm_m6_ksplit)),
                   (6, (VK.vk_qmm_m6, VK.vk_qmm_m6_ksplit))):
        x = randn_bf16(rng, (m, 2048))
        want = qmm_affine4(bits(x), w, s, b, 64)
        for fn in fns:
            y = fn(x, wt, st_, bt, bits=4, group_size=64)
            assert tuple(y.shape) == (m, 1024)
            assert_close(bf16_values(y), want, what=f"{fn.__name__} m={m}")


def _switch(rng, E, n, k, gs=64):
    from mtplx_amd.moe_sorted_gather import QuantizedSwitchLinear
    w, s, b = make_affine4_weights(rng, E * n, k, gs)
    w, s, b = w.reshape(E, n, -1), s.reshape(E, n, -1), b.reshape(E, n, -1)
    return QuantizedSwitchLinear(u32(w), from_bits(s), from_bits(b), group_size=gs), (w, s, b)


def test_switch_glu_rows_patch(gpu):
    """SwitchGLU through the installed row-map patch equals the stock call
    within the bar and the per-expert oracle loop; install is idempotent; the
    row-pad guard is inactive on gfx950 (installs nothing)."""
    from mtplx_amd import moe_sorted_gather as MG
    rng = np.random.default_rng(8)
    E, F, D, T, k = 16, 256, 512, 24, 4
    gate, (wg, sg, bg) = _switch(rng, E, F, D)
    up, (wu, su, bu) = _switch(rng, E, F, D)
    down, (wd, sd, bd) = _switch(rng, E, D, F)
    glu = MG.SwitchGLU(gate, up, down)
    x = randn_bf16(rng, (T, D))
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    ind = torch.from_numpy(idx).cuda()
    stock = glu(x, ind)
    assert tuple(stock.shape) == (T, k, D)
    original = MG.SwitchGLU.__call__
    assert MG.install_switch_linear_guard() is False
    try:
        assert MG.install_switch_glu_rows() is True
        patched = MG.SwitchGLU.__call__
        assert getattr(patched, "_mtplx_switch_glu_rows", False)
        assert MG.install_switch_glu_rows() is True and MG.SwitchGLU.__call__ is patched   # idempotent
        y = glu(x, ind)
        small = glu(x[:8], ind[:8])                     # 32 routed rows: the original call
    finally:
        MG.SwitchGLU.__call__ = original
    torch.cuda.synchronize()
    assert tuple(y.shape) == (T, k, D)
    # per (token, expert) oracle: down(silu(gate) * up) with bf16 storage of the gathers
    want = np.zeros((T, k, D))
    for t in range(T):
        for j in range(k):
            e = int(idx[t, j])
            g = round_to_bf16(qmm_affine4(bits(x[t:t + 1]), wg[e], sg[e], bg[e], 64))
            u = round_to_bf16(qmm_affine4(bits(x[t:t + 1]), wu[e], su[e], bu[e], 64))
            h = round_to_bf16(round_to_bf16(OM.silu(g)) * u)
            want[t, j] = qmm_affine4(f32_to_bf16_bits(h.astype(np.float32)), wd[e], sd[e], bd[e], 64)[0]
    assert_close(bf16_values(y), want, what="switch_glu_rows")
    assert_close(bf16_values(stock), want, what="stock SwitchGLU")
    assert_close(bf16_values(small), want[:8], what="SwitchGLU below the row threshold")


def test_fast_sampling_surface(gpu):
    from mtplx_amd import fast_sampling as FS
    from mtplx_amd.sampling import NonFiniteLogitsError, SamplerConfig
    rng = np.random.default_rng(12)
    V = 32000
    lg = rng.normal(0, 3, (5, V)).astype(np.float32)
    t = torch.from_numpy(lg).cuda()
    cfg = SamplerConfig(0.7, 0.9, 20)
    oc = S.SamplerConfig(0.7, 0.9, 20)
    assert FS.sparse_distribution_from_mlx_logits(t[0], SamplerConfig(0.0, 1.0, 20)) is None
    assert FS.sparse_distribution_from_mlx_logits(t[0], SamplerConfig(0.7, 0.9, 0)) is None
    assert FS.sparse_distribution_rows_from_mlx_logits(t, SamplerConfig(0.0)) is None
    d0 = FS.sparse_distribution_from_mlx_logits(t[0], cfg)
    w0 = S.sparse_distribution(lg[0], oc)
    assert d0.token_ids.tolist() == w0.ids.tolist() and np.allclose(d0.probs, w0.probs, rtol=0, atol=1e-12)
    rows = FS.sparse_distribution_rows_from_mlx_logits(t, cfg)
    lst = FS.sparse_distributions_from_mlx_logits(t, cfg)
    bat = FS.batched_sparse_distributions_from_mlx_logits(t, cfg)
    assert len(rows) == 5 and len(lst) == 5
    for r in range(5):
        w = S.sparse_distribution(lg[r], oc)
        for d in (rows[r], lst[r], bat.to_distribution(r)):
            assert d.token_ids.tolist() == w.ids.tolist()
            assert np.allclose(d.probs, w.probs, rtol=0, atol=1e-12)
        assert abs(bat.probability(r, int(w.ids[0])) - float(w.probs[0])) < 1e-12
    u = rng.random(5)
    ids = FS.sample_token_ids_from_mlx_logits(t, cfg, uniforms=torch.from_numpy(u).cuda()).cpu().numpy()
    assert ids.tolist() == [S.choice(S.sparse_distribution(lg[r], oc), u[r]) for r in range(5)]
    g = FS.sample_token_ids_from_mlx_logits(t, SamplerConfig(0.0)).cpu().numpy()
    assert g.tolist() == lg.argmax(axis=1).tolist()
    assert FS.sample_token_ids_from_mlx_logits(t, SamplerConfig(0.7, 0.9, 0)) is None
    # penalties on one raw row, then the law
    counts = {int(w0.ids[0]): 3, 7: 1}
    row0 = t[0]
    pen = FS.apply_penalties_mlx(row0, counts, 1.0, 0.5)
    assert pen is not row0
    assert FS.apply_penalties_mlx(row0, None, 1.0, 0.5) is row0
    np.testing.assert_array_equal(pen.cpu().numpy(), S.apply_penalties_f32(lg[0], counts, 1.0, 0.5))
    bad = lg.copy()
    bad[2, 3] = np.nan
    rows_bad = FS.sparse_distribution_rows_from_mlx_logits(torch.from_numpy(bad).cuda(), cfg)
    rows_bad[1]                                                    # a finite row reads fine
    with pytest.raises(NonFiniteLogitsError):
        rows_bad[2]
