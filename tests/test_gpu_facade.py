"""The reference call surface on the GPU: verify_qmv, nax_verify, ragged KV
cache gates, ragged attention, sampling facade."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import sampler as S
from oracle.moe import silu
from oracle.qmv import qmm_affine4
from tests.gpu_util import assert_close, bf16_values, bits, randn_bf16

pytestmark = pytest.mark.gpu


def _ql(n, k, seed):
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(seed)
    return QuantizedLinear.random(n, k, 64, generator=g)


def _np(q):
    return (q.weight.cpu().numpy().view(np.uint32), bits(q.scales), bits(q.biases))


def test_verify_qmv_surface(gpu):
    from mtplx_amd import verify_qmv as V
    rng = np.random.default_rng(0)
    q = _ql(1024, 2048, 1)
    x = randn_bf16(rng, (1, 4, 2048))
    assert V.is_multi3_qmv4_eligible(q)
    y = V.multi3_qmv4_matmul(x, q)
    assert y.shape == (1, 4, 1024)
    assert_close(bf16_values(y).reshape(4, -1), qmm_affine4(bits(x).reshape(4, -1), *_np(q), 64), what="multi3")
    g, u = _ql(1024, 2048, 2), _ql(1024, 2048, 3)
    yg, yu = V.multi3_dual_qmv4_matmul(x, g, u)
    assert_close(bf16_values(yg).reshape(4, -1), qmm_affine4(bits(x).reshape(4, -1), *_np(g), 64), what="dual g")
    d = _ql(2048, 1024, 4)
    gate, up = randn_bf16(rng, (4, 1024)), randn_bf16(rng, (4, 1024))
    yd = V.multi3_swiglu_down_qmv4_matmul(gate, up, d)
    from oracle.bf16 import f32_to_bf16_bits, round_to_bf16
    act = round_to_bf16(round_to_bf16(silu(bf16_values(gate))) * bf16_values(up))
    assert_close(bf16_values(yd), qmm_affine4(f32_to_bf16_bits(act.astype(np.float32)), *_np(d), 64), what="swiglu down")
    # ineligible (M > 32 rows) falls back to module(x), still on the GPU
    x40 = randn_bf16(rng, (40, 2048))
    assert_close(bf16_values(V.multi3_qmv4_matmul(x40, q)), qmm_affine4(bits(x40), *_np(q), 64), what="fallback")
    pair_l, pair_r = _ql(48, 1024, 5), _ql(48, 1024, 6)
    assert V.is_smalln_pair_qmv4_eligible(pair_l, pair_r)
    yl, yr = V.smalln_pair_qmv4_matmul(randn_bf16(rng, (4, 1024)), pair_l, pair_r)
    assert yl.shape == (4, 48) and yr.shape == (4, 48)


@pytest.mark.parametrize("m", [4, 8])
def test_verify_qmv_surface_on_packed_modules(gpu, m):
    """Modules packed once (layouts 1 and 2) take the tile-major kernels
    through the same facade calls, also after their MLX triples are released;
    the oracle is computed from the triples before the release. m = 4 runs
    layout 2 (16x16x32 MFMA), m = 8 layout 1."""
    from oracle.bf16 import f32_to_bf16_bits, round_to_bf16
    from mtplx_amd import verify_qmv as V
    rng = np.random.default_rng(10 + m)
    q, g, u, d = _ql(1024, 2048, 11), _ql(1024, 2048, 12), _ql(1024, 2048, 13), _ql(2048, 1024, 14)
    ref = {name: _np(mod) for name, mod in (("q", q), ("g", g), ("u", u), ("d", d))}
    for mod in (q, g, u, d):
        mod.pack()
        mod.pack(layout=2)
        mod.release_source()
    x = randn_bf16(rng, (m, 2048))
    xb = bits(x)
    assert_close(bf16_values(V.multi3_qmv4_matmul(x, q)), qmm_affine4(xb, *ref["q"], 64), what=f"packed m={m}")
    yg, yu = V.multi3_dual_qmv4_matmul(x, g, u)
    assert_close(bf16_values(yg), qmm_affine4(xb, *ref["g"], 64), what=f"packed dual gate m={m}")
    assert_close(bf16_values(yu), qmm_affine4(xb, *ref["u"], 64), what=f"packed dual up m={m}")
    gate, up = randn_bf16(rng, (m, 1024)), randn_bf16(rng, (m, 1024))
    act = round_to_bf16(round_to_bf16(silu(bf16_values(gate))) * bf16_values(up))
    assert_close(bf16_values(V.multi3_swiglu_down_qmv4_matmul(gate, up, d)),
                 qmm_affine4(f32_to_bf16_bits(act.astype(np.float32)), *ref["d"], 64), what=f"packed swiglu down m={m}")


def test_nax_patch_routes_and_counts(gpu):
    from mtplx_amd import nax_verify
    from mtplx_amd.quant import QuantizedLinear
    q = _ql(512, 1024, 7)
    rng = np.random.default_rng(1)
    x = randn_bf16(rng, (4, 1024))
    nax_verify.install_nax_qlinear_patch()
    try:
        assert getattr(QuantizedLinear.__call__, "_mtplx_amd_patch", False)
        assert_close(bf16_values(q(x)), qmm_affine4(bits(x), *_np(q), 64), what="patched call")
        # a packed module (source released) takes its pack through the patch;
        # K = 768 is not a multiple of 512 (no verify_qmv route), so only the
        # pack serves it
        q2 = _ql(256, 768, 8)
        ref = _np(q2)
        q2.pack()
        q2.release_source()
        x2 = randn_bf16(rng, (4, 768))
        assert_close(bf16_values(q2(x2)), qmm_affine4(bits(x2), *ref, 64), what="patched call on a pack")
    finally:
        nax_verify.uninstall_nax_qlinear_patch()


def test_ragged_cache_gates(gpu):
    """Gates of tests/test_ragged_kv_cache.py: uniform offsets == scalar append,
    per-row independence, REPLAY rewrite in place, masked restore bitwise."""
    from mtplx_amd.ragged_kv_cache import RaggedBatchKVCache
    rng = np.random.default_rng(2)
    B, H, D, q = 3, 2, 128, 4
    c = RaggedBatchKVCache(batch_size=B, step=64)
    k0, v0 = randn_bf16(rng, (B, H, 20, D)), randn_bf16(rng, (B, H, 20, D))
    keys, vals = c.update_and_fetch(k0, v0)                       # uniform append at 0
    assert keys.shape[2] == 64 and c.offset.cpu().tolist() == [20, 20, 20]
    assert torch.equal(keys[:, :, :20].view(torch.int16), k0.view(torch.int16))
    snap = c.snapshot()
    k1, v1 = randn_bf16(rng, (B, H, q, D)), randn_bf16(rng, (B, H, q, D))
    c.update_and_fetch(k1, v1, write_start=[20, 19, 20], new_offsets=[24, 23, 21])   # row 1 REPLAY at offset-1
    assert c.offset.cpu().tolist() == [24, 23, 21]
    kb = bits(c.keys)
    assert np.array_equal(kb[1, :, 19:23], bits(k1)[1]) and np.array_equal(kb[1, :, :19], bits(k0)[1, :, :19])
    c.restore_masked(snap, [True, False, True])
    assert c.offset.cpu().tolist() == [20, 23, 20]
    kb2 = bits(c.keys)
    assert np.array_equal(kb2[0], bits(snap.keys)[0]) and np.array_equal(kb2[1], kb[1])
    m = c.make_mask(q)
    assert m.dtype == torch.bool and m.shape == (B, 1, q, 64)
    assert np.array_equal(m.cpu().numpy(), A.ragged_causal_mask([20, 23, 20], q, 64))
    assert c.trim(5) == 5 and c.offset.cpu().tolist() == [15, 18, 15]


def test_ragged_sdpa_facade(gpu):
    from mtplx_amd.ragged_attention import ragged_sdpa
    rng = np.random.default_rng(3)
    q = randn_bf16(rng, (2, 16, 4, 128)); k = randn_bf16(rng, (2, 4, 300, 128)); v = randn_bf16(rng, (2, 4, 300, 128))
    out = ragged_sdpa(q, k, v, torch.tensor([100, 250], dtype=torch.int32, device="cuda"))
    assert_close(bf16_values(out), A.ragged_gqa_attention(bits(q), bits(k), bits(v), [100, 250]), what="sdpa")


def test_sampling_facade(gpu):
    from mtplx_amd import sampling as GS
    rng = np.random.default_rng(4)
    lg = rng.normal(0, 3, (3, 50000)).astype(np.float32)
    dists = GS.sparse_distributions_from_logits(torch.from_numpy(lg).cuda(), GS.SamplerConfig())
    for r in range(3):
        w = S.sparse_distribution(lg[r], S.SamplerConfig())
        assert dists[r].token_ids.tolist() == w.ids.tolist()
        assert np.allclose(dists[r].probs, w.probs, atol=1e-12)
    lg[1, 5] = np.inf
    with pytest.raises(GS.NonFiniteLogitsError):
        GS.sparse_distributions_from_logits(torch.from_numpy(lg).cuda(), GS.SamplerConfig())
