"""GPU parity of the composed verify step at the BASELINE shapes against the
float64 oracle (``oracle.model.verify_forward``), at the north-star bf16 bar
rtol = atol = 1e-2: two dense layers of the 27B shape (hidden 5120, SwiGLU
17408, 40/8 heads of 128, vocab 151936), one request, 4 verify rows at
positions 4092..4095 of a 4096-token context, with the K/V rows each layer
writes and token-exact accept/reject on the produced logits.

The full 64-layer step and the MoE shape are held to the bar layer by layer
in ``test_gpu_model_depth.py``.
"""

import numpy as np
import pytest
import torch

from oracle import sampler as S
from oracle.model import verify_forward
from tests.gpu_util import assert_close
from tests.model_util import model_params_numpy

pytestmark = pytest.mark.gpu


def assert_rope_close(got, want, D=128, what="k rows"):
    """RoPE'd rows: each rotate-half pair (d, d + D/2) is a rotation of the
    bf16-rounded projection, so the error scales with the pair's norm, not
    with the (possibly cancelled) component: |got - want| <= 1e-2 * |pair| + 1e-2."""
    half = D // 2
    r = np.sqrt(want[..., :half] ** 2 + want[..., half:] ** 2)
    r = np.concatenate([r, r], axis=-1)
    bad = np.abs(got - want) > 1e-2 + 1e-2 * r
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside 1e-2 of the pair norm; first "
                             f"{idx.tolist()} got {got[tuple(idx[0])]} want {want[tuple(idx[0])]}")


def _caches(model, layers):
    kc = [model.k_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(layers)]
    vc = [model.v_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(layers)]
    return kc, vc


def test_cfg3_width_two_layers_match_oracle(gpu):
    from mtplx_amd.verify_step import DENSE_27B, VerifyModel
    from dataclasses import replace
    cfg = replace(DENSE_27B, layers=2)
    model = VerifyModel(cfg, device="cuda", seed=17)
    model.allocate_cache(1, 4096)
    kc, vc = _caches(model, cfg.layers)
    gen = torch.Generator(device="cuda").manual_seed(18)
    tokens = torch.randint(0, cfg.vocab, (1, 4), device="cuda", dtype=torch.int32, generator=gen)
    qs = torch.tensor([4092], dtype=torch.int32, device="cuda")
    logits = model.verify_logits(tokens, qs, check=True)
    got = logits.cpu().numpy().astype(np.float64)
    want = verify_forward(model_params_numpy(model), cfg, tokens.cpu().numpy(), np.array([4092]), kc, vc)
    assert_close(got, want, rtol=1e-2, atol=1e-2, what="cfg3-width logits")
    for li in range(cfg.layers):
        k = model.k_cache_standard(li).float().cpu().numpy()
        v = model.v_cache_standard(li).float().cpu().numpy()
        assert_rope_close(k[0, :, 4092:4096], kc[li][0, :, 4092:4096])
        assert_close(v[0, :, 4092:4096], vc[li][0, :, 4092:4096], rtol=1e-2, atol=1e-2, what="v rows")
    # accept/reject at the full vocabulary, token-exact against the oracle law
    from mtplx_amd.sampling import SamplerConfig, spec_accept
    draft = (logits[:3] + 0.5 * torch.randn((3, cfg.vocab), device="cuda", generator=gen)).contiguous()
    u = torch.rand((1, 4), device="cuda", dtype=torch.float64, generator=gen)
    res = spec_accept(logits.reshape(1, 4, -1), draft.reshape(1, 3, -1), tokens[:, 1:], u, SamplerConfig())
    w = S.spec_accept(got.astype(np.float32), draft.cpu().numpy(), tokens[0, 1:].cpu().numpy(), u[0].cpu().numpy(),
                      S.SamplerConfig())
    assert res.tokens[0].cpu().numpy().tolist()[: len(w.tokens)] == w.tokens
    assert int(res.n_accepted[0]) == w.n_accepted


@pytest.mark.parametrize("B,L", [(4, 4), (8, 4), (3, 1), (5, 2)])
def test_cfg3_width_uniform_batches(gpu, B, L):
    """B requests x L rows on the uniform cache at the 27B width, one layer
    against the oracle at the bar. From 16 rows on, x at hidden 5120 does not
    fit in one workgroup's LDS, so the streaming matmuls take the full K split
    (sized by the step's workspace query with each projection's real K) and
    q|k|v runs without the fused RoPE epilogue; M = 3 and 10 cover row
    counts off the tile multiples."""
    from mtplx_amd.verify_step import DENSE_27B, VerifyModel
    from dataclasses import replace
    cfg = replace(DENSE_27B, layers=1)
    model = VerifyModel(cfg, device="cuda", seed=19 + B)
    model.allocate_cache(B, 2048)
    kc, vc = _caches(model, cfg.layers)
    gen = torch.Generator(device="cuda").manual_seed(20 + B)
    tokens = torch.randint(0, cfg.vocab, (B, L), device="cuda", dtype=torch.int32, generator=gen)
    qs_np = np.random.default_rng(B).integers(0, 2048 - L, B)
    qs = torch.from_numpy(qs_np.astype(np.int32)).cuda()
    logits = model.verify_logits(tokens, qs, check=True)
    want = verify_forward(model_params_numpy(model), cfg, tokens.cpu().numpy(), qs_np, kc, vc)
    assert_close(logits.cpu().numpy().astype(np.float64), want, rtol=1e-2, atol=1e-2, what=f"B={B} L={L} logits")
