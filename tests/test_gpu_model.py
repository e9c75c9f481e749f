"""GPU parity of the full verify step (dense and MoE decoders, tiny shapes)
against oracle.model, plus the accept/reject on the produced logits."""

import numpy as np
import pytest
import torch

from oracle import sampler as S
from oracle.model import verify_forward
from tests.gpu_util import assert_close
from tests.model_util import model_params_numpy

pytestmark = pytest.mark.gpu


def _run(cfg, B, L, starts, seed, moe_tokens=None, cap=320):
    from mtplx_amd.verify_step import VerifyModel
    model = VerifyModel(cfg, device="cuda", seed=seed, keep_expert_source=True)
    model.allocate_cache(B, cap)
    kc = [model.k_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(cfg.layers)]
    vc = [model.v_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(cfg.layers)]
    gen = torch.Generator(device="cuda").manual_seed(seed + 1)
    tokens = torch.randint(0, cfg.vocab, (B, L), device="cuda", dtype=torch.int32, generator=gen)
    qs = torch.tensor(starts, dtype=torch.int32, device="cuda")
    logits = model.verify_logits(tokens, qs)
    torch.cuda.synchronize()
    want = verify_forward(model_params_numpy(model), cfg, tokens.cpu().numpy(), np.array(starts), kc, vc)
    return model, tokens, logits, want, kc, vc


def test_dense_verify_step_matches_oracle(gpu):
    from mtplx_amd.verify_step import DecoderConfig
    cfg = DecoderConfig(layers=2, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096)
    model, tokens, logits, want, kc, vc = _run(cfg, 2, 4, [37, 200], 3)
    assert_close(logits.cpu().numpy().astype(np.float64), want, rtol=1e-2, atol=1e-2, what="dense logits")
    # the K/V rows the step wrote are the oracle's (RoPE'd k, raw v) within bf16 tolerance
    for li in range(cfg.layers):
        got_k = model.k_cache_standard(li).float().cpu().numpy()
        for b, s in enumerate([37, 200]):
            assert_close(got_k[b, :, s:s + 4], kc[li][b, :, s:s + 4], rtol=1e-2, atol=1e-2, what="k rows")
    # accept/reject on the GPU logits is token-exact against the oracle law
    from mtplx_amd.sampling import SamplerConfig, spec_accept
    B, L = 2, 4
    gen = torch.Generator(device="cuda").manual_seed(11)
    draft = (logits.reshape(B, L, -1)[:, :3] + 0.3 * torch.randn((B, 3, cfg.vocab), device="cuda",
                                                                 generator=gen)).contiguous()
    u = torch.rand((B, 4), device="cuda", dtype=torch.float64, generator=gen)
    res = spec_accept(logits.reshape(B, L, -1), draft, tokens[:, 1:], u, SamplerConfig())
    torch.cuda.synchronize()
    for b in range(B):
        w = S.spec_accept(logits.reshape(B, L, -1)[b].cpu().numpy(), draft[b].cpu().numpy(),
                          tokens[b, 1:].cpu().numpy(), u[b].cpu().numpy(), S.SamplerConfig())
        assert res.tokens[b].cpu().numpy().tolist()[: len(w.tokens)] == w.tokens
        assert int(res.n_accepted[b]) == w.n_accepted


@pytest.mark.parametrize("B,L", [(2, 4), (1, 1), (3, 3), (8, 4)])
def test_moe_verify_step_matches_oracle(gpu, B, L):
    """The MoE block at 1 to 32 rows (the sort, both expert row classes on two
    streams, the combine and its statistics for the next layer's norm)."""
    from mtplx_amd.verify_step import DecoderConfig
    cfg = DecoderConfig(layers=2, hidden=512, ffn=0, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                        n_experts=16, top_k=4, expert_ffn=256, shared_ffn=256)
    starts = [int(v) for v in np.random.default_rng(B * 10 + L).integers(0, 320 - L, B)]
    model, tokens, logits, want, kc, vc = _run(cfg, B, L, starts, 7)
    assert_close(logits.cpu().numpy().astype(np.float64), want, rtol=1e-2, atol=1e-2, what=f"moe logits B={B} L={L}")


def test_moe_verify_step_balanced_attention_short_contexts(gpu):
    """A cache large enough for the balanced attention (B * Hkv * cap >= 65536
    key-heads) holding short contexts: fewer 32-key tiles than workgroups,
    several per head (the split then runs over as many workgroups as tiles)."""
    from mtplx_amd.verify_step import DecoderConfig
    cfg = DecoderConfig(layers=2, hidden=512, ffn=0, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                        n_experts=16, top_k=4, expert_ffn=256, shared_ffn=256)
    B, L = 8, 4
    starts = [int(v) for v in np.random.default_rng(3).integers(20, 300, B)]
    model, tokens, logits, want, kc, vc = _run(cfg, B, L, starts, 9, cap=4096)
    assert B * cfg.n_kv_heads * model.cap >= 65536
    assert_close(logits.cpu().numpy().astype(np.float64), want, rtol=1e-2, atol=1e-2,
                 what="moe logits, balanced attention over short contexts")


def test_status_word_flags_bad_token_and_position(gpu):
    """An out-of-vocabulary token and a K/V write past the cache capacity set
    the forward's status word; check=True raises instead of returning logits
    that look valid."""
    from mtplx_amd import _lib
    from mtplx_amd.verify_step import DecoderConfig, VerifyModel
    cfg = DecoderConfig(layers=1, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1024)
    model = VerifyModel(cfg, device="cuda", seed=4)
    model.allocate_cache(1, 256)
    ok = torch.tensor([[1, 2, 3, 4]], dtype=torch.int32, device="cuda")
    model.verify_logits(ok, torch.tensor([10], dtype=torch.int32, device="cuda"), check=True)
    assert int(model.status().item()) == 0
    bad_tok = torch.tensor([[1, 2, cfg.vocab + 5, 4]], dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.MtpError):
        model.verify_logits(bad_tok, torch.tensor([10], dtype=torch.int32, device="cuda"), check=True)
    model.verify_logits(ok, torch.tensor([model.cap - 2], dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert int(model.status().item()) != 0
    with pytest.raises(_lib.MtpError):
        model.check_status()
