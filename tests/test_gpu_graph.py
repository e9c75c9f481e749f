"""HIP-graph replay of the verify step equals eager execution, bit for bit,
on every replay, with eager work and input updates between replays."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["dense", "moe"])
def test_captured_step_matches_eager_every_replay(gpu, kind):
    """dense: the cfg3-style layer; moe: router, expert sort, both routed
    row classes (experts with 1-4 and with 5+ rows over 32 routed rows on 8
    experts), shared expert and combine inside the captured step."""
    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import CapturedVerifyStep, DecoderConfig, VerifyModel
    if kind == "dense":
        cfg = DecoderConfig(layers=2, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096)
    else:
        cfg = DecoderConfig(layers=2, hidden=512, ffn=0, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096,
                            n_experts=8, top_k=4, expert_ffn=256, shared_ffn=256)
    model = VerifyModel(cfg, device="cuda", seed=21)
    B, L = 2, 4
    model.allocate_cache(B, 512)
    gen = torch.Generator(device="cuda").manual_seed(4)
    tokens = torch.randint(0, cfg.vocab, (B, L), device="cuda", dtype=torch.int32, generator=gen)
    qs = torch.tensor([100, 300], dtype=torch.int32, device="cuda")
    draft = torch.randn((B, L - 1, cfg.vocab), device="cuda", generator=gen) * 3
    u = torch.rand((B, L), device="cuda", dtype=torch.float64, generator=gen)
    sampler = SamplerConfig()
    cap = CapturedVerifyStep(model, tokens, qs, draft, u, sampler)
    for rep in range(3):
        res = cap.replay()
        torch.cuda.synchronize()
        got_logits = cap.logits.clone()                             # graph-owned buffer
        got_tokens = res.tokens.clone()
        # eager on the same inputs (and some unrelated eager work in between)
        torch.randn(1000, device="cuda").sum().item()
        eager = model.verify_step(tokens, qs, draft, u, sampler)
        torch.cuda.synchronize()
        assert torch.equal(model.last_logits, got_logits), f"replay {rep}: logits differ"
        assert torch.equal(eager.tokens, got_tokens), f"replay {rep}: tokens differ"
        # new inputs for the next replay, written in place
        tokens.copy_(torch.randint(0, cfg.vocab, (B, L), device="cuda", dtype=torch.int32, generator=gen))
        u.copy_(torch.rand((B, L), device="cuda", dtype=torch.float64, generator=gen))
