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


def test_captured_ragged_step_matches_eager_every_replay(gpu):
    """The continuous-batched ragged step (per-request capacities, depths and
    q lengths, the 9..64-row matmuls, block attention, ragged accept) replayed
    from one graph equals eager execution, bit for bit, on every replay."""
    import numpy as np

    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import CapturedRaggedVerifyStep, DecoderConfig, VerifyModel
    cfg = DecoderConfig(layers=2, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096)
    model = VerifyModel(cfg, device="cuda", seed=23)
    depths = np.array([1, 3, 2, 3, 1, 2, 3, 2, 1, 3, 2, 1])
    lens = depths + 1
    ctx = np.array([300, 1200, 700, 2100, 96, 513, 1800, 64, 950, 1500, 260, 3000])
    B = len(depths)
    q_start = (ctx - lens).astype(np.int32)
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d_off = np.concatenate([[0], np.cumsum(depths)]).astype(np.int32)
    draft_index = np.concatenate([np.arange(row_off[b] + 1, row_off[b + 1]) for b in range(B)])
    M, Lmax = int(row_off[-1]), int(lens.max())
    model.allocate_cache_blocks(ctx)
    gen = torch.Generator(device="cuda").manual_seed(6)
    t = lambda a, dt=torch.int32: torch.from_numpy(np.ascontiguousarray(a)).to(device="cuda", dtype=dt)  # noqa: E731
    tokens = torch.randint(0, cfg.vocab, (M,), device="cuda", dtype=torch.int32, generator=gen)
    draft = 3.0 * torch.randn((int(d_off[-1]), cfg.vocab), device="cuda", generator=gen)
    u = torch.rand((B, 4), device="cuda", dtype=torch.float64, generator=gen)
    args = (tokens, t(row_off), t(q_start), t(lens), Lmax, draft, t(d_off), t(draft_index, torch.int64), u,
            SamplerConfig(0.6, 0.95, 20))
    cap = CapturedRaggedVerifyStep(model, *args)
    for rep in range(3):
        res = cap.replay()
        torch.cuda.synchronize()
        got_logits = cap.logits.clone()
        got_tokens, got_n = res.tokens.clone(), res.n_accepted.clone()
        torch.randn(1000, device="cuda").sum().item()
        eager = model.verify_step_ragged(*args)
        torch.cuda.synchronize()
        model.check_status()
        assert torch.equal(model.last_logits, got_logits), f"replay {rep}: logits differ"
        assert torch.equal(eager.tokens, got_tokens), f"replay {rep}: tokens differ"
        assert torch.equal(eager.n_accepted, got_n), f"replay {rep}: accepted counts differ"
        tokens.copy_(torch.randint(0, cfg.vocab, (M,), device="cuda", dtype=torch.int32, generator=gen))
        u.copy_(torch.rand((B, 4), device="cuda", dtype=torch.float64, generator=gen))
