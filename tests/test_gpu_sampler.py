"""GPU parity: exact accept/reject + sparse sampler law vs the oracle.

Bar (north star): token ids bit-exact given identical uniforms; probabilities
within 1e-5 (the GPU law is fp64 like the oracle, so the test uses 1e-9).
"""

import numpy as np
import pytest
import torch

from oracle import sampler as S
from mtplx_amd import _lib

pytestmark = pytest.mark.gpu


def _ws(rows, V):
    nb = _lib.query("mtp_sampler_workspace_bytes", rows, V)
    return torch.empty(nb, dtype=torch.uint8, device="cuda"), nb


def _sample_rows(logits: np.ndarray, cfg: S.SamplerConfig, uniforms: np.ndarray):
    rows, V = logits.shape
    k = max(cfg.top_k, 1)
    tl = torch.from_numpy(logits.astype(np.float32)).cuda()
    u = torch.from_numpy(uniforms.astype(np.float64)).cuda()
    ids = torch.empty((rows, k), dtype=torch.int32, device="cuda")
    probs = torch.empty((rows, k), dtype=torch.float64, device="cuda")
    cnt = torch.empty(rows, dtype=torch.int32, device="cuda")
    smp = torch.empty(rows, dtype=torch.int32, device="cuda")
    st = torch.empty(rows, dtype=torch.int32, device="cuda")
    ws, nb = _ws(rows, V)
    _lib.call("mtp_sample_rows", tl.data_ptr(), rows, V, cfg.temperature, cfg.top_k, cfg.top_p, u.data_ptr(),
              ids.data_ptr(), probs.data_ptr(), cnt.data_ptr(), smp.data_ptr(), st.data_ptr(), ws.data_ptr(), nb,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), probs.cpu().numpy(), cnt.cpu().numpy(), smp.cpu().numpy(), st.cpu().numpy()


@pytest.mark.parametrize("V,cfg", [
    (151936, S.SamplerConfig(0.6, 0.95, 20)),
    (1000, S.SamplerConfig(1.0, 0.8, 8)),
    (5000, S.SamplerConfig(0.3, 1.0, 40)),
    (4097, S.SamplerConfig(1.5, 0.5, 64)),
])
def test_sparse_law_and_draws_match_oracle(gpu, V, cfg):
    rng = np.random.default_rng(V)
    rows = 6
    logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
    logits[1, 10:20] = logits[1].max() + 1.0     # ties at the top: id order decides
    u = rng.random(rows)
    ids, probs, cnt, smp, st = _sample_rows(logits, cfg, u)
    assert (st == 0).all()
    for r in range(rows):
        want = S.sparse_distribution(logits[r], cfg)
        n = int(cnt[r])
        assert ids[r, :n].tolist() == want.ids.tolist(), r
        assert np.allclose(probs[r, :n], want.probs, rtol=0, atol=1e-9), r
        assert int(smp[r]) == S.choice(want, u[r]), r


def test_greedy_and_nonfinite(gpu):
    rng = np.random.default_rng(3)
    V = 3000
    logits = rng.normal(0, 1, (3, V)).astype(np.float32)
    logits[0, 7] = logits[0, 900] = 50.0                       # tie -> lower id
    logits[2, 5] = np.nan
    ids, probs, cnt, smp, st = _sample_rows(logits, S.SamplerConfig(0.0, 1.0, 0), np.zeros(3))
    assert smp[0] == 7 and smp[1] == int(np.argmax(logits[1]))
    assert st.tolist() == [0, 0, 1]


def _spec(target, draft, drafts, uniforms, cfg):
    B, K1, V = target.shape
    K = K1 - 1
    t = torch.from_numpy(target.reshape(-1, V).astype(np.float32)).cuda()
    d = torch.from_numpy(draft.reshape(-1, V).astype(np.float32)).cuda()
    di = torch.from_numpy(drafts.astype(np.int32)).cuda()
    u = torch.from_numpy(uniforms.astype(np.float64)).cuda()
    out = torch.empty((B, K + 1), dtype=torch.int32, device="cuda")
    nacc = torch.empty(B, dtype=torch.int32, device="cuda")
    ap = torch.empty((B, K), dtype=torch.float64, device="cuda")
    st = torch.empty(B, dtype=torch.int32, device="cuda")
    ws, nb = _ws(B * (2 * K + 1), V)
    _lib.call("mtp_spec_accept", t.data_ptr(), d.data_ptr(), di.data_ptr(), u.data_ptr(), B, K, V, cfg.temperature,
              cfg.top_k, cfg.top_p, out.data_ptr(), nacc.data_ptr(), ap.data_ptr(), st.data_ptr(), ws.data_ptr(), nb,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out.cpu().numpy(), nacc.cpu().numpy(), ap.cpu().numpy(), st.cpu().numpy()


@pytest.mark.parametrize("V,B,K,corr", [(151936, 4, 3, 0.5), (151936, 8, 3, 3.0), (2048, 16, 5, 0.3), (999, 8, 1, 1.0)])
def test_spec_accept_token_exact(gpu, V, B, K, corr):
    cfg = S.SamplerConfig(0.6, 0.95, 20)
    rng = np.random.default_rng(V + B + K)
    target = rng.normal(0, 3, (B, K + 1, V)).astype(np.float32)
    draft = (target[:, :K] + rng.normal(0, corr, (B, K, V))).astype(np.float32)
    drafts = np.stack([S.sample_rows(draft[b], rng.random(K), cfg) for b in range(B)])
    uniforms = rng.random((B, K + 1))
    out, nacc, ap, st = _spec(target, draft, drafts, uniforms, cfg)
    assert (st == 0).all()
    for b in range(B):
        want = S.spec_accept(target[b], draft[b], drafts[b], uniforms[b], cfg)
        assert int(nacc[b]) == want.n_accepted, b
        assert out[b, : len(want.tokens)].tolist() == want.tokens, b
        assert (out[b, len(want.tokens):] == -1).all()
        assert np.allclose(ap[b, : len(want.accept_probs)], want.accept_probs, rtol=0, atol=1e-9)


def test_spec_accept_greedy_lane(gpu):
    cfg = S.SamplerConfig(0.0, 1.0, 0)
    rng = np.random.default_rng(9)
    B, K, V = 4, 3, 5000
    target = rng.normal(0, 1, (B, K + 1, V)).astype(np.float32)
    draft = target[:, :K].copy()
    drafts = target[:, :K].argmax(axis=2)
    drafts[1, 1] = (drafts[1, 1] + 1) % V                       # force a mismatch
    out, nacc, ap, st = _spec(target, draft, drafts, np.zeros((B, K + 1)), cfg)
    assert nacc.tolist() == [3, 1, 3, 3]
    assert out[1, :2].tolist() == [drafts[1, 0], target[1, 1].argmax()]
    assert out[0].tolist() == [*drafts[0].tolist(), int(target[0, K].argmax())]
