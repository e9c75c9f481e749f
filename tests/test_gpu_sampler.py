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


def _ws(rows, V, top_k):
    nb = _lib.query("mtp_sampler_workspace_bytes", rows, V, top_k)
    return torch.empty(nb, dtype=torch.uint8, device="cuda"), nb


def _bound(cfg, V):
    if not cfg.temperature > 0:
        return 1
    return cfg.top_k if 0 < cfg.top_k < V else V


def _sample_rows(logits: np.ndarray, cfg: S.SamplerConfig, uniforms: np.ndarray, ld=None):
    rows, V = logits.shape
    k = _bound(cfg, V) if ld is None else ld
    tl = torch.from_numpy(logits.astype(np.float32)).cuda()
    u = torch.from_numpy(uniforms.astype(np.float64)).cuda()
    ids = torch.empty((rows, k), dtype=torch.int32, device="cuda")
    probs = torch.empty((rows, k), dtype=torch.float64, device="cuda")
    cnt = torch.empty(rows, dtype=torch.int32, device="cuda")
    smp = torch.empty(rows, dtype=torch.int32, device="cuda")
    st = torch.empty(rows, dtype=torch.int32, device="cuda")
    ws, nb = _ws(rows, V, cfg.top_k)
    _lib.call("mtp_sample_rows", tl.data_ptr(), rows, V, cfg.temperature, cfg.top_k, cfg.top_p, u.data_ptr(),
              ids.data_ptr(), probs.data_ptr(), k, cnt.data_ptr(), smp.data_ptr(), st.data_ptr(), ws.data_ptr(), nb,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), probs.cpu().numpy(), cnt.cpu().numpy(), smp.cpu().numpy(), st.cpu().numpy()


@pytest.mark.parametrize("V,cfg", [
    (151936, S.SamplerConfig(0.6, 0.95, 20)),
    (1000, S.SamplerConfig(1.0, 0.8, 8)),
    (5000, S.SamplerConfig(0.3, 1.0, 40)),
    (4097, S.SamplerConfig(1.5, 0.5, 64)),
    # wide laws: no top-k bound (pure nucleus / full softmax) and top_k > 64
    (151936, S.SamplerConfig(0.6, 0.95, 0)),
    (151936, S.SamplerConfig(1.0, 1.0, 0)),
    (20000, S.SamplerConfig(2.0, 0.9, 0)),
    (151936, S.SamplerConfig(0.8, 0.95, 100)),
    (5000, S.SamplerConfig(1.0, 0.999, 1000)),
    (48, S.SamplerConfig(1.0, 0.9, 0)),
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


@pytest.mark.parametrize("case", ["k20", "k64", "ties", "one_chunk"])
def test_narrow_top_k_selection_paths(gpu, case):
    """The narrow law's top k is a k-way merge of the chunks' sorted lists,
    one wave maximum of the list heads per round (high words first, the low
    words only when several heads share the maximal high word). Cases: plain
    k = 20 over 38 chunks, k = 64, 20 equal values spread over 10 chunks (the
    id decides every round), one chunk with every key selected; ids and draws
    exact, against the oracle."""
    rng = np.random.default_rng(11)
    V, k, rows = 151936, 20, 4
    if case == "one_chunk":
        V, k = 50, 50          # top_k = V: one chunk, every key selected
    logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
    if case == "k64":
        k = 64
    elif case == "ties":
        # 20 equal top values spread over 10 chunks, two each: the id decides
        for c in range(10):
            logits[:, 4096 * (3 * c + 1) + 7 * c] = 20.0
            logits[:, 4096 * (3 * c + 1) + 7 * c + 1000] = 20.0
    cfg = S.SamplerConfig(0.6, 0.95, k)
    u = rng.random(rows)
    ids, probs, cnt, smp, st = _sample_rows(logits, cfg, u)
    assert (st == 0).all()
    for r in range(rows):
        want = S.sparse_distribution(logits[r], cfg)
        n = int(cnt[r])
        assert ids[r, :n].tolist() == want.ids.tolist(), (case, r)
        assert np.allclose(probs[r, :n], want.probs, rtol=0, atol=1e-9), (case, r)
        assert int(smp[r]) == S.choice(want, u[r]), (case, r)


def test_wide_law_tie_group_cut(gpu):
    """A tie group straddling the top-k cut keeps its lowest ids, and one
    straddling the nucleus cut is cut inside the group (same mass each)."""
    V = 3000
    logits = np.full((3, V), -5.0, np.float32)
    logits[0, 100:400] = 2.0              # 300 tied at the top, top_k = 150: ids 100..249
    logits[1, 50:1050] = 1.0              # 1000 tied: nucleus 0.5 keeps about half of them
    logits[2] = np.random.default_rng(1).normal(0, 1, V).astype(np.float32)
    logits[2, 10:20] = 9.0
    for cfg in (S.SamplerConfig(1.0, 1.0, 150), S.SamplerConfig(1.0, 0.5, 0), S.SamplerConfig(1.0, 0.3, 200)):
        # Uniforms off the cdf steps k/150, k/503, ...: equal probabilities
        # put steps at exact fractions, where any two summation orders of
        # the cdf may round to opposite sides of u.
        u = np.array([0.3137, 0.6071, 0.9023])
        ids, probs, cnt, smp, st = _sample_rows(logits, cfg, u)
        assert (st == 0).all()
        for r in range(3):
            want = S.sparse_distribution(logits[r], cfg)
            assert ids[r, : cnt[r]].tolist() == want.ids.tolist(), (cfg, r)
            assert np.allclose(probs[r, : cnt[r]], want.probs, rtol=0, atol=1e-9)
            assert int(smp[r]) == S.choice(want, u[r])


def test_output_rows_use_the_given_stride(gpu):
    """Greedy with top_k = 20 (support 1) written at a row stride of 20: every
    row's slot 0 is its argmax and the rest is padded (-1, 0)."""
    rng = np.random.default_rng(12)
    logits = rng.normal(0, 1, (5, 3000)).astype(np.float32)
    ids, probs, cnt, smp, st = _sample_rows(logits, S.SamplerConfig(0.0, 0.95, 20), np.zeros(5), ld=20)
    assert cnt.tolist() == [1] * 5 and (st == 0).all()
    assert ids[:, 0].tolist() == logits.argmax(axis=1).tolist()
    assert (ids[:, 1:] == -1).all() and (probs[:, 1:] == 0).all() and (probs[:, 0] == 1).all()
    # the facade allocates [rows, top_k] for the same law
    from mtplx_amd.sampling import SamplerConfig, sparse_distributions_from_logits
    laws = sparse_distributions_from_logits(torch.from_numpy(logits).cuda(), SamplerConfig(0.0, 0.95, 20))
    assert [int(d.token_ids[0]) for d in laws] == logits.argmax(axis=1).tolist()


def test_penalties_match_device_twin(gpu):
    from mtplx_amd.sampling import SamplerConfig, row_laws
    rng = np.random.default_rng(13)
    V = 151936
    logits = rng.normal(0, 3, (3, V)).astype(np.float32)
    top = np.argsort(-logits, axis=1)[:, :6]
    counts = [{int(top[0, 0]): 3, int(top[0, 2]): 1, 7: 2}, None, {int(top[2, 1]): 1}]
    overlay = [None, {int(top[1, 0]): 0.75}, {int(top[2, 0]): 5.0}]
    for pres, freq, k in ((1.5, 0.5, 20), (2.5, -0.5, 0), (0.0, 0.0, 20)):
        cfg = SamplerConfig(0.6, 0.95, k, presence_penalty=pres, frequency_penalty=freq)
        u = rng.random(3)
        laws = row_laws(torch.from_numpy(logits).cuda(), cfg, torch.from_numpy(u).cuda(), token_counts=counts,
                        penalty_overlay=overlay)
        torch.cuda.synchronize()
        ids, probs, cnt = laws.ids.cpu().numpy(), laws.probs.cpu().numpy(), laws.count.cpu().numpy()
        oc = S.SamplerConfig(0.6, 0.95, k)
        for r in range(3):
            pen = S.apply_penalties_f32(logits[r], counts[r], pres, freq, overlay[r])
            want = S.sparse_distribution(pen, oc)
            assert ids[r, : cnt[r]].tolist() == want.ids.tolist(), (pres, r)
            assert np.allclose(probs[r, : cnt[r]], want.probs, rtol=0, atol=1e-9)
            assert int(laws.sampled[r]) == S.choice(want, u[r])
    # the caller's logits are left as they were
    t = torch.from_numpy(logits).cuda()
    row_laws(t, SamplerConfig(0.6, 0.95, 20, presence_penalty=2.0), token_counts={0: 1})
    assert torch.equal(t.cpu(), torch.from_numpy(logits))


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
    ws, nb = _ws(B * (2 * K + 1), V, cfg.top_k)
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


@pytest.mark.parametrize("V,B,K,cfg", [
    (151936, 2, 3, S.SamplerConfig(0.6, 0.95, 0)),
    (151936, 2, 3, S.SamplerConfig(1.0, 1.0, 0)),
    (30000, 4, 3, S.SamplerConfig(0.8, 0.9, 200)),
    (4000, 3, 5, S.SamplerConfig(1.2, 0.98, 0)),
])
def test_spec_accept_wide_laws_token_exact(gpu, V, B, K, cfg):
    rng = np.random.default_rng(V + 7 * B + K)
    target = rng.normal(0, 3, (B, K + 1, V)).astype(np.float32)
    draft = (target[:, :K] + rng.normal(0, 1.0, (B, K, V))).astype(np.float32)
    drafts = np.stack([S.sample_rows(draft[b], rng.random(K), cfg) for b in range(B)])
    uniforms = rng.random((B, K + 1))
    out, nacc, ap, st = _spec(target, draft, drafts, uniforms, cfg)
    assert (st == 0).all()
    for b in range(B):
        want = S.spec_accept(target[b], draft[b], drafts[b], uniforms[b], cfg)
        assert int(nacc[b]) == want.n_accepted, b
        assert out[b, : len(want.tokens)].tolist() == want.tokens, b
        assert np.allclose(ap[b, : len(want.accept_probs)], want.accept_probs, rtol=0, atol=1e-9)


def test_spec_accept_penalties_per_position(gpu):
    """Target and draft row d of a request are penalised with its committed
    counts plus drafts[:d] (mtplx/generation.py:15590-15595)."""
    from collections import Counter

    from mtplx_amd.sampling import SamplerConfig, spec_accept
    rng = np.random.default_rng(21)
    B, K, V = 3, 3, 151936
    cfg = SamplerConfig(0.6, 0.95, 20, presence_penalty=1.5, frequency_penalty=0.25)
    oc = S.SamplerConfig(0.6, 0.95, 20)
    target = rng.normal(0, 3, (B, K + 1, V)).astype(np.float32)
    draft = (target[:, :K] + rng.normal(0, 0.3, (B, K, V))).astype(np.float32)
    drafts = np.stack([np.argsort(-draft[b], axis=1)[:, 0] for b in range(B)]).astype(np.int32)
    counts = [{int(drafts[b, 1]): 2, 5: 1} for b in range(B)]
    uniforms = rng.random((B, K + 1))
    res = spec_accept(torch.from_numpy(target).cuda(), torch.from_numpy(draft).cuda(),
                      torch.from_numpy(drafts).cuda(), torch.from_numpy(uniforms).cuda(), cfg, token_counts=counts)
    torch.cuda.synchronize()
    for b in range(B):
        tl, dl = np.empty_like(target[b]), np.empty_like(draft[b])
        for d in range(K + 1):
            c = Counter(counts[b])
            c.update(int(t) for t in drafts[b, :d])
            tl[d] = S.apply_penalties_f32(target[b, d], c, 1.5, 0.25)
            if d < K:
                dl[d] = S.apply_penalties_f32(draft[b, d], c, 1.5, 0.25)
        want = S.spec_accept(tl, dl, drafts[b], uniforms[b], oc)
        assert int(res.n_accepted[b]) == want.n_accepted
        assert res.tokens[b].cpu().numpy().tolist()[: len(want.tokens)] == want.tokens


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


def _spec_ragged(target_rows, draft_rows, t_off, d_off, k_lens, drafts, uniforms, cfg):
    """mtp_spec_accept_ragged through the facade on host arrays."""
    from mtplx_amd.sampling import SamplerConfig, spec_accept_ragged
    c = SamplerConfig(cfg.temperature, cfg.top_p, cfg.top_k)
    cu = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).astype(dt)).cuda()   # noqa: E731
    res = spec_accept_ragged(cu(target_rows, np.float32), cu(t_off, np.int32), cu(draft_rows, np.float32),
                             cu(d_off, np.int32), cu(k_lens, np.int32), cu(drafts, np.int32), cu(uniforms, np.float64), c)
    torch.cuda.synchronize()
    return (res.tokens.cpu().numpy(), res.n_accepted.cpu().numpy(), res.accept_probs.cpu().numpy(),
            res.status.cpu().numpy())


def _ragged_case(rng, V, k_lens, scale=3.0, corr=0.5):
    """Packed target rows (K_b + 1 per request) and draft rows (K_b per request)."""
    t_off = np.concatenate([[0], np.cumsum(np.asarray(k_lens) + 1)])
    d_off = np.concatenate([[0], np.cumsum(k_lens)])
    target = rng.normal(0, scale, (int(t_off[-1]), V)).astype(np.float32)
    draft = np.concatenate([target[t_off[b]:t_off[b] + k] + rng.normal(0, corr, (k, V))
                            for b, k in enumerate(k_lens)]).astype(np.float32)
    return target, draft, t_off, d_off


def test_spec_accept_ragged_out_of_range_request(gpu):
    """A request whose depth or offsets point outside the buffers is skipped
    on the device with status 2 (tokens -1, nothing accepted); the other
    requests are token-exact against the oracle."""
    cfg = S.SamplerConfig(0.6, 0.95, 20)
    rng = np.random.default_rng(77)
    V = 4096
    k_lens = [3, 2, 1, 3]
    target, draft, t_off, d_off = _ragged_case(rng, V, k_lens)
    drafts = np.concatenate([S.sample_rows(draft[d_off[b]:d_off[b] + k], rng.random(k), cfg)
                             for b, k in enumerate(k_lens)]).astype(np.int32)
    uniforms = rng.random((len(k_lens), 4))
    bad_k = np.array(k_lens, np.int32)
    bad_k[1] = 7                                   # deeper than K_max = 3
    bad_t = t_off[:-1].copy()
    bad_t[2] = int(t_off[-1]) - 1                  # its 2 target rows run past n_target
    bad_d = d_off[:-1].copy()
    bad_d[3] = -1                                  # negative draft offset
    for kl, to, do, hit in ((bad_k, t_off[:-1], d_off[:-1], 1), (np.array(k_lens, np.int32), bad_t, d_off[:-1], 2),
                            (np.array(k_lens, np.int32), t_off[:-1], bad_d, 3)):
        out, nacc, ap, st = _spec_ragged(target, draft, to, do, kl, drafts, uniforms, cfg)
        assert st[hit] == 2 and nacc[hit] == 0 and (out[hit] == -1).all() and (ap[hit] == -1).all()
        for b, k in enumerate(k_lens):
            if b == hit:
                continue
            assert st[b] == 0
            want = S.spec_accept(target[t_off[b]:t_off[b] + k + 1], draft[d_off[b]:d_off[b] + k],
                                 drafts[d_off[b]:d_off[b] + k], uniforms[b], cfg)
            assert int(nacc[b]) == want.n_accepted and out[b, : len(want.tokens)].tolist() == want.tokens


def test_spec_accept_greedy_lane_ragged(gpu):
    """The greedy lane over a ragged batch: each request accepts its drafts
    while they equal the target argmax, corrects with the argmax at the first
    mismatch, and takes the argmax of row K_b as its bonus."""
    cfg = S.SamplerConfig(0.0, 1.0, 0)
    rng = np.random.default_rng(19)
    V = 5000
    k_lens = [3, 1, 2, 3, 1]
    target, draft, t_off, d_off = _ragged_case(rng, V, k_lens, scale=1.0, corr=0.0)
    drafts = np.concatenate([target[t_off[b]:t_off[b] + k].argmax(axis=1) for b, k in enumerate(k_lens)])
    drafts[d_off[3] + 1] = (drafts[d_off[3] + 1] + 1) % V      # request 3 rejects at depth 1
    drafts[d_off[1]] = (drafts[d_off[1]] + 3) % V              # request 1 rejects at depth 0
    out, nacc, ap, st = _spec_ragged(target, draft, t_off[:-1], d_off[:-1], np.array(k_lens), drafts,
                                     np.zeros((len(k_lens), 4)), cfg)
    assert (st == 0).all()
    assert nacc.tolist() == [3, 0, 2, 1, 1]
    for b, k in enumerate(k_lens):
        arg = target[t_off[b]:t_off[b] + k + 1].argmax(axis=1)
        want = []
        for d in range(k + 1):
            if d == k or drafts[d_off[b] + d] != arg[d]:
                want.append(int(arg[d]))
                break
            want.append(int(drafts[d_off[b] + d]))
        assert out[b, : len(want)].tolist() == want, b
        assert (out[b, len(want):] == -1).all()
    assert out[3, :2].tolist() == [drafts[d_off[3]], int(target[t_off[3] + 1].argmax())]
    assert out[0, 3] == int(target[t_off[0] + 3].argmax())
