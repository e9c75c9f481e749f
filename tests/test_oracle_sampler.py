"""Pins for oracle.sampler: the reference's known answers, NumPy's choice, the law."""

import itertools

import numpy as np
import pytest

from oracle import sampler as S


def test_distribution_normalizes_after_filtering():
    # tests/test_sampling.py:22-26
    p = S.distribution_from_logits(np.array([4.0, 3.0, 2.0, 1.0]), S.SamplerConfig(0.6, 0.9, 2))
    assert np.isclose(p.sum(), 1.0) and np.count_nonzero(p) <= 2


def test_acceptance_caps_at_one():
    # tests/test_sampling.py:29-33
    assert S.acceptance_probability(0.8, 0.4) == 1.0
    assert np.isclose(S.acceptance_probability(0.2, 0.6), 1 / 3)
    assert S.acceptance_probability(0.3, 0.0) == 1.0 and S.acceptance_probability(0.0, 0.0) == 0.0


def test_residual_positive_mass():
    # tests/test_sampling.py:36-42
    r = S.residual(S.sparse_from_dense(np.array([0.6, 0.3, 0.1])), S.sparse_from_dense(np.array([0.2, 0.5, 0.3])))
    assert r.ids.tolist() == [0] and r.probs.tolist() == [1.0]


def test_sparse_residual_union():
    # tests/test_sampling.py:62-75
    t = S.Sparse.make(np.array([2, 5, 9]), np.array([0.5, 0.3, 0.2]))
    d = S.Sparse.make(np.array([5]), np.array([1.0]))
    assert np.isclose(S.acceptance_probability(t.probability(5), d.probability(5)), 0.3)
    r = S.residual(t, d)
    assert r.ids.tolist() == [2, 9] and np.allclose(r.probs, [5 / 7, 2 / 7])


def test_zero_mass_is_hard_error():
    # tests/test_sampling.py:86-94
    with pytest.raises(S.NonFiniteLogitsError):
        S.Sparse.make(np.array([7, 11]), np.array([0.0, np.nan]))


def test_residual_without_mass_falls_back_to_target():
    t = S.Sparse.make(np.array([1, 3]), np.array([0.25, 0.75]))
    assert S.residual(t, t) is t


def test_choice_matches_numpy_generator_draw_for_draw():
    rng = np.random.default_rng(7)
    for trial in range(200):
        n = int(rng.integers(1, 30))
        ids = np.sort(rng.choice(1000, size=n, replace=False))
        p = rng.random(n) ** 3
        dist = S.Sparse.make(ids, p)
        seed = 1000 + trial
        want = int(np.random.default_rng(seed).choice(dist.ids, p=dist.probs))
        u = float(np.random.default_rng(seed).random())
        assert S.choice(dist, u) == want


def test_uniform_stream_equals_sequential_random_calls():
    a = np.random.default_rng(11)
    seq = [a.random() for _ in range(5)]
    assert np.array_equal(np.random.default_rng(11).random(5), np.array(seq))


def test_top_p_uses_full_vocab_mass_in_topk_order():
    logits = np.log(np.array([0.5, 0.3, 0.1, 0.06, 0.04]))
    p = S.distribution_from_logits(logits, S.SamplerConfig(1.0, 0.85, 3))
    # cumulative-before: 0, .5, .8 (< .85) -> all three of the top-3 kept
    assert np.count_nonzero(p) == 3
    p = S.distribution_from_logits(logits, S.SamplerConfig(1.0, 0.79, 3))
    assert np.count_nonzero(p) == 2


def test_ties_break_by_lower_id():
    logits = np.array([1.0, 3.0, 3.0, 3.0, 0.0])
    p = S.distribution_from_logits(logits, S.SamplerConfig(1.0, 1.0, 2))
    assert np.nonzero(p)[0].tolist() == [1, 2]


def test_output_marginal_recovers_target():
    # tests/test_sampling.py:55-59
    t = np.array([0.55, 0.25, 0.15, 0.05]); d = np.array([0.10, 0.55, 0.20, 0.15])
    assert np.allclose(S.output_marginal(t, d), t)


def test_spec_accept_law_by_enumeration():
    """Depth-2 law on a 4-token vocabulary: summing over draft paths weighted by
    q and over accept/reject outcomes reproduces the target law at depth 0,
    and the committed-prefix law factorises (method of
    tests/test_block_verify_exact_law.py)."""
    cfg = S.SamplerConfig(1.0, 1.0, 0)
    rng = np.random.default_rng(5)
    V, K = 4, 2
    tl = rng.normal(size=(K + 1, V)); dl = rng.normal(size=(K, V))
    p = [S.distribution_from_logits(tl[d], cfg) for d in range(K + 1)]
    q = [S.distribution_from_logits(dl[d], cfg) for d in range(K)]
    law0 = np.zeros(V)
    # Uniform integration by fine stratification of u for each stage.
    grid = (np.arange(400) + 0.5) / 400
    for d0, d1 in itertools.product(range(V), repeat=2):
        w = q[0][d0] * q[1][d1]
        for u0 in grid:
            if u0 <= S.acceptance_probability(p[0][d0], q[0][d0]):
                law0[d0] += w / len(grid)
            else:
                r = S.residual(S.sparse_from_dense(p[0]), S.sparse_from_dense(q[0]))
                for t, pr in zip(r.ids, r.probs):
                    law0[t] += w * pr / len(grid)
    assert np.allclose(law0, p[0], atol=3e-3)


def _law_logits(*rows):
    """Logit rows whose T=1 softmax is the given law exactly (log p; -inf for 0)."""
    with np.errstate(divide="ignore"):
        return np.log(np.array(rows, dtype=np.float64))


_FULL = S.SamplerConfig(1.0, 1.0, 0)   # no top-k, no nucleus: the law is softmax(l)


@pytest.mark.parametrize("u1,want", [(0.5, 0), (0.7, 1)])
def test_spec_accept_reject_at_depth0_known_answer(u1, want):
    """p0 = [.5,.3,.2,0], q0 = [.1,.1,.8,0], draft 2: a = .2/.8 = .25; u0 = .6
    rejects; residual max(p-q,0) = [.4,.2] -> [2/3,1/3] over ids [0,1];
    Generator.choice with u1 picks #{cdf <= u1}."""
    tl = _law_logits([.5, .3, .2, 0], [.25, .25, .25, .25], [.25, .25, .25, .25])
    dl = _law_logits([.1, .1, .8, 0], [.25, .25, .25, .25])
    res = S.spec_accept(tl, dl, np.array([2, 1]), np.array([0.6, u1, 0.0]), _FULL)
    assert res.n_accepted == 0 and res.uniforms_used == 2
    assert res.tokens == [want]
    assert np.isclose(res.accept_probs[0], 0.25) and len(res.accept_probs) == 1


@pytest.mark.parametrize("u2,want", [(0.2, 2), (0.3, 3)])
def test_spec_accept_reject_at_depth1_known_answer(u2, want):
    """Depth 0 accepts (u0 = .2 <= a0 = .25); depth 1: p1 = [.1,.2,.3,.4],
    q1 = [.4,.3,.2,.1], draft 0: a1 = .25, u1 = .9 rejects; residual
    [0,0,.1,.3] -> [.25,.75] over ids [2,3], drawn with u2."""
    tl = _law_logits([.5, .3, .2, 0], [.1, .2, .3, .4], [.25, .25, .25, .25])
    dl = _law_logits([.1, .1, .8, 0], [.4, .3, .2, .1])
    res = S.spec_accept(tl, dl, np.array([2, 0]), np.array([0.2, 0.9, u2]), _FULL)
    assert res.n_accepted == 1 and res.uniforms_used == 3 and res.tokens == [2, want]
    assert np.allclose(res.accept_probs, [0.25, 0.25])


@pytest.mark.parametrize("u2,want", [(0.1, 0), (0.3, 1), (0.6, 2)])
def test_spec_accept_all_accept_bonus_known_answer(u2, want):
    """Every draft accepted (u = 0 <= a > 0): the bonus is
    choice(law of target row K, u[K]); row K = [.25,.25,.5,0] has cdf
    [.25,.5,1]."""
    tl = _law_logits([.5, .3, .2, 0], [.1, .2, .3, .4], [.25, .25, .5, 0])
    dl = _law_logits([.1, .1, .8, 0], [.4, .3, .2, .1])
    res = S.spec_accept(tl, dl, np.array([2, 3]), np.array([0.0, 0.0, u2]), _FULL)
    assert res.n_accepted == 2 and res.uniforms_used == 3 and res.tokens == [2, 3, want]
    assert np.allclose(res.accept_probs, [0.25, 1.0])


def test_spec_accept_uniform_consumption():
    cfg = S.SamplerConfig(0.6, 0.95, 20)
    rng = np.random.default_rng(9)
    V, K = 64, 3
    tl = rng.normal(0, 3, (K + 1, V)); dl = tl[:K] + rng.normal(0, 0.3, (K, V))
    drafts = S.sample_rows(dl, rng.random(K), cfg)
    # all-accept path: uniforms 0 accept everything -> bonus uses u[K]
    res = S.spec_accept(tl, dl, drafts, np.array([0.0] * K + [0.5]), cfg)
    assert res.n_accepted == K and res.uniforms_used == K + 1 and res.tokens[:K] == drafts.tolist()
    # a draft outside the target's support has a = 0: u0 = 1 rejects it and
    # exactly two uniforms are consumed
    p0 = S.sparse_distribution(tl[0], cfg)
    outside = next(t for t in range(V) if p0.probability(t) == 0.0)
    res = S.spec_accept(tl, dl, np.array([outside] + drafts[1:].tolist()), np.array([1.0, 0.3, 0.0, 0.0]), cfg)
    assert res.accept_probs[0] == 0.0
    assert res.n_accepted == 0 and res.uniforms_used == 2 and len(res.tokens) == 1
    assert res.tokens[0] == S.choice(S.residual(p0, S.sparse_distribution(dl[0], cfg)), 0.3)


# -- penalties: tests/test_penalties.py:31-95 known answers -------------------

_PEN = S.SamplerConfig(1.0, 1.0, 0)


def test_presence_penalty_demotes_a_seen_token():
    p = S.distribution_from_logits(np.array([5.0, 4.0, 0.0, 0.0]), _PEN, {0: 3}, presence=2.0)
    assert int(np.argmax(p)) == 1


def test_frequency_penalty_scales_with_count():
    lg = np.array([5.0, 4.0, 0.0, 0.0])
    assert int(np.argmax(S.distribution_from_logits(lg, _PEN, {0: 4}, frequency=0.5))) == 1
    assert int(np.argmax(S.distribution_from_logits(lg, _PEN, {0: 1}, frequency=0.5))) == 0


def test_zero_penalties_are_identical_and_clamped_range():
    lg = np.array([5.0, 4.0, 3.0, 2.0, 1.0])
    cfg = S.SamplerConfig(0.7, 0.9, 3)
    assert np.array_equal(S.distribution_from_logits(lg, cfg),
                          S.distribution_from_logits(lg, cfg, {0: 3, 1: 2}, 0.0, 0.0))
    assert S.apply_penalties(lg, {0: 3}, 0.0, 0.0) is lg
    # presence 100 clamps to 2: 5 -> 3 still above 2
    assert int(np.argmax(S.distribution_from_logits(np.array([5.0, 2.0]), _PEN, {0: 1}, presence=100.0))) == 0


def test_device_twin_matches_host_law():
    raw = np.array([5.0, 4.0, 3.0, 1.0, 0.0])
    counts = {0: 3, 2: 1}
    host = S.apply_penalties(raw, counts, 1.5, 0.5)
    twin = S.apply_penalties_f32(raw, counts, 1.5, 0.5)
    assert twin.dtype == np.float32 and np.allclose(twin, host, atol=1e-5)
    assert host.tolist() == [5.0 - 1.5 - 1.5, 4.0, 3.0 - 0.5 - 1.5, 1.0, 0.0]
    ov = S.apply_penalties_f32(raw, None, 0.0, 0.0, {1: 0.25})
    assert ov.tolist() == [5.0, 3.75, 3.0, 1.0, 0.0]
