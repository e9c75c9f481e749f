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


def test_spec_accept_uniform_consumption():
    cfg = S.SamplerConfig(0.6, 0.95, 20)
    rng = np.random.default_rng(9)
    V, K = 64, 3
    tl = rng.normal(0, 3, (K + 1, V)); dl = tl[:K] + rng.normal(0, 0.3, (K, V))
    drafts = S.sample_rows(dl, rng.random(K), cfg)
    # all-accept path: uniforms 0 accept everything -> bonus uses u[K]
    res = S.spec_accept(tl, dl, drafts, np.array([0.0] * K + [0.5]), cfg)
    assert res.n_accepted == K and res.uniforms_used == K + 1 and res.tokens[:K] == drafts.tolist()
    # a reject at depth 0 consumes exactly two uniforms
    res = S.spec_accept(tl, dl, drafts, np.array([1.0, 0.3, 0.0, 0.0]), cfg)
    if res.accept_probs[0] < 1.0:
        assert res.n_accepted == 0 and res.uniforms_used == 2 and len(res.tokens) == 1
