"""Sampler law and the depth-K speculative accept/reject step, float64.

Restates the reference's NumPy sampler (``mtplx/sampling.py``) and the order
in which ``generate_mtpk`` consumes uniforms (``mtplx/generation.py:15560-15790``
for the per-depth accept, ``:16085-16110`` for the all-accept bonus), with
NumPy's weighted ``Generator.choice`` written out as the cdf/searchsorted rule
the reference documents (``mtplx/qwen4_draft_device_chain.py:294-305``).

Penalties: the host law (``apply_penalties``, fp64) and the runtime's
device twin (``apply_penalties_f32``, fp32 deltas), which the GPU path
follows.

Parity pins (tests/test_oracle_sampler.py): the reference's own known-answer
tests (``tests/test_sampling.py:22-103``) re-expressed; penalty closed forms; ``choice`` checked
against ``numpy.random.Generator.choice`` draw for draw; the output-marginal
law (``mtplx/sampling.py:372-391``) and exhaustive enumeration of draft paths
on a tiny vocabulary (the method of ``tests/test_block_verify_exact_law.py``).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


class NonFiniteLogitsError(RuntimeError):
    """A row had no finite positive mass (``mtplx/sampling.py:32-70``)."""


@dataclass(frozen=True)
class SamplerConfig:
    """``mtplx/sampling.py:22-29`` defaults; penalties are a no-op at 0."""

    temperature: float = 0.6
    top_p: float = 0.95
    top_k: int = 20


PENALTY_MIN, PENALTY_MAX = -2.0, 2.0


def apply_penalties(logits: np.ndarray, token_counts, presence: float = 0.0, frequency: float = 0.0,
                    overlay=None) -> np.ndarray:
    """Host law ``mtplx/sampling.py:212-256``: in fp64, ``l[j] -= frequency *
    count[j] + presence * (count[j] > 0)`` (penalties clamped to [-2, 2]),
    then ``l[j] -= overlay[j]``; a no-op (same array) when nothing is active."""
    pres = float(np.clip(presence, PENALTY_MIN, PENALTY_MAX))
    freq = float(np.clip(frequency, PENALTY_MIN, PENALTY_MAX))
    counts_on = bool(token_counts) and (pres != 0.0 or freq != 0.0)
    if not counts_on and not overlay:
        return logits
    out = np.array(logits, dtype=np.float64, copy=True)
    if counts_on:
        ids = np.fromiter(token_counts.keys(), dtype=np.int64, count=len(token_counts))
        c = np.fromiter(token_counts.values(), dtype=np.float64, count=len(token_counts))
        out[ids] -= freq * c + pres * (c > 0)
    if overlay:
        ids = np.fromiter(overlay.keys(), dtype=np.int64, count=len(overlay))
        out[ids] -= np.fromiter(overlay.values(), dtype=np.float64, count=len(overlay))
    return out


def apply_penalties_f32(logits: np.ndarray, token_counts, presence: float = 0.0, frequency: float = 0.0,
                        overlay=None) -> np.ndarray:
    """The runtime's device twin ``mtplx/fast_sampling.py:42-81``
    (``apply_penalties_mlx``): the same deltas computed in fp64, cast to fp32,
    and added negated to the fp32 logits in fp32 (counts first, then the
    overlay, each one rounding)."""
    pres = float(np.clip(presence, PENALTY_MIN, PENALTY_MAX))
    freq = float(np.clip(frequency, PENALTY_MIN, PENALTY_MAX))
    counts_on = bool(token_counts) and (pres != 0.0 or freq != 0.0)
    out = np.array(logits, dtype=np.float32, copy=True)
    if counts_on:
        ids = np.fromiter(token_counts.keys(), dtype=np.int64, count=len(token_counts))
        c = np.fromiter(token_counts.values(), dtype=np.float64, count=len(token_counts))
        out[ids] = out[ids] + (-(freq * c + pres * (c > 0.0)).astype(np.float32))
    if overlay:
        ids = np.fromiter(overlay.keys(), dtype=np.int64, count=len(overlay))
        v = np.fromiter(overlay.values(), dtype=np.float64, count=len(overlay)).astype(np.float32)
        out[ids] = out[ids] + (-v)
    return out


def softmax(logits: np.ndarray, temperature: float = 1.0) -> np.ndarray:
    """``mtplx/sampling.py:131-143``: fp64 ``exp(l/T - max)/sum``; T<=0 -> one-hot argmax."""
    logits = np.asarray(logits, dtype=np.float64)
    if temperature <= 0:
        out = np.zeros_like(logits)
        out[int(np.argmax(logits))] = 1.0
        return out
    scaled = logits / float(temperature)
    scaled = scaled - np.max(scaled)
    e = np.exp(scaled)
    total = e.sum()
    if not np.isfinite(total) or total <= 0:
        raise NonFiniteLogitsError("non-finite logits in softmax")
    return e / total


def deterministic_top_k_order(values: np.ndarray, top_k: int) -> np.ndarray:
    """Ids of the ``top_k`` largest values, value descending then id ascending
    (``mtplx/sampling.py:146-163``)."""
    values = np.asarray(values, dtype=np.float64)
    count = min(max(int(top_k), 0), values.shape[0])
    if count == 0:
        return np.empty(0, dtype=np.int64)
    ids = np.arange(values.shape[0], dtype=np.int64)
    # lexsort: last key primary -> (-value) then id.
    order = np.lexsort((ids, -values))
    return order[:count].astype(np.int64)


def apply_top_p_top_k(probs: np.ndarray, top_p: float = 1.0, top_k: int = 0) -> np.ndarray:
    """``mtplx/sampling.py:166-201``. Nucleus over the full-vocab probabilities
    in top-k order (``cumulative_before < top_p``), intersected with top-k,
    renormalised; an empty result falls back to the argmax one-hot."""
    probs = np.asarray(probs, dtype=np.float64)
    size = probs.shape[0]
    bounded_k = int(top_k) if top_k and 0 < int(top_k) < size else 0
    mask = np.ones(size, dtype=bool)
    ranked = deterministic_top_k_order(probs, bounded_k) if bounded_k else None
    if 0 < top_p < 1.0:
        order = ranked if ranked is not None else deterministic_top_k_order(probs, size)
        cum = np.cumsum(probs[order])
        before = np.concatenate(([0.0], cum[:-1]))
        nucleus = np.zeros(size, dtype=bool)
        nucleus[order[before < top_p]] = True
        mask &= nucleus
    if bounded_k:
        top = np.zeros(size, dtype=bool)
        top[ranked] = True
        mask &= top
    filtered = np.where(mask, probs, 0.0)
    total = filtered.sum()
    if total <= 0:
        filtered[int(np.argmax(probs))] = 1.0
        return filtered
    return filtered / total


def distribution_from_logits(logits: np.ndarray, config: SamplerConfig, token_counts=None, presence: float = 0.0,
                             frequency: float = 0.0, overlay=None) -> np.ndarray:
    """Dense law ``mtplx/sampling.py:259-276``: penalties (host law) on the raw
    logits, softmax with temperature, then top-p / top-k."""
    logits = apply_penalties(logits, token_counts, presence, frequency, overlay)
    return apply_top_p_top_k(softmax(logits, config.temperature), config.top_p, config.top_k)


@dataclass(frozen=True)
class Sparse:
    """Ids ascending + probabilities, normalised on construction
    (``mtplx/sampling.py:86-128``; ascending ids as ``fast_sampling.py:619-634`` emits)."""

    ids: np.ndarray
    probs: np.ndarray

    @staticmethod
    def make(ids: np.ndarray, probs: np.ndarray) -> "Sparse":
        ids = np.asarray(ids, dtype=np.int64)
        probs = np.asarray(probs, dtype=np.float64)
        clean = np.where(np.isfinite(probs) & (probs > 0), probs, 0.0)
        total = clean.sum()
        if not np.isfinite(total) or total <= 0:
            raise NonFiniteLogitsError("SparseDistribution without finite mass")
        return Sparse(ids, clean / total)

    def probability(self, token: int) -> float:
        hit = np.nonzero(self.ids == int(token))[0]
        return 0.0 if hit.size == 0 else float(self.probs[hit[0]])


def sparse_from_dense(dense: np.ndarray) -> Sparse:
    keep = np.nonzero(dense > 0)[0]
    return Sparse.make(keep, dense[keep])


def sparse_distribution(logits: np.ndarray, config: SamplerConfig) -> Sparse:
    """The runtime's sparse law: the dense law's support, ids ascending."""
    return sparse_from_dense(distribution_from_logits(logits, config))


def acceptance_probability(p: float, q: float) -> float:
    """``mtplx/sampling.py:295-300``: ``min(1, p/q)``; q<=0 -> 1 if p>0 else 0."""
    if q <= 0:
        return 1.0 if p > 0 else 0.0
    return min(1.0, p / q)


def residual(target: Sparse, draft: Sparse) -> Sparse:
    """``mtplx/sampling.py:303-315``: ``max(p-q, 0)`` over the union of supports
    (ids ascending), renormalised; no positive mass -> the target itself."""
    ids = np.union1d(target.ids, draft.ids).astype(np.int64)
    r = np.array([max(target.probability(t) - draft.probability(t), 0.0) for t in ids], dtype=np.float64)
    r = np.where(np.isfinite(r) & (r > 0), r, 0.0)
    keep = r > 0
    total = r[keep].sum()
    if not np.isfinite(total) or total <= 0:
        return target
    return Sparse.make(ids[keep], r[keep] / total)


def choice(dist: Sparse, u: float) -> int:
    """``Generator.choice(ids, p=probs)`` given its one uniform:
    ``cdf = cumsum(p); cdf /= cdf[-1]; idx = searchsorted(cdf, u, 'right')``
    (``mtplx/qwen4_draft_device_chain.py:294-305``)."""
    cdf = np.cumsum(dist.probs)
    cdf = cdf / cdf[-1]
    idx = int(np.searchsorted(cdf, float(u), side="right"))
    return int(dist.ids[min(idx, dist.ids.shape[0] - 1)])


@dataclass(frozen=True)
class AcceptResult:
    tokens: list          # committed ids: accepted drafts then correction/bonus
    n_accepted: int
    accept_probs: list    # min(1, p/q) per examined depth
    uniforms_used: int


def spec_accept(target_logits: np.ndarray, draft_logits: np.ndarray, draft_ids: np.ndarray,
                uniforms: np.ndarray, config: SamplerConfig) -> AcceptResult:
    """One request's depth-K accept/reject step.

    ``target_logits`` [K+1, V] (verify rows; row K is the bonus row),
    ``draft_logits`` [K, V], ``draft_ids`` [K], ``uniforms`` [>=K+1] consumed in
    stream order exactly as ``generate_mtpk`` consumes ``rng.random()``:
    depth d draws u for ``u <= a_d`` (``generation.py:15630-15640``); the first
    rejection samples the residual with the next uniform and stops; if every
    draft is accepted the bonus is drawn from row K with the next uniform
    (``generation.py:16085-16110``). Stop tokens are out of scope here.
    """
    K = int(np.asarray(draft_ids).shape[0])
    tokens: list[int] = []
    probs: list[float] = []
    ui = 0
    for d in range(K):
        p_dist = sparse_distribution(target_logits[d], config)
        q_dist = sparse_distribution(draft_logits[d], config)
        tok = int(draft_ids[d])
        a = acceptance_probability(p_dist.probability(tok), q_dist.probability(tok))
        probs.append(a)
        u = float(uniforms[ui]); ui += 1
        if u <= a:
            tokens.append(tok)
            continue
        tokens.append(choice(residual(p_dist, q_dist), float(uniforms[ui]))); ui += 1
        return AcceptResult(tokens, d, probs, ui)
    bonus = sparse_distribution(target_logits[K], config)
    tokens.append(choice(bonus, float(uniforms[ui]))); ui += 1
    return AcceptResult(tokens, K, probs, ui)


def sample_rows(logits: np.ndarray, uniforms: np.ndarray, config: SamplerConfig) -> np.ndarray:
    """One draw per row from the sparse law (``sample_from_distribution``,
    ``mtplx/sampling.py:342-349``), uniform ``uniforms[r]`` for row ``r``."""
    return np.array([choice(sparse_distribution(logits[r], config), float(uniforms[r]))
                     for r in range(logits.shape[0])], dtype=np.int64)


def output_marginal(p: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Exact output law of one-token speculative sampling
    (``mtplx/sampling.py:372-391``); must equal ``p``."""
    p = np.asarray(p, dtype=np.float64); p = p / p.sum()
    q = np.asarray(q, dtype=np.float64); q = q / q.sum()
    pd, qd = sparse_from_dense(p), sparse_from_dense(q)
    res = residual(pd, qd)
    r_dense = np.zeros_like(p); r_dense[res.ids] = res.probs
    out = np.zeros_like(p)
    for t, qv in enumerate(q):
        a = acceptance_probability(p[t], qv)
        out[t] += qv * a
        if a < 1.0:
            out += qv * (1.0 - a) * r_dense
    return out / out.sum()
