"""Speculative accept/reject primitives (``mtplx/speculative.py`` re-exports).

The batched GPU step is :func:`mtplx_amd.sampling.spec_accept` (logits in,
committed ids out). The per-token helpers below keep the reference's host
API on :class:`SparseDistribution` supports (at most top_k + top_k ids), with
the reference's semantics (``mtplx/sampling.py:295-391``); they are the
bookkeeping a caller uses after the GPU has built the laws.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .sampling import SparseDistribution, spec_accept  # noqa: F401

__all__ = ["SpeculativeDecision", "acceptance_probability", "residual_distribution", "sample_from_distribution",
           "speculative_output_marginal", "verify_one_token", "spec_accept"]


@dataclass(frozen=True)
class SpeculativeDecision:
    accepted: bool
    token_id: int
    accept_probability: float


def acceptance_probability(target_p: SparseDistribution, draft_q: SparseDistribution, token_id: int) -> float:
    p, q = target_p.probability(token_id), draft_q.probability(token_id)
    if q <= 0:
        return 1.0 if p > 0 else 0.0
    return min(1.0, p / q)


def residual_distribution(target_p: SparseDistribution, draft_q: SparseDistribution) -> SparseDistribution:
    ids = np.union1d(target_p.token_ids, draft_q.token_ids).astype(np.int64)
    r = np.array([max(target_p.probability(int(t)) - draft_q.probability(int(t)), 0.0) for t in ids])
    r = np.where(np.isfinite(r) & (r > 0), r, 0.0)
    keep = r > 0
    total = r[keep].sum()
    if not np.isfinite(total) or total <= 0:
        return target_p
    return SparseDistribution(ids[keep], r[keep] / total, target_p.vocab_size)


def sample_from_distribution(probs: SparseDistribution, rng: np.random.Generator | None = None) -> int:
    rng = rng or np.random.default_rng()
    return int(rng.choice(probs.token_ids, p=probs.probs))


def verify_one_token(target_p: SparseDistribution, draft_q: SparseDistribution, draft_token: int,
                     rng: np.random.Generator | None = None) -> SpeculativeDecision:
    rng = rng or np.random.default_rng()
    a = acceptance_probability(target_p, draft_q, draft_token)
    if float(rng.random()) <= a:
        return SpeculativeDecision(True, int(draft_token), a)
    return SpeculativeDecision(False, sample_from_distribution(residual_distribution(target_p, draft_q), rng), a)


def speculative_output_marginal(target_p: SparseDistribution, draft_q: SparseDistribution) -> np.ndarray:
    p, q = target_p.to_dense(), draft_q.to_dense()
    res = residual_distribution(target_p, draft_q).to_dense()
    out = np.zeros_like(p)
    for t, qv in enumerate(q):
        a = acceptance_probability(target_p, draft_q, t) if qv > 0 else 0.0
        out[t] += qv * a
        if a < 1.0:
            out += qv * (1.0 - a) * res
    return out / out.sum()
