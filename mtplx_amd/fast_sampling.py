"""The runtime sampler's device surface (``mtplx/fast_sampling.py``) on gfx950.

Same names, arguments and ``None`` conventions as the reference's MLX twin of
``sampling.py``; the arrays are torch tensors on the GPU instead of MLX
arrays, and the device work is the HIP sampler (``mtp_sample_rows``:
full-vocabulary softmax statistics in fp64, deterministic top-k with ties to
the lower id, top-p over the full-vocabulary mass, the support's ids
ascending, fp64 probabilities), so every row's law is the host reference's
(``mtplx/sampling.py:259``) bit for bit in its ids.

* ``apply_penalties_mlx`` (:42): the additive presence/frequency penalty and
  the overlay on one raw logit row (``mtp_apply_logit_deltas``);
* ``sparse_distribution_from_mlx_logits`` (:637) and the batched readers
  ``SparseDistributionRows`` (:716), ``sparse_distribution_rows_from_mlx_logits``
  (:780), ``sparse_distributions_from_mlx_logits`` (:795),
  ``batched_sparse_distributions_from_mlx_logits`` (:826) with
  ``BatchedSparseDistributions`` (:84): ``None`` when greedy or without a
  top-k bound, as in the reference; a non-finite row raises
  ``NonFiniteLogitsError`` when it is read;
* ``sample_token_ids_from_mlx_logits`` (:861): one id per row on the device;
  greedy is the argmax, otherwise a draw from the row's exact law with
  uniforms from ``generator`` (or the ``uniforms`` given), where the
  reference draws from MLX's global generator.
"""

from __future__ import annotations

from typing import Mapping

import numpy as np
import torch

from .sampling import (NonFiniteLogitsError, SamplerConfig, SparseDistribution, apply_penalties, row_laws,
                       sparse_distributions_from_logits)

MAX_DEVICE_TOP_K_ORDER = 32   # the reference's device bound (:22); the gfx950 sampler takes any top_k


def apply_penalties_mlx(logits: torch.Tensor, token_counts: Mapping[int, int] | None, presence_penalty: float = 0.0,
                        frequency_penalty: float = 0.0,
                        penalty_overlay: Mapping[int, float] | None = None) -> torch.Tensor:
    """One raw logit row ``[V]`` with the additive penalty subtracted on the
    device (penalties clamped to [-2, 2]; the overlay unclamped). Returns the
    same tensor when nothing is active (the exact no-op)."""
    cfg = SamplerConfig(presence_penalty=float(presence_penalty), frequency_penalty=float(frequency_penalty))
    row = logits.reshape(1, -1).to(torch.float32).contiguous()
    out = apply_penalties(row, cfg, [token_counts], [penalty_overlay])
    return logits if out is row else out.reshape(logits.shape)


def _bounded(config: SamplerConfig) -> bool:
    return float(config.temperature) > 0.0 and int(config.top_k) > 0


def sparse_distribution_from_mlx_logits(logits: torch.Tensor, config: SamplerConfig, *,
                                        token_counts: Mapping[int, int] | None = None,
                                        penalty_overlay: Mapping[int, float] | None = None
                                        ) -> SparseDistribution | None:
    """The exact sparse law of one logit row (penalties applied to the raw
    logits first), or None when greedy or without a top-k bound."""
    if not _bounded(config):
        return None
    return sparse_distributions_from_logits(logits.reshape(1, -1), config, token_counts=token_counts,
                                            penalty_overlay=penalty_overlay)[0]


class SparseDistributionRows:
    """Per-row exact sparse laws of a block of logit rows, row ``i`` equal to
    ``sparse_distribution_from_mlx_logits(logits[i], config)``. The device
    builds every row's law in one launch on the first read (one host round
    trip for the block); a non-finite row raises ``NonFiniteLogitsError``
    only when that row is read."""

    __slots__ = ("_logits", "_config", "_ids", "_probs", "_count", "_status")

    def __init__(self, logits: torch.Tensor, config: SamplerConfig) -> None:
        self._logits = logits.reshape(-1, logits.shape[-1])
        self._config = config
        self._ids = None
        self._probs = self._count = self._status = None

    def __len__(self) -> int:
        return int(self._logits.shape[0])

    def _read(self) -> None:
        laws = row_laws(self._logits, self._config)
        self._ids = laws.ids.cpu().numpy()
        self._probs = laws.probs.cpu().numpy()
        self._count = laws.count.cpu().numpy()
        self._status = laws.status.cpu().numpy()

    def __getitem__(self, index: int) -> SparseDistribution:
        index = int(index)
        if not 0 <= index < len(self):
            raise IndexError(f"row {index} of {len(self)}")
        if self._ids is None:
            self._read()
        if self._status[index]:
            raise NonFiniteLogitsError(f"logits row {index} has no finite mass")
        n = int(self._count[index])
        return SparseDistribution(self._ids[index, :n], self._probs[index, :n], int(self._logits.shape[-1]))


def sparse_distribution_rows_from_mlx_logits(logits: torch.Tensor,
                                             config: SamplerConfig) -> SparseDistributionRows | None:
    """Per-row laws read as a block, or None exactly where
    ``sparse_distribution_from_mlx_logits`` returns None."""
    if not _bounded(config):
        return None
    return SparseDistributionRows(logits, config)


def sparse_distributions_from_mlx_logits(logits: torch.Tensor,
                                         config: SamplerConfig) -> list[SparseDistribution] | None:
    """Exact sparse laws of a batch of logit rows (one device pass)."""
    if not _bounded(config):
        return None
    return sparse_distributions_from_logits(logits.reshape(-1, logits.shape[-1]), config)


class BatchedSparseDistributions:
    """Sparse laws of several rows as ``[rows, k]`` arrays: ids ascending
    within a row, probabilities renormalised per row (slots past a row's
    support hold id -1 and probability 0)."""

    def __init__(self, token_ids: np.ndarray, probs: np.ndarray, *, vocab_size: int) -> None:
        token_ids = np.asarray(token_ids, dtype=np.int64)
        probs = np.asarray(probs, dtype=np.float64)
        if token_ids.ndim != 2 or probs.ndim != 2:
            raise ValueError("BatchedSparseDistributions expects 2D arrays")
        if token_ids.shape != probs.shape:
            raise ValueError("token_ids/probs shape mismatch")
        row_sums = probs.sum(axis=1)
        if np.any(row_sums <= 0) or not np.all(np.isfinite(row_sums)):
            raise ValueError("each sparse distribution row needs positive mass")
        self.token_ids = token_ids
        self.probs = probs / row_sums[:, None]
        self.vocab_size = int(vocab_size)

    def probability(self, row: int, token_id: int) -> float:
        hits = np.nonzero(self.token_ids[int(row)] == int(token_id))[0]
        return 0.0 if hits.size == 0 else float(self.probs[int(row), int(hits[0])])

    def to_distribution(self, row: int) -> SparseDistribution:
        keep = self.probs[int(row)] > 0
        return SparseDistribution(self.token_ids[int(row), keep], self.probs[int(row), keep], self.vocab_size)

    def sample(self, row: int, rng: np.random.Generator) -> int:
        keep = self.probs[int(row)] > 0
        return int(rng.choice(self.token_ids[int(row), keep], p=self.probs[int(row), keep]))


def batched_sparse_distributions_from_mlx_logits(logits: torch.Tensor,
                                                 config: SamplerConfig) -> BatchedSparseDistributions | None:
    """The batch's laws without per-row Python objects, or None when greedy
    or without a top-k bound."""
    if not _bounded(config):
        return None
    rows = logits.reshape(-1, logits.shape[-1])
    laws = row_laws(rows, config)
    st = laws.status.cpu().numpy()
    if st.any():
        raise NonFiniteLogitsError(f"non-finite logits in rows {np.nonzero(st)[0].tolist()}")
    ids = laws.ids.cpu().numpy().astype(np.int64)
    probs = laws.probs.cpu().numpy()
    cnt = laws.count.cpu().numpy()
    for r in range(ids.shape[0]):   # slots past the support: id -1, probability 0
        probs[r, cnt[r]:] = 0.0
        ids[r, cnt[r]:] = -1
    return BatchedSparseDistributions(ids, probs, vocab_size=int(rows.shape[-1]))


def sample_token_ids_from_mlx_logits(logits: torch.Tensor, config: SamplerConfig, *,
                                     uniforms: torch.Tensor | None = None,
                                     generator: torch.Generator | None = None) -> torch.Tensor | None:
    """One token id per row on the device (int32 ``[rows]``): the argmax when
    greedy; otherwise a draw from the row's exact top-k / top-p law with one
    uniform per row (``uniforms``, or drawn from ``generator`` on the
    logits' device). None without a top-k bound and with a nucleus, as in
    the reference."""
    rows = logits.reshape(-1, logits.shape[-1])
    if not float(config.temperature) > 0.0:
        return row_laws(rows, config).ids[:, 0].contiguous()   # the greedy one-hot law: argmax, ties to the lower id
    if int(config.top_k) <= 0 and 0.0 < float(config.top_p) < 1.0:
        return None
    if uniforms is None:
        uniforms = torch.rand(int(rows.shape[0]), dtype=torch.float64, device=rows.device, generator=generator)
    return row_laws(rows, config, uniforms).sampled
