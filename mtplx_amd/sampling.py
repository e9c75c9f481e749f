"""Sampler law on the GPU (``mtplx/sampling.py`` / ``mtplx/fast_sampling.py`` contract).

``SamplerConfig`` and ``SparseDistribution`` keep the reference's fields
(``mtplx/sampling.py:22-128``). The device work — full-vocabulary softmax
statistics, deterministic top-k (value desc, id asc), top-p over the
full-vocabulary mass, renormalisation, draws from fixed uniforms — is the HIP
sampler (``csrc/sampler.hip``); results are bit-exact ids and fp64
probabilities. Non-finite rows raise :class:`NonFiniteLogitsError` as the
reference does (``mtplx/sampling.py:32-70``).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

PENALTY_MIN = -2.0
PENALTY_MAX = 2.0


@dataclass(frozen=True)
class SamplerConfig:
    temperature: float = 0.6
    top_p: float = 0.95
    top_k: int = 20
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0


class NonFiniteLogitsError(RuntimeError):
    """A logits row carried NaN/+inf (no finite mass)."""


@dataclass(frozen=True)
class SparseDistribution:
    token_ids: np.ndarray
    probs: np.ndarray
    vocab_size: int

    def __post_init__(self):
        ids = np.asarray(self.token_ids, dtype=np.int64)
        p = np.asarray(self.probs, dtype=np.float64)
        if ids.ndim != 1 or p.ndim != 1 or ids.shape != p.shape or ids.size == 0:
            raise ValueError("SparseDistribution expects equal-length non-empty 1D ids/probs")
        if np.any(np.isfinite(p) & (p < 0)):
            raise ValueError("SparseDistribution probabilities must be non-negative")
        clean = np.where(np.isfinite(p) & (p > 0), p, 0.0)
        total = clean.sum()
        if not np.isfinite(total) or total <= 0:
            raise NonFiniteLogitsError("SparseDistribution without finite positive mass")
        object.__setattr__(self, "token_ids", ids)
        object.__setattr__(self, "probs", clean / total)

    @classmethod
    def one_hot(cls, token_id: int, vocab_size: int) -> "SparseDistribution":
        return cls(np.array([int(token_id)]), np.array([1.0]), vocab_size)

    def probability(self, token_id: int) -> float:
        hit = np.nonzero(self.token_ids == int(token_id))[0]
        return 0.0 if hit.size == 0 else float(self.probs[int(hit[0])])

    def to_dense(self) -> np.ndarray:
        d = np.zeros(int(self.vocab_size), dtype=np.float64)
        d[self.token_ids] = self.probs
        return d


def _check_penalties(config: SamplerConfig) -> None:
    if config.presence_penalty or config.frequency_penalty:
        raise NotImplementedError("penalties are outside the gfx950 sampler (exact no-op at 0 only)")


def _rows(logits: torch.Tensor) -> torch.Tensor:
    if not logits.is_cuda:
        raise RuntimeError("the sampler runs on the GPU only")
    return logits.reshape(-1, logits.shape[-1]).to(torch.float32).contiguous()


@dataclass
class RowLaws:
    ids: torch.Tensor        # int32 [R, k], ids ascending, -1 padded
    probs: torch.Tensor      # fp64 [R, k]
    count: torch.Tensor      # int32 [R]
    sampled: torch.Tensor | None
    status: torch.Tensor     # int32 [R], 1 = non-finite


def row_laws(logits: torch.Tensor, config: SamplerConfig, uniforms: torch.Tensor | None = None) -> RowLaws:
    """Sparse law of every row (and one draw per row when ``uniforms`` is given)."""
    _check_penalties(config)
    rows = _rows(logits)
    R, V = rows.shape
    k = max(int(config.top_k), 1)
    dev = rows.device
    ids = torch.empty((R, k), dtype=torch.int32, device=dev)
    probs = torch.empty((R, k), dtype=torch.float64, device=dev)
    cnt = torch.empty(R, dtype=torch.int32, device=dev)
    status = torch.empty(R, dtype=torch.int32, device=dev)
    sampled = None
    u = None
    if uniforms is not None:
        u = uniforms.to(device=dev, dtype=torch.float64).reshape(-1).contiguous()
        sampled = torch.empty(R, dtype=torch.int32, device=dev)
    nb = _lib.query("mtp_sampler_workspace_bytes", R, V)
    ws = _lib.WORKSPACES.get(nb, "sampler", dev)
    _lib.call("mtp_sample_rows", rows.data_ptr(), R, V, float(config.temperature), int(config.top_k),
              float(config.top_p), _lib.ptr(u), ids.data_ptr(), probs.data_ptr(), cnt.data_ptr(),
              _lib.ptr(sampled), status.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    return RowLaws(ids, probs, cnt, sampled, status)


def sparse_distributions_from_logits(logits: torch.Tensor, config: SamplerConfig) -> list[SparseDistribution]:
    """Per-row ``SparseDistribution`` (``mtplx/fast_sampling.py:637``, ``:826``)."""
    laws = row_laws(logits, config)
    st = laws.status.cpu().numpy()
    if st.any():
        raise NonFiniteLogitsError(f"non-finite logits in rows {np.nonzero(st)[0].tolist()}")
    ids, probs, cnt = laws.ids.cpu().numpy(), laws.probs.cpu().numpy(), laws.count.cpu().numpy()
    V = int(logits.shape[-1])
    return [SparseDistribution(ids[r, : cnt[r]], probs[r, : cnt[r]], V) for r in range(ids.shape[0])]


def sample_token_ids(logits: torch.Tensor, config: SamplerConfig, uniforms: torch.Tensor) -> torch.Tensor:
    """One draw per row from its sparse law with the given uniforms
    (``mtplx/fast_sampling.py:861`` with explicit uniforms). Stays on the GPU."""
    return row_laws(logits, config, uniforms).sampled


@dataclass
class AcceptResult:
    tokens: torch.Tensor        # int32 [B, K+1], committed ids, -1 padded
    n_accepted: torch.Tensor    # int32 [B]
    accept_probs: torch.Tensor  # fp64 [B, K], -1 where not examined
    status: torch.Tensor        # int32 [B]


def spec_accept(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_ids: torch.Tensor,
                uniforms: torch.Tensor, config: SamplerConfig) -> AcceptResult:
    """Depth-K accept/reject with residual correction for ``B`` requests.

    ``target_logits`` ``[B, K+1, V]`` (verify rows), ``draft_logits`` ``[B, K, V]``,
    ``draft_ids`` ``[B, K]``, ``uniforms`` fp64 ``[B, K+1]`` consumed in the
    order ``generate_mtpk`` draws them (``mtplx/generation.py:15560-15790``,
    ``:16085-16110``). Asynchronous: nothing is read back here.
    """
    _check_penalties(config)
    B, K1, V = (int(s) for s in target_logits.shape)
    K = K1 - 1
    t = _rows(target_logits)
    d = _rows(draft_logits)
    dev = t.device
    di = draft_ids.to(device=dev, dtype=torch.int32).contiguous()
    u = uniforms.to(device=dev, dtype=torch.float64).contiguous()
    out = torch.empty((B, K + 1), dtype=torch.int32, device=dev)
    nacc = torch.empty(B, dtype=torch.int32, device=dev)
    ap = torch.empty((B, K), dtype=torch.float64, device=dev)
    st = torch.empty(B, dtype=torch.int32, device=dev)
    nb = _lib.query("mtp_sampler_workspace_bytes", B * (2 * K + 1), V)
    ws = _lib.WORKSPACES.get(nb, "sampler", dev)
    _lib.call("mtp_spec_accept", t.data_ptr(), d.data_ptr(), di.data_ptr(), u.data_ptr(), B, K, V,
              float(config.temperature), int(config.top_k), float(config.top_p), out.data_ptr(), nacc.data_ptr(),
              ap.data_ptr(), st.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    return AcceptResult(out, nacc, ap, st)
