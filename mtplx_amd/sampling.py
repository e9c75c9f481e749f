"""Sampler law on the GPU (``mtplx/sampling.py`` / ``mtplx/fast_sampling.py`` contract).

``SamplerConfig`` and ``SparseDistribution`` keep the reference's fields
(``mtplx/sampling.py:22-128``). The device work — full-vocabulary softmax
statistics, deterministic top-k (value desc, id asc), top-p over the
full-vocabulary mass, renormalisation, draws from fixed uniforms — is the HIP
sampler (``csrc/sampler.hip``); results are bit-exact ids and fp64
probabilities. Any ``top_k`` (0 = no bound) and ``top_p``; presence /
frequency penalties and overlays are sparse fp32 deltas on the raw logits
(the runtime's device twin, ``mtplx/fast_sampling.py:42-81``). Non-finite rows
raise :class:`NonFiniteLogitsError` as the reference does
(``mtplx/sampling.py:32-70``).
"""

from __future__ import annotations

from collections import Counter
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


def _clamp(v: float) -> float:
    return float(min(max(float(v), PENALTY_MIN), PENALTY_MAX))


def penalties_active(config: SamplerConfig, token_counts=None, penalty_overlay=None) -> bool:
    """``mtplx/sampling.py:236-241``: penalties apply only with counts and a
    non-zero (clamped) penalty, or with an overlay."""
    counts_on = bool(token_counts) and (_clamp(config.presence_penalty) != 0.0 or
                                        _clamp(config.frequency_penalty) != 0.0)
    return counts_on or bool(penalty_overlay)


def _delta_lists(config: SamplerConfig, per_row_counts, per_row_overlay):
    """Host half of the device penalty (``mtplx/fast_sampling.py:42-81``):
    per (row, token) fp32 deltas ``frequency * count + presence * (count > 0)``
    (penalties clamped to [-2, 2]) and overlay values, as two lists so each is
    one fp32 addition on the device, in that order."""
    pres, freq = _clamp(config.presence_penalty), _clamp(config.frequency_penalty)
    lists = []
    for which in ("counts", "overlay"):
        rows, ids, vals = [], [], []
        src = per_row_counts if which == "counts" else per_row_overlay
        for r, m in enumerate(src):
            if not m:
                continue
            if which == "counts" and pres == 0.0 and freq == 0.0:
                continue
            k = np.fromiter(m.keys(), dtype=np.int64, count=len(m))
            v = np.fromiter(m.values(), dtype=np.float64, count=len(m))
            if which == "counts":
                v = freq * v + pres * (v > 0.0)
            rows.append(np.full(k.shape, r, np.int32))
            ids.append(k.astype(np.int32))
            vals.append(v.astype(np.float32))
        lists.append(None if not rows else (np.concatenate(rows), np.concatenate(ids), np.concatenate(vals)))
    return lists


def apply_penalties(logits: torch.Tensor, config: SamplerConfig, per_row_counts, per_row_overlay=None,
                    *, inplace: bool = False) -> torch.Tensor:
    """fp32 logit rows ``[R, V]`` with the sparse penalties applied on the GPU
    (``mtp_apply_logit_deltas``). ``per_row_counts[r]`` / ``per_row_overlay[r]``
    are mappings token -> count / subtraction for row ``r`` (or None).
    Returns a new tensor unless ``inplace``; returns ``logits`` itself when
    nothing is active (the exact no-op)."""
    R, V = (int(s) for s in logits.shape)
    counts = list(per_row_counts) if per_row_counts is not None else [None] * R
    overlay = list(per_row_overlay) if per_row_overlay is not None else [None] * R
    if len(counts) != R or len(overlay) != R:
        raise ValueError(f"penalty maps for {len(counts)}/{len(overlay)} rows, logits have {R}")
    lists = _delta_lists(config, counts, overlay)
    if all(x is None for x in lists):
        return logits
    out = logits if inplace else logits.clone()
    dev = out.device
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    for item in lists:
        if item is None:
            continue
        rows, ids, vals = (torch.from_numpy(a).to(dev) for a in item)
        _lib.call("mtp_apply_logit_deltas", out.data_ptr(), int(out.stride(0)), R, V, rows.data_ptr(),
                  ids.data_ptr(), vals.data_ptr(), int(vals.numel()), status.data_ptr(), _lib.stream_handle(dev))
    if int(status.item()):
        raise ValueError("penalty token id outside the vocabulary")
    return out


def _rows(logits: torch.Tensor) -> torch.Tensor:
    if not logits.is_cuda:
        raise RuntimeError("the sampler runs on the GPU only")
    return logits.reshape(-1, logits.shape[-1]).to(torch.float32).contiguous()


def support_bound(config: SamplerConfig, V: int) -> int:
    """Largest support a row law can have: 1 when greedy, else the top-k bound
    (``0 < top_k < V``), else the vocabulary."""
    if not config.temperature > 0:
        return 1
    k = int(config.top_k)
    return k if 0 < k < V else V


@dataclass
class RowLaws:
    ids: torch.Tensor        # int32 [R, support_bound], ids ascending, -1 padded
    probs: torch.Tensor      # fp64 [R, support_bound]
    count: torch.Tensor      # int32 [R]
    sampled: torch.Tensor | None
    status: torch.Tensor     # int32 [R], 1 = non-finite


def row_laws(logits: torch.Tensor, config: SamplerConfig, uniforms: torch.Tensor | None = None, *,
             token_counts=None, penalty_overlay=None) -> RowLaws:
    """Sparse law of every row (and one draw per row when ``uniforms`` is
    given). ``token_counts`` / ``penalty_overlay``: one mapping for every row,
    or a list with one per row (``mtplx/sampling.py:259`` keywords)."""
    rows = _rows(logits)
    R, V = rows.shape
    if penalties_active(config, token_counts, penalty_overlay) or isinstance(token_counts, (list, tuple)) or \
            isinstance(penalty_overlay, (list, tuple)):
        per_c = token_counts if isinstance(token_counts, (list, tuple)) else [token_counts] * R
        per_o = penalty_overlay if isinstance(penalty_overlay, (list, tuple)) else [penalty_overlay] * R
        rows = apply_penalties(rows, config, per_c, per_o, inplace=rows.data_ptr() != logits.data_ptr())
    k = support_bound(config, V)
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
    nb = _lib.query("mtp_sampler_workspace_bytes", R, V, int(config.top_k))
    ws = _lib.WORKSPACES.get(nb, "sampler", dev)
    _lib.call("mtp_sample_rows", rows.data_ptr(), R, V, float(config.temperature), int(config.top_k),
              float(config.top_p), _lib.ptr(u), ids.data_ptr(), probs.data_ptr(), k, cnt.data_ptr(),
              _lib.ptr(sampled), status.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    return RowLaws(ids, probs, cnt, sampled, status)


def sparse_distributions_from_logits(logits: torch.Tensor, config: SamplerConfig, *, token_counts=None,
                                     penalty_overlay=None) -> list[SparseDistribution]:
    """Per-row ``SparseDistribution`` (``mtplx/fast_sampling.py:637``, ``:826``)."""
    laws = row_laws(logits, config, token_counts=token_counts, penalty_overlay=penalty_overlay)
    st = laws.status.cpu().numpy()
    if st.any():
        raise NonFiniteLogitsError(f"non-finite logits in rows {np.nonzero(st)[0].tolist()}")
    ids, probs, cnt = laws.ids.cpu().numpy(), laws.probs.cpu().numpy(), laws.count.cpu().numpy()
    V = int(logits.shape[-1])
    return [SparseDistribution(ids[r, : cnt[r]], probs[r, : cnt[r]], V) for r in range(ids.shape[0])]


def sample_token_ids(logits: torch.Tensor, config: SamplerConfig, uniforms: torch.Tensor, *, token_counts=None,
                     penalty_overlay=None) -> torch.Tensor:
    """One draw per row from its sparse law with the given uniforms
    (``mtplx/fast_sampling.py:861`` with explicit uniforms). Stays on the GPU."""
    return row_laws(logits, config, uniforms, token_counts=token_counts, penalty_overlay=penalty_overlay).sampled


@dataclass
class AcceptResult:
    tokens: torch.Tensor        # int32 [B, K+1], committed ids, -1 padded
    n_accepted: torch.Tensor    # int32 [B]
    accept_probs: torch.Tensor  # fp64 [B, K], -1 where not examined
    status: torch.Tensor        # int32 [B]


def _position_counts(base, drafts_b, K):
    """Counts of depth d: the committed completion plus drafts[:d]
    (``mtplx/generation.py:15590-15595``, per-position prefix counts)."""
    out = []
    for d in range(K + 1):
        c = Counter(base or {})
        c.update(int(t) for t in drafts_b[:d])
        out.append(c)
    return out


def sampler_workspace(B: int, K: int, V: int, config: SamplerConfig, device) -> torch.Tensor:
    """The accept step's workspace (the rows' chunk partials, then the laws)."""
    nb = _lib.query("mtp_sampler_workspace_bytes", B * (2 * K + 1), V, int(config.top_k))
    return _lib.WORKSPACES.get(nb, "sampler", device)


def spec_accept(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_ids: torch.Tensor,
                uniforms: torch.Tensor, config: SamplerConfig, *, token_counts=None,
                penalty_overlay=None) -> AcceptResult:
    """Depth-K accept/reject with residual correction for ``B`` requests.

    ``target_logits`` ``[B, K+1, V]`` (verify rows), ``draft_logits`` ``[B, K, V]``,
    ``draft_ids`` ``[B, K]``, ``uniforms`` fp64 ``[B, K+1]`` consumed in the
    order ``generate_mtpk`` draws them (``mtplx/generation.py:15560-15790``,
    ``:16085-16110``). Asynchronous unless penalties are active.

    Penalties: ``token_counts[b]`` is request b's committed completion counts
    (one mapping is used for every request); target row d and draft row d of
    request b are penalised with those counts plus ``draft_ids[b, :d]``
    (per-position prefix counts). ``penalty_overlay[b]``: one mapping for all
    of request b's rows, or a list of K+1 (one per depth).
    """
    B, K1, V = (int(s) for s in target_logits.shape)
    K = K1 - 1
    t = _rows(target_logits)
    d = _rows(draft_logits)
    dev = t.device
    di = draft_ids.to(device=dev, dtype=torch.int32).contiguous()
    pen = penalties_active(config, token_counts if not isinstance(token_counts, (list, tuple)) else any(token_counts),
                           penalty_overlay if not isinstance(penalty_overlay, (list, tuple)) else any(penalty_overlay))
    if pen:
        base = token_counts if isinstance(token_counts, (list, tuple)) else [token_counts] * B
        ovl = penalty_overlay if isinstance(penalty_overlay, (list, tuple)) else [penalty_overlay] * B
        drafts = di.cpu().numpy()
        t_counts, d_counts, t_ovl, d_ovl = [], [], [], []
        for b in range(B):
            pc = _position_counts(base[b], drafts[b], K)
            ob = ovl[b] if isinstance(ovl[b], (list, tuple)) else [ovl[b]] * (K + 1)
            t_counts += pc
            d_counts += pc[:K]
            t_ovl += list(ob)
            d_ovl += list(ob[:K])
        t = apply_penalties(t, config, t_counts, t_ovl, inplace=t.data_ptr() != target_logits.data_ptr())
        d = apply_penalties(d, config, d_counts, d_ovl, inplace=d.data_ptr() != draft_logits.data_ptr())
    u = uniforms.to(device=dev, dtype=torch.float64).contiguous()
    out = torch.empty((B, K + 1), dtype=torch.int32, device=dev)
    nacc = torch.empty(B, dtype=torch.int32, device=dev)
    ap = torch.empty((B, K), dtype=torch.float64, device=dev)
    st = torch.empty(B, dtype=torch.int32, device=dev)
    ws = sampler_workspace(B, K, V, config, dev)
    _lib.call("mtp_spec_accept", t.data_ptr(), d.data_ptr(), di.data_ptr(), u.data_ptr(), B, K, V,
              float(config.temperature), int(config.top_k), float(config.top_p), out.data_ptr(), nacc.data_ptr(),
              ap.data_ptr(), st.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    return AcceptResult(out, nacc, ap, st)


def spec_accept_ragged(target_rows: torch.Tensor, t_off: torch.Tensor, draft_rows: torch.Tensor, d_off: torch.Tensor,
                       k_lens: torch.Tensor, draft_ids: torch.Tensor, uniforms: torch.Tensor,
                       config: SamplerConfig) -> AcceptResult:
    """Accept/reject for a ragged batch (per-request depths K_b, the
    continuous-batched lane of ``mtplx/batched_decode.py:338-395``): request
    b's K_b + 1 target rows start at row ``t_off[b]`` of ``target_rows``
    ``[n_target, V]``, its K_b draft rows (and draft ids) at ``d_off[b]`` of
    ``draft_rows`` ``[n_draft, V]`` / ``draft_ids`` ``[n_draft]``; uniforms
    ``[B, K_max + 1]``. Outputs are ``[B, K_max + 1]`` tokens (-1 padded) and
    ``[B, K_max]`` accept probabilities. No penalties on this lane."""
    t = _rows(target_rows)
    d = _rows(draft_rows)
    dev = t.device
    B = int(k_lens.numel())
    K = int(uniforms.shape[-1]) - 1
    V = int(t.shape[-1])
    i32 = dict(device=dev, dtype=torch.int32)
    to, do, kl = (x.to(**i32).contiguous() for x in (t_off, d_off, k_lens))
    di = draft_ids.to(**i32).contiguous()
    u = uniforms.to(device=dev, dtype=torch.float64).contiguous()
    out = torch.empty((B, K + 1), **i32)
    nacc = torch.empty(B, **i32)
    ap = torch.empty((B, K), dtype=torch.float64, device=dev)
    st = torch.empty(B, **i32)
    nb = _lib.query("mtp_sampler_workspace_bytes", int(t.shape[0]) + int(d.shape[0]), V, int(config.top_k))
    ws = _lib.WORKSPACES.get(nb, "sampler", dev)
    _lib.call("mtp_spec_accept_ragged", t.data_ptr(), int(t.shape[0]), d.data_ptr(), int(d.shape[0]), to.data_ptr(),
              do.data_ptr(), kl.data_ptr(), di.data_ptr(), u.data_ptr(), B, K, V, float(config.temperature),
              int(config.top_k), float(config.top_p), out.data_ptr(), nacc.data_ptr(), ap.data_ptr(), st.data_ptr(),
              ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    return AcceptResult(out, nacc, ap, st)
