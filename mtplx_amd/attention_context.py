"""Forward-scoped switches of the verify path (``mtplx/attention_context.py``).

``exact_verify(required)`` marks a forward whose logits must not depend on
the batch it runs in: the reference's generation loop enters it with
``sampler.temperature <= 0`` (``mtplx/generation.py:11527``, ``:15121``) so
that a greedy verify picks the same argmax as autoregressive decode, and its
operator patch then drops to one stock matmul (``mtplx/nax_verify.py:755``).

Here the greedy lane is the *exact lane*: every projection runs on the
9..64-row MFMA matmul, whose K split is planned from (N, K, CUs) alone, and
attention runs a fixed split length with the per-head merge, so each row's
arithmetic is the same at M = 1, at M = 4 and inside a ragged batch
(bit-identical logits). The reference arms its guard only under
``MTPLX_EXACT_T0_GUARD=1`` because its stock kernels still flip across M;
this build's lane keeps the promise, so the guard is armed by default and
``MTPLX_EXACT_T0_GUARD=0`` disarms it.
"""

from __future__ import annotations

import os
from collections import Counter
from contextlib import contextmanager
from contextvars import ContextVar
from typing import Iterator

_EXACT_VERIFY_REQUIRED: ContextVar[bool] = ContextVar("mtplx_amd_exact_verify_required", default=False)

# Forwards and matmuls routed to the exact lane, by caller ("verify_step",
# "verify_step_ragged", "qlinear_m<M>").
exact_lane_counts: Counter = Counter()


def exact_t0_guard_armed() -> bool:
    """Whether greedy (temperature <= 0) verify forwards take the exact lane."""
    return (os.environ.get("MTPLX_EXACT_T0_GUARD") or "1").strip().lower() not in {"0", "false", "off", "no"}


def exact_verify_required() -> bool:
    """True inside ``exact_verify(True)`` while the guard is armed."""
    return exact_t0_guard_armed() and bool(_EXACT_VERIFY_REQUIRED.get())


@contextmanager
def exact_verify(required: bool) -> Iterator[None]:
    token = _EXACT_VERIFY_REQUIRED.set(bool(required))
    try:
        yield
    finally:
        _EXACT_VERIFY_REQUIRED.reset(token)
