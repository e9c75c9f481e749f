"""Float64 restatement of one verify forward of the synthetic 4-bit decoder.

Follows the mlx-lm decoder layer the reference verifies with
(``mtplx/runtime.py:161`` forward_ar → per layer: input RMSNorm, q|k|v, RoPE
at the cache offset, ``update_and_fetch`` then SDPA with the ragged mask,
o_proj + residual, post-attention RMSNorm, SwiGLU MLP + residual; final norm
and lm_head). Values are rounded to bf16 wherever the GPU path stores a bf16
tensor, so the comparison isolates arithmetic error, not storage format.

The MoE layer follows the reference's verify call of the sparse block
(``mtplx/models/qwen4_exp.py:1416-1445`` ``_verify_call``, routed chain
``:1544-1577``): router logits (bf16, a quantized projection whose last row
is the shared-expert gate) plus the synthetic per-expert Zipf skew pick the
top-k experts (value desc, id asc) with softmax weights renormalised over the
k; routed rows go through the sorted SwiGLU chain, stored as bf16 where
the reference's chain stores them (gate|up product, silu, SwiGLU rows, each
expert's down rows); the shared expert is
``sigmoid(gate) * shared_mlp(x)``; the block output ``routed + shared`` is
added to the residual stream.

``decoder_layer`` is the one-layer restatement both forwards run; a test
can feed it the GPU's own hidden rows (teacher forcing) to hold every layer
of a deep model to the bar separately.

Parity pins (tests/test_oracle_model.py): a zero-layer model equals a
closed form of norm + lm_head over the embedding rows; a layer whose o and
down projections are zero leaves the residual stream unchanged, so its
logits equal the zero-layer ones; one dense and one MoE layer equal an
independent scalar-loop restatement of the decoder layer; RoPE at position 0
is the identity and preserves norms; the attention and qmv pieces are pinned
in their own files.
"""

from __future__ import annotations

import numpy as np

from .attention import ragged_gqa_attention
from .bf16 import round_to_bf16
from .moe import moe_forward, silu
from .qmv import dequantize_affine4, qmm_affine4


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * np.asarray(w, dtype=np.float64)


def rope_rotate_half(x: np.ndarray, pos: np.ndarray, base: float) -> np.ndarray:
    """Non-interleaved RoPE: pairs (j, j + D/2), theta_j = pos * base^(-2j/D).
    ``x`` [..., n, D] with ``pos`` broadcastable to [..., n]."""
    D = x.shape[-1]
    half = D // 2
    inv = base ** (-(2.0 * np.arange(half)) / D)
    ang = np.asarray(pos, dtype=np.float64)[..., None] * inv
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def verify_forward(params: dict, cfg, tokens: np.ndarray, q_start: np.ndarray, k_cache: list, v_cache: list,
                   routes: list | None = None) -> np.ndarray:
    """Logits [B*L, V] (float64 of bf16 values). ``params`` holds numpy copies of
    the GPU model (bf16 values as float64, weight triples for 4-bit layers).
    ``k_cache``/``v_cache`` are per-layer float64 arrays [B, Hkv, cap, D],
    updated in place at ``q_start[b] + i``. ``routes``, if a list, receives
    each MoE layer's ``(ids, weights)``."""
    tokens = np.asarray(tokens)
    return verify_forward_ragged(params, cfg, list(tokens), q_start, k_cache, v_cache, routes)


def verify_forward_ragged(params: dict, cfg, tokens: list, q_start, k_cache: list, v_cache: list,
                          routes: list | None = None) -> np.ndarray:
    """The same forward over a ragged batch: request b has ``len(tokens[b])``
    rows at positions ``q_start[b] + i``; rows are packed request after
    request (logits [sum_b L_b, V]). ``k_cache[li][b]`` is request b's
    float64 [Hkv, cap_b, D] cache of layer li (a [B, Hkv, cap, D] array or a
    list of per-request arrays), updated in place."""
    lens = [len(t) for t in tokens]
    flat = np.concatenate([np.asarray(t).reshape(-1) for t in tokens])
    h = embed_rows(params, cfg, flat)
    for li, lay in enumerate(params["layers"]):
        h = decoder_layer(lay, cfg, h, lens, q_start, k_cache[li], v_cache[li], routes)
    return final_logits(params, cfg, h)


def embed_rows(params: dict, cfg, flat_tokens) -> np.ndarray:
    """Embedding rows (bf16 values) of the flattened tokens."""
    gs = cfg.group_size
    emb = params["embed"]
    return round_to_bf16(np.stack([dequantize_affine4(emb[0][t:t + 1], emb[1][t:t + 1], emb[2][t:t + 1], gs)[0]
                                   for t in np.asarray(flat_tokens).reshape(-1)]))


def final_logits(params: dict, cfg, h: np.ndarray) -> np.ndarray:
    """Final RMSNorm and lm_head of the hidden rows (bf16 values)."""
    xn = round_to_bf16(rmsnorm(h, params["final_norm"], cfg.rms_eps))
    return round_to_bf16(qmm_affine4(xn, *params["lm_head"], cfg.group_size))


def decoder_layer(lay: dict, cfg, h: np.ndarray, lens, q_start, k_cache_layer, v_cache_layer,
                  routes: list | None = None, trace: dict | None = None) -> np.ndarray:
    """One decoder layer on the packed rows ``h`` [sum(lens), H] (bf16
    values): request b's ``lens[b]`` rows at positions ``q_start[b] + i``.
    ``k_cache_layer[b]`` / ``v_cache_layer[b]`` are request b's float64
    [Hkv, cap_b, D] caches of this layer, updated in place. Returns the
    layer's output rows (bf16 values). ``trace``, if a dict, receives the
    two rounded block outputs added to the residual stream: ``"attn_out"``
    (the o projection) and ``"mlp_out"`` (down projection, or routed +
    shared for an MoE layer)."""
    gs = cfg.group_size
    H, D, Hq, Hkv = cfg.hidden, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    M = int(offs[-1])
    h = np.asarray(h, dtype=np.float64)
    xn = round_to_bf16(rmsnorm(h, lay["in_norm"], cfg.rms_eps))
    qkv = round_to_bf16(qmm_affine4(xn, *lay["qkv"], gs)).reshape(M, Hq + 2 * Hkv, D)
    att = np.zeros((M, Hq * D))
    for b, L in enumerate(lens):
        if L == 0:
            continue
        rows = slice(int(offs[b]), int(offs[b + 1]))
        pos = int(q_start[b]) + np.arange(L)
        blk = qkv[rows].transpose(1, 0, 2)                       # [heads, L, D]
        q = round_to_bf16(rope_rotate_half(blk[:Hq], pos[None, :], cfg.rope_theta))
        k = round_to_bf16(rope_rotate_half(blk[Hq:Hq + Hkv], pos[None, :], cfg.rope_theta))
        v = blk[Hq + Hkv:]
        kc, vc = k_cache_layer[b], v_cache_layer[b]
        kc[:, pos[0]:pos[0] + L] = k
        vc[:, pos[0]:pos[0] + L] = v
        o = round_to_bf16(ragged_gqa_attention(q[None], kc[None], vc[None], [int(q_start[b])]))[0]
        att[rows] = o.transpose(1, 0, 2).reshape(L, Hq * D)
    o_out = round_to_bf16(qmm_affine4(att, *lay["o"], gs))
    h = round_to_bf16(o_out + h)
    xn = round_to_bf16(rmsnorm(h, lay["post_norm"], cfg.rms_eps))
    if cfg.n_experts:
        E = cfg.n_experts
        rl = round_to_bf16(qmm_affine4(xn, *lay["router"], gs))          # [M, E + 1]
        skew = lay.get("router_skew")
        logits = rl[:, :E].astype(np.float32)
        if skew is not None:
            logits = logits + np.asarray(skew, np.float32)[None, :]
        ids, wts = route_topk(logits.astype(np.float64), cfg.top_k)
        if routes is not None:
            routes.append((ids, wts))
        routed = round_to_bf16(moe_forward(xn, ids, wts, lay["expert_gate_up"], lay["expert_down"], gs,
                                           bf16_storage=True))
        sg = round_to_bf16(qmm_affine4(xn, *lay["shared_gate"], gs))
        su = round_to_bf16(qmm_affine4(xn, *lay["shared_up"], gs))
        sa = round_to_bf16(round_to_bf16(silu(sg)) * su)
        sd = round_to_bf16(qmm_affine4(sa, *lay["shared_down"], gs))
        gate = 1.0 / (1.0 + np.exp(-rl[:, E]))
        shared = round_to_bf16(gate[:, None] * sd)
        mlp_out = round_to_bf16(routed + shared)
    else:
        g = round_to_bf16(qmm_affine4(xn, *lay["gate"], gs))
        u = round_to_bf16(qmm_affine4(xn, *lay["up"], gs))
        a = round_to_bf16(round_to_bf16(silu(g)) * u)
        mlp_out = round_to_bf16(qmm_affine4(a, *lay["down"], gs))
    if trace is not None:
        trace["attn_out"] = o_out
        trace["mlp_out"] = mlp_out
    return round_to_bf16(h + mlp_out)


def route_topk(logits: np.ndarray, top_k: int):
    """Top-k experts (value desc, id asc) and softmax weights over the chosen k."""
    logits = np.asarray(logits, dtype=np.float64)
    ids = np.stack([np.lexsort((np.arange(r.size), -r))[:top_k] for r in logits])
    sel = np.take_along_axis(logits, ids, axis=1)
    e = np.exp(sel - sel[:, :1])
    return ids, e / e.sum(axis=1, keepdims=True)
