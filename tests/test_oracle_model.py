"""Pins for oracle.model (CPU).

``verify_forward`` is the checker of every composed-step GPU test, so its
layer composition is pinned three ways: a zero-layer closed form, a layer
whose o and down projections are zero (the residual stream must pass through
untouched), and an independent scalar-loop restatement of one dense and one
MoE decoder layer (pre-norm placement, GQA head mapping, rotate-half RoPE at
the cache offset, the two residual adds, routed + gated shared expert).
"""

from types import SimpleNamespace

import numpy as np

from oracle.bf16 import bf16_bits_to_f32, round_to_bf16
from oracle.model import rmsnorm, rope_rotate_half, route_topk, verify_forward
from oracle.qmv import make_affine4_weights, qmm_affine4_groupwise, unpack_affine4


def test_rope_position_zero_is_identity_and_preserves_norm():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(3, 128))
    assert np.allclose(rope_rotate_half(x, np.zeros(3), 1e6), x)
    y = rope_rotate_half(x, np.array([5, 77, 4000]), 1e6)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1))
    # rotate-half pairing: dims j and j+64 rotate together by pos * base^(-2j/128)
    e = np.zeros(128); e[0] = 1.0
    r = rope_rotate_half(e[None], np.array([2.0]), 1e6)[0]
    assert np.isclose(r[0], np.cos(2.0)) and np.isclose(r[64], np.sin(2.0))


def test_rmsnorm_closed_form():
    x = np.array([[3.0, 4.0]])
    assert np.allclose(rmsnorm(x, np.array([1.0, 2.0]), 0.0), [[3 / np.sqrt(12.5), 8 / np.sqrt(12.5)]])


def test_route_topk_ties_and_weights():
    ids, w = route_topk(np.array([[1.0, 3.0, 3.0, 0.0]]), 2)
    assert ids.tolist() == [[1, 2]] and np.allclose(w, [[0.5, 0.5]])


# ---------------------------------------------------------------------------
# Composition pins.

def _cfg(**kw):
    base = dict(layers=1, hidden=64, ffn=128, n_heads=4, n_kv_heads=2, head_dim=16, vocab=40, rope_theta=1.0e4,
                rms_eps=1.0e-6, group_size=64, n_experts=0, top_k=0, expert_ffn=0, shared_ffn=0)
    base.update(kw)
    return SimpleNamespace(**base)


def _norm(rng, n):
    return round_to_bf16(1.0 + 0.1 * rng.normal(size=n))


def _lin(rng, n, k, lead=None):
    if lead is None:
        return make_affine4_weights(rng, n, k, 64, scale_std=0.05, bias_std=0.02)
    w = make_affine4_weights(rng, lead * n, k, 64, scale_std=0.05, bias_std=0.02)
    return tuple(a.reshape(lead, n, -1) for a in w)


def _zero_lin(n, k):
    w, s, b = make_affine4_weights(np.random.default_rng(0), n, k, 64)
    return w, np.zeros_like(s), np.zeros_like(b)


def _params(cfg, rng):
    H, D = cfg.hidden, cfg.head_dim
    layers = []
    for _ in range(cfg.layers):
        lay = {"in_norm": _norm(rng, H), "qkv": _lin(rng, (cfg.n_heads + 2 * cfg.n_kv_heads) * D, H),
               "o": _lin(rng, H, cfg.n_heads * D), "post_norm": _norm(rng, H)}
        if cfg.n_experts:
            E, F = cfg.n_experts, cfg.expert_ffn
            lay.update(router=_lin(rng, E + 1, H), router_skew=-1.1 * np.log(1.0 + rng.permutation(E)),
                       expert_gate_up=_lin(rng, 2 * F, H, E), expert_down=_lin(rng, H, F, E),
                       shared_gate=_lin(rng, cfg.shared_ffn, H), shared_up=_lin(rng, cfg.shared_ffn, H),
                       shared_down=_lin(rng, H, cfg.shared_ffn))
        else:
            lay.update(gate=_lin(rng, cfg.ffn, H), up=_lin(rng, cfg.ffn, H), down=_lin(rng, H, cfg.ffn))
        layers.append(lay)
    return {"embed": _lin(rng, cfg.vocab, H), "layers": layers, "final_norm": _norm(rng, H),
            "lm_head": _lin(rng, cfg.vocab, H)}


def _caches(cfg, rng, B, cap):
    shape = (B, cfg.n_kv_heads, cap, cfg.head_dim)
    return ([round_to_bf16(rng.normal(size=shape)) for _ in range(cfg.layers)],
            [round_to_bf16(rng.normal(size=shape)) for _ in range(cfg.layers)])


def _bfv(bits):
    return bf16_bits_to_f32(np.asarray(bits)).astype(np.float64)


def _deq_scalar(lin, n, k, gs=64):
    """One weight w[n, k] from the packed triple by explicit nibble extraction."""
    w, s, b = lin
    q = (int(w[n, k // 8]) >> (4 * (k % 8))) & 0xF
    return q * float(_bfv(s[n, k // gs])) + float(_bfv(b[n, k // gs]))


def _matvec_scalar(lin, x):
    w = lin[0]
    n_out, k_in = w.shape[0], w.shape[1] * 8
    q = unpack_affine4(w).astype(np.float64)
    s = np.repeat(_bfv(lin[1]), 64, axis=1)
    b = np.repeat(_bfv(lin[2]), 64, axis=1)
    out = np.zeros(n_out)
    for n in range(n_out):
        acc = 0.0
        for k in range(k_in):
            acc += x[k] * (q[n, k] * s[n, k] + b[n, k])
        out[n] = acc
    return out


def _rb(v):
    return float(round_to_bf16(np.array([v]))[0])


def _rmsnorm_scalar(x, w, eps):
    ms = sum(v * v for v in x) / len(x)
    inv = 1.0 / np.sqrt(ms + eps)
    return np.array([_rb(x[i] * inv * w[i]) for i in range(len(x))])


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _layer_scalar(cfg, lay, h, tokens_shape, q_start, kc, vc):
    """One decoder layer, written element by element from its definition:
    x = bf16(rmsnorm(h)); q|k|v = x W^T; RoPE (pairs d, d + D/2, angle
    pos * theta^(-2d/D)) on q and k; K/V written at pos; query head hq reads kv
    head hq // (Hq/Hkv) over keys j <= pos; h1 = h + o(attn); then the MLP
    (SwiGLU, or the routed + gated shared MoE block) on bf16(rmsnorm(h1)),
    h2 = h1 + mlp. Every stored tensor rounded to bf16."""
    B, L = tokens_shape
    H, D, Hq, Hkv = cfg.hidden, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    rep = Hq // Hkv
    M = B * L
    q_rows = np.zeros((B, Hq, L, D))
    for r in range(M):
        b, i = divmod(r, L)
        pos = int(q_start[b]) + i
        x = _rmsnorm_scalar(h[r], lay["in_norm"], cfg.rms_eps)
        qkv = np.array([_rb(v) for v in _matvec_scalar(lay["qkv"], x)])
        for head in range(Hq + 2 * Hkv):
            vec = qkv[head * D:(head + 1) * D]
            if head < Hq + Hkv:
                rot = np.zeros(D)
                for d in range(D // 2):
                    ang = pos * cfg.rope_theta ** (-2.0 * d / D)
                    x1, x2 = vec[d], vec[d + D // 2]
                    rot[d] = _rb(x1 * np.cos(ang) - x2 * np.sin(ang))
                    rot[d + D // 2] = _rb(x1 * np.sin(ang) + x2 * np.cos(ang))
                vec = rot
            if head < Hq:
                q_rows[b, head, i] = vec
            elif head < Hq + Hkv:
                kc[b, head - Hq, pos] = vec
            else:
                vc[b, head - Hq - Hkv, pos] = vec
    h1 = np.zeros_like(h)
    for r in range(M):
        b, i = divmod(r, L)
        pos = int(q_start[b]) + i
        att = np.zeros(Hq * D)
        for hq in range(Hq):
            kv = hq // rep
            sc = [sum(q_rows[b, hq, i, d] * kc[b, kv, j, d] for d in range(D)) / np.sqrt(D) for j in range(pos + 1)]
            mx = max(sc)
            e = [np.exp(v - mx) for v in sc]
            tot = sum(e)
            for d in range(D):
                att[hq * D + d] = _rb(sum(e[j] * vc[b, kv, j, d] for j in range(pos + 1)) / tot)
        o = _matvec_scalar(lay["o"], att)
        h1[r] = [_rb(_rb(o[n]) + h[r, n]) for n in range(H)]
    h2 = np.zeros_like(h)
    for r in range(M):
        x = _rmsnorm_scalar(h1[r], lay["post_norm"], cfg.rms_eps)
        if not cfg.n_experts:
            g = _matvec_scalar(lay["gate"], x)
            u = _matvec_scalar(lay["up"], x)
            a = np.array([_rb(_rb(_silu(_rb(g[f]))) * _rb(u[f])) for f in range(cfg.ffn)])
            dn = _matvec_scalar(lay["down"], a)
            h2[r] = [_rb(_rb(dn[n]) + h1[r, n]) for n in range(H)]
            continue
        E, F = cfg.n_experts, cfg.expert_ffn
        rl = [_rb(v) for v in _matvec_scalar(lay["router"], x)]
        score = [float(np.float32(rl[e]) + np.float32(lay["router_skew"][e])) for e in range(E)]
        chosen = sorted(range(E), key=lambda e: (-score[e], e))[: cfg.top_k]
        ex = [np.exp(score[e] - score[chosen[0]]) for e in chosen]
        routed = np.zeros(H)
        for j, e in enumerate(chosen):
            gu = [_rb(v) for v in _matvec_scalar(tuple(a[e] for a in lay["expert_gate_up"]), x)]
            hh = np.array([_rb(_rb(_silu(gu[f])) * gu[F + f]) for f in range(F)])
            y = np.array([_rb(v) for v in _matvec_scalar(tuple(a[e] for a in lay["expert_down"]), hh)])
            routed += (ex[j] / sum(ex)) * y
        sg = _matvec_scalar(lay["shared_gate"], x)
        su = _matvec_scalar(lay["shared_up"], x)
        sa = np.array([_rb(_rb(_silu(_rb(sg[f]))) * _rb(su[f])) for f in range(cfg.shared_ffn)])
        sd = _matvec_scalar(lay["shared_down"], sa)
        gate = 1.0 / (1.0 + np.exp(-rl[E]))
        h2[r] = [_rb(h1[r, n] + _rb(_rb(routed[n]) + _rb(gate * _rb(sd[n])))) for n in range(H)]
    return h2


def _embed_scalar(params, cfg, tokens):
    return np.array([[_rb(_deq_scalar(params["embed"], int(t), k)) for k in range(cfg.hidden)]
                     for t in tokens.reshape(-1)])


def _head_scalar(params, cfg, h):
    out = []
    for r in range(h.shape[0]):
        x = _rmsnorm_scalar(h[r], params["final_norm"], cfg.rms_eps)
        out.append([_rb(v) for v in _matvec_scalar(params["lm_head"], x)])
    return np.array(out)


def test_zero_layer_model_is_norm_then_lm_head():
    """Closed form: logits = bf16(bf16(rmsnorm(E[t])) . W_lm), with the embedding
    row dequantized nibble by nibble and the head through the group-wise
    route (scale * sum(x q) + bias * sum(x) per group)."""
    cfg = _cfg(layers=0)
    rng = np.random.default_rng(1)
    params = _params(cfg, rng)
    tokens = np.array([[3, 17, 39], [0, 5, 5]])
    got = verify_forward(params, cfg, tokens, np.array([0, 4]), [], [])
    h = _embed_scalar(params, cfg, tokens)
    xn = np.stack([_rmsnorm_scalar(h[r], params["final_norm"], cfg.rms_eps) for r in range(h.shape[0])])
    want = round_to_bf16(qmm_affine4_groupwise(xn, *params["lm_head"], 64))
    assert np.allclose(got, want, rtol=2 ** -7, atol=1e-9)
    # rows of the same token give the same logits; different tokens differ
    assert np.array_equal(got[4], got[5]) and not np.allclose(got[0], got[1])


def test_zero_o_and_down_leave_the_residual_stream():
    """A layer whose o and down projections are zero (scales = biases = 0)
    adds nothing to h: its logits equal the zero-layer model's bit for bit
    (a dropped residual add, or a norm applied to the stream itself, fails)."""
    cfg = _cfg(layers=2)
    rng = np.random.default_rng(2)
    params = _params(cfg, rng)
    for lay in params["layers"]:
        lay["o"] = _zero_lin(cfg.hidden, cfg.n_heads * cfg.head_dim)
        lay["down"] = _zero_lin(cfg.hidden, cfg.ffn)
    kc, vc = _caches(cfg, rng, 2, 16)
    tokens = np.array([[1, 2, 3], [30, 31, 32]])
    got = verify_forward(params, cfg, tokens, np.array([2, 9]), kc, vc)
    base = dict(params, layers=[])
    want = verify_forward(base, _cfg(layers=0), tokens, np.array([2, 9]), [], [])
    assert np.array_equal(got, want)


def test_dense_layer_equals_scalar_restatement():
    cfg = _cfg(layers=1)
    rng = np.random.default_rng(3)
    params = _params(cfg, rng)
    B, L, cap = 2, 3, 16
    kc, vc = _caches(cfg, rng, B, cap)
    kc2, vc2 = [a.copy() for a in kc], [a.copy() for a in vc]
    tokens = np.array([[4, 9, 11], [22, 0, 37]])
    q_start = np.array([5, 11])
    got = verify_forward(params, cfg, tokens, q_start, kc, vc)
    h = _embed_scalar(params, cfg, tokens)
    h = _layer_scalar(cfg, params["layers"][0], h, tokens.shape, q_start, kc2[0], vc2[0])
    want = _head_scalar(params, cfg, h)
    assert np.allclose(got, want, rtol=2 ** -7, atol=1e-9)
    assert np.allclose(kc[0], kc2[0], rtol=2 ** -7, atol=1e-9) and np.allclose(vc[0], vc2[0], rtol=2 ** -7,
                                                                                 atol=1e-9)


def test_moe_layer_equals_scalar_restatement():
    cfg = _cfg(layers=1, n_experts=6, top_k=2, expert_ffn=64, shared_ffn=64, ffn=0)
    rng = np.random.default_rng(4)
    params = _params(cfg, rng)
    B, L, cap = 2, 2, 8
    kc, vc = _caches(cfg, rng, B, cap)
    kc2, vc2 = [a.copy() for a in kc], [a.copy() for a in vc]
    tokens = np.array([[3, 8], [21, 39]])
    q_start = np.array([1, 5])
    routes = []
    got = verify_forward(params, cfg, tokens, q_start, kc, vc, routes)
    assert len(routes) == 1 and routes[0][0].shape == (4, 2)
    h = _embed_scalar(params, cfg, tokens)
    h = _layer_scalar(cfg, params["layers"][0], h, tokens.shape, q_start, kc2[0], vc2[0])
    want = _head_scalar(params, cfg, h)
    assert np.allclose(got, want, rtol=2 ** -7, atol=1e-9)


def test_moe_block_halves_are_both_added():
    """Zero expert-down and zero shared-down weights leave the stream untouched
    (logits equal the zero-layer model's bit for bit); either half alone
    changes them, so neither the routed sum nor the gated shared expert is
    dropped from the combine."""
    cfg = _cfg(layers=1, n_experts=4, top_k=2, expert_ffn=64, shared_ffn=64, ffn=0)
    rng = np.random.default_rng(5)
    params = _params(cfg, rng)
    lay = params["layers"][0]
    lay["o"] = _zero_lin(cfg.hidden, cfg.n_heads * cfg.head_dim)
    kc, vc = _caches(cfg, rng, 1, 8)
    tokens = np.array([[7, 8]])
    zero_routed = tuple(np.zeros_like(a) if i else a for i, a in enumerate(lay["expert_down"]))
    zero_shared = _zero_lin(cfg.hidden, cfg.shared_ffn)

    def run(layer):
        return verify_forward(dict(params, layers=[layer]), cfg, tokens, np.array([2]), [a.copy() for a in kc],
                              [a.copy() for a in vc])

    want = verify_forward(dict(params, layers=[]), _cfg(layers=0), tokens, np.array([2]), [], [])
    assert np.array_equal(run(dict(lay, expert_down=zero_routed, shared_down=zero_shared)), want)
    assert not np.allclose(run(dict(lay, expert_down=zero_routed)), want)
    assert not np.allclose(run(dict(lay, shared_down=zero_shared)), want)


def test_ragged_batch_equals_scalar_restatement_per_request():
    """The ragged forward (requests of 1, 3 and 2 rows, capacities 8, 16 and
    24, rows packed request after request) equals the scalar restatement run
    on each request alone, so no row reads another request's tokens, cache
    or positions."""
    from oracle.model import verify_forward_ragged
    cfg = _cfg(layers=1)
    rng = np.random.default_rng(8)
    params = _params(cfg, rng)
    caps, lens, q_start = [8, 16, 24], [1, 3, 2], np.array([7, 2, 20])
    kc = [[round_to_bf16(rng.normal(size=(cfg.n_kv_heads, c, cfg.head_dim))) for c in caps]]
    vc = [[round_to_bf16(rng.normal(size=(cfg.n_kv_heads, c, cfg.head_dim))) for c in caps]]
    kc2 = [[a.copy() for a in kc[0]]]
    vc2 = [[a.copy() for a in vc[0]]]
    tokens = [rng.integers(0, cfg.vocab, size=L) for L in lens]
    got = verify_forward_ragged(params, cfg, tokens, q_start, kc, vc)
    assert got.shape == (sum(lens), cfg.vocab)
    r = 0
    for b, L in enumerate(lens):
        tb = tokens[b].reshape(1, L)
        h = _embed_scalar(params, cfg, tb)
        h = _layer_scalar(cfg, params["layers"][0], h, tb.shape, q_start[b:b + 1], kc2[0][b][None],
                          vc2[0][b][None])
        want = _head_scalar(params, cfg, h)
        assert np.allclose(got[r:r + L], want, rtol=2 ** -7, atol=1e-9), b
        r += L
