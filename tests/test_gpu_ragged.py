"""GPU parity of the continuous-batched ragged verify lane (BASELINE cfg4):
per-request depths K_b in {1, 2, 3} packed as M = sum_b (K_b + 1) rows,
per-request KV capacities in one block cache (kv_off), the ragged RoPE
writer, block attention with per-request lengths, the 9..64-row MFMA
matmul, and accept/reject with per-request depths.

Bars: attention and logits within rtol/atol 1e-2 of the float64 oracle
(``oracle.model.verify_forward_ragged``: the same forward, request by
request); RoPE'd K within 1e-2 of the rotate-half pair norm; the ragged
writer bit-exact against the uniform writer on each request; accepted ids
token-exact against the oracle law per request.
"""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import sampler as S
from oracle.model import verify_forward_ragged
from tests.gpu_util import assert_close, bf16_values
from tests.model_util import model_params_numpy
from tests.test_gpu_model_full import assert_rope_close

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _batch(rng, B, max_ctx=65536, min_ctx=1024):
    """Depths uniform in {1,2,3}, contexts log-uniform in [min_ctx, max_ctx]
    (the largest request pinned to max_ctx), capacities = context + rows."""
    depths = rng.integers(1, 4, size=B)
    ctx = np.exp(rng.uniform(np.log(min_ctx), np.log(max_ctx), size=B)).astype(np.int64)
    ctx[int(rng.integers(0, B))] = max_ctx - 4
    lens = depths + 1
    q_start = ctx - lens
    caps = ((ctx + 31) // 32) * 32
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    return depths, lens, q_start.astype(np.int32), caps, row_off


def test_block_attention_matches_oracle(gpu):
    from mtplx_amd import _lib
    rng = np.random.default_rng(3)
    B, Hq, Hkv, D = 6, 40, 8, 128
    depths, lens, q_start, caps, row_off = _batch(rng, B, max_ctx=40000, min_ctx=300)
    Lmax = int(lens.max())
    nblk = caps // 32
    kv_off = np.concatenate([[0], np.cumsum(Hkv * nblk)]).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(4)
    kb = torch.randn(int(kv_off[-1]) * 4096, device="cuda", generator=g).to(torch.bfloat16)
    vb = torch.randn(int(kv_off[-1]) * 4096, device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn((B, Hq, Lmax, D), device="cuda", generator=g).to(torch.bfloat16)
    M = int(row_off[-1])
    out = torch.full((M, Hq * D), float("nan"), dtype=torch.bfloat16, device="cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()  # noqa: E731
    nb = _lib.query("mtp_attn_blocks_workspace_bytes", B, Hkv, int(caps.max()), int(caps.sum()), 0)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    _lib.attn_blocks(_st(), q=q, k_blk=kb, v_blk=vb, q_start=t(q_start), q_lens=t(lens), row_off=t(row_off),
                     kv_off=t(kv_off), out=out, B=B, Hq=Hq, Hkv=Hkv, Lmax=Lmax, D=D, cap=int(caps.max()),
                     split_keys=0, scale=1.0 / np.sqrt(D), total_cap=int(caps.sum()), ws=ws, ws_bytes=ws.numel())
    torch.cuda.synchronize()
    from mtplx_amd.verify_step import kv_from_blocks
    got = bf16_values(out)
    for b in range(B):
        o0, o1 = int(kv_off[b]), int(kv_off[b + 1])
        kr = kv_from_blocks(kb[o0 * 4096:o1 * 4096].reshape(1, Hkv, int(caps[b]), D), "k").float().cpu().numpy()
        vr = kv_from_blocks(vb[o0 * 4096:o1 * 4096].reshape(1, Hkv, int(caps[b]), D), "v").float().cpu().numpy()
        L = int(lens[b])
        want = A.ragged_gqa_attention(q[b:b + 1, :, :L].float().cpu().numpy(), kr, vr, [int(q_start[b])])[0]
        rows = got[row_off[b]:row_off[b + 1]].reshape(L, Hq, D).transpose(1, 0, 2)
        assert_close(rows, want, what=f"request {b} (ctx {q_start[b] + L})")


def test_ragged_rope_writer_matches_uniform_writer(gpu):
    from mtplx_amd import _lib
    rng = np.random.default_rng(5)
    B, Hq, Hkv, D = 4, 8, 2, 128
    lens = np.array([2, 4, 1, 3], np.int32)
    caps = np.array([96, 256, 64, 160])
    q_start = np.array([10, 250, 0, 100], np.int32)
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    kv_off = np.concatenate([[0], np.cumsum(Hkv * (caps // 32))]).astype(np.int32)
    Lmax, M = int(lens.max()), int(row_off[-1])
    g = torch.Generator(device="cuda").manual_seed(6)
    qkv = torch.randn((M, (Hq + 2 * Hkv) * D), device="cuda", generator=g).to(torch.bfloat16)
    kb = torch.zeros(int(kv_off[-1]) * 4096, dtype=torch.bfloat16, device="cuda")
    vb = torch.zeros_like(kb)
    qo = torch.zeros((B, Hq, Lmax, D), dtype=torch.bfloat16, device="cuda")
    st = torch.zeros(1, dtype=torch.int32, device="cuda")
    # Device copies held in names: a temporary's memory could be handed to
    # the next temporary before the (asynchronous) kernel reads it.
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()  # noqa: E731
    d_row, d_qs, d_kv = t(row_off), t(q_start), t(kv_off)
    _lib.call("mtp_rope_qkv_to_blocks", qkv.data_ptr(), M, d_row.data_ptr(), d_qs.data_ptr(), d_kv.data_ptr(),
              qo.data_ptr(), kb.data_ptr(), vb.data_ptr(), B, Lmax, Hq, Hkv, D, 0, 1.0e6, st.data_ptr(), _st())
    for b in range(B):
        L, cap = int(lens[b]), int(caps[b])
        k1 = torch.zeros((1, Hkv, cap, D), dtype=torch.bfloat16, device="cuda")
        v1 = torch.zeros_like(k1)
        q1 = torch.zeros((1, Hq, L, D), dtype=torch.bfloat16, device="cuda")
        rows = qkv[row_off[b]:row_off[b + 1]].contiguous()
        qs1 = t([q_start[b]])
        _lib.call("mtp_rope_qkv_to_cache_vt", rows.data_ptr(), qs1.data_ptr(), None, q1.data_ptr(), k1.data_ptr(),
                  v1.data_ptr(), 1, L, Hq, Hkv, D, cap, 1.0e6, st.data_ptr(), _st())
        torch.cuda.synchronize()
        o0, o1 = int(kv_off[b]) * 4096, int(kv_off[b + 1]) * 4096
        assert torch.equal(kb[o0:o1], k1.reshape(-1)) and torch.equal(vb[o0:o1], v1.reshape(-1)), b
        assert torch.equal(qo[b, :, :L], q1[0]), b
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    # a position past a request's capacity is skipped and flagged
    bad = t(np.array([10, 250, 64, 100]))   # request 2: capacity 64, one row at 64
    _lib.call("mtp_rope_qkv_to_blocks", qkv.data_ptr(), M, d_row.data_ptr(), bad.data_ptr(), d_kv.data_ptr(),
              qo.data_ptr(), kb.data_ptr(), vb.data_ptr(), B, Lmax, Hq, Hkv, D, 0, 1.0e6, st.data_ptr(), _st())
    torch.cuda.synchronize()
    assert int(st.item()) == 1


def test_cfg4_ragged_verify_step_matches_oracle(gpu):
    """One 27B-width layer, 16 requests, depths U{1,2,3}, contexts
    log-uniform in [1k, 64k] (M = sum of K_b + 1 rows, at most 64)."""
    from dataclasses import replace

    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import DENSE_27B, VerifyModel
    rng = np.random.default_rng(11)
    B = 16
    depths, lens, q_start, caps, row_off = _batch(rng, B)
    cfg = replace(DENSE_27B, layers=1)
    model = VerifyModel(cfg, device="cuda", seed=12)
    model.allocate_cache_blocks(caps)
    kc = [[model.cache_request(0, b, "k").float().cpu().numpy().astype(np.float64) for b in range(B)]]
    vc = [[model.cache_request(0, b, "v").float().cpu().numpy().astype(np.float64) for b in range(B)]]
    M = int(row_off[-1])
    tokens = rng.integers(0, cfg.vocab, size=M).astype(np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()  # noqa: E731
    Lmax = int(lens.max())
    # draft rows/ids: the rows after each request's primary
    d_off = np.concatenate([[0], np.cumsum(depths)]).astype(np.int32)
    draft_index = np.concatenate([np.arange(row_off[b] + 1, row_off[b + 1]) for b in range(B)]).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(13)
    draft_logits = 3.0 * torch.randn((int(d_off[-1]), cfg.vocab), device="cuda", generator=g)
    uniforms = torch.rand((B, 4), device="cuda", dtype=torch.float64, generator=g)
    sampler = SamplerConfig(0.6, 0.95, 20)
    res = model.verify_step_ragged(t(tokens), t(row_off), t(q_start), t(lens), Lmax, draft_logits, t(d_off),
                                   t(draft_index).long(), uniforms, sampler)
    torch.cuda.synchronize()
    model.check_status()
    got = model.last_logits.cpu().numpy().astype(np.float64)
    toks = [tokens[row_off[b]:row_off[b + 1]] for b in range(B)]
    want = verify_forward_ragged(model_params_numpy(model), cfg, toks, q_start, kc, vc)
    assert_close(got, want, what="cfg4 ragged logits")
    for b in (0, 7, 15):
        k = model.cache_request(0, b, "k").float().cpu().numpy()
        s0, L = int(q_start[b]), int(lens[b])
        assert_rope_close(k[:, s0:s0 + L], kc[0][b][:, s0:s0 + L])
    # accept/reject, request by request, token-exact against the oracle law
    dl = draft_logits.cpu().numpy()
    u = uniforms.cpu().numpy()
    lg = model.last_logits.cpu().numpy()
    for b in range(B):
        K = int(depths[b])
        w = S.spec_accept(lg[row_off[b]:row_off[b + 1]], dl[d_off[b]:d_off[b + 1]],
                          tokens[draft_index[d_off[b]:d_off[b + 1]]], u[b], S.SamplerConfig(0.6, 0.95, 20))
        assert int(res.n_accepted[b]) == w.n_accepted, b
        assert res.tokens[b].cpu().numpy().tolist()[: len(w.tokens)] == w.tokens, b
        assert (res.tokens[b, K + 1:].cpu().numpy() == -1).all()
        assert int(res.status[b]) == 0


def _blocks_attention(ctx, lens, split_keys, seed, Hq=40, Hkv=8, ws_fill=None):
    """Block attention over requests with contexts ``ctx`` (keys before the
    new rows) and ``lens`` query rows; returns (output rows, inputs).
    ``ws_fill``: a float every word of the workspace holds beforehand (stale
    partials that must never be read)."""
    from mtplx_amd import _lib
    D = 128
    B = len(ctx)
    lens = np.asarray(lens, np.int32)
    q_start = np.asarray(ctx, np.int32)
    caps = ((q_start + lens + 31) // 32) * 32
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    Lmax = int(lens.max())
    kv_off = np.concatenate([[0], np.cumsum(Hkv * (caps // 32))]).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(seed)
    kb = torch.randn(int(kv_off[-1]) * 4096, device="cuda", generator=g).to(torch.bfloat16)
    vb = torch.randn(int(kv_off[-1]) * 4096, device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn((B, Hq, Lmax, D), device="cuda", generator=g).to(torch.bfloat16)
    out = torch.full((int(row_off[-1]), Hq * D), float("nan"), dtype=torch.bfloat16, device="cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()  # noqa: E731
    d_qs, d_lens, d_row, d_kv = t(q_start), t(lens), t(row_off), t(kv_off)
    nb = _lib.query("mtp_attn_blocks_workspace_bytes", B, Hkv, int(caps.max()), int(caps.sum()), split_keys)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    if ws_fill is not None:
        ws.view(torch.float32)[: nb // 4].fill_(ws_fill)
    _lib.attn_blocks(_st(), q=q, k_blk=kb, v_blk=vb, q_start=d_qs, q_lens=d_lens, row_off=d_row, kv_off=d_kv,
                     out=out, B=B, Hq=Hq, Hkv=Hkv, Lmax=Lmax, D=D, cap=int(caps.max()), split_keys=split_keys,
                     scale=1.0 / np.sqrt(D), total_cap=int(caps.sum()), ws=ws, ws_bytes=ws.numel())
    torch.cuda.synchronize()
    return bf16_values(out), (q, kb, vb, q_start, lens, caps, row_off, kv_off)


@pytest.mark.parametrize("case", ["long_among_short", "tiny_total", "single", "uniform", "many", "short_multi_tile"])
@pytest.mark.parametrize("split_keys", [0, 1024])
@pytest.mark.parametrize("merge", ["auto", "column"])
def test_block_attention_balanced_shapes(gpu, case, split_keys, merge, monkeypatch):
    """split_keys 0 runs the balanced kernel (equal shares of all tiles per
    workgroup, per-head partial slots); 1024 the per-unit kernel. Both
    against the float64 oracle, request by request. merge "auto" merges the
    partials per (request, kv head) when the batch has 64 heads or more
    (long_among_short: 96), "column" per (request, kv head, query column)
    everywhere."""
    from mtplx_amd.verify_step import kv_from_blocks
    if merge == "column":
        monkeypatch.setenv("MTPLX_AMD_ATTN_MERGE_HEAD", "0")
    rng = np.random.default_rng(17)
    if case == "long_among_short":
        ctx = list(rng.integers(0, 97, size=11)) + [20000]
        lens = list(rng.integers(1, 5, size=12))
    elif case == "tiny_total":
        ctx, lens = [3, 0], [2, 4]
    elif case == "single":
        ctx, lens = [30000], [4]
    elif case == "many":   # 130 requests: the prologue's request scans run in three rounds of 64
        ctx = list(rng.integers(0, 400, size=130))
        lens = list(rng.integers(1, 5, size=130))
    elif case == "short_multi_tile":   # fewer tiles (72) than workgroups, several per head
        ctx, lens = [60, 200], [4, 2]
    else:
        ctx, lens = [4093] * 4, [3] * 4
    Hq, Hkv, D = 40, 8, 128
    # every workspace word 1e4 beforehand: a partial slot the merge reads but
    # no workgroup wrote would dominate the merged rows
    got, (q, kb, vb, q_start, lens, caps, row_off, kv_off) = _blocks_attention(ctx, lens, split_keys, seed=23,
                                                                             ws_fill=1e4)
    assert np.isfinite(got).all()
    for b in range(len(ctx)):
        o0, o1 = int(kv_off[b]), int(kv_off[b + 1])
        kr = kv_from_blocks(kb[o0 * 4096:o1 * 4096].reshape(1, Hkv, int(caps[b]), D), "k").float().cpu().numpy()
        vr = kv_from_blocks(vb[o0 * 4096:o1 * 4096].reshape(1, Hkv, int(caps[b]), D), "v").float().cpu().numpy()
        L = int(lens[b])
        want = A.ragged_gqa_attention(q[b:b + 1, :, :L].float().cpu().numpy(), kr, vr, [int(q_start[b])])[0]
        rows = got[row_off[b]:row_off[b + 1]].reshape(L, Hq, D).transpose(1, 0, 2)
        assert_close(rows, want, what=f"{case} request {b} (ctx {q_start[b] + L})")
