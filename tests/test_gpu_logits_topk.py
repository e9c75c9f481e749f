"""GPU parity of the lm_head with the sampler's vocabulary reduction fused
into its epilogue (emode 5) and of the accept step that consumes it
(``mtp_spec_accept_parts``).

Bars: the fused call's fp32 logits bit-exact against the plain lm_head's;
its partial records, merged over each row on the host, against the accept
step's own chunk records over those logits (``mtp_sample_rows`` writes them),
merged the same way: the top-k keys, the maximum and the non-finite flag
bit-exact, the fp64 total sum(exp(l/T - max)) within 1e-12 relative
(another summation order); no id in two records of a row; the verify step
with and without the fusion token-exact, accept probabilities within 1e-12;
arrival counters back at zero."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

PART = np.dtype([("m", "<f8"), ("s", "<f8"), ("nf", "<i4"), ("pad", "<i4"), ("keys", "<u8", (64,))])


def _st():
    return torch.cuda.current_stream().cuda_stream


def _parts(buf: torch.Tensor, rows: int, per_row: int, used: int) -> np.ndarray:
    b = buf[: rows * per_row * PART.itemsize].cpu().numpy()
    return b.view(PART).reshape(rows, per_row)[:, :used]


def _merge(recs: np.ndarray, ksel: int, greedy: bool):
    """One row's records -> (top-ksel keys, max, total sum, flag); key 0 is
    an empty slot (never a valid key: its id field would be 2^32-1)."""
    keys = recs["keys"][:, :ksel].reshape(-1)
    keys = np.sort(keys[keys != 0])[::-1][:ksel]
    nf = int(recs["nf"].max())
    if greedy:
        return keys, None, None, nf
    m = float(recs["m"].max())
    tot = float(sum(r["s"] * np.exp(r["m"] - m) for r in recs if r["s"] > 0))
    return keys, m, tot, nf


def _fused(q, layout, x, M, V, K, temp, top_k):
    from mtplx_amd import _lib
    pb = _lib.query("mtp_logits_topk_parts_bytes", M)
    parts = torch.zeros(pb, dtype=torch.uint8, device="cuda")
    tb = _lib.query("mtp_logits_topk_workspace_bytes", M, V)
    tws = torch.zeros(tb, dtype=torch.uint8, device="cuda")
    logits = torch.full((M, V), float("nan"), dtype=torch.float32, device="cuda")
    w = q.pack(layout=layout)
    tk = dict(parts=parts, ws=tws, ws_bytes=tws.numel(), temperature=temp, top_k=top_k)
    _lib.qmv_ex(_st(), x=x, w0=w, yf=logits, M=M, N=V, K=K, group_size=64, xmode=0, emode=5, packed=layout, topk=tk)
    torch.cuda.synchronize()
    n = tk["n_parts"]
    assert 1 <= n <= 64
    return logits, _parts(parts, M, 64, n), tws


def _reference_parts(logits, M, V, temp, top_k):
    from mtplx_amd import _lib
    n_chunks = (V + 4095) // 4096
    nb = _lib.query("mtp_sampler_workspace_bytes", M, V, top_k)
    ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    u = torch.full((M,), 0.5, dtype=torch.float64, device="cuda")
    ids = torch.empty((M, 64), dtype=torch.int32, device="cuda")
    probs = torch.empty((M, 64), dtype=torch.float64, device="cuda")
    cnt = torch.empty(M, dtype=torch.int32, device="cuda")
    smp = torch.empty(M, dtype=torch.int32, device="cuda")
    st = torch.empty(M, dtype=torch.int32, device="cuda")
    _lib.call("mtp_sample_rows", logits.data_ptr(), M, V, temp, top_k, 1.0, u.data_ptr(), ids.data_ptr(),
              probs.data_ptr(), 64, cnt.data_ptr(), smp.data_ptr(), st.data_ptr(), ws.data_ptr(), ws.numel(), _st())
    torch.cuda.synchronize()
    return _parts(ws, M, n_chunks, n_chunks)


@pytest.mark.parametrize("M,layout,V,K,temp,top_k", [
    (4, 2, 151936, 5120, 0.6, 20),     # the cfg3 lm_head
    (4, 2, 151936, 5120, 0.0, 20),     # greedy
    (8, 1, 151936, 5120, 1.0, 64),
    (1, 2, 1000, 1024, 0.7, 7),        # one partial chunk
    (3, 2, 12000, 2048, 1.3, 33),
])
def test_fused_partials_match_first_pass(gpu, M, layout, V, K, temp, top_k):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(M * 31 + V + top_k)
    q = QuantizedLinear.random(V, K, 64, generator=g)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    logits, got, tws = _fused(q, layout, x, M, V, K, temp, top_k)
    plain = torch.full((M, V), float("nan"), dtype=torch.float32, device="cuda")
    nb = _lib.query("mtp_qmv_workspace_bytes", M, V, K, 0)
    qws = torch.zeros(max(nb, 256), dtype=torch.uint8, device="cuda")
    _lib.qmv_ex(_st(), x=x, w0=q.pack(layout=layout), yf=plain, M=M, N=V, K=K, group_size=64, xmode=0, emode=0,
                packed=layout, ws=qws, ws_bytes=qws.numel())
    torch.cuda.synchronize()
    assert torch.equal(logits.view(torch.int32), plain.view(torch.int32))
    want = _reference_parts(plain, M, V, temp, top_k)
    greedy = temp <= 0
    ksel = 1 if greedy else top_k
    for r in range(M):
        gk, gm, gs, gnf = _merge(got[r], ksel, greedy)
        wk, wm, ws, wnf = _merge(want[r], ksel, greedy)
        assert np.array_equal(gk, wk) and gnf == wnf, f"row {r}"
        if not greedy:
            assert gm == wm and abs(gs - ws) <= 1e-12 * ws, f"row {r}"
        # the records' id sets are disjoint: no id appears in two records
        k = got[r]["keys"][:, :ksel].reshape(-1)
        k = k[k != 0]
        assert len(np.unique(k & 0xFFFFFFFF)) == len(k), f"row {r}: an id in two records"
    # the arrival counters (the scratch's first 256 bytes) are back at zero
    assert int(torch.count_nonzero(tws[:256])) == 0


def test_fused_lm_head_refuses_wide_laws_and_many_rows(gpu):
    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear
    g = torch.Generator(device="cuda").manual_seed(3)
    q = QuantizedLinear.random(4096, 1024, 64, generator=g)
    for M, top_k in ((4, 0), (4, 65), (9, 20)):
        x = torch.randn((M, 1024), device="cuda", generator=g).to(torch.bfloat16)
        with pytest.raises(_lib.MtpError):
            _fused(q, 1, x, M, 4096, 1024, 0.6, top_k)


@pytest.mark.parametrize("B,K,cfg", [(1, 3, (0.6, 0.95, 20)), (1, 3, (0.0, 1.0, 1)), (2, 3, (1.0, 0.8, 64)),
                                     (1, 2, (0.7, 1.0, 40))])
def test_verify_step_with_and_without_fusion(gpu, B, K, cfg):
    from dataclasses import replace

    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import DENSE_27B, VerifyModel
    c = replace(DENSE_27B, layers=1, hidden=1024, ffn=2048, n_heads=8, n_kv_heads=2)
    model = VerifyModel(c, device="cuda", seed=B * 10 + K)
    model.allocate_cache(B, 512)
    g = torch.Generator(device="cuda").manual_seed(77)
    L = K + 1
    tokens = torch.randint(0, c.vocab, (B, L), device="cuda", dtype=torch.int32, generator=g)
    qs = torch.full((B,), 300, dtype=torch.int32, device="cuda")
    sampler = SamplerConfig(*cfg)
    # drafts close to the target so accepts and rejects both happen
    base = model.verify_logits(tokens, qs).reshape(B, L, -1)
    draft = (base[:, :K] + 0.3 * torch.randn((B, K, c.vocab), device="cuda", generator=g)).contiguous()
    for seed in range(4):
        u = torch.rand((B, L), device="cuda", dtype=torch.float64,
                       generator=torch.Generator(device="cuda").manual_seed(seed))
        a = model.verify_step(tokens, qs, draft, u, sampler, fuse_topk=True)
        ta, na, pa = a.tokens.clone(), a.n_accepted.clone(), a.accept_probs.clone()
        b = model.verify_step(tokens, qs, draft, u, sampler, fuse_topk=False)
        torch.cuda.synchronize()
        assert torch.equal(ta, b.tokens) and torch.equal(na, b.n_accepted)
        assert torch.allclose(pa, b.accept_probs, rtol=1e-12, atol=1e-15)
        assert int(a.status.max()) == 0
