"""The greedy exact lane: a request's verify logits do not depend on the batch.

The reference promises that a greedy (temperature <= 0) verify picks the
argmax autoregressive decode would (``mtplx/nax_verify.py:755-763``,
``mtplx/attention_context.py:99``). Here one request (27B widths, two
layers) is verified

* alone with one row (its primary token only: the decode step),
* alone with its 4 verify rows,
* as request 5 of a 16-request ragged batch (45 rows, depths 1..3, contexts
  1k..40k, per-request capacities),
* through ``verify_step`` at temperature 0 on the uniform cache,

on the same cache contents; the logits of every shared row must be
bit-identical, and the K/V rows written too. The greedy accept on the batch
is checked against the greedy rule.
"""

import numpy as np
import pytest
import torch

from oracle.model import verify_forward
from tests.gpu_util import assert_close
from tests.model_util import model_params_numpy

pytestmark = pytest.mark.gpu


def _set_request_cache(model, li, b, k_std, v_std):
    """Write request b's [Hkv, cap_b, D] K/V into a block cache."""
    from mtplx_amd.verify_step import kv_to_blocks
    o0, o1 = model._kv_off_host[b], model._kv_off_host[b + 1]
    model.k_cache[li][o0 * 4096:o1 * 4096] = kv_to_blocks(k_std[None], "k").reshape(-1)
    model.v_cache[li][o0 * 4096:o1 * 4096] = kv_to_blocks(v_std[None], "v").reshape(-1)


@pytest.mark.timeout(600)
def test_greedy_logits_bit_identical_across_batches(gpu):
    from dataclasses import replace

    from mtplx_amd.attention_context import exact_lane_counts
    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import DENSE_27B, VerifyModel
    cfg = replace(DENSE_27B, layers=2)
    model = VerifyModel(cfg, device="cuda", seed=31)
    dev = "cuda"
    gen = torch.Generator(device=dev).manual_seed(32)
    ctx_r, L = 3000, 4
    cap_r = 3072
    Hkv, D = cfg.n_kv_heads, cfg.head_dim
    kstd = [torch.randn((Hkv, cap_r, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(cfg.layers)]
    vstd = [torch.randn((Hkv, cap_r, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(cfg.layers)]
    toks_r = torch.randint(0, cfg.vocab, (L,), device=dev, dtype=torch.int32, generator=gen)
    qs_r = ctx_r - L

    def alone(nrows):
        model.allocate_cache_blocks([cap_r], fill_random=False)
        for li in range(cfg.layers):
            _set_request_cache(model, li, 0, kstd[li], vstd[li])
        ro = torch.tensor([0, nrows], dtype=torch.int32, device=dev)
        logits = model.verify_logits_ragged(toks_r[:nrows].contiguous(), ro,
                                            torch.tensor([qs_r], dtype=torch.int32, device=dev),
                                            torch.tensor([nrows], dtype=torch.int32, device=dev), nrows, exact=True,
                                            check=True)
        k_rows = [model.cache_request(li, 0, "k")[:, qs_r:qs_r + nrows].clone() for li in range(cfg.layers)]
        return logits.clone(), k_rows

    l1, k1 = alone(1)
    l4, k4 = alone(4)
    # the ragged batch: request 5 is the one above
    rng = np.random.default_rng(33)
    B, slot = 16, 5
    depths = rng.integers(1, 4, B)
    depths[slot] = L - 1
    ctxs = np.exp(rng.uniform(np.log(1024), np.log(40000), B)).astype(int)
    ctxs[slot] = ctx_r
    lens = depths + 1
    caps = [int(((c + 31) // 32) * 32) for c in ctxs]
    caps[slot] = cap_r
    model.allocate_cache_blocks(caps)
    for li in range(cfg.layers):
        _set_request_cache(model, li, slot, kstd[li], vstd[li])
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    M = int(row_off[-1])
    tokens = torch.randint(0, cfg.vocab, (M,), device=dev, dtype=torch.int32, generator=gen)
    tokens[row_off[slot]:row_off[slot] + L] = toks_r
    qstart = torch.tensor(ctxs - lens, dtype=torch.int32, device=dev)
    ro = torch.from_numpy(row_off).to(dev)
    ql = torch.from_numpy(lens.astype(np.int32)).to(dev)
    lb = model.verify_logits_ragged(tokens, ro, qstart, ql, int(lens.max()), exact=True, check=True)
    kb = [model.cache_request(li, slot, "k")[:, qs_r:qs_r + L].clone() for li in range(cfg.layers)]
    r0 = int(row_off[slot])
    bitw = lambda t: t.contiguous().view(torch.int32)   # noqa: E731
    assert torch.equal(bitw(l4), bitw(lb[r0:r0 + L])), "request logits differ alone and inside the batch"
    assert torch.equal(bitw(l1[0]), bitw(l4[0])), "the primary row differs at M=1 and M=4"
    for li in range(cfg.layers):
        assert torch.equal(k4[li].view(torch.int16), kb[li].view(torch.int16))
        assert torch.equal(k1[li][:, 0].view(torch.int16), k4[li][:, 0].view(torch.int16))
    # greedy accept on the batch: each request follows the argmax rule
    from mtplx_amd.sampling import spec_accept_ragged
    V = cfg.vocab
    d_off = np.concatenate([[0], np.cumsum(depths)]).astype(np.int32)
    draft_rows = torch.randn((int(d_off[-1]), V), device=dev, generator=gen)
    draft_ids = torch.empty(int(d_off[-1]), dtype=torch.int32, device=dev)
    arg = lb.argmax(dim=1).to(torch.int32)
    for b in range(B):          # drafts equal the target argmax except request 2's depth 0
        for d in range(int(depths[b])):
            draft_ids[d_off[b] + d] = arg[row_off[b] + d] if b != 2 or d else (arg[row_off[b]] + 1) % V
    res = spec_accept_ragged(lb, ro[:-1], draft_rows, torch.from_numpy(d_off[:-1]).to(dev),
                             torch.from_numpy(depths.astype(np.int32)).to(dev), draft_ids,
                             torch.zeros((B, 4), dtype=torch.float64, device=dev), SamplerConfig(0.0, 1.0, 0))
    torch.cuda.synchronize()
    nacc = res.n_accepted.cpu().numpy()
    assert nacc[2] == 0 and all(nacc[b] == depths[b] for b in range(B) if b != 2)
    toks = res.tokens.cpu().numpy()
    a = arg.cpu().numpy()
    assert toks[2, 0] == a[row_off[2]]
    assert toks[slot, L - 1] == a[r0 + L - 1]
    # verify_step at temperature 0 on the uniform cache takes the exact lane: same logits
    model.allocate_cache(1, cap_r, fill_random=False)
    from mtplx_amd.verify_step import kv_to_blocks
    for li in range(cfg.layers):
        model.k_cache[li].copy_(kv_to_blocks(kstd[li][None], "k"))
        model.v_cache[li].copy_(kv_to_blocks(vstd[li][None], "v"))
    n0 = exact_lane_counts["verify_step"]
    dl = torch.randn((1, L - 1, V), device=dev, generator=gen)
    model.verify_step(toks_r[None], torch.tensor([qs_r], dtype=torch.int32, device=dev), dl,
                      torch.zeros((1, L), dtype=torch.float64, device=dev), SamplerConfig(0.0, 1.0, 0))
    torch.cuda.synchronize()
    assert exact_lane_counts["verify_step"] == n0 + 1
    assert torch.equal(bitw(model.last_logits), bitw(l4))
    # and the exact lane meets the oracle bar
    kc = [kstd[li][None].float().cpu().numpy().astype(np.float64) for li in range(cfg.layers)]
    vc = [vstd[li][None].float().cpu().numpy().astype(np.float64) for li in range(cfg.layers)]
    want = verify_forward(model_params_numpy(model), cfg, toks_r[None].cpu().numpy(), np.array([qs_r]), kc, vc)
    assert_close(l4.cpu().numpy().astype(np.float64), want, what="exact lane logits")
