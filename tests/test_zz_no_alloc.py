"""GPU test of mtp_spec_accept_noalloc (workspace in a file-scope device
array): the same outputs as mtp_spec_accept with a caller workspace, bit for
bit, on two calls in a row (the second smaller, so it runs over the first's
leftover scratch contents), and a clear refusal above the array's size."""

import numpy as np
import pytest
import torch

from mtplx_amd import _lib
from oracle import sampler as S

pytestmark = pytest.mark.gpu


def _inputs(seed, B, K, V, cfg):
    rng = np.random.default_rng(seed)
    target = rng.normal(0, 3, (B, K + 1, V)).astype(np.float32)
    draft = (target[:, :K] + rng.normal(0, 0.7, (B, K, V))).astype(np.float32)
    drafts = np.stack([S.sample_rows(draft[b], rng.random(K), cfg) for b in range(B)]).astype(np.int32)
    u = rng.random((B, K + 1))
    return [torch.from_numpy(a).cuda() for a in (target.reshape(-1, V), draft.reshape(-1, V), drafts, u)]


def _outs(B, K):
    return (torch.full((B, K + 1), -7, dtype=torch.int32, device="cuda"),
            torch.full((B,), -7, dtype=torch.int32, device="cuda"),
            torch.full((B, K), -7.0, dtype=torch.float64, device="cuda"),
            torch.full((B,), -7, dtype=torch.int32, device="cuda"))


def _run(noalloc, ins, B, K, V, cfg):
    t, d, di, u = ins
    out, nacc, ap, st = _outs(B, K)
    stream = torch.cuda.current_stream().cuda_stream
    common = (t.data_ptr(), d.data_ptr(), di.data_ptr(), u.data_ptr(), B, K, V, cfg.temperature, cfg.top_k,
              cfg.top_p, out.data_ptr(), nacc.data_ptr(), ap.data_ptr(), st.data_ptr())
    if noalloc:
        _lib.call("mtp_spec_accept_noalloc", *common, stream)
    else:
        nb = _lib.query("mtp_sampler_workspace_bytes", B * (2 * K + 1), V, cfg.top_k)
        ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
        _lib.call("mtp_spec_accept", *common, ws.data_ptr(), nb, stream)
    torch.cuda.synchronize()
    return [x.cpu() for x in (out, nacc, ap, st)]


@pytest.mark.parametrize("cfg,shapes", [
    (S.SamplerConfig(0.6, 0.95, 20), ((4, 3, 151936), (2, 2, 30000))),
    (S.SamplerConfig(1.0, 0.9, 200), ((3, 3, 8000), (1, 1, 3000))),     # wide laws
])
def test_noalloc_equals_workspace_entry_two_calls(gpu, cfg, shapes):
    for seed, (B, K, V) in enumerate(shapes):
        ins = _inputs(seed, B, K, V, cfg)
        want = _run(False, ins, B, K, V, cfg)
        got = _run(True, ins, B, K, V, cfg)
        for w, g in zip(want, got):
            assert torch.equal(w, g), (seed, B, K, V)
        assert (got[3] == 0).all()


def test_noalloc_refuses_beyond_its_scratch(gpu):
    cfg = S.SamplerConfig(0.6, 0.95, 0)      # wide laws at the full vocabulary: about 25 MB
    B, K, V = 1, 3, 151936
    ins = _inputs(3, B, K, V, S.SamplerConfig(0.6, 0.95, 20))
    with pytest.raises(_lib.MtpError) as e:
        _run(True, ins, B, K, V, cfg)
    assert e.value.code == -2 and "scratch" in str(e.value)
