"""GPU parity: ragged KV cache mechanics (bit-exact) and ragged GQA attention
(bf16 within rtol/atol 1e-2 of the float64 oracle)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import kv_cache as KV
from mtplx_amd import _lib
from tests.gpu_util import assert_close, bf16_values, bits, randn_bf16

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _attn(q, k, v, q_start, q_lens=None, split_keys=0, rows_layout=False):
    B, Hq, L, D = q.shape
    Hkv, cap = k.shape[1], k.shape[2]
    qs = torch.tensor(q_start, dtype=torch.int32, device="cuda")
    ql = None if q_lens is None else torch.tensor(q_lens, dtype=torch.int32, device="cuda")
    out = torch.full((B, L, Hq, D) if rows_layout else (B, Hq, L, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    nb = _lib.query("mtp_attn_workspace_bytes", B, Hkv, cap, split_keys)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    fn = "mtp_ragged_gqa_attn_rows" if rows_layout else "mtp_ragged_gqa_attn"
    _lib.call(fn, q.data_ptr(), k.data_ptr(), v.data_ptr(), qs.data_ptr(), None if ql is None else ql.data_ptr(),
              out.data_ptr(), B, Hq, Hkv, L, D, cap, 1.0 / math.sqrt(D), split_keys, ws.data_ptr(), nb, _st())
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("B,Hq,Hkv,L,cap,starts,split", [
    (2, 4, 1, 4, 96, [0, 60], 32),
    (3, 40, 8, 4, 700, [17, 300, 640], 0),
    (2, 32, 4, 4, 1300, [1000, 5], 64),
    (1, 8, 8, 1, 64, [40], 0),
    (2, 16, 2, 2, 128, [33, 90], 32),
])
def test_ragged_attention_matches_oracle(gpu, B, Hq, Hkv, L, cap, starts, split):
    rng = np.random.default_rng(B * 100 + cap)
    q = randn_bf16(rng, (B, Hq, L, 128)); k = randn_bf16(rng, (B, Hkv, cap, 128)); v = randn_bf16(rng, (B, Hkv, cap, 128))
    out = _attn(q, k, v, starts, split_keys=split)
    want = A.ragged_gqa_attention(bits(q), bits(k), bits(v), starts)
    got = bf16_values(out)
    assert np.isfinite(got).all()
    assert_close(got, want, what="attention")
    rows = _attn(q, k, v, starts, split_keys=split, rows_layout=True)
    assert torch.equal(rows.permute(0, 2, 1, 3).contiguous().view(torch.int16), out.view(torch.int16))


def test_cfg2_ragged_lengths(gpu):
    """BASELINE cfg2 shape class: 8 requests, lengths U[512, 32768], 4 rows, 40/8 heads."""
    rng = np.random.default_rng(2024)
    B, Hq, Hkv, L, D = 8, 40, 8, 4, 128
    lens = rng.integers(512, 32769, size=B)
    cap = int(lens.max())
    starts = (lens - L).tolist()
    g = torch.Generator(device="cuda").manual_seed(7)
    q = randn_bf16(rng, (B, Hq, L, D))
    k = torch.randn((B, Hkv, cap, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, Hkv, cap, D), generator=g, device="cuda").to(torch.bfloat16)
    out = _attn(q, k, v, starts)
    # Oracle on a subset of (request, head) pairs keeps the float64 check in seconds.
    qb, kb, vb = bits(q), bits(k), bits(v)
    got = bf16_values(out)
    for b in (0, 3, 7):
        for h in (0, 13, 39):
            kv = h // (Hq // Hkv)
            want = A.ragged_gqa_attention(qb[b:b + 1, h:h + 1], kb[b:b + 1, kv:kv + 1], vb[b:b + 1, kv:kv + 1], [starts[b]])
            assert_close(got[b, h], want[0, 0], what=f"cfg2 b={b} h={h}")


def test_per_request_q_lens(gpu):
    rng = np.random.default_rng(8)
    B, Hq, Hkv, L, cap = 3, 8, 2, 4, 256
    q = randn_bf16(rng, (B, Hq, L, 128)); k = randn_bf16(rng, (B, Hkv, cap, 128)); v = randn_bf16(rng, (B, Hkv, cap, 128))
    starts, lens = [10, 100, 200], [1, 3, 4]
    got = bf16_values(_attn(q, k, v, starts, q_lens=lens))
    want = A.ragged_gqa_attention(bits(q), bits(k), bits(v), starts)
    for b in range(B):
        assert_close(got[b, :, : lens[b]], want[b, :, : lens[b]], what=f"b={b}")
        assert (got[b, :, lens[b]:] == 0).all()


def test_kv_scatter_restore_and_mask_bit_exact(gpu):
    rng = np.random.default_rng(4)
    B, H, cap, q, D = 3, 2, 64, 4, 128
    kc = torch.zeros((B, H, cap, D), dtype=torch.bfloat16, device="cuda"); vc = torch.zeros_like(kc)
    kn = randn_bf16(rng, (B, H, q, D)); vn = randn_bf16(rng, (B, H, q, D))
    ws = torch.tensor([0, 17, 60], dtype=torch.int32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    snap_k = kc.clone()
    _lib.call("mtp_kv_scatter", kc.data_ptr(), vc.data_ptr(), kn.data_ptr(), vn.data_ptr(), ws.data_ptr(),
              B, H, cap, q, D, status.data_ptr(), _st())
    torch.cuda.synchronize()
    assert status.item() == 0
    assert np.array_equal(bits(kc), KV.scatter(bits(snap_k), bits(kn), [0, 17, 60]))
    # out-of-range write is skipped and flagged
    bad = torch.tensor([0, 0, 62], dtype=torch.int32, device="cuda")
    before = bits(kc)
    _lib.call("mtp_kv_scatter", kc.data_ptr(), vc.data_ptr(), kn.data_ptr(), vn.data_ptr(), bad.data_ptr(),
              B, H, cap, q, D, status.data_ptr(), _st())
    torch.cuda.synchronize()
    assert status.item() == 1
    after = bits(kc)
    knb = bits(kn)
    assert np.array_equal(after[0], KV.scatter(before, knb, [0, 0, 0])[0])
    assert np.array_equal(after[2, :, :62], before[2, :, :62])
    assert np.array_equal(after[2, :, 62:64], knb[2, :, 0:2])      # in-range part written
    # masked restore, snapshot capacity smaller than the buffer (zero padded)
    snap = randn_bf16(rng, (B, H, 48, D))
    mask = torch.tensor([1, 0, 1], dtype=torch.uint8, device="cuda")
    cur = kc.clone()
    _lib.call("mtp_kv_restore_masked", cur.data_ptr(), snap.data_ptr(), mask.data_ptr(), B, H, cap, 48, D, 0, cap, _st())
    torch.cuda.synchronize()
    assert np.array_equal(bits(cur), KV.restore_masked(bits(kc), bits(snap), [True, False, True]))
    # mask materialisation
    qs = torch.tensor([0, 5, 9], dtype=torch.int32, device="cuda")
    m = torch.empty((B, 1, 4, 20), dtype=torch.uint8, device="cuda")
    _lib.call("mtp_ragged_causal_mask", m.data_ptr(), qs.data_ptr(), B, 4, 20, _st())
    torch.cuda.synchronize()
    assert np.array_equal(m.cpu().numpy().astype(bool), A.ragged_causal_mask([0, 5, 9], 4, 20))


from mtplx_amd.verify_step import kv_to_blocks


@pytest.mark.parametrize("B,Hq,Hkv,L,cap,starts,lens", [
    (1, 40, 8, 4, 4096, [4092], None),                     # cfg3 verify shape
    (3, 40, 8, 4, 736, [17, 300, 700], None),
    (2, 32, 4, 4, 1312, [1000, 5], [4, 2]),
    (2, 16, 2, 2, 128, [33, 90], None),
    (1, 8, 8, 1, 64, [40], None),
])
def test_blocked_v_attention_matches_oracle(gpu, B, Hq, Hkv, L, cap, starts, lens):
    """The verify step's attention over the operand-major K/V block cache:
    oracle within the bf16 bar, and within one bf16 ulp of the reference-layout
    kernel."""
    rng = np.random.default_rng(B * 1000 + cap + L)
    q = randn_bf16(rng, (B, Hq, L, 128)); k = randn_bf16(rng, (B, Hkv, cap, 128)); v = randn_bf16(rng, (B, Hkv, cap, 128))
    qs = torch.tensor(starts, dtype=torch.int32, device="cuda")
    ql = None if lens is None else torch.tensor(lens, dtype=torch.int32, device="cuda")
    # stale bits past every request's keys must not leak in: poison them in the blocked copy
    vt_std = v.clone()
    for b, s in enumerate(starts):
        end = s + (L if lens is None else lens[b])
        vt_std[b, :, end:] = float("nan")
    kb = kv_to_blocks(k, "k")
    vt = kv_to_blocks(vt_std, "v")
    out = torch.full((B, L, Hq, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    nb = _lib.query("mtp_attn_vt_workspace_bytes", B, Hkv, cap)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    _lib.call("mtp_ragged_gqa_attn_rows_vt", q.data_ptr(), kb.data_ptr(), vt.data_ptr(), qs.data_ptr(),
              None if ql is None else ql.data_ptr(), out.data_ptr(), B, Hq, Hkv, L, 128, cap,
              1.0 / math.sqrt(128), ws.data_ptr(), nb, _st())
    torch.cuda.synchronize()
    got = bf16_values(out.permute(0, 2, 1, 3).contiguous())
    qlen = [L] * B if lens is None else lens
    for b in range(B):
        want = A.ragged_gqa_attention(bits(q[b:b + 1]), bits(k[b:b + 1]), bits(v[b:b + 1]), [starts[b]])
        assert_close(got[b:b + 1, :, :qlen[b]], want[:, :, :qlen[b]], what=f"blocked-V attention b={b}")
    ref = bf16_values(_attn(q, k, v, starts, q_lens=lens).float().to(torch.bfloat16))
    for b in range(B):
        a, r = got[b, :, :qlen[b]], ref[b, :, :qlen[b]]
        tol = np.maximum(np.abs(a), np.abs(r)) * 2.0 ** -7 + 1e-3
        assert (np.abs(a - r) <= tol).all(), np.abs(a - r).max()


def test_blocked_v_rope_writer(gpu):
    """mtp_rope_qkv_to_cache_vt writes the same q, K and V values as the
    reference-layout writer, K and V in the operand-major block layout."""
    rng = np.random.default_rng(9)
    B, L, Hq, Hkv, D, cap = 2, 4, 8, 2, 128, 256
    qkv = randn_bf16(rng, (B * L, (Hq + 2 * Hkv) * D))
    qs = torch.tensor([30, 250], dtype=torch.int32, device="cuda")
    outs = []
    for fn in ("mtp_rope_qkv_to_cache", "mtp_rope_qkv_to_cache_vt"):
        qo = torch.zeros((B, Hq, L, D), dtype=torch.bfloat16, device="cuda")
        kc = torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device="cuda")
        vc = torch.zeros_like(kc)
        st = torch.zeros(1, dtype=torch.int32, device="cuda")
        _lib.call(fn, qkv.data_ptr(), qs.data_ptr(), None, qo.data_ptr(), kc.data_ptr(), vc.data_ptr(), B, L, Hq, Hkv,
                  D, cap, 1e6, st.data_ptr(), _st())
        torch.cuda.synchronize()
        outs.append((qo, kc, vc, int(st.item())))
    (q0, k0, v0, s0), (q1, k1, v1, s1) = outs
    assert torch.equal(q0.view(torch.int16), q1.view(torch.int16))
    assert torch.equal(kv_to_blocks(k0, "k").view(torch.int16), k1.view(torch.int16))
    assert torch.equal(kv_to_blocks(v0, "v").view(torch.int16), v1.view(torch.int16))
    assert s0 == 0 and s1 == 0
