"""GPU parity of the fused verify layer (mtp_verify_layer: one persistent
kernel per dense layer, grid barriers between its six phases).

Bars: logits within the north-star tolerance of the float64 oracle (the same
bar as the per-phase path in test_gpu_model.py); bit-exact against the
per-phase kernels where both use the same tiling (small shapes), within one
bf16 ulp per matmul where gate/up's K-split differs (27B shapes); graph
replays equal to the eager step; the barrier's error flag never set; unsafe
buffer chains refused on the host.
"""

import numpy as np
import pytest
import torch

from oracle.model import verify_forward
from tests.gpu_util import assert_close
from tests.model_util import model_params_numpy

pytestmark = pytest.mark.gpu


def _model(cfg, seed, cap=320):
    from mtplx_amd.verify_step import VerifyModel
    model = VerifyModel(cfg, device="cuda", seed=seed)
    model.allocate_cache(1, cap)
    return model


def _tokens(cfg, seed, L=4):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(0, cfg.vocab, (1, L), device="cuda", dtype=torch.int32, generator=gen)


def test_fused_layer_matches_oracle(gpu):
    from mtplx_amd.verify_step import DecoderConfig
    cfg = DecoderConfig(layers=2, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096)
    model = _model(cfg, 5)
    model.fused_layer = True
    kc = [model.k_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(cfg.layers)]
    vc = [model.v_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(cfg.layers)]
    tokens = _tokens(cfg, 6)
    qs = torch.tensor([57], dtype=torch.int32, device="cuda")
    logits = model.verify_logits(tokens, qs)
    torch.cuda.synchronize()
    assert not model.layer_sync_error()
    want = verify_forward(model_params_numpy(model), cfg, tokens.cpu().numpy(), np.array([57]), kc, vc, None)
    assert_close(logits.cpu().numpy().astype(np.float64), want, rtol=3e-2, atol=3e-2, what="fused dense logits")
    for li in range(cfg.layers):
        got_k = model.k_cache_standard(li).float().cpu().numpy()
        assert_close(got_k[0, :, 57:61], kc[li][0, :, 57:61], rtol=2e-2, atol=2e-2, what="k rows")


@pytest.mark.parametrize("L,start", [(4, 100), (3, 250), (1, 31)])
def test_fused_layer_bit_exact_vs_phase_kernels(gpu, L, start):
    """Same tiling as the per-phase kernels (every matmul below 256 tiles, 8
    waves): logits and the K/V rows written are bit-identical."""
    from mtplx_amd.verify_step import DecoderConfig
    cfg = DecoderConfig(layers=3, hidden=1024, ffn=2048, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048)
    model = _model(cfg, 7)
    tokens = _tokens(cfg, 8, L)
    qs = torch.tensor([start], dtype=torch.int32, device="cuda")
    model.fused_layer = False
    ref = model.verify_logits(tokens, qs).clone()
    kref = [k.clone() for k in model.k_cache]
    vref = [v.clone() for v in model.v_cache]
    model.fused_layer = True
    got = model.verify_logits(tokens, qs)
    torch.cuda.synchronize()
    assert not model.layer_sync_error()
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
    for li in range(cfg.layers):
        assert torch.equal(model.k_cache[li].view(torch.int16), kref[li].view(torch.int16))
        assert torch.equal(model.v_cache[li].view(torch.int16), vref[li].view(torch.int16))


def test_fused_layer_27b_shapes_vs_phase_kernels(gpu):
    """The 27B layer shapes (gate/up 544 tiles: 512 whole + 32 split 8 ways by
    K), two layers: the fused kernel's gate/up runs 8 waves per tile where the
    standalone kernel runs 4, so sums reassociate; logits stay within the
    north-star rtol/atol 1e-2 of the per-phase path."""
    from mtplx_amd.verify_step import DecoderConfig
    cfg = DecoderConfig(layers=2, hidden=5120, ffn=17408, n_heads=40, n_kv_heads=8, head_dim=128, vocab=4096)
    model = _model(cfg, 9, cap=4352)
    tokens = _tokens(cfg, 10)
    qs = torch.tensor([4092], dtype=torch.int32, device="cuda")
    model.fused_layer = False
    ref = model.verify_logits(tokens, qs).clone()
    model.fused_layer = True
    got = model.verify_logits(tokens, qs)
    torch.cuda.synchronize()
    assert not model.layer_sync_error()
    a, b = got.cpu().numpy().astype(np.float64), ref.cpu().numpy().astype(np.float64)
    assert_close(a, b, rtol=1e-2, atol=1e-2, what="fused vs per-phase logits (27B shapes)")


def test_fused_layer_graph_replays(gpu):
    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import CapturedVerifyStep, DecoderConfig
    cfg = DecoderConfig(layers=2, hidden=1024, ffn=2048, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048)
    model = _model(cfg, 11)
    model.fused_layer = True
    tokens = _tokens(cfg, 12)
    qs = torch.tensor([90], dtype=torch.int32, device="cuda")
    eager = model.verify_logits(tokens, qs).clone()
    gen = torch.Generator(device="cuda").manual_seed(13)
    draft = torch.randn((1, 3, cfg.vocab), device="cuda", generator=gen)
    u = torch.rand((1, 4), device="cuda", dtype=torch.float64, generator=gen)
    step = CapturedVerifyStep(model, tokens, qs, draft, u, SamplerConfig())
    for _ in range(3):
        step.replay()
        torch.cuda.synchronize()
        assert torch.equal(step.logits.view(torch.int32), eager.view(torch.int32))
        eager2 = model.verify_logits(tokens, qs)   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager2.view(torch.int32), eager.view(torch.int32))
    assert not model.layer_sync_error()


def test_fused_layer_refuses_unsafe_buffers(gpu):
    """o_proj writing into its own residual input (the per-phase path's
    in-place h) is refused: another XCD's L2 may still hold h's old lines."""
    from mtplx_amd import _lib
    from mtplx_amd.verify_step import DecoderConfig
    cfg = DecoderConfig(layers=1, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1024)
    model = _model(cfg, 14)
    L = model.layers[0]
    M, H = 4, cfg.hidden
    dev = "cuda"
    h = torch.randn((M, H), device=dev).to(torch.bfloat16)
    attn = torch.empty((M, cfg.n_heads * 128), dtype=torch.bfloat16, device=dev)
    act = torch.empty((M, cfg.ffn), dtype=torch.bfloat16, device=dev)
    sums = torch.empty(cfg.ffn, dtype=torch.float32, device=dev)
    ss_a = torch.empty(H, dtype=torch.float32, device=dev)
    ss_b = torch.empty(H, dtype=torch.float32, device=dev)
    qh = torch.empty((1, cfg.n_heads, 4, 128), dtype=torch.bfloat16, device=dev)
    qs = torch.tensor([10], dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(_lib.query("mtp_qmv_workspace_bytes", M, cfg.ffn, H, 1), dtype=torch.uint8, device=dev)
    aws = torch.zeros(_lib.query("mtp_attn_vt_workspace_bytes", 1, cfg.n_kv_heads, model.cap), dtype=torch.uint8,
                      device=dev)
    sync = torch.zeros(_lib.query("mtp_verify_layer_sync_bytes"), dtype=torch.uint8, device=dev)
    rope = dict(q_start=qs, q_out=qh, k_cache=model.k_cache[0], v_cache=model.v_cache[0], status=status, L=4,
                Hq=cfg.n_heads, Hkv=cfg.n_kv_heads, D=128, cap=model.cap, blocked=1, rope_base=1e6)
    st = torch.cuda.current_stream().cuda_stream
    with pytest.raises(_lib.MtpError) as e:
        _lib.verify_layer(
            st, rope=rope,
            qkv=dict(x=h, x2=L.in_norm, eps=1e-6, w0=L.qkv_rope2, M=M, N=cfg.qkv_out, K=H, group_size=64, xmode=2,
                     emode=4, packed=2),
            o=dict(x=attn, w0=L.o.packed_mf16, resid=h, y0=h, ss_out=ss_a, M=M, N=H, K=1024, group_size=64,
                   xmode=0, emode=1, packed=2),
            gate_up=dict(x=h, x2=L.post_norm, ss_in=ss_a, eps=1e-6, w0=L.gate.packed_mf16, w1=L.up.packed_mf16,
                         y0=act, y_sums=sums, M=M, N=cfg.ffn, K=H, group_size=64, xmode=2, emode=3, packed=2, ws=ws,
                         ws_bytes=ws.numel()),
            down=dict(x=act, x_sums=sums, w0=L.down.packed_mf16, resid=h, y0=h, ss_out=ss_b, M=M, N=H, K=cfg.ffn,
                      group_size=64, xmode=3, emode=1, packed=2),
            attn_out=attn, attn_scale=0.088, attn_ws=aws, sync=sync)
    assert e.value.code == -1
