"""Benchmark of the MI355X speculative-verify hot path (one GPU).

Default workload (BASELINE cfg3): one depth-3 verify step (B=1, 4 rows) of the
27B-shaped 4-bit dense decoder at 4096-token context, random init, synthetic
inputs resident in HBM: embedding -> 64 layers (fused norm+q|k|v, RoPE+KV write,
ragged GQA attention, o_proj+residual, fused norm+gate/up+SwiGLU,
down_proj+residual) -> norm+lm_head (fp32 logits) -> exact accept/reject.

Prints one JSON line. ``value`` = verify rows/s = B*(K+1)/t_step. The
``roofline`` object times the step's dominant kernel (the fused norm+gate/up
quantized matmul, one launch per layer's weights, so no launch re-reads
cached weights) with HIP events on the stream it runs on; ``cpu_baseline``
times an fp32 NumPy/BLAS port of the same step (weights dequantised ahead of
time) on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import time

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
ROOT = os.path.dirname(os.path.abspath(__file__))


def _gate_up_bytes(M: int, N: int, K: int, gs: int) -> int:
    w = N * K // 2
    sb = 2 * N * (K // gs) * 2
    return 2 * (w + sb) + M * K * 2 + K * 2 + M * N * 2


def _qmv_bytes(M: int, N: int, K: int, gs: int) -> int:
    return N * K // 2 + 2 * N * (K // gs) * 2 + M * K * 2 + M * N * 2


def roofline_gate_up(model, M: int, reps: int = 5) -> dict:
    """Average duration of the fused norm+gate/up launch over every layer's
    weights: the verify step's own call (packed weights, norm statistics from
    the residual epilogue, the shared workspace), one launch per layer captured
    in a HIP graph and replayed, timed with events on the capture stream."""
    import torch

    c = model.cfg
    dev = model.device
    x = torch.randn((M, c.hidden), device=dev).to(torch.bfloat16)
    xf = x.float()
    ss = torch.zeros(((c.hidden + 31) // 32) * 32, dtype=torch.float32, device=dev)
    ss.view(-1, 32)[:, :M] = (xf * xf).view(M, -1, 32).sum(dim=2).t()
    y = torch.empty((M, c.ffn), dtype=torch.bfloat16, device=dev)
    ysum = torch.empty(((c.ffn + 31) // 32) * 32, dtype=torch.float32, device=dev)
    launch = _gate_up_launcher(model, M, x, ss, y, ysum)

    for L in model.layers:
        launch(L)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for L in model.layers:
            launch(L)
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    n = reps * len(model.layers)
    us = e0.elapsed_time(e1) * 1000.0 / n
    byts = _gate_up_bytes(M, c.ffn, c.hidden, c.group_size)
    gbs = byts / us / 1e3
    return {"bound": "hbm",
            "kernel": "qmv_stream_kernel<NW=4,R=4,X_RMSNORM,E_DUAL_SWIGLU,packed,MF> (mtp_qmv_affine4_ex, packed layout 2, "
                      "tail split)",
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(), "algorithmic_bytes_per_launch": byts, "avg_launch_us": round(us, 3),
            "launches_timed": n}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gate_up_cfg3_traffic.md")


def measured_traffic() -> int | None:
    """HBM bytes per launch of the roofline kernel, from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (each scaled by the copy-kernel
    calibration stated there), or None when absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"\s*traffic_bytes_per_launch:\s*(\d+)", line)
                if m:
                    return int(m.group(1))
    except OSError:
        pass
    return None


def profile_roofline(model, M: int) -> None:
    """The counter workload: the roofline kernel over every layer twice, eager
    (one dispatch each), then a 256 MiB device copy whose FETCH_SIZE /
    WRITE_SIZE readings calibrate the counters (256 MiB read + written)."""
    import torch

    c = model.cfg
    dev = model.device
    x = torch.randn((M, c.hidden), device=dev).to(torch.bfloat16)
    xf = x.float()
    ss = torch.zeros(((c.hidden + 31) // 32) * 32, dtype=torch.float32, device=dev)
    ss.view(-1, 32)[:, :M] = (xf * xf).view(M, -1, 32).sum(dim=2).t()
    y = torch.empty((M, c.ffn), dtype=torch.bfloat16, device=dev)
    ysum = torch.empty(((c.ffn + 31) // 32) * 32, dtype=torch.float32, device=dev)
    launch = _gate_up_launcher(model, M, x, ss, y, ysum)
    for _ in range(2):
        for L in model.layers:
            launch(L)
    _calibration_copy(dev)
    print("roofline counter workload done", flush=True)


def _calibration_copy(dev) -> None:
    """A 256 MiB device-to-device copy, twice: reads and writes exactly
    268,435,456 B, so its FETCH_SIZE / WRITE_SIZE readings scale the counters."""
    import torch

    src = torch.ones(64 << 20, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()


def profile_step(model, tokens, q_start, draft_logits, uniforms, sampler) -> None:
    """The counter workload for every kernel of the step: one eager verify
    step (one dispatch per kernel and layer, each layer on its own weights),
    then the calibration copy."""
    import torch

    model.verify_step(tokens, q_start, draft_logits, uniforms, sampler)
    torch.cuda.synchronize()
    _calibration_copy(model.device)
    print("step counter workload done", flush=True)


def _gate_up_launcher(model, M, x, ss, y, ysum):
    """The verify step's own gate/up call (packed weights, norm statistics
    handed over, SwiGLU output sums for down_proj, the shared workspace)."""
    from mtplx_amd import _lib

    c = model.cfg
    dev = model.device
    nb = _lib.query("mtp_qmv_workspace_bytes", M, c.ffn, c.hidden, 1)
    ws = _lib.WORKSPACES.get(nb, "qmv", dev)

    def launch(L):
        lay = 2 if M <= 4 else 1   # as the verify step chooses
        _lib.qmv_ex(_lib.stream_handle(dev), x=x, x2=L.post_norm, ss_in=ss, eps=c.rms_eps,
                    w0=L.gate.packed_mf16 if lay == 2 else L.gate.packed,
                    w1=L.up.packed_mf16 if lay == 2 else L.up.packed, y0=y, y_sums=ysum, M=M, N=c.ffn, K=c.hidden,
                    group_size=c.group_size, xmode=2, emode=3, packed=lay, ws=ws, ws_bytes=ws.numel())
    return launch


def roofline_qmv_cfg1(reps: int = 64, nsets: int = 8) -> dict:
    """BASELINE cfg1 qmv (x [4,5120] . W [17408,5120] 4-bit g64) on the verify
    step's own path: packed layout 2 (the 16x16x32 MFMA form for 4 rows), the
    tail split over all CUs with the step's shared workspace, launches
    replayed from a HIP graph; 8 rotating weight sets (400 MB > the 256 MB
    MALL) so every launch streams from HBM. Timed with HIP events on the
    replay stream."""
    import torch

    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear

    M, N, K, gs = 4, 17408, 5120, 64
    gen = torch.Generator(device="cuda").manual_seed(1)
    sets = [QuantizedLinear.random(N, K, gs, generator=gen) for _ in range(nsets)]
    for q in sets:
        q.pack(layout=2)
        q.release_source()
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ws = _lib.WORKSPACES.get(_lib.query("mtp_qmv_workspace_bytes", M, N, K, 1), "bench_cfg1")
    stream = torch.cuda.Stream()

    def launch(q):
        _lib.qmv_ex(_lib.stream_handle(), x=x, w0=q.packed_mf16, y0=y, M=M, N=N, K=K, group_size=gs, xmode=0,
                    emode=0, packed=2, ws=ws, ws_bytes=ws.numel())

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for q in sets:
            launch(q)
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for q in sets:
                launch(q)
    us = _replay_us(graph, stream, max(1, reps // nsets)) / nsets
    byts = _qmv_bytes(M, N, K, gs)
    gbs = byts / us / 1e3
    return {"kernel": "qmv_stream_kernel<NW=4,R=4,X_PLAIN,E_STORE,packed,MF> (mtp_qmv_affine4_ex, packed layout 2, "
                      "tail split, graph replay)",
            "achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "avg_launch_us": round(us, 3),
            "algorithmic_bytes_per_launch": byts, "target_us_at_70pct": round(byts / (0.7 * HBM_PEAK_GBS) / 1e3, 2)}


def accept_leg_cfg1(reps: int = 64, nsets: int = 64) -> dict:
    """BASELINE cfg1's accept leg: rejection sampling with residual
    correction for 3 drafts over fp32 logits, target [4, 151936] and draft
    [3, 151936] ~N(0, 3), temperature 0.6, top-k 20, top-p 0.95, seeded
    uniforms (``mtp_spec_accept``: ``vocab_partials`` over the 7 rows, then
    ``accept_laws``). 64 rotating logit sets (272 MB > the 256 MB MALL),
    launches replayed from a HIP graph, HIP events on the replay stream.
    Algorithmic bytes: the 7 logit rows read once (4,254,208 B)."""
    import torch

    from mtplx_amd.sampling import SamplerConfig, spec_accept

    B, K, V = 1, 3, 151936
    gen = torch.Generator(device="cuda").manual_seed(3)
    tl = [(torch.randn((B, K + 1, V), device="cuda", generator=gen) * 3.0) for _ in range(nsets)]
    dl = [(t[:, :K] + 0.5 * torch.randn((B, K, V), device="cuda", generator=gen)).contiguous() for t in tl]
    ids = torch.randint(0, V, (B, K), device="cuda", dtype=torch.int32, generator=gen)
    u = torch.rand((B, K + 1), device="cuda", dtype=torch.float64, generator=gen)
    cfg = SamplerConfig(0.6, 0.95, 20)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for i in range(nsets):
            res = spec_accept(tl[i], dl[i], ids, u, cfg)
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(nsets):
                res = spec_accept(tl[i], dl[i], ids, u, cfg)
    us = _replay_us(graph, stream, max(1, reps // nsets)) / nsets
    assert int(res.status.max().item()) == 0
    byts = (2 * K + 1) * B * V * 4
    return {"kernels": "vocab_partials + accept_laws (mtp_spec_accept)", "rows": "target [4,151936] + draft [3,151936]",
            "avg_step_us": round(us, 3), "algorithmic_bytes": byts, "achieved_gbs": round(byts / us / 1e3, 1),
            "frac_hbm": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}


def qmm_rows(M: int, reps: int = 64, nsets: int = 8) -> dict:
    """The M >= 16 path (cfg4's ragged batches reach 64 rows):
    mtp_qmm_affine4_mfma, x [M,5120] . W [17408,5120] 4-bit g64 (packed
    layout 1), each weight quad read once for all M rows on the 32x32x16
    MFMA, x streamed through LDS; 8 rotating weight sets (400 MB > the
    256 MB MALL). Launches replayed from a HIP graph (host set-up untimed).
    Reported against the dense bf16 MFMA peak (2.5 PFLOP/s) and HBM."""
    import torch

    from mtplx_amd import _lib
    from mtplx_amd.quant import QuantizedLinear

    N, K, gs = 17408, 5120, 64
    gen = torch.Generator(device="cuda").manual_seed(2)
    sets = [QuantizedLinear.random(N, K, gs, generator=gen) for _ in range(nsets)]
    for q in sets:
        q.pack()
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ws = _lib.WORKSPACES.get(max(256, _lib.query("mtp_qmm_workspace_bytes", M, N, K, 0)), "bench_qmm")
    gs_stream = torch.cuda.Stream()

    def launch(q):
        _lib.qmm_mfma(_lib.stream_handle(), x=x, w0=q.packed, y=y, M=M, N=N, K=K, group_size=gs, emode=0, ws=ws,
                      ws_bytes=ws.numel())

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(gs_stream):
        for q in sets:
            launch(q)
        gs_stream.synchronize()
        with torch.cuda.graph(graph, stream=gs_stream):
            for q in sets:
                launch(q)
    us = _replay_us(graph, gs_stream, max(1, reps // nsets)) / nsets
    flops = 2.0 * M * N * K
    tfs = flops / us / 1e6
    byts = _qmv_bytes(M, N, K, gs)
    return {"kernel": f"qmm_rows_kernel<R2={1 if M <= 32 else 2},store> (mtp_qmm_affine4_mfma)",
            "rows": M, "avg_launch_us": round(us, 3), "achieved_tflops": round(tfs, 1),
            "frac_mfma_bf16": round(tfs / MFMA_BF16_PEAK_TFLOPS, 4), "achieved_gbs": round(byts / us / 1e3, 1),
            "frac_hbm": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}


def _replay_us(graph, stream, rounds: int) -> float:
    """Average microseconds per replay of ``graph`` on ``stream`` (HIP events
    recorded on that stream, one untimed replay first)."""
    import torch

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        graph.replay()
        stream.synchronize()
        e0.record(stream)
        for _ in range(rounds):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / rounds


def _matrix_bytes(*qs) -> int:
    """MLX-layout bytes of the layers (the packed copies hold the same bytes;
    a layer whose source was released is counted from its shape)."""
    total = 0
    for q in qs:
        if q is None:
            continue
        lead = 1
        for d in q._shape[:-2]:
            lead *= d
        n, k = q.out_features, q.in_features
        total += lead * (n * k * q.bits // 8 + 2 * n * (k // q.group_size) * 2)
    return total


def _randn_bf16(n: int, gen, dev):
    """n N(0,1) bf16 values, generated in slices (bounded fp32 temporaries)."""
    import torch

    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    step = 1 << 26
    for i in range(0, n, step):
        m = min(step, n - i)
        out[i:i + m] = torch.randn(m, generator=gen, device=dev).to(torch.bfloat16)
    return out


def cfg4_ragged(model, steps: int = 5, warmup: int = 2, seed: int = 11, eager: bool = False) -> dict:
    """BASELINE cfg4 on the same 27B-shaped weights: 16 requests, depths
    U{1,2,3}, contexts log-uniform in [1k, 64k] (seeded), packed into one
    ragged batch of M = sum(K_b + 1) rows; per-request capacities in one
    block cache (each request's verify rows are its context's last rows).
    One step = embedding -> 64 layers (RMSNorm, q|k|v on the rows kernel,
    ragged RoPE + K/V write, block attention, o + residual, RMSNorm, gate/up
    + SwiGLU, down + residual) -> norm + lm_head -> accept/reject with
    per-request depths, replayed from one HIP graph (``eager``: launched
    kernel by kernel). Algorithmic bytes per step: every
    layer matrix and the lm_head once, each request's K/V (ctx_b keys x
    Hkv x 128 x 2 x 2 B per layer) once, plus the M new K/V rows written."""
    import numpy as np
    import torch

    from mtplx_amd.sampling import SamplerConfig

    c = model.cfg
    dev = model.device
    rng = np.random.default_rng(seed)
    B = 16
    depths = rng.integers(1, 4, size=B)
    ctx = np.exp(rng.uniform(np.log(1024), np.log(65536), size=B)).astype(np.int64)
    lens = depths + 1
    q_start = (ctx - lens).astype(np.int32)
    row_off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d_off = np.concatenate([[0], np.cumsum(depths)]).astype(np.int32)
    draft_index = np.concatenate([np.arange(row_off[b] + 1, row_off[b + 1]) for b in range(B)]).astype(np.int64)
    M, Lmax = int(row_off[-1]), int(lens.max())
    model.allocate_cache_blocks(ctx)
    gen = torch.Generator(device=dev).manual_seed(seed)

    def t(a, dtype=torch.int32):
        return torch.from_numpy(np.ascontiguousarray(a)).to(device=dev, dtype=dtype)

    tokens = torch.randint(0, c.vocab, (M,), device=dev, dtype=torch.int32, generator=gen)
    draft_logits = 3.0 * torch.randn((int(d_off[-1]), c.vocab), device=dev, generator=gen)
    uniforms = torch.rand((B, 4), device=dev, dtype=torch.float64, generator=gen)
    args = (tokens, t(row_off), t(q_start), t(lens), Lmax, draft_logits, t(d_off), t(draft_index, torch.int64),
            uniforms, SamplerConfig(0.6, 0.95, 20))
    from mtplx_amd.verify_step import CapturedRaggedVerifyStep
    if eager:
        stream = torch.cuda.current_stream()

        def step():
            return model.verify_step_ragged(*args)
    else:
        cap = CapturedRaggedVerifyStep(model, *args)
        stream = cap.stream
        step = cap.replay
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            res = step()
        torch.cuda.synchronize()
        model.check_status()
        e0.record(stream)
        for _ in range(steps):
            res = step()
        e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    assert int(res.status.max().item()) == 0
    kv_row = c.n_kv_heads * c.head_dim * 2 * 2
    w_bytes = sum(_matrix_bytes(L.qkv, L.o, L.gate, L.up, L.down) for L in model.layers) + \
        _matrix_bytes(model.lm_head)
    kv_bytes = c.layers * (int(ctx.sum()) + M) * kv_row
    mm_flops = 2.0 * M * sum(c.qkv_out * c.hidden + c.hidden * c.n_heads * c.head_dim + 3 * c.ffn * c.hidden
                             for _ in range(c.layers)) + 2.0 * M * c.vocab * c.hidden
    keys = sum(int(q_start[b]) * int(lens[b]) + int(lens[b]) * (int(lens[b]) + 1) // 2 for b in range(B))
    at_flops = c.layers * 4.0 * c.n_heads * c.head_dim * keys
    s = ms / 1e3
    total = w_bytes + kv_bytes
    return {"workload": "cfg4: 16 requests, depths U{1,2,3}, contexts log-uniform [1k, 64k] (seed %d), one ragged "
                        "batch, 27B-shaped 4-bit dense decoder, " % seed +
                        ("eager launches" if eager else "launches replayed from one HIP graph"),
            "rows": M, "depths": depths.tolist(), "contexts": ctx.tolist(), "ms_per_step": round(ms, 4),
            "verify_rows_per_s": round(M / s, 2), "weight_bytes": w_bytes, "kv_bytes": kv_bytes,
            "achieved_gbs": round(total / s / 1e9, 1), "frac_hbm": round(total / s / 1e9 / HBM_PEAK_GBS, 4),
            "achieved_tflops": round((mm_flops + at_flops) / s / 1e12, 2),
            "frac_mfma_bf16": round((mm_flops + at_flops) / s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 5)}


def cfg2_attention(nsets: int = 8, reps: int = 4, seed: int = 21) -> dict:
    """BASELINE cfg2: 8 requests, KV lengths U[512, 32768] (seeded), 4 verify
    rows each (the context's last 4 keys), 40/8 heads, head_dim 128, bf16.
    Two kernels: the verify step's block attention (per-request capacities,
    operand-major 32-key blocks) and the facade's split kernel over the
    reference's contiguous [B, Hkv, cap, 128] cache. 8 rotating K/V sets
    (> the 256 MB MALL) so every launch streams from HBM; achieved GB/s =
    sum_b L_b x 4096 B (K and V of 8 heads x 128 x bf16) per launch."""
    import numpy as np
    import torch

    from mtplx_amd import _lib

    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(seed)
    B, Hq, Hkv, D, L = 8, 40, 8, 128, 4
    kv_len = rng.integers(512, 32769, size=B)
    caps = ((kv_len + 31) // 32) * 32
    q_start = (kv_len - L).astype(np.int32)
    lens = np.full(B, L, np.int32)
    row_off = (np.arange(B + 1) * L).astype(np.int32)
    kv_off = np.concatenate([[0], np.cumsum(Hkv * (caps // 32))]).astype(np.int32)
    gen = torch.Generator(device=dev).manual_seed(seed)

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)

    d_qs, d_lens, d_row, d_kv = t(q_start), t(lens), t(row_off), t(kv_off)
    q = torch.randn((B, Hq, L, D), device=dev, generator=gen).to(torch.bfloat16)
    algo = int(kv_len.sum()) * Hkv * D * 2 * 2
    scale = 1.0 / np.sqrt(D)
    out = {"workload": f"cfg2: 8 requests, KV lengths {kv_len.tolist()} (seed {seed}), 4 rows each, 40/8 heads",
           "kv_bytes_per_launch": algo}

    def timed(launch, n):
        launch(0)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            launch(i % nsets)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / n

    # the verify step's block attention
    nblk = int(kv_off[-1])
    kb = [_randn_bf16(nblk * 4096, gen, dev) for _ in range(nsets)]
    vb = [_randn_bf16(nblk * 4096, gen, dev) for _ in range(nsets)]
    o = torch.empty((B * L, Hq * D), dtype=torch.bfloat16, device=dev)
    nb = _lib.query("mtp_attn_blocks_workspace_bytes", B, Hkv, int(caps.max()), int(caps.sum()), 0)
    ws = _lib.WORKSPACES.get(nb, "bench_attn_blocks", dev)
    st = _lib.stream_handle(dev)

    def blocks(i):
        _lib.attn_blocks(st, q=q, k_blk=kb[i], v_blk=vb[i], q_start=d_qs, q_lens=d_lens, row_off=d_row, kv_off=d_kv,
                         out=o, B=B, Hq=Hq, Hkv=Hkv, Lmax=L, D=D, cap=int(caps.max()), split_keys=0, scale=scale,
                         total_cap=int(caps.sum()), ws=ws, ws_bytes=ws.numel())

    us = timed(blocks, reps * nsets)
    out["blocks"] = {"kernel": "attn_bal_kernel + attn_merge_head_kernel (mtp_ragged_gqa_attn_blocks)",
                     "avg_launch_us": round(us, 3), "achieved_gbs": round(algo / us / 1e3, 1),
                     "frac_hbm": round(algo / us / 1e3 / HBM_PEAK_GBS, 4)}
    del kb, vb
    # the facade kernel over the reference's contiguous layout
    cap = int(caps.max())
    kc = [_randn_bf16(B * Hkv * cap * D, gen, dev).view(B, Hkv, cap, D) for _ in range(nsets)]
    vc = [_randn_bf16(B * Hkv * cap * D, gen, dev).view(B, Hkv, cap, D) for _ in range(nsets)]
    o2 = torch.empty((B, Hq, L, D), dtype=torch.bfloat16, device=dev)
    nb = _lib.query("mtp_attn_workspace_bytes", B, Hkv, cap, 0)
    ws2 = _lib.WORKSPACES.get(nb, "bench_attn", dev)

    def split(i):
        _lib.call("mtp_ragged_gqa_attn", q.data_ptr(), kc[i].data_ptr(), vc[i].data_ptr(), d_qs.data_ptr(),
                  d_lens.data_ptr(), o2.data_ptr(), B, Hq, Hkv, L, D, cap, scale, 0, ws2.data_ptr(), ws2.numel(), st)

    us = timed(split, reps * nsets)
    out["contiguous"] = {"kernel": "attn_split_kernel + attn_merge_head_kernel (mtp_ragged_gqa_attn, ragged_sdpa)",
                         "avg_launch_us": round(us, 3), "achieved_gbs": round(algo / us / 1e3, 1),
                         "frac_hbm": round(algo / us / 1e3 / HBM_PEAK_GBS, 4)}
    del kc, vc
    torch.cuda.empty_cache()
    return out


def cfg5_moe(steps: int = 5, warmup: int = 2, seed: int = 5, eager: bool = False) -> dict:
    """BASELINE cfg5: the 125B-class MoE decoder (48 layers, hidden 4096,
    256 experts top-8 + 1 gated shared expert, expert FFN 1536, 32/4 heads,
    vocab 151936), random init, router skew Zipf(1.1), 4 requests x depth 3
    (16 rows) at 8k context, experts sorted before the gathered matmuls.
    Algorithmic bytes per step from the seeded routing: the distinct
    (layer, expert) pairs the step routes to x one expert's gate/up + down
    bytes, plus every dense matrix (q|k|v, o, router, shared expert) and the
    lm_head once, plus the K/V read (8k keys x 4 heads x 128 x 2 x 2 B per
    request and layer)."""
    import torch

    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import MOE_125B, VerifyModel

    dev = torch.device("cuda", 0)
    c = MOE_125B
    B, K, ctx = 4, 3, 8192
    L = K + 1
    model = VerifyModel(c, device=dev, seed=seed)
    model.allocate_cache(B, ctx)
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    tokens = torch.randint(0, c.vocab, (B, L), device=dev, dtype=torch.int32, generator=gen)
    q_start = torch.full((B,), ctx - L, dtype=torch.int32, device=dev)
    draft_logits = (torch.randn((B, K, c.vocab), device=dev, generator=gen) * 3.0).contiguous()
    uniforms = torch.rand((B, L), device=dev, dtype=torch.float64, generator=gen)
    sampler = SamplerConfig(0.6, 0.95, 20)
    model.route_log = []
    res = model.verify_step(tokens, q_start, draft_logits, uniforms, sampler)
    torch.cuda.synchronize()
    model.check_status()
    distinct = [int(torch.unique(ids).numel()) for ids in model.route_log]
    counts = [torch.bincount(ids.reshape(-1).long(), minlength=c.n_experts) for ids in model.route_log]
    few = sum(int(((n > 0) & (n <= 4)).sum()) for n in counts) / len(counts)
    many = sum(int((n > 4).sum()) for n in counts) / len(counts)
    rows_many = sum(int(n[n > 4].sum()) for n in counts) / len(counts)
    model.route_log = None
    # The step (router, sort, both expert row classes, shared expert, combine)
    # replayed from one HIP graph, as the cfg3 line; eager launches of its
    # ~770 short kernels would add ~0.9 ms of host gaps per step.
    from mtplx_amd.verify_step import CapturedVerifyStep
    if eager:
        cap = None
        stream = torch.cuda.current_stream()

        def step():
            return model.verify_step(tokens, q_start, draft_logits, uniforms, sampler)
    else:
        cap = CapturedVerifyStep(model, tokens, q_start, draft_logits, uniforms, sampler)
        stream = cap.stream
        step = cap.replay
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            res = step()
        e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    assert int(res.status.max().item()) == 0
    model.check_status()
    L0 = model.layers[0]
    expert_bytes = (_matrix_bytes(L0.expert_gate_up) + _matrix_bytes(L0.expert_down)) // c.n_experts
    dense = sum(_matrix_bytes(x.qkv, x.o, x.router, x.shared_gate, x.shared_up, x.shared_down)
                for x in model.layers) + _matrix_bytes(model.lm_head)
    kv = c.layers * B * ctx * c.n_kv_heads * c.head_dim * 2 * 2
    total = sum(distinct) * expert_bytes + dense + kv
    s = ms / 1e3
    del cap, model
    torch.cuda.empty_cache()
    return {"workload": "cfg5: 125B-class MoE decoder, 4 requests x depth 3 (16 rows), 8k context, Zipf(1.1) "
                        "router skew, " + ("eager launches" if eager else "launches replayed from one HIP graph"),
            "rows": B * L, "ms_per_step": round(ms, 4), "verify_rows_per_s": round(B * L / s, 2),
            "distinct_experts_per_layer_mean": round(sum(distinct) / len(distinct), 2),
            "experts_with_1_to_4_rows_mean": round(few, 2), "experts_with_5_plus_rows_mean": round(many, 2),
            "rows_in_5_plus_experts_mean": round(rows_many, 2),
            "expert_bytes": expert_bytes, "bytes_per_step": total, "achieved_gbs": round(total / s / 1e9, 1),
            "frac_hbm": round(total / s / 1e9 / HBM_PEAK_GBS, 4)}


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the GPU box's CPU share (16 for one
    GPU), or fewer if the machine has fewer."""
    return max(1, min(16, os.cpu_count() or 1))


def cpu_baseline(layers: int, timeout_s: int = 300) -> dict | None:
    """The CPU port on a bounded sample in a child process, its BLAS on
    cpu_threads() threads."""
    t = str(cpu_threads())
    env = dict(os.environ, OMP_NUM_THREADS=t, OPENBLAS_NUM_THREADS=t, MKL_NUM_THREADS=t)
    cmd = [sys.executable, "-c", f"import sys; sys.path.insert(0, {ROOT!r}); import bench; bench._cpu_child({layers})"]
    try:
        out = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        return None
    for line in out.stdout.splitlines()[::-1]:
        if line.startswith("{"):
            return json.loads(line)
    sys.stderr.write(out.stderr[-2000:])
    return None


def _cpu_child(layers: int) -> None:
    """A CPU port of the depth-3 verify step of the 27B shape in fp32 with
    the weights dequantised ahead of time (untimed; a CPU serving the model
    would hold them so): per layer RMSNorm, q|k|v, RoPE, GQA attention over
    the 4096-token cache, o, RMSNorm, gate/up + SwiGLU, down, every matmul a
    multithreaded fp32 BLAS product; then 1/4 of the lm_head and the
    sampler's accept step (the fp64 oracle). Three passes of one layer (every
    layer has the same shapes) are timed and extrapolated to the step."""
    import numpy as np

    from oracle import sampler as S
    from oracle.qmv import dequantize_affine4, make_affine4_weights

    SAMPLE_LAYERS, LM_PART = 3, 4
    rng = np.random.default_rng(0)
    M, H, F, Hq, Hkv, D, V, ctx = 4, 5120, 17408, 40, 8, 128, 151936, 4096
    rep = Hq // Hkv

    def deq(n, k):
        return dequantize_affine4(*make_affine4_weights(rng, n, k), 64).astype(np.float32)

    W = {n: deq(o, i) for n, o, i in
         [("qkv", (Hq + 2 * Hkv) * D, H), ("o", H, Hq * D), ("g", F, H), ("u", F, H), ("d", H, F)]}
    lm = deq(V // LM_PART, H)
    kc = rng.standard_normal((Hkv, ctx, D)).astype(np.float32)
    vc = rng.standard_normal((Hkv, ctx, D)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    h = rng.standard_normal((M, H)).astype(np.float32)
    pos = np.arange(ctx - M, ctx, dtype=np.float32)
    inv = (1.0e6 ** (-(np.arange(D // 2, dtype=np.float32) * 2.0) / D)).astype(np.float32)
    cos, sin = np.cos(pos[:, None] * inv), np.sin(pos[:, None] * inv)
    mask = np.where(np.arange(ctx)[None, :] <= (ctx - M + np.arange(M))[:, None], 0.0, -np.inf).astype(np.float32)

    def norm(x):
        return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-6) * nw

    def rope(x):   # [M, heads, D]
        x1, x2 = x[..., : D // 2], x[..., D // 2:]
        c, s_ = cos[:, None, :], sin[:, None, :]
        return np.concatenate([x1 * c - x2 * s_, x1 * s_ + x2 * c], axis=-1)

    t0 = time.perf_counter()
    for _ in range(SAMPLE_LAYERS):
        qkv = (norm(h) @ W["qkv"].T).reshape(M, Hq + 2 * Hkv, D)
        q, k, v = rope(qkv[:, :Hq]), rope(qkv[:, Hq:Hq + Hkv]), qkv[:, Hq + Hkv:]
        kc[:, ctx - M:] = k.transpose(1, 0, 2)
        vc[:, ctx - M:] = v.transpose(1, 0, 2)
        att = np.empty((M, Hq, D), np.float32)
        for g in range(Hkv):
            qg = q[:, g * rep:(g + 1) * rep].transpose(1, 0, 2).reshape(rep * M, D)
            sc = (qg @ kc[g].T) / np.float32(np.sqrt(D)) + np.tile(mask, (rep, 1))
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            o = (p @ vc[g]) / p.sum(axis=1, keepdims=True)
            att[:, g * rep:(g + 1) * rep] = o.reshape(rep, M, D).transpose(1, 0, 2)
        h = h + att.reshape(M, Hq * D) @ W["o"].T
        xn = norm(h)
        gt, up = xn @ W["g"].T, xn @ W["u"].T
        h = h + (gt / (1.0 + np.exp(-gt)) * up) @ W["d"].T
    t_layer = (time.perf_counter() - t0) / SAMPLE_LAYERS
    t0 = time.perf_counter()
    norm(h) @ lm.T
    t_lm = (time.perf_counter() - t0) * LM_PART
    logits = rng.normal(0, 3, (7, V))
    t0 = time.perf_counter()
    S.spec_accept(logits[:4], logits[4:], np.array([1, 2, 3]), rng.random(4), S.SamplerConfig())
    t_acc = time.perf_counter() - t0
    t_step = layers * t_layer + t_lm + t_acc
    threads = int(os.environ.get("OPENBLAS_NUM_THREADS", "1"))
    print(json.dumps({"value": round(M / t_step, 4), "unit": "verify rows/s", "cores": threads, "kind": "port",
                      "sample": f"fp32 NumPy/BLAS port on {threads} threads, weights dequantised ahead of time "
                                f"(untimed): {SAMPLE_LAYERS} passes of one 27B-shaped decoder layer at 4096 context "
                                f"({t_layer * 1e3:.1f} ms each; the step has {layers}) + 1/{LM_PART} of lm_head "
                                f"({t_lm / LM_PART * 1e3:.1f} ms) + the fp64 oracle's accept step "
                                f"({t_acc * 1e3:.1f} ms), extrapolated to the full step ({t_step * 1e3:.0f} ms)",
                      "host_cpu_count": os.cpu_count()}))


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--parts", default="",
                    help="comma list of the extra measurements to run (cfg1,qmm,cfg4,cfg2,cfg5; default all)")
    ap.add_argument("--eager", action="store_true", help="launch kernel by kernel instead of one HIP graph per step")
    ap.add_argument("--profile-roofline", action="store_true",
                    help="only launch the roofline kernel (2 passes over the layers, eager) and a 256 MiB copy, "
                         "for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--profile-step", action="store_true",
                    help="only run one eager verify step and a 256 MiB copy, for rocprofv3 --pmc over every kernel")
    ap.add_argument("--workload", choices=["cfg1", "cfg2", "cfg4", "cfg5"], default=None,
                    help="only run that configuration's measurement (its sub-line, printed alone; for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the hot path is single-GPU); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        return 2

    import torch

    from mtplx_amd import _lib
    from mtplx_amd.sampling import SamplerConfig
    from mtplx_amd.verify_step import DENSE_27B, CapturedVerifyStep, VerifyModel

    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.workload == "cfg1":
        print(json.dumps({"cfg1_qmv": roofline_qmv_cfg1(), "cfg1_accept": accept_leg_cfg1()}), flush=True)
        return 0
    if args.workload == "cfg2":
        print(json.dumps(cfg2_attention()), flush=True)
        return 0
    if args.workload == "cfg5":
        print(json.dumps(cfg5_moe(steps=args.steps, warmup=args.warmup, eager=args.eager)), flush=True)
        return 0
    if args.workload == "cfg4":
        print(json.dumps(cfg4_ragged(VerifyModel(DENSE_27B, device=dev, seed=0), eager=args.eager, steps=args.steps,
                                     warmup=args.warmup)), flush=True)
        return 0
    cfg = DENSE_27B
    B, K = 1, 3
    L = K + 1
    model = VerifyModel(cfg, device=dev, seed=0)
    if args.profile_roofline:
        profile_roofline(model, B * L)
        return 0
    model.allocate_cache(B, args.ctx)
    gen = torch.Generator(device=dev).manual_seed(123)
    tokens = torch.randint(0, cfg.vocab, (B, L), device=dev, dtype=torch.int32, generator=gen)
    q_start = torch.full((B,), args.ctx - L, dtype=torch.int32, device=dev)
    draft_logits = (torch.randn((B, K, cfg.vocab), device=dev, generator=gen) * 3.0).contiguous()
    uniforms = torch.rand((B, K + 1), device=dev, dtype=torch.float64, generator=gen)
    sampler = SamplerConfig(0.6, 0.95, 20)
    if args.profile_step:
        profile_step(model, tokens, q_start, draft_logits, uniforms, sampler)
        return 0

    if args.eager:
        def step():
            return model.verify_step(tokens, q_start, draft_logits, uniforms, sampler)
        stream = torch.cuda.current_stream()
    else:
        cap = CapturedVerifyStep(model, tokens, q_start, draft_logits, uniforms, sampler)
        step = cap.replay
        stream = cap.stream
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            res = step()
        e1.record(stream)
        torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    assert int(res.status.max().item()) == 0, "non-finite logits in the verify step"
    value = B * L / (ms / 1e3)

    roof = roofline_gate_up(model, B * L)
    parts = set(args.parts.split(",")) if args.parts else {"cfg1", "qmm", "cfg4", "cfg2", "cfg5"}
    parts.discard("none")
    if "cfg1" in parts:
        roof["cfg1_qmv"] = roofline_qmv_cfg1()
        roof["cfg1_accept"] = accept_leg_cfg1()
    if "qmm" in parts:
        for m in (16, 32, 64):
            roof[f"m{m}_qmm"] = qmm_rows(m)
    others = {}
    if not args.eager:
        del cap
    if "cfg4" in parts:
        others["cfg4"] = cfg4_ragged(model, eager=args.eager)
        print(f"cfg4 done: {others['cfg4']['ms_per_step']} ms/step", file=sys.stderr, flush=True)
    del model
    torch.cuda.empty_cache()
    if "cfg2" in parts:
        others["cfg2_attention"] = cfg2_attention()
        print("cfg2 done", file=sys.stderr, flush=True)
    if "cfg5" in parts:
        others["cfg5"] = cfg5_moe(eager=args.eager)
        print(f"cfg5 done: {others['cfg5']['ms_per_step']} ms/step", file=sys.stderr, flush=True)
    cpu = None if args.no_cpu_baseline else cpu_baseline(cfg.layers)

    line = {
        "metric": "verify tokens/s at MTP depth 3; qmv achieved HBM GB/s (% of peak)",
        "value": round(value, 2),
        "unit": "verify rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations x 4-bit affine weights, fp32 accumulate; fp64 sampler",
        "data": "synthetic (random-init weights, random tokens/KV/draft logits, seeded)",
        "config": {"workload": "cfg3: depth-3 verify step, 27B-shaped 4-bit dense decoder, batch 1, "
                               f"{args.ctx}-token context, 4 verify rows + accept/reject",
                   "layers": cfg.layers, "hidden": cfg.hidden, "ffn": cfg.ffn, "heads": f"{cfg.n_heads}/{cfg.n_kv_heads}",
                   "head_dim": cfg.head_dim, "vocab": cfg.vocab, "group_size": cfg.group_size, "batch": B,
                   "verify_rows": L, "context": args.ctx, "wall_s_timed": round(wall, 3),
                   "launch": "eager" if args.eager else "hip_graph"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "other_configs": others,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
