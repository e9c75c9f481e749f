"""One speculative verify step of a 4-bit decoder on gfx950 (random init).

This is the forward the reference runs on ``[primary, d1..dK]``
(``mtplx/generation.py:15027-15066`` → ``MTPLXRuntime.forward_ar``,
``mtplx/runtime.py:161``) followed by the accept/reject of
``mtplx/generation.py:15560-15790``, for a dense GQA decoder (the 27B shape:
64 layers, hidden 5120, SwiGLU 17408, 40/8 heads of 128, RMSNorm, RoPE 1e6,
vocab 151936, every linear 4-bit affine g64, bf16 KV cache) or its MoE variant.

Per layer the kernels are (every matmul is ``mtp_qmv_affine4_ex`` on the
layer's packed weights; the mode names the fused work):
  1. xmode 2, emode 4   input RMSNorm fused into the q|k|v matmul, whose
                        epilogue applies RoPE at per-request offsets and
                        writes K/V into the cache (where the epilogue does not
                        fit: the q|k|v matmul, then ``mtp_rope_qkv_to_cache_vt``)
  2. ``mtp_ragged_gqa_attn_rows_vt``  ragged GQA attention (split-KV + merge;
                        the balanced ``mtp_ragged_gqa_attn_blocks`` for long
                        total contexts)
  3. emode 1            o_proj + residual add (``mtp_qmv_affine4_residual``'s work)
  4. xmode 2, emode 3   post-attention RMSNorm + gate/up + SwiGLU
                        (``mtp_qmv_affine4_rmsnorm_dual``'s work)
  5. xmode 3, emode 1   down_proj + residual add, the row sums of its input
                        handed over by step 4
  (MoE layers replace 4-5 with RMSNorm → router projection (its last row
  is the shared-expert gate) → top-k route → expert sort → gathered SwiGLU →
  gathered down, the shared expert's SwiGLU MLP, and one combine: residual +
  routed + sigmoid(gate) * shared, ``mtplx/models/qwen4_exp.py:1416-1445``.)
then the final RMSNorm fused into the lm_head (fp32 logits) and
``mtp_spec_accept`` on the verify rows.
"""

from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass

import torch

from . import _lib
from .moe_sorted_gather import expert_sort, moe_combine
from .quant import QuantizedLinear, rope_row_order
from .attention_context import exact_lane_counts, exact_t0_guard_armed, exact_verify_required
from .sampling import SamplerConfig, spec_accept

# Keys per attention work unit on the exact lane: a fixed split length (a
# multiple of 128) makes each request's partials and merge independent of the
# rest of the batch; 1024 keeps at most 256 splits up to 256k-key contexts.
EXACT_SPLIT_KEYS = 1024


# MoE layers run the 5+-row experts and the shared expert on a second stream
# beside the 1-4-row experts (MTPLX_AMD_MOE_SIDE_STREAM=0: one stream).
MOE_SIDE_STREAM = (os.environ.get("MTPLX_AMD_MOE_SIDE_STREAM") or "1").strip() not in {"0", "false", "off", "no"}
# Rows up to which the dense projections take packed layout 2 (the
# 16x16x32 MFMA form, at most 16; MTPLX_AMD_LAYOUT2_ROWS=4 keeps 5..16 rows on
# layout 1's 32x32x16 form).
LAYOUT2_ROWS = min(16, int(os.environ.get("MTPLX_AMD_LAYOUT2_ROWS") or "16"))
# Packed layout of the routed expert stacks: 2 (16x16x32 quads, the default)
# or 1 (MTPLX_AMD_MOE_LAYOUT=1: 32x32x16 quads). One layout is kept.
MOE_LAYOUT = 1 if (os.environ.get("MTPLX_AMD_MOE_LAYOUT") or "2").strip() == "1" else 2


def qmv_ws_bytes(M: int, c: "DecoderConfig") -> int:
    """Split-K workspace of the streaming matmul for every projection of the
    step (the tail split's, or the full split's where x does not fit in LDS)."""
    ffn = c.expert_ffn if c.n_experts else c.ffn
    H = c.hidden
    nk = [(c.qkv_out, H), (H, c.n_heads * c.head_dim), (ffn, H), (H, ffn), (c.vocab, H)]
    if c.n_experts:
        nk += [(c.shared_ffn, H), (H, c.shared_ffn), (c.n_experts + 1, H)]
    return max(_lib.query("mtp_qmv_workspace_bytes", M, n, k, 1) for n, k in nk)


def _exact_lane(sampler: SamplerConfig) -> bool:
    """Greedy verify forwards (or any forward inside ``exact_verify(True)``)
    take the exact lane while the guard is armed."""
    return exact_verify_required() or (not float(sampler.temperature) > 0.0 and exact_t0_guard_armed())


@dataclass
class DecoderConfig:
    layers: int = 64
    hidden: int = 5120
    ffn: int = 17408
    n_heads: int = 40
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6
    group_size: int = 64
    # MoE variant (n_experts > 0): routed experts top-k + one shared expert.
    n_experts: int = 0
    top_k: int = 0
    expert_ffn: int = 0
    shared_ffn: int = 0
    router_zipf_s: float = 1.1
    # Weight recipe. False: every linear as the single-linear benchmark
    # (nibbles U{0..15}, scales |N(0,0.02)|, biases N(0,0.01)). Its groups
    # have mean 7.5 x scale, so each output column carries an offset common
    # to all tokens; layer after layer the hidden rows become nearly the same
    # vector and every token routes to the same top-k experts. True: centered
    # groups (bias -7.5 x scale) with unit gain (scale std 1/sqrt(21.25 K),
    # so an rms-1 input gives rms-1 outputs): hidden rows stay token-specific
    # and routing follows the Zipf skew plus per-token spread.
    centered_init: bool = False

    @property
    def qkv_out(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


DENSE_27B = DecoderConfig()
MOE_125B = DecoderConfig(layers=48, hidden=4096, ffn=0, n_heads=32, n_kv_heads=4, n_experts=256, top_k=8,
                         expert_ffn=1536, shared_ffn=1536, centered_init=True)


def _norm_weight(n: int, gen, device) -> torch.Tensor:
    return (1.0 + 0.1 * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16)


@dataclass
class Layer:
    in_norm: torch.Tensor
    qkv: QuantizedLinear
    o: QuantizedLinear
    post_norm: torch.Tensor
    gate: QuantizedLinear | None = None
    up: QuantizedLinear | None = None
    down: QuantizedLinear | None = None
    # MoE
    router: QuantizedLinear | None = None       # [E + 1, H]: E router rows, then the shared-expert gate row
    router_skew: torch.Tensor | None = None     # fp32 [E]: synthetic Zipf popularity added to the router logits
                                                # (None: the logits as they are, as for loaded weights)
    expert_gate_up: QuantizedLinear | None = None   # [E, 2F, K/8] fused [gate | up]
    expert_down: QuantizedLinear | None = None      # [E, H, F/8]
    shared_gate: QuantizedLinear | None = None
    shared_up: QuantizedLinear | None = None
    shared_down: QuantizedLinear | None = None
    qkv_rope: torch.Tensor | None = None    # q|k|v packed in RoPE tile order (fused RoPE epilogue), layout 1
    qkv_rope2: torch.Tensor | None = None   # the same in layout 2


def kv_block_offsets(kind: str) -> list[int]:
    """Offset inside a 4096-element block of (key % 32, d) = index key%32*128 + d,
    for the operand-major K ("k") or V ("v") cache blocks (head dim 128)."""
    offs = []
    for kk in range(32):
        for d in range(128):
            if kind == "k":
                c = d // 8
                offs.append(((c % 8) * 2 + c // 8) * 256 + kk * 8 + d % 8)
            else:
                jj, r = kk // 16, kk % 16
                h2 = (r % 8) // 4
                e = r % 4 if r < 8 else 4 + r % 4
                offs.append(((d // 32) * 2 + jj) * 512 + (h2 * 32 + d % 32) * 8 + e)
    return offs


def kv_to_blocks(std: torch.Tensor, kind: str) -> torch.Tensor:
    """[B, Hkv, cap, 128] -> operand-major blocks (same shape and storage size)."""
    B, H, cap, D = std.shape
    src = std.reshape(B, H, cap // 32, 4096)
    out = torch.empty_like(src)
    out[..., torch.tensor(kv_block_offsets(kind), device=std.device)] = src
    return out.reshape(B, H, cap, D)


def kv_from_blocks(blk: torch.Tensor, kind: str) -> torch.Tensor:
    """Inverse of :func:`kv_to_blocks`."""
    B, H, cap, D = blk.shape
    src = blk.reshape(B, H, cap // 32, 4096)
    return src.index_select(3, torch.tensor(kv_block_offsets(kind), device=blk.device)).reshape(B, H, cap, D)


class VerifyModel:
    """Random-init weights of ``cfg`` resident in HBM plus a ragged KV cache."""

    def __init__(self, cfg: DecoderConfig, *, device="cuda", seed: int = 0, keep_expert_source: bool = False):
        self.cfg = cfg
        self.keep_expert_source = keep_expert_source
        self.device = torch.device(device)
        gen = torch.Generator(device=self.device).manual_seed(seed)
        self.gen = gen
        c = cfg
        gs = c.group_size

        def lin(n, k, experts=None, gain=1.0):
            if c.centered_init:
                return QuantizedLinear.random(n, k, gs, generator=gen, device=device, experts=experts,
                                              scale_std=gain / math.sqrt(21.25 * k), centered=True)
            return QuantizedLinear.random(n, k, gs, generator=gen, device=device, experts=experts)

        # embedding rows: rms ~1 under the centered recipe (gain sqrt(K))
        self.embed = lin(c.vocab, c.hidden, gain=math.sqrt(c.hidden))
        self.layers: list[Layer] = []
        for _ in range(c.layers):
            L = Layer(in_norm=_norm_weight(c.hidden, gen, device), qkv=lin(c.qkv_out, c.hidden),
                      o=lin(c.hidden, c.n_heads * c.head_dim), post_norm=_norm_weight(c.hidden, gen, device))
            if c.n_experts:
                # Zipf-skewed routing: rank r (a per-layer permutation) gets
                # -s * log(r) added to the router logits; the router weights
                # are zero-mean (centered groups) with a scale that gives the
                # logits a per-token spread near the standard Gumbel's (std
                # 1.28), the noise under which top-k of (skew + noise) draws
                # experts with Zipf(s) popularity.
                L.router = QuantizedLinear.random(c.n_experts + 1, c.hidden, gs, generator=gen, device=device,
                                                  scale_std=0.0065, centered=True)
                rank = torch.randperm(c.n_experts, generator=gen, device=device).to(torch.float32) + 1.0
                L.router_skew = (-c.router_zipf_s * torch.log(rank)).contiguous()
                L.expert_gate_up = lin(2 * c.expert_ffn, c.hidden, experts=c.n_experts)
                L.expert_down = lin(c.hidden, c.expert_ffn, experts=c.n_experts)
                L.shared_gate = lin(c.shared_ffn, c.hidden)
                L.shared_up = lin(c.shared_ffn, c.hidden)
                L.shared_down = lin(c.hidden, c.shared_ffn)
            else:
                L.gate = lin(c.ffn, c.hidden)
                L.up = lin(c.ffn, c.hidden)
                L.down = lin(c.hidden, c.ffn)
            self.layers.append(L)
        self.final_norm = _norm_weight(c.hidden, gen, device)
        self.lm_head = lin(c.vocab, c.hidden)
        self._finish_init()

    @classmethod
    def from_weights(cls, cfg: DecoderConfig, embed: QuantizedLinear, layers: list[Layer], final_norm: torch.Tensor,
                     lm_head: QuantizedLinear, *, device="cuda", keep_expert_source: bool = False) -> "VerifyModel":
        """A model over given weights (e.g. an MLX pack read by
        :func:`mtplx_amd.mlx_pack.load_verify_model`) instead of random init."""
        self = cls.__new__(cls)
        self.cfg = cfg
        self.keep_expert_source = keep_expert_source
        self.device = torch.device(device)
        self.gen = torch.Generator(device=self.device).manual_seed(0)
        self.embed = embed
        self.layers = layers
        self.final_norm = final_norm
        self.lm_head = lm_head
        self._finish_init()
        return self

    def _finish_init(self) -> None:
        c = self.cfg
        # Tile-major copies for the streaming verify matmul (one pass at load
        # time), in layout 1 (any M) and layout 2 (M <= 16, 16x16x32 MFMA);
        # q|k|v also in RoPE tile order for the fused RoPE epilogue.
        rope_order = rope_row_order(c.n_heads + 2 * c.n_kv_heads, c.head_dim)
        for L in self.layers:
            for q in (L.qkv, L.o, L.gate, L.up, L.down, L.router, L.shared_gate, L.shared_up, L.shared_down):
                if q is not None:
                    q.pack()
                    q.pack(layout=2)
            L.qkv_rope = L.qkv.pack(rope_order)
            L.qkv_rope2 = L.qkv.pack(rope_order, layout=2)
            # Expert stacks: one packed layout (MOE_LAYOUT), and (unless asked
            # to keep it) the MLX-layout source is freed, so a 125B-class MoE
            # holds its experts once (2.7 GB per layer at the cfg5 shape).
            for q in (L.expert_gate_up, L.expert_down):
                if q is not None:
                    q.pack(layout=MOE_LAYOUT)
                    if not self.keep_expert_source:
                        q.release_source()
        self.lm_head.pack()
        self.lm_head.pack(layout=2)
        self._side = None
        self.k_cache: list[torch.Tensor] = []
        self.v_cache: list[torch.Tensor] = []
        self.cap = 0
        self._status: torch.Tensor | None = None
        # A list here receives each MoE layer's routed expert ids (int32
        # [M, top_k], on the device) as the forward runs; None records nothing.
        self.route_log: list | None = None

    def _side_stream(self) -> torch.Stream:
        """The model's second stream (default priority), made on first use."""
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.device)
        return self._side

    # -- cache ----------------------------------------------------------------
    def allocate_cache(self, batch: int, capacity: int, *, fill_random: bool = True) -> None:
        c = self.cfg
        cap = ((capacity + 255) // 256) * 256
        self.k_cache, self.v_cache = [], []
        for _ in range(c.layers):
            shape = (batch, c.n_kv_heads, cap, c.head_dim)
            if fill_random:
                k = torch.randn(shape, generator=self.gen, device=self.device).to(torch.bfloat16)
                v = torch.randn(shape, generator=self.gen, device=self.device).to(torch.bfloat16)
            else:
                k = torch.zeros(shape, dtype=torch.bfloat16, device=self.device)
                v = torch.zeros_like(k)
            self.k_cache.append(k)
            self.v_cache.append(v)
        self.cap = cap
        self.batch = batch

    def allocate_cache_blocks(self, capacities, *, fill_random: bool = True) -> None:
        """A ragged cache for the continuous-batched lane: request b gets its
        own capacity (rounded up to 32 keys) inside one packed buffer of
        operand-major 32-key blocks per layer; ``kv_off`` int32 [B+1] holds
        each request's first block (head h at kv_off[b] + h * nblk_b)."""
        c = self.cfg
        caps = [((int(x) + 31) // 32) * 32 for x in capacities]
        offs = [0]
        for cp in caps:
            offs.append(offs[-1] + c.n_kv_heads * (cp // 32))
        nblocks = offs[-1]
        self.k_cache, self.v_cache = [], []
        for _ in range(c.layers):
            if fill_random:
                k = torch.empty(nblocks * 4096, dtype=torch.bfloat16, device=self.device)
                v = torch.empty_like(k)
                step = 1 << 26   # fill in slices: bounded fp32 temporaries
                for t in (k, v):
                    for i in range(0, t.numel(), step):
                        n = min(step, t.numel() - i)
                        t[i:i + n] = torch.randn(n, generator=self.gen, device=self.device).to(torch.bfloat16)
            else:
                k = torch.zeros(nblocks * 4096, dtype=torch.bfloat16, device=self.device)
                v = torch.zeros_like(k)
            self.k_cache.append(k)
            self.v_cache.append(v)
        self.caps = caps
        self.cap = max(caps)
        self.total_cap = sum(caps)
        self.batch = len(caps)
        self.kv_off = torch.tensor(offs, dtype=torch.int32, device=self.device)
        self._kv_off_host = offs

    def cache_request(self, li: int, b: int, kind: str) -> torch.Tensor:
        """Request b's K ("k") or V ("v") cache of layer li in the reference
        layout [Hkv, cap_b, D] (from a block cache made by allocate_cache_blocks)."""
        c = self.cfg
        o0, o1 = self._kv_off_host[b], self._kv_off_host[b + 1]
        buf = (self.k_cache if kind == "k" else self.v_cache)[li]
        blk = buf[o0 * 4096:o1 * 4096].reshape(1, c.n_kv_heads, (o1 - o0) // c.n_kv_heads * 32, c.head_dim)
        return kv_from_blocks(blk, kind)[0]

    # K and V caches are kept in the operand-major 32-key block layout
    # (include/mtplx_amd.h); these give the reference [B, Hkv, cap, D] view.
    def k_cache_standard(self, li: int) -> torch.Tensor:
        return kv_from_blocks(self.k_cache[li], "k")

    def v_cache_standard(self, li: int) -> torch.Tensor:
        return kv_from_blocks(self.v_cache[li], "v")

    def status(self) -> torch.Tensor | None:
        """The last forward's device status word (int32 [1]): bit 0 is set when
        a token id was outside the vocabulary (its embedding row reads as zero)
        or a K/V write fell outside the cache capacity (skipped; attention then
        stops at the capacity). Nonzero means that forward's logits are invalid."""
        return self._status

    def check_status(self) -> None:
        """Raise :class:`MtpError` if the last forward flagged its status word
        (synchronises with the device)."""
        if self._status is not None and int(self._status.item()) != 0:
            raise _lib.MtpError("verify_logits", -1, "token id outside the vocabulary or a K/V position outside "
                                "the cache capacity (status word set)")

    # -- forward --------------------------------------------------------------
    def verify_logits(self, tokens: torch.Tensor, q_start: torch.Tensor, q_lens: torch.Tensor | None = None,
                      *, logits_out: torch.Tensor | None = None, check: bool = False,
                      exact: bool = False, layer_log: list | None = None) -> torch.Tensor:
        """``tokens`` int32 ``[B, L]`` (GPU), ``q_start`` int32 ``[B]`` (GPU):
        writes K/V of the L rows at ``q_start[b] + i`` and returns fp32 logits ``[B*L, V]``.
        The device status word (:meth:`status`) flags invalid tokens or
        positions; ``check=True`` synchronises and raises on it. ``exact``: the exact lane
        (:meth:`verify_logits_ragged` with ``exact=True`` over this uniform
        cache), whose rows do not depend on B or L. ``layer_log``: a list
        that receives a copy of the hidden rows (bf16 ``[B*L, H]``) entering
        every layer and the final norm (layers + 1 entries)."""
        c = self.cfg
        B, Lq = (int(s) for s in tokens.shape)
        M = B * Lq
        if exact:
            if c.n_experts:
                raise ValueError("the exact lane serves the dense model")
            dev = self.device
            nblk = self.cap // 32
            kv_off = torch.arange(B + 1, dtype=torch.int32, device=dev) * (c.n_kv_heads * nblk)
            row_off = torch.arange(B + 1, dtype=torch.int32, device=dev) * Lq
            ql = torch.full((B,), Lq, dtype=torch.int32, device=dev) if q_lens is None else q_lens
            return self._ragged_forward(tokens.reshape(-1), row_off, q_start, ql, Lq, kv_off, B * self.cap,
                                        logits_out=logits_out, check=check, split_keys=EXACT_SPLIT_KEYS,
                                        layer_log=layer_log)
        dev = self.device
        st = _lib.stream_handle(dev)
        gs = c.group_size
        H = c.hidden
        call = _lib.call
        eps = ctypes.c_float(c.rms_eps)
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        h = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
        tok = tokens.reshape(-1).to(torch.int32).contiguous()
        call("mtp_embed_affine4", tok.data_ptr(), self.embed.weight.data_ptr(), self.embed.scales.data_ptr(),
             self.embed.biases.data_ptr(), h.data_ptr(), M, H, c.vocab, gs, status.data_ptr(), st)
        qkv = torch.empty((M, c.qkv_out), dtype=torch.bfloat16, device=dev)
        qh = torch.empty((B, c.n_heads, Lq, c.head_dim), dtype=torch.bfloat16, device=dev)
        attn = torch.empty((M, c.n_heads * c.head_dim), dtype=torch.bfloat16, device=dev)
        ffn = c.expert_ffn if c.n_experts else c.ffn
        act = torch.empty((M, ffn), dtype=torch.bfloat16, device=dev)
        # Sum-of-squares statistics of h handed from each residual epilogue to the
        # next fused RMSNorm (two buffers so a producer never overwrites what its
        # consumer has not read yet). None for the embedding output.
        ss_a = torch.empty(((H + 31) // 32) * 32, dtype=torch.float32, device=dev)
        ss_b = torch.empty_like(ss_a)
        ss_h = None
        # gate/up also writes the 32-column row sums of its SwiGLU output, so
        # down_proj stages its x without a pass over it (xmode 3).
        act_sums = torch.empty(((ffn + 31) // 32) * 32, dtype=torch.float32, device=dev)
        nb = _lib.query("mtp_attn_vt_workspace_bytes", B, c.n_kv_heads, self.cap)
        aws = _lib.WORKSPACES.get(nb, "attn", dev)
        # Long total contexts (B * Hkv * cap >= 65536 key-heads: cfg5's 4 x 4 x
        # 8k) run the balanced block attention (one workgroup per CU, equal
        # shares of all tiles): cfg5 13.84 -> 13.70 ms per step. The cfg3 step
        # (1 x 8 x 4k) keeps the split kernel (4.95 against 5.34 ms).
        balanced = B * c.n_kv_heads * self.cap >= 65536
        if balanced:
            bnb = _lib.query("mtp_attn_blocks_workspace_bytes", B, c.n_kv_heads, self.cap, 0, 0)
            bws = _lib.WORKSPACES.get(bnb, "attn_blocks", dev)
        scale = 1.0 / math.sqrt(c.head_dim)
        ql = None if q_lens is None else q_lens.to(torch.int32).contiguous()
        # Per-tile streaming kernel with a workspace: its leftover tiles (e.g.
        # the last 32 of gate/up's 544 on 256 CUs) are split by K over all CUs.
        qws = _lib.WORKSPACES.get(qmv_ws_bytes(M, c), "qmv", dev)

        def qmv(stream, **kw):
            _lib.qmv_ex(stream, ws=qws, ws_bytes=qws.numel(), **kw)

        # The RoPE epilogue covers up to 16 rows with all of x in LDS.
        fused_rope = bool(_lib.query("mtp_qmv_rope_fusable", M, c.qkv_out, H))
        lay = 2 if M <= LAYOUT2_ROWS else 1   # layout 2: the 16x16x32 MFMA form for up to 16 rows

        def W(q):
            return q.packed_mf16 if lay == 2 else q.packed

        for li, L in enumerate(self.layers):
            if layer_log is not None:
                layer_log.append(h.clone())
            xin = dict(x=h, x2=L.in_norm, xmode=2)   # input RMSNorm fused into the staging
            if fused_rope:
                rope = dict(q_start=q_start, q_lens=ql, q_out=qh, k_cache=self.k_cache[li], v_cache=self.v_cache[li],
                            status=status, L=Lq, Hq=c.n_heads, Hkv=c.n_kv_heads, D=c.head_dim, cap=self.cap,
                            blocked=1, rope_base=c.rope_theta)
                qmv(st, rope=rope, ss_in=ss_h, eps=c.rms_eps, w0=L.qkv_rope2 if lay == 2 else L.qkv_rope, M=M,
                    N=c.qkv_out, K=H, group_size=gs, emode=4, packed=lay, **xin)
            else:
                qmv(st, ss_in=ss_h, eps=c.rms_eps, w0=W(L.qkv), y0=qkv, M=M, N=c.qkv_out, K=H, group_size=gs,
                    emode=0, packed=lay, **xin)
                call("mtp_rope_qkv_to_cache_vt", qkv.data_ptr(), q_start.data_ptr(), _lib.ptr(ql), qh.data_ptr(),
                     self.k_cache[li].data_ptr(), self.v_cache[li].data_ptr(), B, Lq, c.n_heads, c.n_kv_heads,
                     c.head_dim, self.cap, ctypes.c_float(c.rope_theta), status.data_ptr(), st)
            if balanced:
                _lib.attn_blocks(st, q=qh, k_blk=self.k_cache[li], v_blk=self.v_cache[li], q_start=q_start, q_lens=ql,
                                 row_off=None, kv_off=None, out=attn, B=B, Hq=c.n_heads, Hkv=c.n_kv_heads, Lmax=Lq,
                                 D=c.head_dim, cap=self.cap, split_keys=0, scale=scale, total_cap=0, ws=bws,
                                 ws_bytes=bws.numel())
            else:
                call("mtp_ragged_gqa_attn_rows_vt", qh.data_ptr(), self.k_cache[li].data_ptr(),
                     self.v_cache[li].data_ptr(), q_start.data_ptr(), _lib.ptr(ql), attn.data_ptr(), B, c.n_heads,
                     c.n_kv_heads, Lq, c.head_dim, self.cap, ctypes.c_float(scale), aws.data_ptr(), aws.numel(), st)
            qmv(st, x=attn, w0=W(L.o), resid=h, y0=h, ss_out=ss_a, M=M, N=H, K=c.n_heads * c.head_dim,
                group_size=gs, xmode=0, emode=1, packed=lay)
            ss_h = ss_a
            if c.n_experts:
                # (the statistics' layout holds up to 32 rows)
                ss_h = ss_b if M <= 32 else None
                self._moe_block(L, h, M, st, qmv, lay, ss_h)
            else:
                qmv(st, x=h, x2=L.post_norm, ss_in=ss_h, eps=c.rms_eps, w0=W(L.gate), w1=W(L.up), y0=act,
                    y_sums=act_sums, M=M, N=c.ffn, K=H, group_size=gs, xmode=2, emode=3, packed=lay)
                qmv(st, x=act, x_sums=act_sums, w0=W(L.down), resid=h, y0=h, ss_out=ss_b, M=M, N=H, K=c.ffn,
                    group_size=gs, xmode=3, emode=1, packed=lay)
                ss_h = ss_b
        if layer_log is not None:
            layer_log.append(h.clone())
        logits = logits_out if logits_out is not None else torch.empty((M, c.vocab), dtype=torch.float32, device=dev)
        qmv(st, x=h, x2=self.final_norm, ss_in=ss_h, eps=c.rms_eps, w0=W(self.lm_head), yf=logits, M=M,
            N=c.vocab, K=H, group_size=gs, xmode=2, emode=0, packed=lay)
        self._status = status
        if check:
            self.check_status()
        return logits

    def _moe_block(self, L: Layer, h: torch.Tensor, M: int, st: int, qmv, lay: int,
                   ss_out: torch.Tensor | None) -> None:
        """The sparse block on the post-attention norm of ``h``, added to ``h``
        in place: routed experts through the sorted chain
        (``mtplx/models/qwen4_exp.py:1544-1577``) plus the sigmoid-gated shared
        expert (``:1438-1445``). The combine writes the output rows' sums of
        squares to ``ss_out`` (when given) for the next fused RMSNorm."""
        c = self.cfg
        call = _lib.call
        gs = c.group_size
        dev = h.device
        H = c.hidden
        E = c.n_experts
        xn = torch.empty_like(h)
        call("mtp_rmsnorm", h.data_ptr(), L.post_norm.data_ptr(), xn.data_ptr(), M, H, c.rms_eps, st)
        # Router logits (bf16-rounded, fp32 storage) [M, E+1]; column E is the
        # shared-expert gate's pre-activation.
        rl = torch.empty((M, E + 1), dtype=torch.float32, device=dev)
        Wr = L.router.packed_mf16 if lay == 2 else L.router.packed
        qmv(st, x=xn, w0=Wr, yf=rl, M=M, N=E + 1, K=H, group_size=gs, xmode=0, emode=0, packed=lay)
        ids = torch.empty((M, c.top_k), dtype=torch.int32, device=dev)
        wts = torch.empty((M, c.top_k), dtype=torch.float32, device=dev)
        call("mtp_moe_route", rl.data_ptr(), E + 1, _lib.ptr(L.router_skew), M, E, c.top_k, ids.data_ptr(),
             wts.data_ptr(), st)
        if self.route_log is not None:
            self.route_log.append(ids)
        es = expert_sort(ids, E)
        R = M * c.top_k
        F = c.expert_ffn
        hsorted = torch.empty((R, F), dtype=torch.bfloat16, device=dev)
        ysorted = torch.empty((R, H), dtype=torch.bfloat16, device=dev)

        # Routed experts over their packed stacks: gate|up + SwiGLU on the
        # token rows gathered by row_map, then down on the sorted rows; one
        # launch per row class (experts with 1-4 rows, with more).
        gfn = "mtp_gather_qmv_affine4_packed_mf16" if MOE_LAYOUT == 2 else "mtp_gather_qmv_affine4_packed_rows"

        def EW(q):
            return q.packed_mf16 if MOE_LAYOUT == 2 else q.packed

        def experts(row_class, stream):
            call(gfn, xn.data_ptr(), es.row_map.data_ptr(), es.expert_off.data_ptr(), es.active.data_ptr(),
                 EW(L.expert_gate_up).data_ptr(), hsorted.data_ptr(), M, E, F, H, gs, 3, 2 * F, row_class, stream)
            call(gfn, hsorted.data_ptr(), None, es.expert_off.data_ptr(), es.active.data_ptr(),
                 EW(L.expert_down).data_ptr(), ysorted.data_ptr(), M, E, H, F, gs, 0, H, row_class, stream)

        # Shared expert (SwiGLU MLP) on the normalised rows, then one combine:
        # h = h + bf16(routed + bf16(sigmoid(gate) * shared)).
        def W(q):
            return q.packed_mf16 if lay == 2 else q.packed

        sh_act = torch.empty((M, c.shared_ffn), dtype=torch.bfloat16, device=dev)
        shared = torch.empty_like(h)

        def shared_expert(stream, run):
            run(stream, x=xn, w0=W(L.shared_gate), w1=W(L.shared_up), y0=sh_act, M=M, N=c.shared_ffn, K=H,
                group_size=gs, xmode=0, emode=3, packed=lay)
            run(stream, x=sh_act, w0=W(L.shared_down), y0=shared, M=M, N=H, K=c.shared_ffn, group_size=gs, xmode=0,
                emode=0, packed=lay)

        side = self._side_stream() if MOE_SIDE_STREAM else None
        if side is None:
            experts(0, st)
            shared_expert(st, qmv)
        else:
            # The latency-bound work (the 5+-row experts, the shared expert)
            # on a second stream beside the 1-4-row experts, which stream
            # most of the bytes; the combine waits for both.
            main = torch.cuda.current_stream(dev)
            fork = torch.cuda.Event()
            fork.record(main)
            side.wait_event(fork)
            with torch.cuda.stream(side):
                sst = side.cuda_stream
                sws = _lib.WORKSPACES.get(qmv_ws_bytes(M, c), "qmv_side", dev)

                def side_qmv(stream, **kw):
                    _lib.qmv_ex(stream, ws=sws, ws_bytes=sws.numel(), **kw)

                experts(2, sst)
                shared_expert(sst, side_qmv)
                join = torch.cuda.Event()
                join.record(side)
            experts(1, st)
            main.wait_event(join)
        moe_combine(ysorted, es, wts, shared, shared_gate=rl[:, E], resid=h, out=h, ss_out=ss_out)

    def verify_logits_ragged(self, tokens: torch.Tensor, row_off: torch.Tensor, q_start: torch.Tensor,
                             q_lens: torch.Tensor, Lmax: int, *, logits_out: torch.Tensor | None = None,
                             check: bool = False, exact: bool = False, layer_log: list | None = None) -> torch.Tensor:
        """The continuous-batched verify forward (dense model, block cache from
        :meth:`allocate_cache_blocks`): ``tokens`` int32 [M] packed request
        after request, request b's ``q_lens[b]`` (<= ``Lmax``) rows at
        ``row_off[b]`` (int32 [B+1]) and positions ``q_start[b] + i``. Every
        projection runs on ``mtp_qmm_affine4_mfma`` (each weight quad read once
        for all M <= 64 rows); RoPE writes K/V into the requests' blocks;
        attention reads per-request capacities. Returns fp32 logits [M, V].

        ``exact``: the exact lane. The matmul's K split never depends on M,
        and attention runs ``EXACT_SPLIT_KEYS``-key units with the per-head
        merge instead of the balanced kernel (whose shares depend on the
        whole batch), so each request's logits are bit-identical to those of
        the same rows verified alone (any L, any batch)."""
        return self._ragged_forward(tokens, row_off, q_start, q_lens, Lmax, self.kv_off, self.total_cap,
                                    logits_out=logits_out, check=check,
                                    split_keys=EXACT_SPLIT_KEYS if exact else 0, layer_log=layer_log)

    def _ragged_forward(self, tokens: torch.Tensor, row_off: torch.Tensor, q_start: torch.Tensor,
                        q_lens: torch.Tensor, Lmax: int, kv_off: torch.Tensor, total_cap: int, *,
                        logits_out: torch.Tensor | None, check: bool, split_keys: int,
                        layer_log: list | None) -> torch.Tensor:
        """The ragged forward over a block cache described by ``kv_off``
        (int32 [B+1], first block of each request) and ``total_cap`` (summed
        capacities); ``split_keys`` 0 = balanced attention."""
        c = self.cfg
        if c.n_experts:
            raise NotImplementedError("the ragged lane serves the dense model")
        M = int(tokens.numel())
        B = int(q_start.numel())
        if M > 64:
            raise ValueError(f"the ragged lane takes at most 64 rows (got {M})")
        dev = self.device
        st = _lib.stream_handle(dev)
        call = _lib.call
        H, gs = c.hidden, c.group_size
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        h = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
        xn = torch.empty_like(h)
        tok = tokens.reshape(-1).to(torch.int32).contiguous()
        call("mtp_embed_affine4", tok.data_ptr(), self.embed.weight.data_ptr(), self.embed.scales.data_ptr(),
             self.embed.biases.data_ptr(), h.data_ptr(), M, H, c.vocab, gs, status.data_ptr(), st)
        qkv = torch.empty((M, c.qkv_out), dtype=torch.bfloat16, device=dev)
        qh = torch.empty((B, c.n_heads, Lmax, c.head_dim), dtype=torch.bfloat16, device=dev)
        attn = torch.empty((M, c.n_heads * c.head_dim), dtype=torch.bfloat16, device=dev)
        act = torch.empty((M, c.ffn), dtype=torch.bfloat16, device=dev)
        ro = row_off.to(torch.int32).contiguous()
        ql = q_lens.to(torch.int32).contiguous()
        qmm_nb = max(_lib.query("mtp_qmm_workspace_bytes", M, n, k, d) for n, k, d in
                     ((c.qkv_out, H, 0), (H, c.n_heads * c.head_dim, 0), (c.ffn, H, 1), (H, c.ffn, 0),
                      (c.vocab, H, 0)))
        qws = _lib.WORKSPACES.get(max(qmm_nb, 256), "qmm", dev)
        anb = _lib.query("mtp_attn_blocks_workspace_bytes", B, c.n_kv_heads, self.cap, total_cap, split_keys)
        aws = _lib.WORKSPACES.get(anb, "attn_blocks", dev)
        scale = 1.0 / math.sqrt(c.head_dim)
        eps = ctypes.c_float(c.rms_eps)

        def mm(**kw):
            _lib.qmm_mfma(st, M=M, group_size=gs, ws=qws, ws_bytes=qws.numel(), **kw)

        def norm(x, w, out):
            call("mtp_rmsnorm", x.data_ptr(), w.data_ptr(), out.data_ptr(), M, H, eps, st)

        kvo = kv_off.to(torch.int32).contiguous()
        for li, L in enumerate(self.layers):
            if layer_log is not None:
                layer_log.append(h.clone())
            norm(h, L.in_norm, xn)
            mm(x=xn, w0=L.qkv.packed, y=qkv, N=c.qkv_out, K=H, emode=0)
            call("mtp_rope_qkv_to_blocks", qkv.data_ptr(), M, ro.data_ptr(), q_start.data_ptr(),
                 kvo.data_ptr(), qh.data_ptr(), self.k_cache[li].data_ptr(), self.v_cache[li].data_ptr(), B,
                 Lmax, c.n_heads, c.n_kv_heads, c.head_dim, self.cap, ctypes.c_float(c.rope_theta),
                 status.data_ptr(), st)
            _lib.attn_blocks(st, q=qh, k_blk=self.k_cache[li], v_blk=self.v_cache[li], q_start=q_start, q_lens=ql,
                             row_off=ro, kv_off=kvo, out=attn, B=B, Hq=c.n_heads, Hkv=c.n_kv_heads, Lmax=Lmax,
                             D=c.head_dim, cap=self.cap, split_keys=split_keys, scale=scale, total_cap=total_cap,
                             ws=aws, ws_bytes=aws.numel())
            mm(x=attn, w0=L.o.packed, y=h, resid=h, N=H, K=c.n_heads * c.head_dim, emode=1)
            norm(h, L.post_norm, xn)
            mm(x=xn, w0=L.gate.packed, w1=L.up.packed, y=act, N=c.ffn, K=H, emode=3)
            mm(x=act, w0=L.down.packed, y=h, resid=h, N=H, K=c.ffn, emode=1)
        if layer_log is not None:
            layer_log.append(h.clone())
        norm(h, self.final_norm, xn)
        logits = logits_out if logits_out is not None else torch.empty((M, c.vocab), dtype=torch.float32, device=dev)
        mm(x=xn, w0=self.lm_head.packed, yf=logits, N=c.vocab, K=H, emode=0)
        self._status = status
        if check:
            self.check_status()
        return logits

    def verify_step_ragged(self, tokens: torch.Tensor, row_off: torch.Tensor, q_start: torch.Tensor,
                           q_lens: torch.Tensor, Lmax: int, draft_logits: torch.Tensor, d_off: torch.Tensor,
                           draft_index: torch.Tensor, uniforms: torch.Tensor, sampler: SamplerConfig = SamplerConfig()):
        """Ragged forward, then accept/reject with per-request depths
        K_b = q_lens[b] - 1: request b's draft ids are ``tokens[draft_index]``
        entries d_off[b] .. d_off[b] + K_b - 1 (the rows after its primary) and
        its draft rows the same rows of ``draft_logits``."""
        from .sampling import spec_accept_ragged

        if int(uniforms.shape[-1]) < int(Lmax) or int(uniforms.shape[0]) != int(q_start.numel()):
            raise ValueError(f"uniforms must be [B, >= Lmax] = [{int(q_start.numel())}, >= {int(Lmax)}] "
                             f"(got {list(uniforms.shape)}): request b consumes up to q_lens[b] of its row")
        exact = _exact_lane(sampler)
        if exact:
            exact_lane_counts["verify_step_ragged"] += 1
        logits = self.verify_logits_ragged(tokens, row_off, q_start, q_lens, Lmax, exact=exact)
        self.last_logits = logits
        drafts = tokens.reshape(-1)[draft_index]
        return spec_accept_ragged(logits, row_off[:-1], draft_logits, d_off, q_lens - 1, drafts, uniforms, sampler)

    def verify_step(self, tokens: torch.Tensor, q_start: torch.Tensor, draft_logits: torch.Tensor,
                    uniforms: torch.Tensor, sampler: SamplerConfig = SamplerConfig()):
        """Forward the ``B x (K+1)`` verify rows, then accept/reject against the drafts
        (``tokens[:, 1:]`` are the draft ids). Returns the device-side accept result."""
        B, L = (int(s) for s in tokens.shape)
        K = L - 1
        c = self.cfg
        if _exact_lane(sampler) and not c.n_experts:
            # Greedy verify: the exact lane, whose rows do not depend on the
            # batch (the argmax the autoregressive decode of the same rows picks).
            exact_lane_counts["verify_step"] += 1
            logits = self.verify_logits(tokens, q_start, exact=True)
            self.last_logits = logits
            return spec_accept(logits.reshape(B, L, -1), draft_logits, tokens[:, 1:].contiguous(), uniforms,
                               sampler)
        logits = self.verify_logits(tokens, q_start)
        self.last_logits = logits
        return spec_accept(logits.reshape(B, L, -1), draft_logits, tokens[:, 1:].contiguous(), uniforms, sampler)


class CapturedVerifyStep:
    """The whole verify step (embedding → layers → lm_head → accept/reject)
    recorded once as a HIP graph on a dedicated stream and replayed per step,
    so the ~7 launches per layer cost no host round trips.

    The graph reads its inputs from the tensors given at capture time: update
    them in place (``tokens.copy_(...)`` etc.) between replays. Workspaces are
    created by an eager warm-up on the same stream, so the capture itself
    allocates nothing but the step's own activations (from the graph pool).
    """

    def __init__(self, model: VerifyModel, tokens: torch.Tensor, q_start: torch.Tensor,
                 draft_logits: torch.Tensor, uniforms: torch.Tensor, sampler: SamplerConfig = SamplerConfig()):
        self.model = model
        self.inputs = (tokens, q_start, draft_logits, uniforms)
        self.stream = torch.cuda.Stream(device=model.device)
        self.graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize(model.device)
        with torch.cuda.stream(self.stream):
            model.verify_step(tokens, q_start, draft_logits, uniforms, sampler)     # warm-up: workspaces
        self.stream.synchronize()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.result = model.verify_step(tokens, q_start, draft_logits, uniforms, sampler)
        self.logits = model.last_logits          # graph-owned output buffer
        torch.cuda.synchronize(model.device)

    def replay(self):
        """Enqueue one step on the current stream's device; returns the (static) accept result."""
        self.graph.replay()
        return self.result


class CapturedRaggedVerifyStep:
    """``verify_step_ragged`` (embedding → layers → lm_head → accept/reject
    with per-request depths) recorded once as a HIP graph, with the same
    contract as :class:`CapturedVerifyStep`: the graph reads the tensors given
    at capture time (update them in place between replays; the host-side
    ``Lmax`` and the sampler configuration are fixed), and an eager warm-up on
    the capture stream creates the workspaces first."""

    def __init__(self, model: VerifyModel, tokens: torch.Tensor, row_off: torch.Tensor, q_start: torch.Tensor,
                 q_lens: torch.Tensor, Lmax: int, draft_logits: torch.Tensor, d_off: torch.Tensor,
                 draft_index: torch.Tensor, uniforms: torch.Tensor, sampler: SamplerConfig = SamplerConfig()):
        self.model = model
        self.args = (tokens, row_off, q_start, q_lens, Lmax, draft_logits, d_off, draft_index, uniforms, sampler)
        self.stream = torch.cuda.Stream(device=model.device)
        self.graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize(model.device)
        with torch.cuda.stream(self.stream):
            model.verify_step_ragged(*self.args)     # warm-up: workspaces
        self.stream.synchronize()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.result = model.verify_step_ragged(*self.args)
        self.logits = model.last_logits          # graph-owned output buffer
        torch.cuda.synchronize(model.device)

    def replay(self):
        """Enqueue one step on the current stream's device; returns the (static) accept result."""
        self.graph.replay()
        return self.result
