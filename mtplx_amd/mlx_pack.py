"""Reader for MLX affine-quantized safetensors packs (the layout mlx-lm's
converter writes) into the verify model, so a real pack can replace random
init.

What is restated from the reference: the quantization block is
``config.json``'s ``quantization_config`` or ``quantization``, at the top
level or in ``text_config`` (``mtplx/artifacts.py:1131-1133``, local packs
``:1327-1329``); weight files are ``model*.safetensors`` (``:1134-1139``) or
the shards a ``model.safetensors.index.json`` names. A quantized linear is the
triple ``<name>.weight`` (uint32 ``[N, K*bits/32]``), ``<name>.scales`` and
``<name>.biases`` (``[N, K/group_size]``), with per-module overrides of
``{group_size, bits}`` keyed by the module name inside the quantization
block (MLX's convention). Tensor names are mlx-lm's for the Qwen decoder
family (``model.layers.{i}.self_attn.q_proj`` ...; MoE layers
``mlp.gate``, ``mlp.switch_mlp.*`` with a leading expert axis,
``mlp.shared_expert.*``, ``mlp.shared_expert_gate``).

Mapping onto :class:`~mtplx_amd.verify_step.VerifyModel` (exact: rows are
independent, so stacking quantized rows changes no value): q|k|v rows are
stacked into one projection; each expert's gate and up rows into one
``[E, 2F, K/8]`` pack; the router's E rows and the shared-expert gate's row
into one ``[E+1, H]`` projection.

Tensors the verify forward does not read are refused unless they cannot change
its logits: the MTP draft head (``mtp.*``) is always skipped, and with
``strict=False`` so are rotary ``inv_freq`` buffers and a multimodal pack's
vision tower and projector. Anything else left over (e.g. Qwen3's per-head
``q_norm``/``k_norm``, projection biases) is part of the decoder's math that
this forward does not apply, so it is refused whatever ``strict`` says.

Shards are opened lazily (``safetensors.safe_open``) and read one layer at a
time: :func:`load_verify_model` uploads and packs each layer on the GPU before
reading the next, so host memory holds one layer's tensors (plus the
embedding and lm_head), not the whole pack.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any

import torch

from .quant import QuantizedLinear
from .verify_step import DecoderConfig, Layer, VerifyModel


class PackError(ValueError):
    """The pack does not describe a model the verify forward can run."""


def text_config(config: dict) -> dict:
    tc = config.get("text_config")
    return tc if isinstance(tc, dict) else config


def quantization(config: dict) -> dict:
    """The pack's quantization block (``mtplx/artifacts.py:1131-1133``)."""
    quant = config.get("quantization_config") or config.get("quantization") or {}
    if not quant:
        tc = text_config(config)
        quant = tc.get("quantization_config") or tc.get("quantization") or {}
    return dict(quant)


def module_quant(quant: dict, name: str) -> tuple[int, int] | None:
    """(group_size, bits) of module ``name``; None when it is not quantized
    (a per-module entry of ``false``)."""
    over = quant.get(name)
    if over is False:
        return None
    if isinstance(over, dict):
        return int(over.get("group_size", quant.get("group_size", 64))), int(over.get("bits", quant.get("bits", 4)))
    if "group_size" not in quant or "bits" not in quant:
        raise PackError("config.json has no quantization {group_size, bits}")
    return int(quant["group_size"]), int(quant["bits"])


def shard_files(path: Path) -> list[Path]:
    index = path / "model.safetensors.index.json"
    if index.exists():
        wm = json.loads(index.read_text()).get("weight_map", {})
        return [path / f for f in sorted(set(wm.values()))]
    files = sorted(p for p in path.glob("model*.safetensors"))
    if not files:
        raise PackError(f"no model*.safetensors in {path}")
    return files


class LazyTensors:
    """Read-only mapping name -> CPU tensor over a pack's shards; a tensor is
    read from its shard when it is looked up, not before."""

    def __init__(self, files: list[Path]):
        from safetensors import safe_open

        self._handles = []
        self._where: dict[str, Any] = {}
        for f in files:
            h = safe_open(str(f), framework="pt", device="cpu")
            self._handles.append(h)
            for k in h.keys():
                self._where[k] = h

    def __contains__(self, key: str) -> bool:
        return key in self._where

    def __getitem__(self, key: str) -> torch.Tensor:
        h = self._where.get(key)
        if h is None:
            raise KeyError(key)
        return h.get_tensor(key)

    def __iter__(self):
        return iter(self._where)

    def keys(self):
        return self._where.keys()


def read_tensors(path: Path) -> LazyTensors:
    return LazyTensors(shard_files(path))


# Names a verify forward may skip without changing its logits (strict=False):
# rotary frequency buffers (the forward computes its own from rope_theta) and
# the vision side of a multimodal pack (the verify rows are text tokens).
_IGNORABLE_PARTS = ("rotary_emb.inv_freq",)
_IGNORABLE_PREFIXES = ("vision_tower.", "visual.", "model.visual.", "multi_modal_projector.", "model.vision_tower.",
                       "model.multi_modal_projector.")


def _ignorable(key: str, outer: str) -> bool:
    k = key[len(outer):] if outer and key.startswith(outer) else key
    return any(p in k for p in _IGNORABLE_PARTS) or any(k.startswith(p) for p in _IGNORABLE_PREFIXES)


def decoder_config(config: dict) -> DecoderConfig:
    tc = text_config(config)
    quant = quantization(config)
    n_heads = int(tc["num_attention_heads"])
    hidden = int(tc["hidden_size"])
    rope = tc.get("rope_theta")
    if rope is None and isinstance(tc.get("rope_parameters"), dict):
        rope = tc["rope_parameters"].get("rope_theta")
    n_experts = int(tc.get("num_experts") or tc.get("n_routed_experts") or 0)
    kw: dict[str, Any] = dict(
        layers=int(tc["num_hidden_layers"]), hidden=hidden, ffn=int(tc.get("intermediate_size") or 0),
        n_heads=n_heads, n_kv_heads=int(tc.get("num_key_value_heads") or n_heads),
        head_dim=int(tc.get("head_dim") or hidden // n_heads), vocab=int(tc["vocab_size"]),
        rope_theta=float(rope if rope is not None else 10000.0), rms_eps=float(tc.get("rms_norm_eps", 1e-6)),
        group_size=int(quant.get("group_size", 64)))
    if n_experts:
        if tc.get("norm_topk_prob") is not True:
            raise PackError("MoE routing without renormalised top-k weights (norm_topk_prob) is not the verify "
                            "model's router")
        kw.update(ffn=0, n_experts=n_experts, top_k=int(tc["num_experts_per_tok"]),
                  expert_ffn=int(tc["moe_intermediate_size"]),
                  shared_ffn=int(tc.get("shared_expert_intermediate_size") or 0))
        if not kw["shared_ffn"]:
            raise PackError("the verify model's MoE block has a gated shared expert; this pack has none")
    return DecoderConfig(**kw)


class _Reader:
    def __init__(self, tensors: dict[str, torch.Tensor], quant: dict, prefix: str, group_size: int):
        self.t = tensors
        self.quant = quant
        self.prefix = prefix
        self.gs = group_size
        self.used: set[str] = set()

    def take(self, key: str) -> torch.Tensor:
        k = self.prefix + key
        if k not in self.t:
            raise PackError(f"missing tensor {k}")
        self.used.add(k)
        return self.t[k]

    def norm(self, name: str) -> torch.Tensor:
        w = self.take(name + ".weight")
        if w.dtype != torch.bfloat16:
            raise PackError(f"{name}.weight is {w.dtype}; the verify kernels take bf16 norm weights")
        return w

    def triple(self, name: str) -> tuple[torch.Tensor, ...]:
        q = module_quant(self.quant, self.prefix + name) if (self.prefix + name) in self.quant else \
            module_quant(self.quant, name)
        if q is None:
            raise PackError(f"{name} is not quantized; the verify matmul takes quantized projections")
        gs, bits = q
        if bits != 4 or gs not in (64, 128) or gs != self.gs:
            raise PackError(f"{name}: {bits}-bit group {gs}; the verify model runs every projection 4-bit with "
                            f"the pack's one group size (64 or 128; here {self.gs})")
        w, s = self.take(name + ".weight"), self.take(name + ".scales")
        b = self.take(name + ".biases")
        if w.dtype not in (torch.uint32, torch.int32):
            raise PackError(f"{name}.weight is {w.dtype}, not packed uint32 words")
        if s.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
            raise PackError(f"{name}: scales/biases must be bf16 (got {s.dtype}/{b.dtype})")
        if (self.prefix + name + ".bias") in self.t:
            raise PackError(f"{name} has an additive bias; the verify model's projections have none")
        return w.view(torch.int32), s, b, torch.tensor(gs)


def _ql(parts, device) -> QuantizedLinear:
    w, s, b, gs = parts
    return QuantizedLinear(w.contiguous().to(device), s.contiguous().to(device), b.contiguous().to(device),
                           group_size=int(gs), bits=4)


def _stack(parts_list, dim: int):
    gss = {int(p[3]) for p in parts_list}
    if len(gss) != 1:
        raise PackError("stacked projections must share one group size")
    return tuple(torch.cat([p[i] for p in parts_list], dim=dim) for i in range(3)) + (parts_list[0][3],)


def _walk(path, strict: bool, on_layer=None) -> tuple[DecoderConfig, dict]:
    """Parse a pack on the CPU into the verify model's structure. Each layer's
    dict (norm weights and triples ``(weight int32, scales, biases,
    group_size)``) goes to ``on_layer(i, layer)`` as soon as it is read, whose
    return value is kept in its place (``None``: the layer dict itself)."""
    path = Path(path)
    config = json.loads((path / "config.json").read_text())
    cfg = decoder_config(config)
    tensors = read_tensors(path)
    emb_keys = [k for k in tensors if k.endswith("embed_tokens.weight")]
    if not emb_keys:
        raise PackError("no embed_tokens.weight in the pack")
    prefix = emb_keys[0][: -len("embed_tokens.weight")]          # e.g. "model."
    outer = prefix[: -len("model.")] if prefix.endswith("model.") else ""
    # Refuse leftovers before reading any weight: names are all it takes.
    r = _Reader(tensors, quantization(config), outer, cfg.group_size)
    m = prefix[len(outer):]
    expected = _expected_names(cfg, outer + m, outer, config)
    left = sorted(k for k in tensors.keys() if k not in expected and not k.startswith(outer + "mtp."))
    math = [k for k in left if not _ignorable(k, outer)]
    if math:
        raise PackError(f"{len(math)} tensors change the decoder's math but the verify forward does not apply them, "
                        f"e.g. {math[:4]}")
    if strict and left:
        raise PackError(f"{len(left)} tensors the verify forward does not use, e.g. {left[:4]} (strict=False "
                        "ignores rotary buffers and a vision tower)")
    out: dict[str, Any] = {"embed": r.triple(m + "embed_tokens"), "layers": []}
    for i in range(cfg.layers):
        p = f"{m}layers.{i}."
        lay: dict[str, Any] = {
            "in_norm": r.norm(p + "input_layernorm"),
            "qkv": _stack([r.triple(p + f"self_attn.{n}_proj") for n in ("q", "k", "v")], 0),
            "o": r.triple(p + "self_attn.o_proj"),
            "post_norm": r.norm(p + "post_attention_layernorm"),
        }
        if cfg.n_experts:
            router = r.triple(p + "mlp.gate")
            sgate = r.triple(p + "mlp.shared_expert_gate")
            lay["router"] = _stack([router, sgate], 0)
            g, u = r.triple(p + "mlp.switch_mlp.gate_proj"), r.triple(p + "mlp.switch_mlp.up_proj")
            lay["expert_gate_up"] = _stack([g, u], 1)
            del g, u
            lay["expert_down"] = r.triple(p + "mlp.switch_mlp.down_proj")
            for n in ("gate", "up", "down"):
                lay[f"shared_{n}"] = r.triple(p + f"mlp.shared_expert.{n}_proj")
        else:
            for n in ("gate", "up", "down"):
                lay[n] = r.triple(p + f"mlp.{n}_proj")
        kept = on_layer(i, lay) if on_layer is not None else None
        out["layers"].append(lay if kept is None else kept)
        del lay
    out["final_norm"] = r.norm(m + "norm")
    if (outer + "lm_head.weight") in tensors:
        out["lm_head"] = r.triple("lm_head")
    elif text_config(config).get("tie_word_embeddings") or config.get("tie_word_embeddings"):
        out["lm_head"] = out["embed"]
    else:
        raise PackError("no lm_head and the embeddings are not tied")
    return cfg, out


def _expected_names(cfg: DecoderConfig, m: str, outer: str, config: dict) -> set[str]:
    """Every tensor name the verify forward reads from a pack of ``cfg``."""
    names: set[str] = set()

    def tri(n):
        names.update(n + x for x in (".weight", ".scales", ".biases"))

    tri(m + "embed_tokens")
    for i in range(cfg.layers):
        p = f"{m}layers.{i}."
        names.update({p + "input_layernorm.weight", p + "post_attention_layernorm.weight"})
        for n in ("q", "k", "v", "o"):
            tri(p + f"self_attn.{n}_proj")
        if cfg.n_experts:
            tri(p + "mlp.gate")
            tri(p + "mlp.shared_expert_gate")
            for n in ("gate", "up", "down"):
                tri(p + f"mlp.switch_mlp.{n}_proj")
                tri(p + f"mlp.shared_expert.{n}_proj")
        else:
            for n in ("gate", "up", "down"):
                tri(p + f"mlp.{n}_proj")
    names.add(m + "norm.weight")
    tri(outer + "lm_head")
    return names


def read_mlx_pack(path, *, strict: bool = True) -> tuple[DecoderConfig, dict]:
    """Parse a pack on the CPU: (config, weights in the verify model's
    structure as CPU tensors: ``embed``/``lm_head``/per-layer triples
    ``(weight int32, scales, biases, group_size)``, norm weights)."""
    return _walk(path, strict)


def load_verify_model(path, *, device="cuda", strict: bool = True) -> VerifyModel:
    """A :class:`VerifyModel` over the pack's weights (on ``device``, packed
    for the streaming kernels; routing without the synthetic skew)."""
    def upload(i, lw):
        L = Layer(in_norm=lw["in_norm"].to(device), qkv=_ql(lw["qkv"], device), o=_ql(lw["o"], device),
                  post_norm=lw["post_norm"].to(device))
        for name in ("gate", "up", "down", "router", "expert_gate_up", "expert_down", "shared_gate", "shared_up",
                     "shared_down"):
            if name in lw:
                setattr(L, name, _ql(lw[name], device))
        return L   # the CPU copies of this layer are dropped here

    cfg, w = _walk(path, strict, upload)
    layers = w["layers"]
    embed = _ql(w["embed"], device)
    lm_head = embed if w["lm_head"] is w["embed"] else _ql(w["lm_head"], device)
    return VerifyModel.from_weights(cfg, embed, layers, w["final_norm"].to(device), lm_head, device=device)
