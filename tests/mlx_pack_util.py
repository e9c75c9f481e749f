"""Writes small synthetic packs in mlx-lm's on-disk layout (tests only)."""

import json

import numpy as np
import torch

from oracle.bf16 import f32_to_bf16_bits
from oracle.qmv import make_affine4_weights


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _triple(out: dict, raw: dict, name: str, w, s, b):
    out[name + ".weight"] = torch.from_numpy(np.ascontiguousarray(w)).view(torch.uint32)
    out[name + ".scales"] = _bf16(s)
    out[name + ".biases"] = _bf16(b)
    raw[name] = (w, s, b)


def write_pack(path, *, layers=2, hidden=512, ffn=1024, n_heads=4, n_kv=2, vocab=1000, experts=0, top_k=2,
               expert_ffn=256, shared_ffn=256, gs=64, seed=0, tie=False, prefix="model.", extra=None,
               config_extra=None, shards=2, scale_std=0.02):
    """A pack with random 4-bit layers; returns the raw numpy arrays by module name."""
    from safetensors.torch import save_file

    rng = np.random.default_rng(seed)
    D = 128
    t: dict[str, torch.Tensor] = {}
    raw: dict = {}

    def lin(name, n, k, lead=None):
        if lead is None:
            _triple(t, raw, name, *make_affine4_weights(rng, n, k, gs, scale_std=scale_std))
        else:
            w, s, b = make_affine4_weights(rng, lead * n, k, gs, scale_std=scale_std)
            _triple(t, raw, name, w.reshape(lead, n, -1), s.reshape(lead, n, -1), b.reshape(lead, n, -1))

    def norm(name, n):
        v = f32_to_bf16_bits((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
        t[name + ".weight"] = _bf16(v)
        raw[name] = v

    lin(prefix + "embed_tokens", vocab, hidden)
    for i in range(layers):
        p = f"{prefix}layers.{i}."
        norm(p + "input_layernorm", hidden)
        lin(p + "self_attn.q_proj", n_heads * D, hidden)
        lin(p + "self_attn.k_proj", n_kv * D, hidden)
        lin(p + "self_attn.v_proj", n_kv * D, hidden)
        lin(p + "self_attn.o_proj", hidden, n_heads * D)
        norm(p + "post_attention_layernorm", hidden)
        if experts:
            lin(p + "mlp.gate", experts, hidden)
            lin(p + "mlp.shared_expert_gate", 1, hidden)
            lin(p + "mlp.switch_mlp.gate_proj", expert_ffn, hidden, lead=experts)
            lin(p + "mlp.switch_mlp.up_proj", expert_ffn, hidden, lead=experts)
            lin(p + "mlp.switch_mlp.down_proj", hidden, expert_ffn, lead=experts)
            lin(p + "mlp.shared_expert.gate_proj", shared_ffn, hidden)
            lin(p + "mlp.shared_expert.up_proj", shared_ffn, hidden)
            lin(p + "mlp.shared_expert.down_proj", hidden, shared_ffn)
        else:
            lin(p + "mlp.gate_proj", ffn, hidden)
            lin(p + "mlp.up_proj", ffn, hidden)
            lin(p + "mlp.down_proj", hidden, ffn)
    norm(prefix + "norm", hidden)
    if not tie:
        lin("lm_head", vocab, hidden)
    if extra:
        t.update(extra)
    cfg = {"model_type": "qwen3_next" if experts else "qwen2", "num_hidden_layers": layers, "hidden_size": hidden,
           "intermediate_size": ffn, "num_attention_heads": n_heads, "num_key_value_heads": n_kv, "head_dim": D,
           "vocab_size": vocab, "rope_theta": 1.0e6, "rms_norm_eps": 1e-6, "tie_word_embeddings": tie,
           "quantization": {"group_size": gs, "bits": 4}}
    if experts:
        cfg.update(num_experts=experts, num_experts_per_tok=top_k, moe_intermediate_size=expert_ffn,
                   shared_expert_intermediate_size=shared_ffn, norm_topk_prob=True)
    if config_extra:
        cfg.update(config_extra)
    (path / "config.json").write_text(json.dumps(cfg))
    keys = sorted(t)
    if shards == 1:
        save_file(t, str(path / "model.safetensors"))
    else:
        wm = {}
        for j in range(shards):
            part = {k: t[k].contiguous() for k in keys[j::shards]}
            fn = f"model-{j + 1:05d}-of-{shards:05d}.safetensors"
            save_file(part, str(path / fn))
            wm.update({k: fn for k in part})
        (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    return raw
