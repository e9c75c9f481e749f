"""CPU tests of the MLX pack reader: config and quantization lookup (the
reference's ``artifacts.py:1131-1133`` order), shard discovery, the exact
stacking of q|k|v, expert gate|up and router|shared-gate rows, and the
refusals (unused tensors, other widths, untied missing lm_head, MoE without
renormalised top-k)."""

import numpy as np
import pytest
import torch

from mtplx_amd.mlx_pack import PackError, module_quant, quantization, read_mlx_pack
from tests.mlx_pack_util import write_pack


def _np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.view(torch.int32).numpy().view(np.uint32)


def test_quantization_lookup_order():
    assert quantization({"quantization_config": {"bits": 4, "group_size": 64}})["bits"] == 4
    assert quantization({"quantization": {"bits": 8, "group_size": 32}})["bits"] == 8
    assert quantization({"text_config": {"quantization": {"bits": 4, "group_size": 128}}})["group_size"] == 128
    q = {"group_size": 64, "bits": 4, "model.layers.0.mlp.down_proj": {"bits": 8}, "lm_head": False}
    assert module_quant(q, "model.layers.0.mlp.up_proj") == (64, 4)
    assert module_quant(q, "model.layers.0.mlp.down_proj") == (64, 8)
    assert module_quant(q, "lm_head") is None


def test_dense_pack_maps_exactly(tmp_path):
    raw = write_pack(tmp_path, layers=2, shards=3)
    cfg, w = read_mlx_pack(tmp_path)
    assert (cfg.layers, cfg.hidden, cfg.ffn, cfg.n_heads, cfg.n_kv_heads, cfg.vocab) == (2, 512, 1024, 4, 2, 1000)
    assert cfg.rope_theta == 1.0e6 and cfg.group_size == 64 and cfg.n_experts == 0
    for i in range(2):
        p = f"model.layers.{i}."
        qkv = w["layers"][i]["qkv"]
        for j in range(3):
            want = np.concatenate([raw[p + f"self_attn.{n}_proj"][j] for n in ("q", "k", "v")], axis=0)
            assert np.array_equal(_np(qkv[j]), want)
        assert np.array_equal(_np(w["layers"][i]["down"][0]), raw[p + "mlp.down_proj"][0])
        assert np.array_equal(_np(w["layers"][i]["in_norm"]), raw[p + "input_layernorm"])
    assert np.array_equal(_np(w["lm_head"][1]), raw["lm_head"][1])
    assert np.array_equal(_np(w["embed"][0]), raw["model.embed_tokens"][0])


def test_moe_pack_stacks_experts_and_router(tmp_path):
    raw = write_pack(tmp_path, layers=1, experts=8, top_k=2, shards=1)
    cfg, w = read_mlx_pack(tmp_path)
    assert (cfg.n_experts, cfg.top_k, cfg.expert_ffn, cfg.shared_ffn, cfg.ffn) == (8, 2, 256, 256, 0)
    L = w["layers"][0]
    p = "model.layers.0.mlp."
    for j in range(3):
        gu = np.concatenate([raw[p + "switch_mlp.gate_proj"][j], raw[p + "switch_mlp.up_proj"][j]], axis=1)
        assert np.array_equal(_np(L["expert_gate_up"][j]), gu)
        rt = np.concatenate([raw[p + "gate"][j], raw[p + "shared_expert_gate"][j]], axis=0)
        assert np.array_equal(_np(L["router"][j]), rt)
    assert _np(L["expert_gate_up"][0]).shape == (8, 512, 512 // 8)


def test_tied_embeddings_and_prefix(tmp_path):
    write_pack(tmp_path, layers=1, tie=True, prefix="language_model.model.")
    cfg, w = read_mlx_pack(tmp_path)
    assert w["lm_head"] is w["embed"]


def test_refusals(tmp_path):
    d = tmp_path / "a"; d.mkdir()
    write_pack(d, layers=1, extra={"model.layers.0.self_attn.q_norm.weight": torch.ones(128, dtype=torch.bfloat16),
                                   "mtp.fc.weight": torch.ones(4, dtype=torch.bfloat16)})
    with pytest.raises(PackError, match="q_norm"):
        read_mlx_pack(d)
    with pytest.raises(PackError, match="change the decoder's math"):
        read_mlx_pack(d, strict=False)                 # per-head q/k norms change the logits: always refused
    d = tmp_path / "r"; d.mkdir()
    write_pack(d, layers=1, extra={"model.layers.0.self_attn.rotary_emb.inv_freq": torch.ones(64),
                                   "mtp.fc.weight": torch.ones(4, dtype=torch.bfloat16)})
    with pytest.raises(PackError, match="inv_freq"):
        read_mlx_pack(d)                               # strict: every unused tensor but mtp.* is refused
    read_mlx_pack(d, strict=False)                     # rotary buffers and mtp.* cannot change the logits
    d = tmp_path / "s"; d.mkdir()
    write_pack(d, layers=1, extra={"model.layers.0.self_attn.q_proj.bias": torch.ones(512, dtype=torch.bfloat16)})
    with pytest.raises(PackError):
        read_mlx_pack(d, strict=False)                 # projection biases: refused
    d = tmp_path / "b"; d.mkdir()
    write_pack(d, layers=1, config_extra={"quantization": {"group_size": 64, "bits": 4,
                                                           "model.layers.0.mlp.down_proj": {"bits": 8}}})
    with pytest.raises(PackError, match="8-bit"):
        read_mlx_pack(d)
    d = tmp_path / "c"; d.mkdir()
    write_pack(d, layers=1, tie=False)
    (d / "model-00001-of-00002.safetensors").unlink()
    with pytest.raises(Exception):
        read_mlx_pack(d)
    d = tmp_path / "e"; d.mkdir()
    write_pack(d, layers=1, experts=4, config_extra={"norm_topk_prob": False})
    with pytest.raises(PackError, match="norm_topk_prob"):
        read_mlx_pack(d)
