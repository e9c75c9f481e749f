"""GPU parity of a verify model loaded from an MLX pack (dense and MoE):
logits of the verify forward against the float64 oracle whose parameters
are built by this test straight from the pack's arrays (q, k, v rows stacked
in the oracle model's head order; each expert's gate rows then up rows; the
router rows then the shared-expert gate row), so the loader's mapping is
checked against the model definition, not against itself.

Bar: rtol/atol 1e-2 (the north-star bf16 bar), routed expert ids equal to
the oracle's."""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from oracle.model import verify_forward
from tests.gpu_util import assert_close
from tests.mlx_pack_util import write_pack

pytestmark = pytest.mark.gpu


def _params(raw, layers, experts, prefix="model."):
    vals = lambda bits: bf16_bits_to_f32(bits).astype(np.float64)  # noqa: E731
    cat = lambda names, axis=0: tuple(np.concatenate([raw[n][j] for n in names], axis=axis)  # noqa: E731
                                      for j in range(3))
    out = {"embed": raw[prefix + "embed_tokens"], "layers": [], "final_norm": vals(raw[prefix + "norm"]),
           "lm_head": raw.get("lm_head", raw[prefix + "embed_tokens"])}
    for i in range(layers):
        p = f"{prefix}layers.{i}."
        d = {"in_norm": vals(raw[p + "input_layernorm"]), "post_norm": vals(raw[p + "post_attention_layernorm"]),
             "qkv": cat([p + f"self_attn.{n}_proj" for n in ("q", "k", "v")]), "o": raw[p + "self_attn.o_proj"]}
        if experts:
            d.update(router=cat([p + "mlp.gate", p + "mlp.shared_expert_gate"]), router_skew=None,
                     expert_gate_up=cat([p + "mlp.switch_mlp.gate_proj", p + "mlp.switch_mlp.up_proj"], axis=1),
                     expert_down=raw[p + "mlp.switch_mlp.down_proj"],
                     shared_gate=raw[p + "mlp.shared_expert.gate_proj"],
                     shared_up=raw[p + "mlp.shared_expert.up_proj"],
                     shared_down=raw[p + "mlp.shared_expert.down_proj"])
        else:
            d.update(gate=raw[p + "mlp.gate_proj"], up=raw[p + "mlp.up_proj"], down=raw[p + "mlp.down_proj"])
        out["layers"].append(d)
    return out


@pytest.mark.parametrize("experts,tie", [(0, False), (0, True), (8, False)])
def test_loaded_model_matches_oracle(gpu, tmp_path, experts, tie):
    from mtplx_amd.mlx_pack import load_verify_model
    layers = 1 if experts else 2
    raw = write_pack(tmp_path, layers=layers, experts=experts, tie=tie, seed=3 + experts, shards=2)
    model = load_verify_model(tmp_path, device="cuda")
    cfg = model.cfg
    B, L, cap = 2, 4, 256
    model.allocate_cache(B, cap)
    kc = [model.k_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(layers)]
    vc = [model.v_cache_standard(li).float().cpu().numpy().astype(np.float64) for li in range(layers)]
    g = torch.Generator(device="cuda").manual_seed(5)
    tokens = torch.randint(0, cfg.vocab, (B, L), device="cuda", dtype=torch.int32, generator=g)
    starts = [100, 37]
    model.route_log = []
    logits = model.verify_logits(tokens, torch.tensor(starts, dtype=torch.int32, device="cuda"), check=True)
    got = logits.cpu().numpy().astype(np.float64)
    routes = []
    want = verify_forward(_params(raw, layers, experts), cfg, tokens.cpu().numpy(), np.array(starts), kc, vc, routes)
    assert_close(got, want, what=f"pack experts={experts} tie={tie}")
    if experts:
        gpu_ids = model.route_log[0].cpu().numpy()
        assert np.array_equal(np.sort(gpu_ids, axis=1), np.sort(routes[0][0], axis=1))
