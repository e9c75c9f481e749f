"""Copy a GPU VerifyModel into the NumPy structures oracle.model expects."""

import numpy as np
import torch


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _vals(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _ql(q):
    if q is None:
        return None
    if q.weight is None:
        raise ValueError("the layer's source weights were released: build the model with keep_expert_source=True")
    return (q.weight.detach().contiguous().cpu().numpy().view(np.uint32), _bits(q.scales), _bits(q.biases))


def model_params_numpy(model) -> dict:
    layers = []
    for L in model.layers:
        d = {"in_norm": _vals(L.in_norm), "qkv": _ql(L.qkv), "o": _ql(L.o), "post_norm": _vals(L.post_norm)}
        if L.gate is not None:
            d.update(gate=_ql(L.gate), up=_ql(L.up), down=_ql(L.down))
        else:
            d.update(router=_ql(L.router), router_skew=None if L.router_skew is None else L.router_skew.cpu().numpy().astype(np.float32),
                     expert_gate_up=_ql(L.expert_gate_up), expert_down=_ql(L.expert_down),
                     shared_gate=_ql(L.shared_gate), shared_up=_ql(L.shared_up), shared_down=_ql(L.shared_down))
        layers.append(d)
    return {"embed": _ql(model.embed), "layers": layers, "final_norm": _vals(model.final_norm),
            "lm_head": _ql(model.lm_head)}
