"""Export a grpo_mi355x Qwen2ForCausalLM to the oracle's numpy weight format (tests only)."""

from __future__ import annotations

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _nf4(lin, bias=None, a=None, b=None):
    qs = lin.weight.quant_state
    d = dict(packed=lin.weight.detach().cpu().numpy().reshape(-1).copy(),
             absmax=qs.absmax.detach().cpu().numpy().copy(),
             n=lin.out_features, k=lin.in_features)
    if bias is not None:
        d["bias"] = bits(bias)
    if a is not None:
        d["A"], d["B"] = bits(a), bits(b)
    return d


def export(model, cfg=None) -> tuple[dict, dict]:
    """Oracle weights/config of ``model``; ``cfg`` overrides ``model.config`` (a
    transformers config lacks the NF4 blocksize and LoRA fields)."""
    cfg = cfg or model.config
    layers = []
    for L in model.model.layers:
        at, mlp = L.self_attn, L.mlp
        e = dict(input_norm=bits(L.input_layernorm.weight),
                 post_norm=bits(L.post_attention_layernorm.weight))
        for name in ("q", "k", "v", "o"):
            m = getattr(at, f"{name}_proj")
            e[name] = _nf4(m.base_layer, m.base_layer.bias, m.lora_A.weight, m.lora_B.weight)
        for name in ("gate", "up", "down"):
            e[name] = _nf4(getattr(mlp, f"{name}_proj"))
        layers.append(e)
    w = dict(embed=bits(model.model.embed_tokens.weight), norm=bits(model.model.norm.weight),
             lm_head=bits(model.lm_head.weight), layers=layers)
    c = dict(hidden=cfg.hidden_size, n_heads=cfg.num_attention_heads,
             n_kv=cfg.num_key_value_heads, head_dim=cfg.head_dim, eps=cfg.rms_norm_eps,
             theta=cfg.rope_theta, blocksize=cfg.nf4_blocksize,
             scaling=cfg.lora_alpha / cfg.lora_rank)
    return w, c
