"""Adapt a transformers-layout Qwen2 model to the decode engine's layout.

The reference trainer hands its own model to ``paged_kv_decode``
(``src/grpo/trainer.py:389-400``): a transformers ``Qwen2ForCausalLM`` whose
linear layers are bitsandbytes ``Linear4bit`` (NF4, ``model_loader.py:15-20``)
and whose q/k/v/o projections are wrapped in ``ManualLoRALayer``
(``src/core/lora.py:166-233``).  The reference walks that tree by attribute
name (``paged_kv.py:459-544``); ``decode_model_from`` does the same and
returns an object with the layout ``DecodeEngine`` needs:

* q|k|v of each layer stacked into ONE NF4 buffer (rows q, k, v) and gate|up
  into another, so each group is one kernel launch.  The packed bytes and
  absmax are copied once (the base weights are frozen during GRPO); the
  per-projection modules become views into the stacked buffers.
* LoRA A/B, biases, norms, embeddings and lm_head are shared with the source
  model by reference, so adapter updates made by the trainer in place are
  seen by the next rollout without re-adapting.

A weight is accepted when it has the bnb ``Params4bit`` surface: a uint8
tensor with ``quant_state.{absmax, code, blocksize, shape}``.  Nested
(double-quantized) absmax is expanded once to the float32 absmax the kernels
read (``_nf4_parts``, ``grpo_nf4_absmax_expand``: lora_forward.py:187-199).  A
model that already has the stacked layout (for example
``rollout.qwen2.Qwen2ForCausalLM``) is returned unchanged.
"""

from __future__ import annotations

import weakref
from types import SimpleNamespace

import torch
import torch.nn as nn

from ..core.nf4 import float_absmax
from .qwen2 import Qwen2Config, Qwen2RotaryEmbedding, StackedNF4, _view_linear

_cache: "weakref.WeakKeyDictionary[nn.Module, object]" = weakref.WeakKeyDictionary()


def _unwrap(mod):
    """(base NF4 linear, LoRA wrapper or None) of a projection."""
    if hasattr(mod, "base_layer") and hasattr(mod, "lora_A"):
        return mod.base_layer, mod
    return mod, None


def _nf4_parts(lin, what: str):
    w = getattr(lin, "weight", None)
    qs = getattr(w, "quant_state", None)
    if w is None or qs is None or w.dtype != torch.uint8:
        raise ValueError(f"{what}: expected an NF4 (Params4bit-like) weight with quant_state")
    n, k = (int(s) for s in qs.shape)
    absmax = float_absmax(qs)  # a nested state is expanded once (frozen weights)
    if absmax.dtype != torch.float32 or absmax.numel() * int(qs.blocksize) < n * k:
        raise ValueError(f"{what}: absmax must be float32 with one entry per block")
    return w.reshape(-1), absmax.reshape(-1), qs.code, int(qs.blocksize), n, k


def _stack(parts, what: str):
    packed = torch.cat([p[0] for p in parts])
    absmax = torch.cat([p[1][: p[4] * p[5] // p[3]] for p in parts])
    code, bs = parts[0][2], parts[0][3]
    for p in parts:
        if p[3] != bs or p[5] != parts[0][5] or not torch.equal(p[2], code):
            raise ValueError(f"{what}: stacked projections need one blocksize, K and codebook")
        if p[4] * p[5] % bs:
            raise ValueError(f"{what}: each projection must hold whole absmax blocks")
    return packed.contiguous(), absmax.contiguous(), code.float().contiguous(), bs


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.bfloat16 else t.detach().to(torch.bfloat16)


def _lora_view(base, wrapper):
    """A LoRA wrapper over a stacked-buffer view, sharing A/B with ``wrapper``."""
    if wrapper is None:
        raise ValueError("q/k/v/o projections must carry LoRA adapters (ManualLoRALayer)")
    for name in ("lora_A", "lora_B"):
        if getattr(wrapper, name).weight.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16 (inject_lora_layers makes it so)")
    return SimpleNamespace(base_layer=base, lora_A=wrapper.lora_A, lora_B=wrapper.lora_B,
                           rank=int(wrapper.rank), scaling=float(wrapper.scaling))


def _config(model, rank: int, alpha: float, blocksize: int) -> Qwen2Config:
    c = model.config
    heads = int(c.num_attention_heads)
    head_dim = int(getattr(c, "head_dim", None) or c.hidden_size // heads)
    theta = getattr(c, "rope_theta", None)
    if theta is None:
        theta = (getattr(c, "rope_parameters", None) or {}).get("rope_theta", 10000.0)
    return Qwen2Config(vocab_size=int(c.vocab_size), hidden_size=int(c.hidden_size),
                       intermediate_size=int(c.intermediate_size),
                       num_hidden_layers=int(c.num_hidden_layers), num_attention_heads=heads,
                       num_key_value_heads=int(c.num_key_value_heads), head_dim=head_dim,
                       rms_norm_eps=float(c.rms_norm_eps), rope_theta=float(theta),
                       lora_rank=rank, lora_alpha=alpha, nf4_blocksize=blocksize)


def _norm(mod):
    eps = getattr(mod, "variance_epsilon", None)
    if eps is None:
        eps = getattr(mod, "eps", 1e-6)
    return SimpleNamespace(weight=_bf16(mod.weight), variance_epsilon=float(eps))


def _adapt(model):
    inner = model.model
    layers = []
    rank = alpha = bs = None
    for li, layer in enumerate(inner.layers):
        at, mlp = layer.self_attn, layer.mlp
        qkv_mods = [_unwrap(getattr(at, f"{n}_proj")) for n in ("q", "k", "v")]
        parts = [_nf4_parts(b, f"layer {li} {n}_proj")
                 for (b, _), n in zip(qkv_mods, ("q", "k", "v"))]
        packed, absmax, code, bs = _stack(parts, f"layer {li} q|k|v")
        k = parts[0][5]
        rows = [p[4] for p in parts]
        qkv = StackedNF4(packed, absmax, code, rows, k, bs)
        views, row0 = {}, 0
        for (base, wrap), n, r in zip(qkv_mods, ("q", "k", "v"), rows):
            bias = None if getattr(base, "bias", None) is None else _bf16(base.bias)
            views[n] = _lora_view(_view_linear(packed, absmax, code, row0, r, k, bs, bias), wrap)
            row0 += r
        o_base, o_wrap = _unwrap(at.o_proj)
        _nf4_parts(o_base, f"layer {li} o_proj")
        o_view = _lora_view(o_base, o_wrap)
        g_parts = [_nf4_parts(_unwrap(getattr(mlp, f"{n}_proj"))[0], f"layer {li} {n}_proj")
                   for n in ("gate", "up")]
        gpk, gab, gcode, _ = _stack(g_parts, f"layer {li} gate|up")
        gate_up = StackedNF4(gpk, gab, gcode, [p[4] for p in g_parts], g_parts[0][5], bs)
        down = _unwrap(mlp.down_proj)[0]
        _nf4_parts(down, f"layer {li} down_proj")
        rank = views["q"].rank if rank is None else rank
        alpha = views["q"].scaling * views["q"].rank if alpha is None else alpha
        for v in (views["q"], views["k"], views["v"], o_view):
            if v.rank != rank or abs(v.scaling * v.rank - alpha) > 1e-6:
                raise ValueError("every q/k/v/o adapter must have the same rank and alpha")
        layers.append(SimpleNamespace(
            self_attn=SimpleNamespace(qkv=qkv, q_proj=views["q"], k_proj=views["k"],
                                      v_proj=views["v"], o_proj=o_view),
            mlp=SimpleNamespace(gate_up=gate_up, down_proj=down),
            input_layernorm=_norm(layer.input_layernorm),
            post_attention_layernorm=_norm(layer.post_attention_layernorm)))
    cfg = _config(model, int(rank), float(alpha), int(bs))
    dev = inner.embed_tokens.weight.device
    out = SimpleNamespace(
        config=cfg,
        model=SimpleNamespace(embed_tokens=SimpleNamespace(weight=_bf16(inner.embed_tokens.weight)),
                              layers=layers, norm=_norm(inner.norm),
                              rotary_emb=Qwen2RotaryEmbedding(cfg, dev)),
        lm_head=SimpleNamespace(weight=_bf16(model.lm_head.weight)))
    return out


@torch.no_grad()
def decode_model_from(model):
    """The decode-engine view of ``model`` (cached per model object)."""
    first = model.model.layers[0]
    if hasattr(first.self_attn, "qkv") and hasattr(first.mlp, "gate_up"):
        return model
    hit = _cache.get(model)
    if hit is None:
        hit = _adapt(model)
        _cache[model] = hit
    return hit


__all__ = ["decode_model_from"]
