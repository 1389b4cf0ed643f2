"""Random-init Qwen2-shaped causal LM with NF4 base weights and LoRA on q/k/v/o.

The module tree uses transformers' attribute names, which the reference's
model-level decode walks (``src/triton_kernels/paged_kv.py:459-544``):
``model.embed_tokens``, ``model.layers[i].{input_layernorm, self_attn.{q,k,v,o}_proj,
post_attention_layernorm, mlp.{gate,up,down}_proj}``, ``model.norm``,
``model.rotary_emb``, ``lm_head``, ``config``.  q/k/v/o are ``ManualLoRALayer``
over ``Linear4bitNF4`` (as ``inject_lora_layers`` leaves a bitsandbytes model,
``src/core/lora.py:166-233``); gate/up/down are plain ``Linear4bitNF4``; q/k/v
carry a bias, o_proj does not (Qwen2).

Layout for the decode step: the q|k|v weights of a layer are ONE stacked NF4
buffer (rows q, then k, then v) and gate|up another; the per-projection
modules hold views into them, so one grouped kernel launch covers them
without any copy.  The stacked quantization equals per-projection
quantization because every projection holds whole absmax blocks.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn as nn

from ..core.lora import ManualLoRALayer
from ..core.nf4 import Linear4bitNF4, Params4bit, QuantState, nf4_code, quantize_nf4


@dataclass
class Qwen2Config:
    vocab_size: int = 151936
    hidden_size: int = 1536
    intermediate_size: int = 8960
    num_hidden_layers: int = 28
    num_attention_heads: int = 12
    num_key_value_heads: int = 2
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 32768
    lora_rank: int = 16
    lora_alpha: int = 32
    nf4_blocksize: int = 64
    extra: dict = field(default_factory=dict)

    @classmethod
    def qwen2_1_5b(cls) -> "Qwen2Config":
        return cls()

    @classmethod
    def qwen2_7b(cls) -> "Qwen2Config":
        return cls(hidden_size=3584, intermediate_size=18944, num_attention_heads=28,
                   num_key_value_heads=4, vocab_size=152064)

    @classmethod
    def tiny(cls, layers: int = 2, heads: int = 4, kv_heads: int = 2, head_dim: int = 128,
             inter: int = 1024, vocab: int = 1000) -> "Qwen2Config":
        return cls(vocab_size=vocab, hidden_size=heads * head_dim, intermediate_size=inter,
                   num_hidden_layers=layers, num_attention_heads=heads,
                   num_key_value_heads=kv_heads, head_dim=head_dim)


class Qwen2RMSNorm(nn.Module):
    def __init__(self, hidden: int, eps: float, device=None):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden, dtype=torch.bfloat16, device=device),
                                   requires_grad=False)
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:  # transformers' Qwen2RMSNorm
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * h.to(x.dtype)


class Qwen2RotaryEmbedding(nn.Module):
    """transformers' default RoPE; ``tables`` returns bf16 cos/sin per position."""

    def __init__(self, cfg: Qwen2Config, device=None):
        super().__init__()
        d = cfg.head_dim
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
        self.register_buffer("inv_freq", inv.to(device), persistent=False)
        self.head_dim = d

    @torch.no_grad()
    def forward(self, x: torch.Tensor, position_ids: torch.Tensor):
        inv = self.inv_freq[None, :, None].float().expand(position_ids.shape[0], -1, 1)
        pos = position_ids[:, None, :].float()
        freqs = (inv.to(pos.device) @ pos).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)

    @torch.no_grad()
    def tables(self, max_pos: int, dtype=torch.bfloat16):
        pos = torch.arange(max_pos, device=self.inv_freq.device)[None]
        cos, sin = self.forward(torch.empty(0, dtype=dtype, device=self.inv_freq.device), pos)
        return cos[0].contiguous(), sin[0].contiguous()


def _view_linear(packed: torch.Tensor, absmax: torch.Tensor, code: torch.Tensor, row0: int,
                 rows: int, k: int, blocksize: int, bias: torch.Tensor | None) -> Linear4bitNF4:
    """A ``Linear4bitNF4`` whose weight/absmax are views into a stacked buffer."""
    lin = Linear4bitNF4.__new__(Linear4bitNF4)
    nn.Module.__init__(lin)
    lin.in_features, lin.out_features, lin.blocksize = k, rows, blocksize
    b0, b1 = row0 * k // 2, (row0 + rows) * k // 2
    a0, a1 = row0 * k // blocksize, (row0 + rows) * k // blocksize
    state = QuantState(absmax[a0:a1], (rows, k), code, blocksize)
    lin.weight = Params4bit(packed[b0:b1], state)
    if bias is not None:
        lin.bias = nn.Parameter(bias, requires_grad=False)
    else:
        lin.register_parameter("bias", None)
    return lin


class StackedNF4(nn.Module):
    """Several NF4 projections of one input stacked row-wise in one buffer."""

    def __init__(self, packed: torch.Tensor, absmax: torch.Tensor, code: torch.Tensor,
                 seg_rows: list[int], k: int, blocksize: int):
        super().__init__()
        self.register_buffer("packed", packed, persistent=True)
        self.register_buffer("absmax", absmax, persistent=True)
        self.register_buffer("code", code, persistent=True)
        self.seg_rows = list(seg_rows)
        self.in_features = k
        self.blocksize = blocksize

    @property
    def out_features(self) -> int:
        return sum(self.seg_rows)


def _stack(weights: list[torch.Tensor], blocksize: int):
    w = torch.cat(weights, 0)
    packed, state = quantize_nf4(w, blocksize)
    return packed.view(-1), state.absmax, state.code


class Qwen2Attention(nn.Module):
    def __init__(self, cfg: Qwen2Config, g: torch.Generator, device, std: float,
                 lora_std: float):
        super().__init__()
        h, d = cfg.hidden_size, cfg.head_dim
        nq, nkv = cfg.num_attention_heads * d, cfg.num_key_value_heads * d
        self.num_heads, self.num_key_value_heads, self.head_dim = (
            cfg.num_attention_heads, cfg.num_key_value_heads, d)
        bs = cfg.nf4_blocksize
        rnd = lambda *s, sd=std: (torch.randn(*s, generator=g, device=device) * sd)
        packed, absmax, code = _stack([rnd(nq, h), rnd(nkv, h), rnd(nkv, h)], bs)
        self.qkv = StackedNF4(packed, absmax, code, [nq, nkv, nkv], h, bs)
        biases = [rnd(n).to(torch.bfloat16) for n in (nq, nkv, nkv)]
        row0 = 0
        for name, rows, b in zip(("q_proj", "k_proj", "v_proj"), (nq, nkv, nkv), biases):
            base = _view_linear(packed, absmax, code, row0, rows, h, bs, b)
            setattr(self, name, self._lora(base, cfg, g, device, lora_std))
            row0 += rows
        opk, ost = quantize_nf4(rnd(h, nq), bs)
        o_base = _view_linear(opk.view(-1), ost.absmax, ost.code, 0, h, nq, bs, None)
        self.o_proj = self._lora(o_base, cfg, g, device, lora_std)

    @staticmethod
    def _lora(base, cfg, g, device, lora_std):
        layer = ManualLoRALayer(base, rank=cfg.lora_rank, alpha=cfg.lora_alpha)
        with torch.no_grad():
            layer.lora_A.weight = nn.Parameter(
                (torch.randn(cfg.lora_rank, base.in_features, generator=g, device=device)
                 * lora_std).to(torch.bfloat16))
            layer.lora_B.weight = nn.Parameter(
                (torch.randn(base.out_features, cfg.lora_rank, generator=g, device=device)
                 * lora_std).to(torch.bfloat16))
        return layer


class Qwen2MLP(nn.Module):
    def __init__(self, cfg: Qwen2Config, g: torch.Generator, device, std: float):
        super().__init__()
        h, i, bs = cfg.hidden_size, cfg.intermediate_size, cfg.nf4_blocksize
        rnd = lambda *s: torch.randn(*s, generator=g, device=device) * std
        packed, absmax, code = _stack([rnd(i, h), rnd(i, h)], bs)
        self.gate_up = StackedNF4(packed, absmax, code, [i, i], h, bs)
        self.gate_proj = _view_linear(packed, absmax, code, 0, i, h, bs, None)
        self.up_proj = _view_linear(packed, absmax, code, i, i, h, bs, None)
        dpk, dst = quantize_nf4(rnd(h, i), bs)
        self.down_proj = _view_linear(dpk.view(-1), dst.absmax, dst.code, 0, h, i, bs, None)


class Qwen2DecoderLayer(nn.Module):
    def __init__(self, cfg, g, device, std, lora_std):
        super().__init__()
        self.self_attn = Qwen2Attention(cfg, g, device, std, lora_std)
        self.mlp = Qwen2MLP(cfg, g, device, std)
        self.input_layernorm = Qwen2RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device)
        self.post_attention_layernorm = Qwen2RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device)
        with torch.no_grad():
            for n in (self.input_layernorm, self.post_attention_layernorm):
                n.weight.add_((torch.randn(cfg.hidden_size, generator=g, device=device) * std)
                              .to(torch.bfloat16))


class Qwen2Model(nn.Module):
    def __init__(self, cfg, g, device, std, lora_std):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size, device=device,
                                         dtype=torch.bfloat16)
        with torch.no_grad():
            self.embed_tokens.weight.copy_(
                (torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=device) * std)
                .to(torch.bfloat16))
        self.embed_tokens.weight.requires_grad_(False)
        self.layers = nn.ModuleList(
            Qwen2DecoderLayer(cfg, g, device, std, lora_std)
            for _ in range(cfg.num_hidden_layers))
        self.norm = Qwen2RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device)
        self.rotary_emb = Qwen2RotaryEmbedding(cfg, device)


class Qwen2ForCausalLM(nn.Module):
    def __init__(self, cfg: Qwen2Config, device=None, seed: int = 0, std: float = 0.02,
                 lora_std: float = 0.01):
        super().__init__()
        g = torch.Generator(device=device if device is not None else "cpu")
        g.manual_seed(seed)
        self.config = cfg
        self.model = Qwen2Model(cfg, g, device, std, lora_std)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False, device=device,
                                 dtype=torch.bfloat16)
        with torch.no_grad():
            self.lm_head.weight.copy_(
                (torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=device) * std)
                .to(torch.bfloat16))
        self.lm_head.weight.requires_grad_(False)
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.hidden_size = cfg.hidden_size
        self.head_dim = cfg.head_dim

    def weight_bytes(self) -> dict:
        """Bytes a decode step must read, per part (NF4 packed, absmax, LoRA, lm_head)."""
        nf4 = absmax = lora = 0
        for layer in self.model.layers:
            for st in (layer.self_attn.qkv, layer.mlp.gate_up):
                nf4 += st.packed.numel()
                absmax += st.absmax.numel() * 4
            for lin in (layer.self_attn.o_proj.base_layer, layer.mlp.down_proj):
                nf4 += lin.weight.numel()
                absmax += lin.weight.quant_state.absmax.numel() * 4
            for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
                m = getattr(layer.self_attn, name)
                lora += (m.lora_A.weight.numel() + m.lora_B.weight.numel()) * 2
                if m.base_layer.bias is not None:
                    lora += 0  # biases are counted with the activations (tiny)
        lm = self.lm_head.weight.numel() * 2
        return {"nf4": nf4, "absmax": absmax, "lora": lora, "lm_head": lm}


def build_random_model(cfg: Qwen2Config, device, seed: int = 0) -> Qwen2ForCausalLM:
    """Random-init NF4+LoRA model (weights N(0, 0.02) before NF4, LoRA N(0, 0.01))."""
    with torch.no_grad():
        return Qwen2ForCausalLM(cfg, device=device, seed=seed).eval()
