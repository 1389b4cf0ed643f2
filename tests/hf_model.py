"""A transformers Qwen2ForCausalLM in the reference's training layout (tests only).

NF4 base weights on every decoder linear (as ``load_in_4bit`` leaves the
model, ``src/core/model_loader.py:15-20``) and ``ManualLoRALayer`` adapters on
q/k/v/o (``inject_lora_layers``, ``src/core/lora.py:166-233``), with non-zero
LoRA B so that the adapter term is observable.
"""

from __future__ import annotations

import torch


def build_hf_nf4_lora_model(seed: int = 0, layers: int = 2, device="cpu", hidden: int = 512,
                            heads: int = 4, kv_heads: int = 2, head_dim: int = 128,
                            inter: int = 1024, vocab: int = 1000):
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2ForCausalLM

    from grpo_mi355x.core.lora import ManualLoRALayer, inject_lora_layers
    from grpo_mi355x.core.nf4 import Linear4bitNF4

    cfg = Qwen2Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                      num_hidden_layers=layers, num_attention_heads=heads,
                      num_key_value_heads=kv_heads, head_dim=head_dim, rms_norm_eps=1e-6,
                      rope_theta=1_000_000.0, tie_word_embeddings=False,
                      max_position_embeddings=4096)
    torch.manual_seed(seed)
    hf = Qwen2ForCausalLM(cfg).to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for layer in hf.model.layers:
            for n in (layer.input_layernorm, layer.post_attention_layernorm):
                n.weight.add_((0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16))
            for parent, names in ((layer.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                                  (layer.mlp, ("gate_proj", "up_proj", "down_proj"))):
                for n in names:
                    lin = getattr(parent, n)
                    w = torch.randn(lin.weight.shape, generator=g) * 0.02
                    bias = None
                    if lin.bias is not None:
                        bias = (torch.randn(lin.bias.shape, generator=g) * 0.02)
                    setattr(parent, n, Linear4bitNF4.from_weight(w, bias, 64))
        inject_lora_layers(hf, ["q_proj", "k_proj", "v_proj", "o_proj"], rank=16, alpha=32,
                           verbose=False)
        for m in hf.modules():
            if isinstance(m, ManualLoRALayer):
                m.lora_A.weight.copy_(torch.randn(m.lora_A.weight.shape, generator=g) * 0.01)
                m.lora_B.weight.copy_(torch.randn(m.lora_B.weight.shape, generator=g) * 0.01)
    return hf.to(device)
