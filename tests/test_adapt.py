"""CPU checks of the transformers-layout -> decode-engine adapter (rollout/adapt.py)."""

import numpy as np
import pytest
import torch

pytest.importorskip("transformers")

from hf_model import build_hf_nf4_lora_model  # noqa: E402


def test_adapter_stacks_qkv_and_gate_up_and_shares_adapters():
    from grpo_mi355x.rollout.adapt import decode_model_from

    hf = build_hf_nf4_lora_model(seed=0, layers=2)
    m = decode_model_from(hf)
    assert decode_model_from(hf) is m  # cached per model object
    c = m.config
    assert (c.hidden_size, c.num_attention_heads, c.num_key_value_heads, c.head_dim) == \
        (512, 4, 2, 128)
    assert (c.lora_rank, c.lora_alpha, c.nf4_blocksize, c.rope_theta) == (16, 32, 64, 1e6)
    for src, dst in zip(hf.model.layers, m.model.layers):
        at = src.self_attn
        qkv = dst.self_attn.qkv
        want = torch.cat([getattr(at, f"{n}_proj").base_layer.weight.reshape(-1)
                          for n in ("q", "k", "v")])
        assert torch.equal(qkv.packed, want)
        want_a = torch.cat([getattr(at, f"{n}_proj").base_layer.weight.quant_state.absmax
                            for n in ("q", "k", "v")])
        assert torch.equal(qkv.absmax, want_a)
        assert qkv.seg_rows == [512, 256, 256]
        lo, hi = qkv.packed.data_ptr(), qkv.packed.data_ptr() + qkv.packed.numel()
        for n in ("q", "k", "v"):
            v = getattr(dst.self_attn, f"{n}_proj")
            assert lo <= v.base_layer.weight.data_ptr() < hi
            s = getattr(at, f"{n}_proj")
            assert v.lora_A.weight.data_ptr() == s.lora_A.weight.data_ptr()
            assert v.lora_B.weight.data_ptr() == s.lora_B.weight.data_ptr()
            assert v.base_layer.bias.data_ptr() == s.base_layer.bias.data_ptr()
            assert v.scaling == 2.0 and v.rank == 16
        gu = dst.mlp.gate_up
        assert torch.equal(gu.packed, torch.cat([src.mlp.gate_proj.weight.reshape(-1),
                                                 src.mlp.up_proj.weight.reshape(-1)]))
        assert dst.mlp.down_proj is src.mlp.down_proj
        assert dst.self_attn.o_proj.base_layer is at.o_proj.base_layer


def test_adapter_rejects_what_the_kernels_cannot_run():
    # (nested absmax states are accepted: tests/test_gpu_nested.py)
    from grpo_mi355x.rollout.adapt import decode_model_from

    hf2 = build_hf_nf4_lora_model(seed=2, layers=1)
    hf2.model.layers[0].self_attn.o_proj = hf2.model.layers[0].self_attn.o_proj.base_layer
    with pytest.raises(ValueError, match="LoRA"):
        decode_model_from(hf2)


def test_engine_layout_model_is_returned_unchanged():
    from grpo_mi355x.rollout.adapt import decode_model_from
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    m = build_random_model(Qwen2Config.tiny(layers=1, inter=256, vocab=64), "cpu")
    assert decode_model_from(m) is m
