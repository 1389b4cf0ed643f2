"""Double-quantized (nested) NF4 states: the reference trainer's default
(``bnb_4bit_use_double_quant=True``, src/core/model_loader.py:19).  Their uint8
absmax expands on the device to float32 as the reference kernel computes it
(lora_forward.py:187-199, one rounding); every consumer then sees exactly the
scales of a plain state holding the expanded values."""

import numpy as np
import pytest
import torch

from oracle import nf4 as O

pytestmark = pytest.mark.gpu


def _nest(qs, bs2=256):
    """Replace a plain state's float32 absmax by its nested form, in place;
    returns the float32 absmax the expansion must give (oracle)."""
    from grpo_mi355x.core.nf4 import QuantState

    a = qs.absmax.float().cpu().numpy()
    q, c2, a2, off = O.quantize_absmax_nested(a, bs2)
    dev = qs.absmax.device
    qs.absmax = torch.from_numpy(q).to(dev)
    qs.state2 = QuantState(torch.from_numpy(a2).to(dev), (a2.size,),
                           torch.from_numpy(c2).to(dev), bs2, dtype=torch.float32)
    qs.offset = torch.tensor(float(off), device=dev)
    qs.nested = True
    return O.nested_absmax(q, c2, a2, bs2, off)


def test_absmax_expansion_bit_exact(dev):
    from grpo_mi355x.kernels import ops

    rng = np.random.default_rng(3)
    a = rng.uniform(1e-3, 0.3, 100_003).astype(np.float32)
    q, c2, a2, off = O.quantize_absmax_nested(a, 256)
    print("nested absmax expansion: 100003 blocks", flush=True)
    got = ops.nf4_absmax_expand(torch.from_numpy(q).to(dev), torch.from_numpy(c2).to(dev),
                                torch.from_numpy(a2).to(dev), 256, float(off))
    want = O.nested_absmax(q, c2, a2, 256, off)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_nested_linear_equals_expanded_plain_state(dev):
    """The fused NF4 + LoRA linear and the dequantize of a nested state equal
    those of a plain state holding the oracle's expanded absmax, bit for bit."""
    from hf_model import build_hf_nf4_lora_model

    from grpo_mi355x.kernels import lora_fused_forward

    a = build_hf_nf4_lora_model(seed=5, layers=1, device=dev)
    b = build_hf_nf4_lora_model(seed=5, layers=1, device=dev)
    la, lb = a.model.layers[0].self_attn.q_proj, b.model.layers[0].self_attn.q_proj
    want = _nest(la.base_layer.weight.quant_state)
    lb.base_layer.weight.quant_state.absmax = torch.from_numpy(want).to(dev)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 8, 512, generator=g).to(torch.bfloat16).to(dev)
    print("nested q_proj [512, 512] + LoRA, 8 rows", flush=True)
    ya = lora_fused_forward(x, lora_layer=la)
    yb = lora_fused_forward(x, lora_layer=lb)
    assert torch.equal(ya, yb)
    wa = la.base_layer.dequantize()
    assert torch.equal(wa, lb.base_layer.dequantize())
    qs = la.base_layer.weight.quant_state
    nested = dict(code=qs.state2.code.cpu().numpy(), absmax=qs.state2.absmax.cpu().numpy(),
                  blocksize=256, offset=float(qs.offset))
    ref = O.dequantize_nf4(la.base_layer.weight.data.cpu().numpy().reshape(-1),
                           qs.absmax.cpu().numpy(), 512 * 512, 64, nested=nested)
    assert np.array_equal(wa.view(torch.int16).cpu().numpy().reshape(-1).view(np.uint16), ref)


def test_nested_model_decodes_like_its_expanded_twin(dev):
    """The trainer's call (trainer.py:389-400) on a transformers model whose every
    NF4 state is nested gives the tokens of the same model with plain states
    holding the expanded scales."""
    from hf_model import build_hf_nf4_lora_model

    from grpo_mi355x.core.nf4 import Linear4bitNF4
    from grpo_mi355x.kernels import paged_kv_decode

    a = build_hf_nf4_lora_model(seed=6, layers=2, device=dev)
    b = build_hf_nf4_lora_model(seed=6, layers=2, device=dev)
    mods_b = dict(b.named_modules())
    n = 0
    for name, mod in a.named_modules():
        if isinstance(mod, Linear4bitNF4):
            want = _nest(mod.weight.quant_state)
            mods_b[name].weight.quant_state.absmax = torch.from_numpy(want).to(dev)
            n += 1
    assert n == 14
    rng = np.random.default_rng(8)
    ids = torch.tensor([rng.integers(0, 1000, 17).tolist()] * 4, device=dev)
    kw = dict(attention_mask=torch.ones_like(ids), max_new_tokens=6, do_sample=False,
              pad_token_id=0, eos_token_id=None, use_cache=True)
    print("nested transformers Qwen2 decode: 2 layers, 4 rows", flush=True)
    ta = paged_kv_decode(a, input_ids=ids, **kw)
    tb = paged_kv_decode(b, input_ids=ids, **kw)
    assert torch.equal(ta, tb)
