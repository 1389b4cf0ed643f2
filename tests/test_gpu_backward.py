"""Backward of the fused NF4 + LoRA linear (FusedLoRAFunction.backward,
src/triton_kernels/lora_forward.py:761-930) against the oracle.

``grpo_nf4_grad_x`` (the NF4 part of grad_x for fewer than 1024 rows,
reduction over the N output features) is compared with the oracle's bf16(g @ W) directly: the two differ
only in float32 summation order, so the bar is one bf16 ulp of max|x| (8e-3)
with >= 95 % of elements bit-identical.  Through autograd, grad_x, grad_A,
grad_B and grad_bias of ``lora_fused_forward`` are within 1e-2 of max|x| of
the oracle's gradients, shapes ragged in M, and the forward output within
1e-2 of the oracle's on both of its paths (split-K kernel up to 64 rows,
dequantize + bf16 GEMMs beyond).
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.lora_linear import nf4_lora_backward, nf4_lora_linear, nf4_weight_bf16
from oracle.nf4 import NF4_CODE, quantize_nf4

from conftest import rel_err
from model_export import bits

pytestmark = pytest.mark.gpu


def _t(b, dev):
    return torch.from_numpy(np.asarray(b).astype(np.int16)).view(torch.bfloat16).to(dev)


@pytest.mark.parametrize("m,n,k", [(1, 256, 512), (77, 1536, 256), (200, 96, 1536),
                                   (64, 8960, 128)])
def test_nf4_grad_x_matches_oracle(dev, m, n, k):
    from grpo_mi355x.kernels import ops

    g = np.random.default_rng(m + n + k)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, 64)
    gr = f32_to_bf16_bits(g.standard_normal((m, n)))
    add = f32_to_bf16_bits(g.standard_normal((m, k)) * 0.05)
    print(f"nf4_grad_x M={m} N={n} K={k}", flush=True)
    args = (_t(gr, dev), torch.from_numpy(packed).to(dev), torch.from_numpy(absmax).to(dev),
            torch.from_numpy(NF4_CODE).to(dev), 64, n, k)
    got = bits(ops.nf4_grad_x(*args))
    wf = nf4_weight_bf16(packed, absmax, n, k, 64).astype(np.float64)
    ref = f32_to_bf16_bits((bf16_bits_to_f32(gr).astype(np.float64) @ wf).astype(np.float32))
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(ref)) <= 8e-3
    assert np.mean(got == ref) >= 0.95
    # the addend is added to the bf16-rounded product and rounded once more
    got2 = bits(ops.nf4_grad_x(*args, addend=_t(add, dev)))
    want2 = f32_to_bf16_bits(bf16_bits_to_f32(got) + bf16_bits_to_f32(add))
    assert np.array_equal(got2, want2)


@pytest.mark.parametrize("m,n,k,r", [(37, 256, 512, 16), (130, 1536, 256, 8),
                                     (1100, 256, 512, 16),   # dequant + GEMM (rows)
                                     (37, 72, 200, 16)])     # dequant + GEMM (shape)
def test_fused_lora_backward_matches_oracle(dev, m, n, k, r):
    from grpo_mi355x.core.nf4 import Linear4bitNF4
    from grpo_mi355x.kernels import lora_fused_forward

    g = np.random.default_rng(7 * m + r)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    base = Linear4bitNF4.from_weight(torch.from_numpy(w).to(dev), bias=torch.from_numpy(
        (g.standard_normal(n) * 0.02).astype(np.float32)).to(dev), blocksize=64)
    base.bias.requires_grad_(True)
    x_b = f32_to_bf16_bits(g.standard_normal((m, k)))
    a_b = f32_to_bf16_bits(g.standard_normal((r, k)) * 0.05)
    b_b = f32_to_bf16_bits(g.standard_normal((n, r)) * 0.05)
    g_b = f32_to_bf16_bits(g.standard_normal((m, n)))
    x = _t(x_b, dev).view(1, m, k).requires_grad_()
    a = _t(a_b, dev).requires_grad_()
    b = _t(b_b, dev).requires_grad_()
    print(f"fused NF4+LoRA backward M={m} N={n} K={k} r={r}", flush=True)
    y = lora_fused_forward(x, base_layer=base, lora_A=a, lora_B=b, scaling=2.0)
    y.backward(_t(g_b, dev).view(1, m, n))
    qs = base.weight.quant_state
    packed = base.weight.data.view(torch.uint8).cpu().numpy().reshape(-1)
    # forward: the split-K kernel (M <= 64) or dequantize + bf16 GEMMs
    y_ref = nf4_lora_linear(x_b, packed, qs.absmax.cpu().numpy(), n, k, 64,
                            bias_bits=bits(base.bias.detach()), a_bits=a_b, b_bits=b_b,
                            scaling=2.0)
    ey = rel_err(bf16_bits_to_f32(bits(y.detach().view(m, n))), bf16_bits_to_f32(y_ref))
    print(f"forward: rel err {ey:.2e}", flush=True)
    assert ey <= 1e-2
    want = nf4_lora_backward(g_b, x_b, packed, qs.absmax.cpu().numpy(), n, k, 64, a_b, b_b,
                             2.0, has_bias=True)
    got = [x.grad.view(m, k), a.grad, b.grad, base.bias.grad]
    for name, gg, ww in zip(("x", "A", "B", "bias"), got, want):
        assert gg is not None, name
        e = rel_err(bf16_bits_to_f32(bits(gg)), ww)
        print(f"grad_{name}: rel err {e:.2e}", flush=True)
        assert e <= 1e-2, name


@pytest.mark.parametrize("m", [48, 1500])
def test_manual_lora_layer_trains_through_the_fused_function(dev, m):
    """ManualLoRALayer (src/core/lora.py:50-163) on the fused path: its
    gradients for x, lora_A and lora_B equal, within 1e-2 of max|x|, those of
    the same layer on the PyTorch branch (use_triton=False: dequantized base
    linear + nn.Linear LoRA, autograd through torch)."""
    from grpo_mi355x.core.lora import ManualLoRALayer
    from grpo_mi355x.core.nf4 import Linear4bitNF4

    torch.manual_seed(m)
    k, n = 512, 1536
    base = Linear4bitNF4.from_weight(torch.randn(n, k, device=dev) * 0.02,
                                     bias=torch.randn(n, device=dev) * 0.02, blocksize=64)
    layers = [ManualLoRALayer(base, rank=16, alpha=32, use_triton=t).to(dev).to(torch.bfloat16)
              for t in (True, False)]
    with torch.no_grad():
        layers[0].lora_A.weight.normal_(0, 0.05)
        layers[0].lora_B.weight.normal_(0, 0.05)
        for name in ("lora_A", "lora_B"):
            getattr(layers[1], name).weight.copy_(getattr(layers[0], name).weight)
    x0 = torch.randn(1, m, k, device=dev).to(torch.bfloat16)
    gr = torch.randn(1, m, n, device=dev).to(torch.bfloat16)
    grads = []
    print(f"ManualLoRALayer backward, fused vs PyTorch branch, M={m}", flush=True)
    for layer in layers:
        x = x0.clone().requires_grad_()
        layer(x).backward(gr)
        grads.append([x.grad, layer.lora_A.weight.grad, layer.lora_B.weight.grad])
    for name, a, b in zip(("x", "A", "B"), grads[0], grads[1]):
        e = rel_err(a.float().cpu().numpy(), b.float().cpu().numpy())
        print(f"grad_{name}: rel err {e:.2e}", flush=True)
        assert e <= 1e-2, name
