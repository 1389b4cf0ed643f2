"""GPU parity of the float16 form of the fused NF4 + LoRA linear: the
reference's ``_lora_forward_kernel`` with X_DTYPE = LORA_DTYPE = float16
(src/triton_kernels/lora_forward.py:141-143, 745-749) and its backward
(``:761-930``, W cast to the gradient's float16, ``:343``).

* ``grpo_nf4_dequant_f16`` equals the oracle's float16(code * absmax) bit for bit;
* ``grpo_nf4_gemm_f16`` (through ``ops.nf4_lora_linear`` with float16 tensors)
  is within 1e-2 of max|y| of the float16 oracle and bit-identical on >= 98 %
  of outputs (only the float32 summation order differs);
* ``lora_fused_forward`` on float16 inputs: forward and the four gradients
  within 1e-2 of the oracle's float16 forward and backward, on the GEMM and on
  the dequantize + GEMM path;
* ``ManualLoRALayer`` in float16 trains through the fused function with the
  gradients of its PyTorch branch.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import f16_bits_to_f32, f32_to_f16_bits
from oracle.lora_linear import nf4_lora_backward, nf4_lora_linear
from oracle.nf4 import NF4_CODE, dequantize_nf4, quantize_nf4

from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _h(b, dev):
    """float16 bit patterns (numpy uint16) -> torch float16 on dev."""
    return torch.from_numpy(np.asarray(b).astype(np.uint16).view(np.int16)).view(
        torch.float16).to(dev)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _code(dev):
    return torch.from_numpy(NF4_CODE.copy()).to(dev)


@pytest.mark.parametrize("numel,bs", [(64 * 1000, 64), (4096, 128), (100_001, 64)])
def test_dequant_f16_bit_exact(dev, numel, bs):
    from grpo_mi355x.kernels import ops

    g = np.random.default_rng(numel)
    packed = g.integers(0, 256, (numel + 1) // 2).astype(np.uint8)
    absmax = (np.abs(g.standard_normal(-(-numel // bs))) * 0.05).astype(np.float32)
    absmax[::7] = 0.0
    out = ops.nf4_dequant(torch.from_numpy(packed).to(dev), torch.from_numpy(absmax).to(dev),
                          _code(dev), numel, bs, dtype=torch.float16)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), dequantize_nf4(packed, absmax, numel, bs, dtype="f16"))


def _case(seed, m, n, k, r, with_bias, bs=64):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    return dict(x=f32_to_f16_bits(g.standard_normal((m, k))), packed=packed, absmax=absmax,
                bias=f32_to_f16_bits(g.standard_normal(n) * 0.02) if with_bias else None,
                a=f32_to_f16_bits(g.standard_normal((r, k)) * 0.01) if r else None,
                b=f32_to_f16_bits(g.standard_normal((n, r)) * 0.01) if r else None,
                m=m, n=n, k=k, r=r, bs=bs)


@pytest.mark.parametrize("m,n,k,r,with_bias", [
    (1, 256, 512, 16, True),      # one decode row
    (8, 1536, 1536, 16, True),    # q_proj at a decode batch
    (65, 1024, 1024, 16, False),
    (300, 256, 512, 32, True),    # two rank tiles
    (130, 200, 96, 5, True),      # ragged N, K % 128 != 0, r % 8 != 0
    (512, 8960, 1536, 0, False),  # gate at a prefill chunk, no LoRA
])
def test_gemm_f16_matches_oracle(dev, m, n, k, r, with_bias):
    from grpo_mi355x.kernels import ops

    c = _case(5 * m + n + k + r, m, n, k, r, with_bias)
    print(f"float16 NF4 GEMM m={m} n={n} k={k} r={r}", flush=True)
    y = ops.nf4_lora_linear(
        _h(c["x"], dev), torch.from_numpy(c["packed"]).to(dev),
        torch.from_numpy(c["absmax"]).to(dev), _code(dev), c["bs"], n,
        bias=None if c["bias"] is None else _h(c["bias"], dev),
        lora_a=None if c["a"] is None else _h(c["a"], dev),
        lora_b=None if c["b"] is None else _h(c["b"], dev), scaling=2.0)
    torch.cuda.synchronize()
    assert y.dtype == torch.float16
    got = _bits(y)
    ref = nf4_lora_linear(c["x"], c["packed"], c["absmax"], n, k, c["bs"], bias_bits=c["bias"],
                          a_bits=c["a"], b_bits=c["b"], scaling=2.0, dtype="f16")
    gf, rf = f16_bits_to_f32(got), f16_bits_to_f32(ref)
    assert np.all(np.isfinite(gf))
    assert rel_err(gf, rf) <= TOL
    assert np.mean(got == ref) >= 0.98


@pytest.mark.parametrize("m,n,k,r", [(37, 256, 512, 16),      # the NF4 GEMM
                                     (4200, 256, 512, 16)])   # dequantize + GEMM (rows)
def test_fused_lora_f16_forward_backward_matches_oracle(dev, m, n, k, r):
    from grpo_mi355x.core.nf4 import Linear4bitNF4
    from grpo_mi355x.kernels import lora_fused_forward

    g = np.random.default_rng(11 * m + r)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    bias32 = (g.standard_normal(n) * 0.02).astype(np.float32)
    base = Linear4bitNF4.from_weight(torch.from_numpy(w).to(dev),
                                     bias=torch.from_numpy(bias32).to(dev), blocksize=64)
    base.bias.requires_grad_(True)
    x_h = f32_to_f16_bits(g.standard_normal((m, k)))
    a_h = f32_to_f16_bits(g.standard_normal((r, k)) * 0.05)
    b_h = f32_to_f16_bits(g.standard_normal((n, r)) * 0.05)
    g_h = f32_to_f16_bits(g.standard_normal((m, n)))
    x = _h(x_h, dev).view(1, m, k).requires_grad_()
    a = _h(a_h, dev).requires_grad_()
    b = _h(b_h, dev).requires_grad_()
    print(f"float16 fused NF4+LoRA M={m} N={n} K={k} r={r}", flush=True)
    y = lora_fused_forward(x, base_layer=base, lora_A=a, lora_B=b, scaling=2.0)
    assert y.dtype == torch.float16
    y.backward(_h(g_h, dev).view(1, m, n))
    qs = base.weight.quant_state
    packed = base.weight.data.view(torch.uint8).cpu().numpy().reshape(-1)
    absmax = qs.absmax.cpu().numpy()
    bias_h = _bits(base.bias.detach().to(torch.float16))  # the reference's bias.to(x.dtype)
    y_ref = nf4_lora_linear(x_h, packed, absmax, n, k, 64, bias_bits=bias_h, a_bits=a_h,
                            b_bits=b_h, scaling=2.0, dtype="f16")
    ey = rel_err(f16_bits_to_f32(_bits(y.view(m, n))), f16_bits_to_f32(y_ref))
    print(f"forward: rel err {ey:.2e}", flush=True)
    assert ey <= TOL
    want = nf4_lora_backward(g_h, x_h, packed, absmax, n, k, 64, a_h, b_h, 2.0, has_bias=True,
                             dtype="f16")
    got = [x.grad.view(m, k), a.grad, b.grad, base.bias.grad]
    for name, gg, ww in zip(("x", "A", "B", "bias"), got, want):
        assert gg is not None, name
        e = rel_err(gg.float().cpu().numpy(), ww)
        print(f"grad_{name}: rel err {e:.2e}", flush=True)
        assert e <= TOL, name


def test_manual_lora_layer_f16_trains_through_the_fused_function(dev):
    """ManualLoRALayer (src/core/lora.py:50-163) in float16: the fused path's
    gradients for x, lora_A and lora_B equal, within 1e-2 of max|x|, those of
    its PyTorch branch (use_triton=False)."""
    from grpo_mi355x.core.lora import ManualLoRALayer
    from grpo_mi355x.core.nf4 import Linear4bitNF4

    torch.manual_seed(3)
    m, k, n = 96, 512, 1536
    base = Linear4bitNF4.from_weight(torch.randn(n, k, device=dev) * 0.02,
                                     bias=torch.randn(n, device=dev) * 0.02, blocksize=64)
    layers = [ManualLoRALayer(base, rank=16, alpha=32, use_triton=t).to(dev).to(torch.float16)
              for t in (True, False)]
    with torch.no_grad():
        layers[0].lora_A.weight.normal_(0, 0.05)
        layers[0].lora_B.weight.normal_(0, 0.05)
        for name in ("lora_A", "lora_B"):
            getattr(layers[1], name).weight.copy_(getattr(layers[0], name).weight)
    x0 = torch.randn(1, m, k, device=dev).to(torch.float16)
    gr = torch.randn(1, m, n, device=dev).to(torch.float16)
    grads, outs = [], []
    print(f"float16 ManualLoRALayer, fused vs PyTorch branch, M={m}", flush=True)
    for layer in layers:
        x = x0.clone().requires_grad_()
        y = layer(x)
        outs.append(y.detach())
        y.backward(gr)
        grads.append([x.grad, layer.lora_A.weight.grad, layer.lora_B.weight.grad])
    assert outs[0].dtype == torch.float16
    assert rel_err(outs[0].float().cpu().numpy(), outs[1].float().cpu().numpy()) <= TOL
    for name, a, b in zip(("x", "A", "B"), grads[0], grads[1]):
        e = rel_err(a.float().cpu().numpy(), b.float().cpu().numpy())
        print(f"grad_{name}: rel err {e:.2e}", flush=True)
        assert e <= TOL, name
