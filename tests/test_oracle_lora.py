"""CPU checks that pin the NF4+LoRA linear oracle.

* the closed-form known answer of the reference's ``tests/test_lora.py:69-91``
  (A = 0.1, B = 0.2, x = 1, r = 4, alpha = 8 -> + 0.2*(0.1*8)*4*2 per output);
* torch float64 ``F.linear`` on the dequantized weight plus the adapter term
  (an independent library routine) within the op's 1e-2 tolerance;
* the rounding points of ``lora_forward.py:246-257`` (bias added after the base
  sum is rounded to bf16).
"""

import numpy as np
import torch
import torch.nn.functional as F

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from oracle.lora_linear import nf4_lora_linear, nf4_weight_bf16
from oracle.nf4 import quantize_nf4

from conftest import rel_err, rng

TOL = 1e-2  # bf16 tolerance for the linear (north star: max rel err 1e-2)


def test_lora_closed_form_known_answer():
    k = n = 8
    r, alpha = 4, 8
    packed = np.full(n * k // 2, 0x77, np.uint8)  # code[7] = 0.0 everywhere: zero base weight
    absmax = np.ones(1, np.float32)
    x = f32_to_bf16_bits(np.ones((1, k)))
    a = f32_to_bf16_bits(np.full((r, k), 0.1))
    b = f32_to_bf16_bits(np.full((n, r), 0.2))
    y = bf16_bits_to_f32(nf4_lora_linear(x, packed, absmax, n, k, 64, a_bits=a, b_bits=b,
                                         scaling=alpha / r))
    expected = 0.2 * (0.1 * 8) * 4 * (alpha / r)  # = 1.28
    assert np.all(np.abs(y - expected) <= TOL * expected)
    bias = f32_to_bf16_bits(np.full(n, 0.5))
    y = bf16_bits_to_f32(nf4_lora_linear(x, packed, absmax, n, k, 64, bias_bits=bias, a_bits=a,
                                         b_bits=b, scaling=alpha / r))
    assert np.all(np.abs(y - (expected + 0.5)) <= TOL * (expected + 0.5))


def test_linear_matches_torch_float64():
    g = rng(20)
    for (m, n, k, r) in [(8, 256, 512, 16), (3, 64, 128, 4), (8, 96, 256, 0)]:
        w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
        packed, absmax = quantize_nf4(w, 64)
        x = f32_to_bf16_bits(g.standard_normal((m, k)))
        bias = f32_to_bf16_bits(g.standard_normal(n) * 0.02)
        a = f32_to_bf16_bits(g.standard_normal((r, k)) * 0.01) if r else None
        b = f32_to_bf16_bits(g.standard_normal((n, r)) * 0.01) if r else None
        y = bf16_bits_to_f32(nf4_lora_linear(x, packed, absmax, n, k, 64, bias_bits=bias,
                                             a_bits=a, b_bits=b, scaling=2.0))
        wd = torch.from_numpy(nf4_weight_bf16(packed, absmax, n, k, 64)).double()
        xt = torch.from_numpy(bf16_bits_to_f32(x)).double()
        ref = F.linear(xt, wd, torch.from_numpy(bf16_bits_to_f32(bias)).double())
        if r:
            at = torch.from_numpy(bf16_bits_to_f32(a)).double()
            bt = torch.from_numpy(bf16_bits_to_f32(b)).double()
            ref = ref + (xt @ at.T) @ bt.T * 2.0
        assert rel_err(y, ref.numpy()) <= TOL


def test_rounding_points_bias_after_base_round():
    # The base sum is rounded to bf16 BEFORE the bias add (lora_forward.py:246-251).
    # x = [1, 2^-8] . w = [1, 1] = 1 + 2^-8, a tie in bf16 (ulp 2^-7) -> 1.0 (even);
    # + bias 2^-8 -> another tie -> 1.0.  Adding the bias first would give
    # bf16(1 + 2^-7) = 1 + 2^-7.
    k = n = 64
    x = np.zeros((1, k), np.float32)
    x[0, 0], x[0, 1] = 1.0, 2.0 ** -8
    packed = np.full(n * k // 2, 0x77, np.uint8)
    packed[0] = 0xFF  # row 0: w[0,0] = w[0,1] = 1.0 (code 15 * absmax 1)
    absmax = np.ones(n * k // 64, np.float32)
    bias = f32_to_bf16_bits(np.full(n, 2.0 ** -8))
    y = bf16_bits_to_f32(nf4_lora_linear(f32_to_bf16_bits(x), packed, absmax, n, k, 64,
                                         bias_bits=bias))
    assert y[0, 0] == np.float32(1.0)
    assert float(round_bf16(np.float32(1 + 2.0 ** -7)).reshape(-1)[0]) == 1 + 2.0 ** -7


def _backward_case(g, m, n, k, r, scale_b=0.01):
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, 64)
    x = f32_to_bf16_bits(g.standard_normal((m, k)))
    a = f32_to_bf16_bits(g.standard_normal((r, k)) * 0.05)
    b = f32_to_bf16_bits(g.standard_normal((n, r)) * scale_b)
    gr = f32_to_bf16_bits(g.standard_normal((m, n)))
    return packed, absmax, x, a, b, gr


def test_backward_matches_torch_autograd_float64():
    """The oracle's gradients against torch.autograd of the same float64 linear
    (an independent differentiation): exact mode to float64 round-off, the
    bf16-rounded mode within the op's tolerance; scaling 2 and a bias make a
    dropped or misplaced term fail."""
    from oracle.lora_linear import nf4_lora_backward

    g = rng(31)
    for (m, n, k, r) in [(5, 64, 128, 4), (17, 96, 256, 16)]:
        packed, absmax, x, a, b, gr = _backward_case(g, m, n, k, r, scale_b=0.2)
        wd = torch.from_numpy(nf4_weight_bf16(packed, absmax, n, k, 64)).double()
        xt = torch.from_numpy(bf16_bits_to_f32(x)).double().requires_grad_()
        at = torch.from_numpy(bf16_bits_to_f32(a)).double().requires_grad_()
        bt = torch.from_numpy(bf16_bits_to_f32(b)).double().requires_grad_()
        bias = torch.zeros(n, dtype=torch.float64, requires_grad=True)
        y = F.linear(xt, wd, bias) + (xt @ at.T) @ bt.T * 2.0
        y.backward(torch.from_numpy(bf16_bits_to_f32(gr)).double())
        want = [xt.grad.numpy(), at.grad.numpy(), bt.grad.numpy(), bias.grad.numpy()]
        ex = nf4_lora_backward(gr, x, packed, absmax, n, k, 64, a, b, 2.0, has_bias=True,
                               exact=True)
        rd = nf4_lora_backward(gr, x, packed, absmax, n, k, 64, a, b, 2.0, has_bias=True)
        for e, q, wt in zip(ex, rd, want):
            assert np.abs(e - wt).max() <= 1e-10 * max(np.abs(wt).max(), 1.0)
            assert rel_err(q, wt) <= TOL


def test_backward_linearity_identities():
    """y is linear in x and in each of A, B: <g, y(x)> = <grad_x, x>,
    <g, y(A) - y(A = 0)> = <grad_A, A>, <g, y(B) - y(B = 0)> = <grad_B, B>, with y
    from the forward oracle (bf16-rounded) and g chosen along the signal so the
    rounding noise is small against it."""
    from oracle.lora_linear import nf4_lora_backward

    m, n, k, r, s = 9, 128, 256, 8, 2.0
    packed, absmax, x, a, b, _ = _backward_case(rng(32), m, n, k, r, scale_b=0.3)
    fwd = lambda aa, bb: bf16_bits_to_f32(nf4_lora_linear(
        x, packed, absmax, n, k, 64, a_bits=aa, b_bits=bb, scaling=s)).astype(np.float64)
    za, zb = np.zeros_like(a), np.zeros_like(b)
    y = fwd(a, b)
    dy_a, dy_b = y - fwd(za, b), y - fwd(a, zb)
    for sig, pick in ((y, 0), (dy_a, 1), (dy_b, 2)):
        gr = f32_to_bf16_bits(sig.astype(np.float32))
        grads = nf4_lora_backward(gr, x, packed, absmax, n, k, 64, a, b, s)
        lhs = float((bf16_bits_to_f32(gr).astype(np.float64) * sig).sum())
        var = (x, a, b)[pick]
        rhs = float((grads[pick].astype(np.float64) * bf16_bits_to_f32(var)).sum())
        assert abs(lhs - rhs) <= 2e-2 * abs(lhs), (pick, lhs, rhs)


# ---- float16 form (the reference kernel with X_DTYPE = LORA_DTYPE = float16)

def _f16(t):
    """float32 numpy -> torch float16 (torch's own rounding)."""
    return torch.from_numpy(np.asarray(t, np.float32)).to(torch.float16)


def test_dequant_f16_all_bytes_against_torch_rounding():
    """float16(code[q] * absmax) per element: the oracle's float16 dequantization
    equals torch's float32 product rounded by ``.to(torch.float16)`` for all
    256 bytes at scales across float16's range (overflow to inf, subnormals)."""
    from oracle.bf16 import f16_bits_to_f32
    from oracle.nf4 import NF4_CODE, dequantize_nf4

    packed = np.tile(np.arange(256, dtype=np.uint8), 8)
    absmax = np.array([0.0, 1e-6, 3e-5, 7e4, 1.0, 0.5, 123.456, 7e-3] * 8, np.float32)
    got = dequantize_nf4(packed, absmax, 4096, 64, dtype="f16")
    q = np.stack([packed >> 4, packed & 15], axis=1).reshape(-1)
    prod = torch.from_numpy(NF4_CODE[q]) * torch.from_numpy(np.repeat(absmax, 64))
    want = prod.to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.isinf(f16_bits_to_f32(got)).any()  # the 7e4 block overflows float16


def test_linear_f16_matches_torch_float16_ops():
    """The float16 oracle against the same linear spelled with torch's float16
    CPU ops (F.linear and elementwise ops each rounding to float16 -- an
    independent implementation of the rounding points): >= 99 % of outputs
    bit-identical, the rest one summation-order ulp away.  Rounding any step to
    bf16 instead would move most outputs."""
    from oracle.bf16 import f16_bits_to_f32, f32_to_f16_bits

    g = rng(40)
    for (m, n, k, r) in [(8, 256, 512, 16), (5, 96, 256, 8), (6, 64, 128, 0)]:
        w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
        packed, absmax = quantize_nf4(w, 64)
        x = f32_to_f16_bits(g.standard_normal((m, k)))
        bias = f32_to_f16_bits(g.standard_normal(n) * 0.02)
        a = f32_to_f16_bits(g.standard_normal((r, k)) * 0.01) if r else None
        b = f32_to_f16_bits(g.standard_normal((n, r)) * 0.01) if r else None
        got = nf4_lora_linear(x, packed, absmax, n, k, 64, bias_bits=bias, a_bits=a, b_bits=b,
                              scaling=2.0, dtype="f16")
        xt = _f16(f16_bits_to_f32(x))
        wt = _f16(nf4_weight_bf16(packed, absmax, n, k, 64, dtype="f16"))
        y = F.linear(xt, wt) + _f16(f16_bits_to_f32(bias))
        if r:
            t = F.linear(xt, _f16(f16_bits_to_f32(a)))
            u = F.linear(t, _f16(f16_bits_to_f32(b))) * torch.tensor(2.0, dtype=torch.float16)
            y = y + u
        want = y.view(torch.int16).numpy().view(np.uint16)
        assert np.mean(got == want) >= 0.99
        assert rel_err(f16_bits_to_f32(got), f16_bits_to_f32(want)) <= 2e-3


def test_backward_f16_matches_torch_float16_ops():
    """The float16 backward oracle against torch's float16 CPU ops at the same
    points (g @ W, g * s, @ B, @ A, x @ A^T, the weight gradients, Σ g):
    within 2e-3 of the larger value, >= 95 % bit-identical per tensor."""
    from oracle.bf16 import f16_bits_to_f32, f32_to_f16_bits
    from oracle.lora_linear import nf4_lora_backward

    g = rng(41)
    m, n, k, r = 9, 96, 256, 16
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, 64)
    x = f32_to_f16_bits(g.standard_normal((m, k)))
    a = f32_to_f16_bits(g.standard_normal((r, k)) * 0.05)
    b = f32_to_f16_bits(g.standard_normal((n, r)) * 0.2)
    gr = f32_to_f16_bits(g.standard_normal((m, n)))
    got = nf4_lora_backward(gr, x, packed, absmax, n, k, 64, a, b, 2.0, has_bias=True,
                            dtype="f16")
    gt, xt = _f16(f16_bits_to_f32(gr)), _f16(f16_bits_to_f32(x))
    at, bt = _f16(f16_bits_to_f32(a)), _f16(f16_bits_to_f32(b))
    wt = _f16(nf4_weight_bf16(packed, absmax, n, k, 64, dtype="f16"))
    sg = gt * torch.tensor(2.0, dtype=torch.float16)
    gi = sg @ bt
    grad_x = gt @ wt + gi @ at
    grad_a = gi.t() @ xt
    grad_b = sg.t() @ (xt @ at.t())
    grad_bias = gt.float().sum(0).half()
    for mine, ref in zip(got, (grad_x, grad_a, grad_b, grad_bias)):
        ref = ref.float().numpy()
        assert rel_err(mine, ref) <= 2e-3
        assert np.mean(np.float32(mine) == ref) >= 0.95
