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
