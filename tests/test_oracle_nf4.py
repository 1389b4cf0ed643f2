"""CPU checks that pin the NF4 oracle (codebook, bf16 rounding, dequant layout).

Each check is chosen so that a plausible mistake fails it: a swapped nibble
order fails the known-answer bytes; an off-by-one block index fails the block
boundary test; truncation instead of round-to-nearest-even fails the torch
rounding comparison; a wrong code constant fails the closed form.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.nf4 import NF4_CODE, dequantize_nf4, nf4_code_closed_form, nibbles, quantize_nf4

from conftest import rng


def test_nf4_code_matches_closed_form():
    cf = nf4_code_closed_form()
    assert np.abs(cf - NF4_CODE).max() <= 2e-7


def test_nf4_code_invariants():
    assert NF4_CODE[0] == -1.0 and NF4_CODE[7] == 0.0 and NF4_CODE[15] == 1.0
    assert np.all(np.diff(NF4_CODE) > 0)
    assert NF4_CODE.dtype == np.float32 and NF4_CODE.size == 16


def test_bf16_rounding_matches_torch():
    g = rng(0)
    x = np.concatenate([
        g.standard_normal(100000).astype(np.float32) * 10.0 ** g.integers(-30, 30, 100000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0, 1.00390625, 1.01171875, 3.4e38, 1e-40, -1e-41],
                 dtype=np.float32),
    ]).astype(np.float32)
    # exact ties (low 16 bits == 0x8000) exercise round-half-to-even
    ties = (g.integers(0, 2**31, 5000).astype(np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, ties.view(np.float32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    ours = f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_dequant_known_answer_nibble_order():
    absmax = np.array([2.0], dtype=np.float32)
    # byte 0x0F: element 0 = high nibble 0 -> code[0] = -1; element 1 = low nibble 15 -> +1
    out = bf16_bits_to_f32(dequantize_nf4(np.array([0x0F], np.uint8), absmax, 2, 64))
    assert out.tolist() == [-2.0, 2.0]
    # byte 0x7F: high nibble 7 -> 0.0; low nibble 15 -> 1.0
    out = bf16_bits_to_f32(dequantize_nf4(np.array([0x7F], np.uint8), absmax, 2, 64))
    assert out.tolist() == [0.0, 2.0]


def test_dequant_block_boundaries():
    # 192 elements, blocksize 64, absmax 1,2,4 per block; every byte = 0xFF (code 1.0)
    packed = np.full(96, 0xFF, np.uint8)
    absmax = np.array([1.0, 2.0, 4.0], np.float32)
    out = bf16_bits_to_f32(dequantize_nf4(packed, absmax, 192, 64))
    assert np.all(out[:64] == 1.0) and np.all(out[64:128] == 2.0) and np.all(out[128:] == 4.0)
    # odd numel: the last element is the high nibble of the last byte
    out = bf16_bits_to_f32(dequantize_nf4(np.array([0xF0, 0x0F], np.uint8), absmax[:1], 3, 64))
    assert out.tolist() == [1.0, -1.0, -1.0]


def test_dequant_all_bytes_against_torch_rounding():
    g = rng(1)
    packed = np.arange(256, dtype=np.uint8)
    for absmax_v in g.standard_normal(8).astype(np.float32) * 3:
        absmax = np.array([absmax_v] * 8, np.float32)
        ours = dequantize_nf4(packed, absmax, 512, 64)
        hi = torch.tensor(NF4_CODE)[torch.arange(256) >> 4]
        lo = torch.tensor(NF4_CODE)[torch.arange(256) & 15]
        vals = torch.stack([hi, lo], 1).reshape(-1) * torch.tensor(absmax_v)
        ref = vals.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(ours, ref)


def test_quantize_roundtrip_error_bound():
    g = rng(2)
    w = (g.standard_normal((64, 256)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, 64)
    deq = bf16_bits_to_f32(dequantize_nf4(packed, absmax, w.size, 64)).reshape(w.shape)
    gap = np.diff(NF4_CODE).max() / 2
    bound = np.repeat(absmax, 64).reshape(w.shape) * (gap + 2 ** -8) + 1e-12
    assert np.all(np.abs(deq - w) <= bound)
    # the nearest code is chosen: every element's code is optimal up to ties
    q = nibbles(packed, w.size).reshape(w.shape)
    a = np.repeat(absmax, 64).reshape(w.shape)
    err = np.abs(NF4_CODE[q] - w / a)
    best = np.abs(NF4_CODE[None, None, :] - (w / a)[..., None]).min(-1)
    assert np.all(err <= best + 1e-6)


def test_quantize_zero_block():
    packed, absmax = quantize_nf4(np.zeros(128, np.float32), 64)
    assert np.all(absmax == 0)
    out = dequantize_nf4(packed, absmax, 128, 64)
    assert np.all(bf16_bits_to_f32(out) == 0)


def test_product_quantizer_matches_oracle_bytes():
    """The product's torch quantizer emits the oracle's bytes (same input)."""
    from grpo_mi355x.core.nf4 import NF4_CODE_VALUES, quantize_nf4 as q_prod

    assert np.array_equal(np.array(NF4_CODE_VALUES, np.float32), NF4_CODE)
    g = rng(3)
    for shape, bs in [((96, 512), 64), ((16, 1536), 128), ((7, 9), 64)]:
        w = (g.standard_normal(shape) * 0.02).astype(np.float32)
        p_or, a_or = quantize_nf4(w, bs)
        p_pr, st = q_prod(torch.from_numpy(w), bs)
        assert np.array_equal(p_pr.numpy().reshape(-1), p_or)
        assert np.array_equal(st.absmax.numpy(), a_or)
        assert tuple(st.shape) == shape and st.blocksize == bs and not st.nested


@pytest.mark.parametrize("numel", [1, 2, 63, 64, 65, 1000])
def test_dequant_shapes(numel):
    g = rng(numel)
    packed = g.integers(0, 256, (numel + 1) // 2).astype(np.uint8)
    absmax = g.random(-(-numel // 64)).astype(np.float32)
    out = dequantize_nf4(packed, absmax, numel, 64)
    assert out.shape == (numel,) and out.dtype == np.uint16


def test_blocked_dequant_equals_elementwise():
    from oracle.nf4 import _dequantize_blocked

    g = rng(9)
    for numel, bs in [(64 * 37, 64), (128 * 5, 128), (256 * 3, 256)]:
        packed = g.integers(0, 256, numel // 2).astype(np.uint8)
        absmax = (g.random(numel // bs) * 3).astype(np.float32)
        q = nibbles(packed, numel)
        ref = f32_to_bf16_bits(NF4_CODE[q] * np.repeat(absmax, bs))
        assert np.array_equal(_dequantize_blocked(packed, absmax, numel, bs, NF4_CODE), ref)
        assert np.array_equal(dequantize_nf4(packed, absmax, numel, bs), ref)


def test_nested_absmax_rounds_once_and_bounds_the_error():
    """nested_absmax = code2[q] * absmax2 + offset rounded once: the nearest
    float32 of the exact value (rational arithmetic); bitsandbytes' two
    roundings differ from it by at most the product's rounding; the double
    quantization keeps
    each scale within half a step of the 256-entry code of its block."""
    from fractions import Fraction

    from oracle import nf4

    rng = np.random.default_rng(11)
    a = rng.uniform(1e-3, 0.3, 4000).astype(np.float32)
    q, c2, a2, off = nf4.quantize_absmax_nested(a, 256)
    got = nf4.nested_absmax(q, c2, a2, 256, off)
    for i in range(0, 4000, 7):
        exact = Fraction(float(c2[q[i]])) * Fraction(float(a2[i // 256])) + Fraction(float(off))
        x = got[i]
        lo = np.nextafter(x, np.float32(-np.inf))
        hi = np.nextafter(x, np.float32(np.inf))
        d = abs(Fraction(float(x)) - exact)
        assert d <= abs(Fraction(float(lo)) - exact) and d <= abs(Fraction(float(hi)) - exact)
    two = nf4.nested_absmax_two_roundings(q, c2, a2, 256, off)
    prod = np.abs(c2[q].astype(np.float64) * a2[np.arange(4000) // 256])
    # the product's rounding (<= 2^-24 of it) plus the two final roundings
    bound = 2.0 ** -24 * prod + 2.0 ** -23 * np.abs(got.astype(np.float64))
    assert np.all(np.abs(got.astype(np.float64) - two) <= bound)
    assert np.mean(got == two) > 0.5
    step = a2[np.arange(4000) // 256] * np.float32(2.0 / 255)
    assert np.all(np.abs(got - a) <= step / 2 * 1.001 + 1e-7)
