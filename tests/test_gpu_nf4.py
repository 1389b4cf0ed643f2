"""GPU parity: NF4 dequant (bit-exact) and the fused NF4+LoRA linear (bf16 tolerance).

All calls go through libgrpo_hip.so's C ABI (ctypes).  Tolerance for the linear:
``max|y - y_ref| <= 1e-2 * max|y_ref|`` (north star: max rel err 1e-2, fp32
accumulation); in addition the fast path must be bit-identical to the oracle on
>= 98% of outputs (its products equal the reference's ``bf16(code*absmax)*x``
exactly; only the float32 summation order differs).
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.lora_linear import nf4_lora_linear as ref_linear
from oracle.nf4 import NF4_CODE, dequantize_nf4, quantize_nf4

from conftest import from_bf16, rel_err, rng, to_dev_bf16

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _ops():
    from grpo_mi355x.kernels import ops

    return ops


def _code(dev):
    return torch.from_numpy(NF4_CODE.copy()).to(dev)


@pytest.mark.parametrize("numel,bs", [(1, 64), (33, 64), (64 * 1000, 64), (4096, 128),
                                      (3 * 4096, 256), (1536 * 1536, 64), (100_001, 64),
                                      (8960 * 1536, 64)])
def test_dequant_bit_exact(dev, numel, bs):
    g = rng(numel + bs)
    packed = g.integers(0, 256, (numel + 1) // 2).astype(np.uint8)
    absmax = (np.abs(g.standard_normal(-(-numel // bs))) * 0.05).astype(np.float32)
    absmax[::7] = 0.0
    out = _ops().nf4_dequant(torch.from_numpy(packed).to(dev), torch.from_numpy(absmax).to(dev),
                             _code(dev), numel, bs)
    torch.cuda.synchronize()
    assert np.array_equal(from_bf16(out), dequantize_nf4(packed, absmax, numel, bs))


def test_dequant_all_bytes_extreme_scales(dev):
    packed = np.tile(np.arange(256, dtype=np.uint8), 8)  # 4096 elements, 64 blocks
    absmax = np.array([0.0, 1e-38, 1e-30, 3e38, 1.0, 0.5, 123.456, 7e-3] * 8, np.float32)
    out = _ops().nf4_dequant(torch.from_numpy(packed).to(dev), torch.from_numpy(absmax).to(dev),
                             _code(dev), 4096, 64)
    torch.cuda.synchronize()
    assert np.array_equal(from_bf16(out), dequantize_nf4(packed, absmax, 4096, 64))


def make_linear_case(seed, m, n, k, r, with_bias, bs=64):
    g = rng(seed)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    x = f32_to_bf16_bits(g.standard_normal((m, k)))
    bias = f32_to_bf16_bits(g.standard_normal(n) * 0.02) if with_bias else None
    a = f32_to_bf16_bits(g.standard_normal((r, k)) * 0.01) if r else None
    b = f32_to_bf16_bits(g.standard_normal((n, r)) * 0.01) if r else None
    return dict(x=x, packed=packed, absmax=absmax, bias=bias, a=a, b=b, m=m, n=n, k=k, r=r, bs=bs)


def run_linear(dev, c, scaling=2.0):
    ops = _ops()
    y = ops.nf4_lora_linear(
        to_dev_bf16(c["x"], dev), torch.from_numpy(c["packed"]).to(dev),
        torch.from_numpy(c["absmax"]).to(dev), _code(dev), c["bs"], c["n"],
        bias=None if c["bias"] is None else to_dev_bf16(c["bias"], dev),
        lora_a=None if c["a"] is None else to_dev_bf16(c["a"], dev),
        lora_b=None if c["b"] is None else to_dev_bf16(c["b"], dev), scaling=scaling)
    torch.cuda.synchronize()
    return from_bf16(y)


def oracle_linear(c, scaling=2.0):
    return ref_linear(c["x"], c["packed"], c["absmax"], c["n"], c["k"], c["bs"],
                      bias_bits=c["bias"], a_bits=c["a"], b_bits=c["b"], scaling=scaling)


FAST = [
    (8, 1536, 1536, 16, True),    # q_proj (cfg 2)
    (8, 256, 1536, 16, True),     # k/v_proj (cfg 2)
    (8, 1536, 1536, 16, False),   # o_proj (cfg 2)
    (8, 8960, 1536, 0, False),    # gate/up (plain NF4)
    (8, 1536, 8960, 0, False),    # down (plain NF4, long K -> split-K)
    (1, 256, 512, 16, True),
    (16, 512, 1024, 16, True),
    (17, 512, 1024, 8, True),
    (33, 256, 768, 16, True),
    (64, 512, 512, 16, True),
    (32, 3584, 3584, 16, True),   # 7B q_proj at G = 32
    (64, 512, 3584, 16, True),    # 7B k/v_proj at G = 64
    (8, 3584, 18944, 0, False),   # 7B down_proj (deepest k-split)
    (64, 3584, 18944, 0, False),  # 7B down_proj at G = 64: 5 k-steps per slice, x chunk-major
    (57, 3584, 18944, 16, True),  # the same with ragged rows (57) and LoRA partials
    (20, 2048, 18944, 16, True),  # 5 k-steps chunk-major on two row tiles (rows 20..31 unused)
    (48, 1536, 18944, 16, True),  # 19 slices of 4 k-steps with LoRA partials
    (64, 3584, 3584, 16, False),  # 7B o_proj at G = 64: 8-wave wide workgroups (224 of them)
    (64, 256, 40960, 16, True),   # x over LDS: 32-row launches (tpart row offsets)
    (64, 256, 4096, 16, True),    # LoRA with two k-steps per wave
    (8, 400, 512, 16, True),      # N not a multiple of 256: the finish's last wave ragged
    (3, 1040, 512, 16, False),    # ... a second finish workgroup with 16 columns
]


@pytest.mark.parametrize("m,n,k,r,with_bias", FAST)
def test_linear_fast_matches_oracle(dev, m, n, k, r, with_bias):
    c = make_linear_case(m * 7 + n + k + r, m, n, k, r, with_bias)
    got = run_linear(dev, c)
    ref = oracle_linear(c)
    gf, rf = bf16_bits_to_f32(got), bf16_bits_to_f32(ref)
    assert np.all(np.isfinite(gf))
    assert rel_err(gf, rf) <= TOL
    assert np.mean(got == ref) >= 0.98


GENERIC = [
    (6, 16, 16, 4, True),      # the reference's tests/test_lora.py:93-122 shape (x [2,3,16])
    (5, 40, 100, 3, False),
    (8, 64, 320, 16, True),    # K not a multiple of 256
    (70, 64, 256, 16, True),   # M > 64
    (4, 48, 512, 32, True),    # r > 16
]


@pytest.mark.parametrize("m,n,k,r,with_bias", GENERIC)
def test_linear_generic_matches_oracle(dev, m, n, k, r, with_bias):
    c = make_linear_case(1000 + m + n + k, m, n, k, r, with_bias)
    got = run_linear(dev, c)
    ref = oracle_linear(c)
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(ref)) <= TOL


def test_linear_blocksize_128(dev):
    c = make_linear_case(77, 8, 512, 1024, 16, True, bs=128)
    got = run_linear(dev, c)
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(oracle_linear(c))) <= TOL


def test_linear_is_deterministic_across_calls(dev):
    """Repeated and interleaved calls of different shapes give bit-identical results."""
    big = make_linear_case(5, 8, 1536, 8960, 0, False)
    small = make_linear_case(6, 8, 256, 1536, 16, True)
    y1 = run_linear(dev, big)
    ys = run_linear(dev, small)
    y2 = run_linear(dev, big)
    ys2 = run_linear(dev, small)
    assert np.array_equal(y1, y2) and np.array_equal(ys, ys2)


def test_linear_scaling_and_zero_lora(dev):
    c = make_linear_case(9, 8, 256, 512, 16, True)
    for s in (0.5, 2.0, 3.7):
        got = run_linear(dev, c, scaling=s)
        assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(oracle_linear(c, s))) <= TOL
    c["b"] = np.zeros_like(c["b"])  # reference init: lora_B = 0 -> pure base + bias
    c0 = dict(c, a=None, b=None, r=0)
    assert np.array_equal(run_linear(dev, c), run_linear(dev, c0))


def test_linear_row_strides(dev):
    """x and y with row strides larger than the row (views into wider buffers)."""
    from grpo_mi355x.kernels import ops

    c = make_linear_case(11, 8, 256, 512, 16, True)
    xw = torch.zeros((8, 512 + 64), dtype=torch.bfloat16, device=dev)
    xw[:, :512] = to_dev_bf16(c["x"], dev)
    yw = torch.zeros((8, 256 + 32), dtype=torch.bfloat16, device=dev)
    ops.nf4_lora_linear(xw[:, :512], torch.from_numpy(c["packed"]).to(dev),
                        torch.from_numpy(c["absmax"]).to(dev), _code(dev), 64, 256,
                        bias=to_dev_bf16(c["bias"], dev), lora_a=to_dev_bf16(c["a"], dev),
                        lora_b=to_dev_bf16(c["b"], dev), scaling=2.0, out=yw[:, :256])
    torch.cuda.synchronize()
    assert np.array_equal(from_bf16(yw[:, :256]), run_linear(dev, c))
    assert torch.all(yw[:, 256:] == 0)
