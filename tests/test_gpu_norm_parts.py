"""grpo_add_rmsnorm_parts through the C ABI against the oracle.

The split-K partial sums come from the GPU linear (grpo_nf4_linear_partials)
on seeded NF4 weights; the reference is the oracle linear
(oracle.lora_linear.nf4_lora_linear, pinned by the golden fixtures) followed
by the residual add and the oracle RMSNorm (oracle.decode.rmsnorm, pinned
against transformers' Qwen2RMSNorm).  Cases cover the register path (rows of
at most 2048 columns), the LDS path for wider rows (3584: Qwen2-7B's hidden
size), the LoRA + bias epilogue, and a norm weight and output that are only
2-byte aligned (the scalar load/store path).
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.decode import rmsnorm
from oracle.lora_linear import nf4_lora_linear
from oracle.nf4 import NF4_CODE, quantize_nf4

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _dev_bf16(bits, dev, offset=0):
    """bf16 tensor holding ``bits``; ``offset`` elements of padding in front make
    the returned view only 2-byte aligned when offset is odd."""
    flat = np.zeros(bits.size + offset, np.uint16)
    flat[offset:] = bits.reshape(-1)
    t = torch.from_numpy(flat.view(np.int16)).view(torch.bfloat16).to(dev)
    return t[offset:].view(bits.shape)


@pytest.mark.parametrize("m,n,k,lora,offset", [(8, 1536, 512, False, 0), (8, 1536, 512, True, 1),
                                               (8, 3584, 512, True, 0), (8, 3584, 512, False, 1),
                                               (64, 3584, 3584, True, 0),
                                               (64, 3584, 18944, False, 0),
                                               (16, 3584, 18944, False, 1),
                                               (4, 1040, 512, True, 0)])
def test_add_rmsnorm_parts_matches_oracle(dev, m, n, k, lora, offset):
    """The 64-row cases are config 5's post-attention norm (7 slices of o_proj
    partials with LoRA) and input norm (15 slices of down_proj partials, no
    LoRA): rows of 3584 columns finished by 1024 threads in one pass; the last
    takes the 16-slice form with a 2-byte aligned weight and output.  1040
    columns leave the LoRA B wave loads one wave of 16 columns."""
    from grpo_mi355x import _lib
    from grpo_mi355x.kernels import ops

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    r, bs, eps = 16, 64, 1e-6
    g = np.random.default_rng(n + 10 * lora + offset + m + k)
    x = f32_to_bf16_bits(g.standard_normal((m, k)).astype(np.float32))
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    bias = f32_to_bf16_bits((g.standard_normal(n) * 0.1).astype(np.float32))
    a = f32_to_bf16_bits((g.standard_normal((r, k)) * 0.05).astype(np.float32))
    b = f32_to_bf16_bits((g.standard_normal((n, r)) * 0.05).astype(np.float32))
    res = f32_to_bf16_bits(g.standard_normal((m, n)).astype(np.float32))
    nw = f32_to_bf16_bits((1 + 0.1 * g.standard_normal(n)).astype(np.float32))

    # split-K partial sums of the linear on the GPU
    rr = r if lora else 0
    plan = ops.nf4_linear_plan(m, n, k, rr, 1, bs)
    assert plan is not None
    splits, pbytes, tbytes = plan
    t = lambda arr: torch.from_numpy(np.ascontiguousarray(arr)).to(dev)
    x_d, a_d, b_d, bias_d = (_dev_bf16(v, dev) for v in (x, a, b, bias))
    pk_d, am_d, code_d = t(packed), t(absmax), t(NF4_CODE.astype(np.float32))
    part = torch.empty(max(pbytes, 16) // 4, dtype=torch.float32, device=dev)
    tpart = torch.empty(max(tbytes, 16) // 4, dtype=torch.float32, device=dev)
    d = _lib.LinearParts()
    d.part, d.tpart = part.data_ptr(), tpart.data_ptr()
    d.splits, d.M, d.N, d.K, d.nseg, d.r = splits, m, n, k, 1, rr
    d.seg_end[0] = n
    d.bias[0] = bias_d.data_ptr()
    d.lora_b[0] = b_d.data_ptr() if lora else None
    d.scaling = 2.0
    la = (ctypes.c_void_p * 1)(a_d.data_ptr() if lora else None)
    _lib.check(lib.grpo_nf4_linear_partials(x_d.data_ptr(), k, pk_d.data_ptr(), am_d.data_ptr(),
                                            code_d.data_ptr(), bs, la, ctypes.byref(d), st),
               "partials")

    # residual add + RMSNorm from the partials, in place on the residual
    h_d = _dev_bf16(res, dev)  # the residual must be 8-byte aligned
    nw_d = _dev_bf16(nw, dev, offset)
    y_d = _dev_bf16(np.zeros((m, n), np.uint16), dev, offset)
    _lib.check(lib.grpo_add_rmsnorm_parts(ctypes.byref(d), h_d.data_ptr(), h_d.data_ptr(),
                                          nw_d.data_ptr(), y_d.data_ptr(), eps, st), "norm")
    torch.cuda.synchronize()

    lin = nf4_lora_linear(x, packed, absmax, n, k, bs, bias_bits=bias,
                          a_bits=a if lora else None, b_bits=b if lora else None, scaling=2.0)
    h_ref = f32_to_bf16_bits(bf16_bits_to_f32(lin) + bf16_bits_to_f32(res))
    y_ref = rmsnorm(h_ref, nw, eps)
    h_got, y_got = _bits(h_d), _bits(y_d)
    # the linear's float32 summation order differs from numpy's: a few outputs
    # differ by an ulp, which the residual add and the norm carry along
    assert np.mean(h_got == h_ref) >= 0.97
    assert rel_err(bf16_bits_to_f32(h_got), bf16_bits_to_f32(h_ref)) <= 1e-2
    assert np.mean(y_got == y_ref) >= 0.95
    assert rel_err(bf16_bits_to_f32(y_got), bf16_bits_to_f32(y_ref)) <= 1e-2


@pytest.mark.parametrize("m,i,k", [(8, 8960, 1536), (3, 256, 512), (16, 512, 1536),
                                   (8, 512, 3584), (8, 17920, 3584), (5, 4112, 512),
                                   (17, 256, 512), (32, 8960, 1536), (40, 8960, 1536),
                                   (64, 2048, 768), (48, 20480, 256), (32, 18944, 3584),
                                   (64, 18944, 3584), (24, 40000, 256)])
def test_gate_up_silu_matches_oracle(dev, m, i, k):
    _check_gate_up_silu(dev, m, i, k, 8)


@pytest.mark.parametrize("m,i,k", [(65, 8960, 1536), (130, 256, 512), (512, 8960, 1536),
                                   (200, 1000, 96)])
def test_gate_up_silu_wide_batches_match_oracle(dev, m, i, k):
    """More than 64 rows (prefill chunks): the NF4 GEMM with 64 gate and the
    same 64 up columns per tile, SiLU*up in its epilogue; ragged row tiles
    (65, 130, 200), I not a multiple of 64 (1000), K not a multiple of 128 (96)."""
    _check_gate_up_silu(dev, m, i, k, 8)
    _check_gate_up_silu(dev, m, i, k, 3)


@pytest.mark.parametrize("m,i,k", [(40, 8960, 1536), (5, 4112, 512), (24, 8960, 1536)])
def test_gate_up_silu_unaligned_act_rows(dev, m, i, k):
    """act rows of I + 3 columns: the wide kernel's epilogue then stores
    column by column instead of 8 columns per 16-byte store."""
    _check_gate_up_silu(dev, m, i, k, 3)


def _check_gate_up_silu(dev, m, i, k, pad):
    """grpo_nf4_gate_up_silu = oracle NF4 linear of the gate and up halves of a
    stacked weight, then oracle SiLU*mul (fused_ops.py:79-112).  The first four
    and the sixth shape run the 8-column-unit kernel (the sixth has 514 units
    over 256 workgroups: two workgroups take a third unit); [8, 17920, 3584]
    has more items per wave than the unit kernel keeps in registers and runs
    one workgroup per 16 columns.  17..32 rows whose x and item tiles fit LDS
    (17 x 256 x 512: one unit per workgroup; config 4's 32 x 8960 x 1536;
    24 x 40000 x 256: 19 or 20 units per workgroup, more than the wide kernel
    takes) run the unit kernel on two 16-row tiles.  The other 17..64-row shapes run the
    wide kernel (x staged in 512-column chunks, unit accumulators in registers
    across K): a 3-row-tile shape (40 rows); an odd number of k-steps, whose
    last chunk has one (64 x 2048 x 768); a single k-step and 10 units per
    workgroup (48 x 20480 x 256); two row tiles whose x exceeds LDS
    (32 x 18944 x 3584); config 5's Qwen2-7B MLP (2368 units: 9 or 10 per
    workgroup)."""
    from grpo_mi355x import _lib

    from oracle.decode import silu_mul

    lib = _lib.device_library()
    bs = 64
    assert lib.grpo_nf4_gate_up_silu_supported(m, i, k, bs) == 1
    g = np.random.default_rng(m * 7 + i + k)
    x = f32_to_bf16_bits(g.standard_normal((m, k)).astype(np.float32))
    w = (g.standard_normal((2 * i, k)) * 0.05).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    t = lambda arr: torch.from_numpy(np.ascontiguousarray(arr)).to(dev)
    # device buffers are kept in names until the kernel has run (a temporary
    # freed before the asynchronous launch may be reused by the next copy)
    x_d, pk_d, am_d = _dev_bf16(x, dev), t(packed), t(absmax)
    code_d = t(NF4_CODE.astype(np.float32))
    act = torch.zeros(m, i + pad, dtype=torch.bfloat16, device=dev)  # lda > I
    _lib.check(lib.grpo_nf4_gate_up_silu(x_d.data_ptr(), k, pk_d.data_ptr(), am_d.data_ptr(),
                                         code_d.data_ptr(), bs, i, k, m, act.data_ptr(), i + pad,
                                         _lib.stream_handle(dev)), "gu")
    torch.cuda.synchronize()
    half = packed.size // 2, absmax.size // 2
    gate = nf4_lora_linear(x, packed[:half[0]], absmax[:half[1]], i, k, bs)
    up = nf4_lora_linear(x, packed[half[0]:], absmax[half[1]:], i, k, bs)
    ref = silu_mul(gate, up)
    got = _bits(act)[:, :i]
    assert np.all(_bits(act)[:, i:] == 0)  # columns past I untouched
    assert np.mean(got == ref) >= 0.97
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(ref)) <= 1e-2


def test_gate_up_silu_rejects_unsupported(dev):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    # more than 64 rows: the NF4 GEMM's form (I % 8, K % 32, blocksize >= 32)
    assert lib.grpo_nf4_gate_up_silu_supported(65, 256, 512, 64) == 1
    assert lib.grpo_nf4_gate_up_silu_supported(65, 250, 512, 64) == 0  # I % 8
    assert lib.grpo_nf4_gate_up_silu_supported(65, 256, 500, 64) == 0  # K % 32
    assert lib.grpo_nf4_gate_up_silu_supported(8, 250, 512, 64) == 0   # I % 16
    assert lib.grpo_nf4_gate_up_silu_supported(32, 250, 512, 64) == 0  # I % 8
    assert lib.grpo_nf4_gate_up_silu_supported(8, 256, 500, 64) == 0   # K % 256
    assert lib.grpo_nf4_gate_up_silu_supported(32, 256, 500, 64) == 0  # K % 256
    assert lib.grpo_nf4_gate_up_silu_supported(8, 256, 6400, 64) == 0  # K > 6144
    assert lib.grpo_nf4_gate_up_silu_supported(32, 256, 512, 32) == 0  # blocksize < 64
    # more than 12 units per CU for the wide kernel, more than 32 rows for the
    # unit kernel (32 rows take it on two row tiles)
    assert lib.grpo_nf4_gate_up_silu_supported(40, 24584, 512, 64) == 0
    assert lib.grpo_nf4_gate_up_silu_supported(32, 24584, 512, 64) == 1
    assert lib.grpo_nf4_gate_up_silu(None, 512, None, None, None, 64, 250, 512, 65, None, 256,
                                     None) == -2  # GRPO_EUNSUPPORTED
    assert lib.grpo_nf4_gate_up_silu(None, 512, None, None, None, 64, 256, 512, 65, None, 256,
                                     None) == -1  # a taken shape, null pointers: GRPO_EINVAL
