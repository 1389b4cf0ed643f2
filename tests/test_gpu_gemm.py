"""GPU parity: the NF4 GEMM (``grpo_nf4_gemm``, ``nf4_gemm_mfma``) that takes the
NF4 + LoRA linear beyond the split-K path's 64 rows -- the reference's
``_lora_forward_kernel`` for any M (src/triton_kernels/lora_forward.py:107-260).

Tolerance as for the split-K linear: ``max|y - y_ref| <= 1e-2 * max|y_ref|``,
and >= 98% of the outputs bit-identical to the oracle (every product equals the
reference's ``bf16(code*absmax) * x``; only the float32 summation order
differs).  Calls go through the C ABI (``ops.nf4_lora_linear`` ->
``grpo_nf4_lora_linear``, which routes M > 64 to the GEMM, and the GEMM's own
entry point).
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32

from conftest import from_bf16, rel_err, to_dev_bf16
from test_gpu_nf4 import _code, make_linear_case, oracle_linear, run_linear

pytestmark = pytest.mark.gpu
TOL = 1e-2

GEMM = [
    (65, 1536, 1536, 16, True),   # q_proj, one row past the split-K path
    (256, 1024, 1024, 16, False), # the reference harness shape: 4 x 64 rows, r 16
    (512, 8960, 1536, 0, False),  # gate at a 512-token prefill chunk (no LoRA)
    (511, 1536, 8960, 16, False), # down_proj: K = 8960 in 70 stages, ragged rows
    (130, 200, 96, 5, True),      # N % 128 != 0, K % 128 != 0, r % 8 != 0 (scalar B rows)
    (129, 136, 160, 24, True),    # two rank tiles (r > 16)
    (300, 256, 512, 32, True),    # r = 32
    (1000, 384, 384, 8, True),    # 8 row tiles, r = 8
    (2048, 1536, 1536, 16, True), # unsplit with LoRA, 16 row tiles
    (70, 64, 256, 16, True),      # N below one column tile
    (97, 1030, 256, 16, True),    # N % 8 != 0: element stores
]


def _check(got, ref):
    gf, rf = bf16_bits_to_f32(got), bf16_bits_to_f32(ref)
    assert np.all(np.isfinite(gf))
    assert rel_err(gf, rf) <= TOL
    assert np.mean(got == ref) >= 0.98


@pytest.mark.parametrize("m,n,k,r,with_bias", GEMM)
def test_gemm_matches_oracle(dev, m, n, k, r, with_bias):
    print(f"nf4 gemm case m={m} n={n} k={k} r={r} bias={with_bias}", flush=True)
    c = make_linear_case(3 * m + n + 7 * k + r, m, n, k, r, with_bias)
    _check(run_linear(dev, c), oracle_linear(c))


def test_gemm_blocksize_32_and_256(dev):
    for bs in (32, 256):
        c = make_linear_case(21 + bs, 200, 512, 768, 16, True, bs=bs)
        _check(run_linear(dev, c), oracle_linear(c))


def test_gemm_deterministic_and_scaling(dev):
    c = make_linear_case(31, 200, 640, 1024, 16, True)
    y1 = run_linear(dev, c)
    y2 = run_linear(dev, c)
    assert np.array_equal(y1, y2)
    for s in (0.5, 3.7):
        _check(run_linear(dev, c, scaling=s), oracle_linear(c, s))
    # lora_B = 0 (the reference's initialisation): the base product alone
    c["b"] = np.zeros_like(c["b"])
    assert np.array_equal(run_linear(dev, c), run_linear(dev, dict(c, a=None, b=None, r=0)))


def _lib():
    from grpo_mi355x import _lib

    return _lib


def test_gemm_entry_strided_and_unaligned_output(dev):
    """grpo_nf4_gemm directly: x and y as views with row strides larger than the
    row; y starting at an odd element (2-byte stores) and at an aligned one
    (16-byte stores) give the same values, and nothing outside the view changes."""
    _l = _lib()
    lib = _l.device_library()
    m, n, k, r = 150, 264, 512, 16
    c = make_linear_case(41, m, n, k, r, True)
    xw = torch.zeros((m, k + 64), dtype=torch.bfloat16, device=dev)
    xw[:, :k] = to_dev_bf16(c["x"], dev)
    packed = torch.from_numpy(c["packed"]).to(dev)
    absmax = torch.from_numpy(c["absmax"]).to(dev)
    code = _code(dev)
    bias, a, b = (to_dev_bf16(c[key], dev) for key in ("bias", "a", "b"))
    outs = []
    for off in (0, 1):
        yw = torch.zeros((m, n + 40), dtype=torch.bfloat16, device=dev)
        rc = lib.grpo_nf4_gemm(xw.data_ptr(), xw.stride(0), packed.data_ptr(), absmax.data_ptr(),
                               code.data_ptr(), 64, bias.data_ptr(), a.data_ptr(), b.data_ptr(), r,
                               2.0, yw[:, off:].data_ptr(), yw.stride(0), m, n, k,
                               _l.stream_handle(dev))
        _l.check(rc, "grpo_nf4_gemm")
        torch.cuda.synchronize()
        assert torch.all(yw[:, :off] == 0) and torch.all(yw[:, off + n:] == 0)
        outs.append(from_bf16(yw[:, off:off + n]))
    assert np.array_equal(outs[0], outs[1])
    _check(outs[0], oracle_linear(c))


def test_gemm_supported_query(dev):
    lib = _lib().device_library()
    assert lib.grpo_nf4_gemm_supported(65, 1536, 1536, 16, 64) == 1
    assert lib.grpo_nf4_gemm_supported(65, 1536, 1540, 16, 64) == 0  # K % 32 != 0
    assert lib.grpo_nf4_gemm_supported(65, 1536, 1536, 33, 64) == 0  # r > 32
    assert lib.grpo_nf4_gemm_supported(65, 1536, 1536, 16, 16) == 0  # blocksize < 32
    assert lib.grpo_nf4_gemm_supported(65, 1536, 1536, 16, 96) == 0  # not a power of two


def test_grouped_qkv_wide_batch(dev):
    """grpo_nf4_lora_linear_grouped at 100 rows: q|k|v of one stacked weight,
    each segment with its own bias and LoRA pair, one GEMM launch for the three
    segments (and K slices + one finish)."""
    _l = _lib()
    lib = _l.device_library()
    m, k, r, bs = 100, 1536, 16, 64
    segs = (1536, 256, 256)
    cases = [make_linear_case(60 + i, m, n, k, r, True) for i, n in enumerate(segs)]
    for cs in cases[1:]:
        cs["x"] = cases[0]["x"]
    packed = torch.from_numpy(np.concatenate([cs["packed"] for cs in cases])).to(dev)
    absmax = torch.from_numpy(np.concatenate([cs["absmax"] for cs in cases])).to(dev)
    x = to_dev_bf16(cases[0]["x"], dev)
    keep = [tuple(to_dev_bf16(cs[key], dev) for key in ("bias", "a", "b")) for cs in cases]
    arr = ctypes.c_void_p * 4
    bias = arr(*[t[0].data_ptr() for t in keep], None)
    la = arr(*[t[1].data_ptr() for t in keep], None)
    lb = arr(*[t[2].data_ptr() for t in keep], None)
    seg_rows = (ctypes.c_int * 4)(*segs, 0)
    y = torch.zeros((m, sum(segs)), dtype=torch.bfloat16, device=dev)
    code = _code(dev)
    # 12 + 2 + 2 column tiles over 12 stages: the K split (partial sums + finish)
    nbytes = int(lib.grpo_nf4_lora_linear_workspace_bytes(m, sum(segs), k, r, 3, bs))
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    rc = lib.grpo_nf4_lora_linear_grouped(
        x.data_ptr(), x.stride(0), packed.data_ptr(), absmax.data_ptr(), code.data_ptr(), bs, 3,
        seg_rows, bias, la, lb, r, 2.0, y.data_ptr(), y.stride(0), m, k, ws.data_ptr(), nbytes,
        _l.stream_handle(dev))
    _l.check(rc, "grpo_nf4_lora_linear_grouped")
    torch.cuda.synchronize()
    got = from_bf16(y)
    start = 0
    for n, cs in zip(segs, cases):
        _check(got[:, start:start + n], oracle_linear(cs))
        start += n
