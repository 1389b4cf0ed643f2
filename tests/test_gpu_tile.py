"""The one-launch NF4 (+ LoRA) linear (``grpo_nf4_tile_linear*``) through the C ABI.

Each case is compared with the oracle linear (``oracle.lora_linear.nf4_lora_linear``,
pinned by the golden fixtures): bf16 tolerance ``max|y - y_ref| <= 1e-2 max|y_ref|``
and >= 97 % bit-identical outputs (the products are the reference's
``bf16(code * absmax) * x``; only the float32 summation order differs).  Shapes:
the Qwen2-1.5B and -7B decode projections (q|k|v as three segments with bias and
LoRA, o_proj with LoRA), ragged row counts (1, 5, 13), two row tiles (17..32
rows), several k-units per wave (K = 4096, 8192), no LoRA, rank 8, no bias.  The RMSNorm
source is compared with the oracle RMSNorm followed by the linear; the residual
form with the oracle's bf16 residual add, and its per-16-column sums of squares
with float64 sums of the kernel's own h.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.decode import bf16_residual, rmsnorm
from oracle.lora_linear import nf4_lora_linear
from oracle.nf4 import NF4_CODE, quantize_nf4

from conftest import from_bf16, rel_err, rng, to_dev_bf16

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _ops():
    from grpo_mi355x.kernels import ops

    return ops


def _case(seed, m, k, seg_rows, r, with_bias, bs=64):
    g = rng(seed)
    n = sum(seg_rows)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    x = f32_to_bf16_bits(g.standard_normal((m, k)))
    segs = []
    for rows in seg_rows:
        segs.append(dict(
            rows=rows,
            bias=f32_to_bf16_bits(g.standard_normal(rows) * 0.02) if with_bias else None,
            a=f32_to_bf16_bits(g.standard_normal((r, k)) * 0.01) if r else None,
            b=f32_to_bf16_bits(g.standard_normal((rows, r)) * 0.01) if r else None))
    return dict(x=x, packed=packed, absmax=absmax, segs=segs, m=m, n=n, k=k, r=r, bs=bs)


def _oracle(c, x_bits, scaling):
    outs = []
    row = 0
    for s in c["segs"]:
        rows = s["rows"]
        # this segment's rows of the packed weight (element e = n * K + k)
        lo, hi = row * c["k"] // 2, (row + rows) * c["k"] // 2
        alo, ahi = row * c["k"] // c["bs"], (row + rows) * c["k"] // c["bs"]
        outs.append(nf4_lora_linear(x_bits, c["packed"][lo:hi], c["absmax"][alo:ahi], rows,
                                    c["k"], c["bs"], bias_bits=s["bias"], a_bits=s["a"],
                                    b_bits=s["b"], scaling=scaling))
        row += rows
    return np.concatenate(outs, axis=1)


def _desc(c, dev, scaling):
    ops = _ops()
    segs = c["segs"]
    return ops.tile_linear_desc(
        c["m"], c["k"], [s["rows"] for s in segs],
        biases=[None if s["bias"] is None else to_dev_bf16(s["bias"], dev) for s in segs],
        lora_a=None if not c["r"] else [to_dev_bf16(s["a"], dev) for s in segs],
        lora_b=None if not c["r"] else [to_dev_bf16(s["b"], dev) for s in segs],
        scaling=scaling)


def _weights(c, dev):
    return (torch.from_numpy(c["packed"]).to(dev), torch.from_numpy(c["absmax"]).to(dev),
            torch.from_numpy(NF4_CODE.copy()).to(dev))


def _check(got, ref, min_identical=0.97):
    err = rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(ref))
    ident = float(np.mean(got == ref))
    assert err <= TOL, f"rel err {err}"
    assert ident >= min_identical, f"bit-identical fraction {ident}"


CASES = [
    # (m, k, segment rows, rank, bias)
    (8, 1536, [1536, 256, 256], 16, True),     # Qwen2-1.5B q|k|v (3 segments)
    (8, 1536, [1536], 16, False),              # Qwen2-1.5B o_proj
    (1, 1536, [1536], 16, True),
    (5, 1536, [1536, 256, 256], 16, True),
    (13, 3584, [3584, 512, 512], 16, True),    # Qwen2-7B q|k|v (7 waves x 2 k-steps)
    (16, 3584, [3584], 16, False),             # Qwen2-7B o_proj
    (32, 1536, [1536, 256, 256], 16, True),    # two row tiles (config 4's 32 rows)
    (19, 1536, [1536], 8, False),              # rank 8 (LoRA B rows not 16-byte vectors)
    (8, 8192, [1536], 0, False),               # folded, 2 k-units per wave
    (12, 4096, [512], 0, False),               # plain, 2 k-steps per wave
    (3, 512, [48, 16], 0, True),               # tiny: 2 waves, no LoRA
]


@pytest.mark.parametrize("m,k,seg_rows,r,with_bias", CASES)
def test_tile_linear_matches_oracle(dev, m, k, seg_rows, r, with_bias):
    ops = _ops()
    c = _case(1000 + m + k + r, m, k, seg_rows, r, with_bias)
    n = c["n"]
    assert _ops()._lib.library().grpo_nf4_tile_supported(m, n, k, r, len(seg_rows), 64) == 1
    pk, am, code = _weights(c, dev)
    desc = _desc(c, dev, 2.0)
    print(f"tile linear m={m} k={k} segs={seg_rows} r={r}", flush=True)
    y = ops.nf4_tile_linear(to_dev_bf16(c["x"], dev), pk, am, code, 64, desc)
    torch.cuda.synchronize()
    _check(from_bf16(y), _oracle(c, c["x"], 2.0))


@pytest.mark.parametrize("m,k,seg_rows", [(8, 1536, [1536, 256, 256]), (16, 3584, [3584, 512, 512]),
                                          (2, 1536, [1536, 256, 256])])
def test_tile_linear_norm_matches_oracle(dev, m, k, seg_rows):
    """x = RMSNorm(h) staged from per-group sums of squares of h: 8-column
    groups (as the folded down_proj writes them) up to 2048 columns, 16-column
    groups (as the residual form writes them) beyond."""
    ops = _ops()
    c = _case(77 + m, m, k, seg_rows, 16, True)
    g = rng(5 + m)
    h = f32_to_bf16_bits(g.standard_normal((m, k)) * 0.7)
    nw = f32_to_bf16_bits(1.0 + g.standard_normal(k) * 0.05)
    hf = bf16_bits_to_f32(h).astype(np.float64)
    gw = 8 if k <= 2048 else 16
    ss = (hf * hf).reshape(m, k // gw, gw).sum(-1).astype(np.float32)
    eps = 1e-6
    pk, am, code = _weights(c, dev)
    desc = _desc(c, dev, 2.0)
    print(f"tile linear norm m={m} k={k}", flush=True)
    y = ops.nf4_tile_linear(to_dev_bf16(h, dev), pk, am, code, 64, desc,
                            norm=(torch.from_numpy(ss).to(dev), to_dev_bf16(nw, dev), eps))
    torch.cuda.synchronize()
    x = rmsnorm(h, nw, eps)
    _check(from_bf16(y), _oracle(c, x, 2.0))


@pytest.mark.parametrize("m,k,n", [(8, 1536, 1536), (16, 3584, 3584), (7, 1536, 1536),
                                   (24, 1536, 1536)])
def test_tile_linear_residual_matches_oracle(dev, m, k, n):
    """o_proj + residual add in place (h aliases the residual) + sums of squares."""
    ops = _ops()
    c = _case(31 + m, m, k, [n], 16, False)
    g = rng(9 + m)
    res = f32_to_bf16_bits(g.standard_normal((m, n)))
    pk, am, code = _weights(c, dev)
    desc = _desc(c, dev, 2.0)
    h = to_dev_bf16(res, dev)
    groups = int(_ops()._lib.library().grpo_nf4_tile_sumsq_groups(m, n, k, 16, 64))
    assert groups == (n // 8 if m <= 8 else n // 16)
    ss = torch.full((m, groups), -1.0, dtype=torch.float32, device=dev)
    print(f"tile linear residual m={m} k={k} n={n}", flush=True)
    ops.nf4_tile_linear(to_dev_bf16(c["x"], dev), pk, am, code, 64, desc, out=h, residual=h,
                        sumsq=ss)
    torch.cuda.synchronize()
    got = from_bf16(h)
    ref = bf16_residual(res, _oracle(c, c["x"], 2.0))
    _check(got, ref)
    hf = bf16_bits_to_f32(got).astype(np.float64)
    want = (hf * hf).reshape(m, groups, n // groups).sum(-1)
    np.testing.assert_allclose(ss.cpu().numpy(), want, rtol=1e-5, atol=1e-6)


def test_tile_linear_repeat_is_deterministic(dev):
    ops = _ops()
    c = _case(4, 8, 1536, [1536, 256, 256], 16, True)
    pk, am, code = _weights(c, dev)
    desc = _desc(c, dev, 2.0)
    x = to_dev_bf16(c["x"], dev)
    a = ops.nf4_tile_linear(x, pk, am, code, 64, desc)
    b = ops.nf4_tile_linear(x, pk, am, code, 64, desc)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
