"""Writes the golden fixtures of tests/golden/ (run from the repository root).

The reference ships no golden files for this path and cannot run here
(bitsandbytes is not installed and its Triton kernels need a GPU), so the
fixtures are produced by the CPU oracle (``oracle/``), which the oracle tests
pin against the reference's closed forms and known-answer tests.  Inputs are
seeded numpy draws shaped like BASELINE configs 1 and 2, cut down so that the
files stay small:

* ``nf4_dequant.npz``   -- every byte value under 32 absmax blocks (zero,
  denormal-range, large and ordinary scales): bit-exact target.
* ``lora_linear_kv.npz`` -- config 2's k/v projection: x [8, 1536] ~ N(0, 1),
  W [256, 1536] ~ N(0, 0.02) quantized to NF4 (blocksize 64), bias, rank-16
  LoRA A/B ~ N(0, 0.01), scaling 2.0 -> y [8, 256] bf16.
* ``paged_attention.npz`` -- config 1's head shape (12 query / 2 KV heads,
  head_dim 128, block 16) for 2 ragged sequences (37 and 70 tokens) on a
  shuffled block table of 10 physical blocks, plus one appended token per
  sequence -> float32 output.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.bf16 import f32_to_bf16_bits  # noqa: E402
from oracle.lora_linear import nf4_lora_linear  # noqa: E402
from oracle.nf4 import NF4_CODE, dequantize_nf4, quantize_nf4  # noqa: E402
from oracle.paged import append_kv, paged_attention_decode  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def nf4_dequant_case():
    packed = np.tile(np.arange(256, dtype=np.uint8), 4)  # 2048 elements
    g = np.random.default_rng(101)
    absmax = (np.abs(g.standard_normal(32)) * 0.05).astype(np.float32)
    absmax[:6] = [0.0, 1e-38, 3e-39, 3e38, 1.0, 0.5]
    out = dequantize_nf4(packed, absmax, packed.size * 2, 64)
    return dict(packed=packed, absmax=absmax, code=NF4_CODE.copy(), blocksize=np.int32(64),
                expected=out)


def lora_linear_case():
    g = np.random.default_rng(202)
    m, n, k, r = 8, 256, 1536, 16
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, 64)
    x = f32_to_bf16_bits(g.standard_normal((m, k)))
    bias = f32_to_bf16_bits(g.standard_normal(n) * 0.02)
    a = f32_to_bf16_bits(g.standard_normal((r, k)) * 0.01)
    b = f32_to_bf16_bits(g.standard_normal((n, r)) * 0.01)
    y = nf4_lora_linear(x, packed, absmax, n, k, 64, bias_bits=bias, a_bits=a, b_bits=b,
                        scaling=2.0)
    return dict(x=x, packed=packed, absmax=absmax, bias=bias, lora_a=a, lora_b=b,
                scaling=np.float32(2.0), blocksize=np.int32(64), n=np.int32(n), k=np.int32(k),
                expected=y)


def paged_attention_case():
    g = np.random.default_rng(303)
    hq, hkv, d, bs, nb = 12, 2, 128, 16, 10
    ctx = np.array([37, 70], dtype=np.int32)
    width = 5
    perm = g.permutation(nb).astype(np.int32)
    tables = np.full((2, width), -1, dtype=np.int32)
    tables[0, :3] = perm[:3]   # 37 tokens + 1 appended -> 3 blocks
    tables[1, :5] = perm[3:8]  # 70 tokens + 1 appended -> 5 blocks
    kc = f32_to_bf16_bits(g.standard_normal((nb, hkv, bs, d)))
    vc = f32_to_bf16_bits(g.standard_normal((nb, hkv, bs, d)))
    q = f32_to_bf16_bits(g.standard_normal((2, hq, d)))
    k_new = f32_to_bf16_bits(g.standard_normal((2, hkv, d)))
    v_new = f32_to_bf16_bits(g.standard_normal((2, hkv, d)))
    k_after, v_after = kc.copy(), vc.copy()
    append_kv(k_after, v_after, k_new, v_new, tables, ctx)
    out = paged_attention_decode(q, k_after, v_after, tables, ctx + 1, 1.0 / np.sqrt(d))
    return dict(q=q, k_cache=kc, v_cache=vc, k_new=k_new, v_new=v_new, block_tables=tables,
                context_lens=ctx, expected=out)


CASES = {"nf4_dequant": nf4_dequant_case, "lora_linear_kv": lora_linear_case,
         "paged_attention": paged_attention_case}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
