"""CPU checks of the committed golden fixtures (tests/golden/*.npz).

Each fixture is reproduced from its stored inputs by the oracle (so a change
to the oracle that alters a pinned result fails here), and checked by a route
that does not share the oracle's code: dense float64 algebra for the linear,
torch's softmax attention on the gathered cache for attention.
"""

import os

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from oracle.lora_linear import nf4_lora_linear
from oracle.nf4 import NF4_CODE, dequantize_nf4
from oracle.paged import append_kv, paged_attention_decode

from conftest import ROOT

GOLDEN = os.path.join(ROOT, "tests", "golden")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False))


def test_nf4_dequant_fixture():
    f = load("nf4_dequant")
    assert np.array_equal(f["code"], NF4_CODE)
    got = dequantize_nf4(f["packed"], f["absmax"], f["packed"].size * 2, int(f["blocksize"]))
    assert np.array_equal(got, f["expected"])
    # independent route: byte b under absmax a gives (code[b >> 4] * a, code[b & 15] * a)
    e = f["expected"].reshape(-1, 2)
    for i in (0, 17, 255, 700, 1023):
        a = f["absmax"][(2 * i) // 64]
        hi = torch.tensor(float(NF4_CODE[f["packed"][i] >> 4]) * float(a), dtype=torch.float32)
        lo = torch.tensor(float(NF4_CODE[f["packed"][i] & 15]) * float(a), dtype=torch.float32)
        want = torch.stack([hi, lo]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(e[i], want)


def test_lora_linear_fixture():
    f = load("lora_linear_kv")
    n, k, bs = int(f["n"]), int(f["k"]), int(f["blocksize"])
    got = nf4_lora_linear(f["x"], f["packed"], f["absmax"], n, k, bs, bias_bits=f["bias"],
                          a_bits=f["lora_a"], b_bits=f["lora_b"], scaling=float(f["scaling"]))
    assert np.array_equal(got, f["expected"])
    # independent route: float64 x W^T + bias + (x A^T) B^T s, no intermediate rounding
    w = bf16_bits_to_f32(dequantize_nf4(f["packed"], f["absmax"], n * k, bs)).reshape(n, k)
    x = bf16_bits_to_f32(f["x"]).astype(np.float64)
    a = bf16_bits_to_f32(f["lora_a"]).astype(np.float64)
    b = bf16_bits_to_f32(f["lora_b"]).astype(np.float64)
    dense = x @ w.T.astype(np.float64) + bf16_bits_to_f32(f["bias"]) + (x @ a.T) @ b.T * 2.0
    y = bf16_bits_to_f32(f["expected"])
    assert np.max(np.abs(y - dense)) <= 1e-2 * np.max(np.abs(dense))


def test_paged_attention_fixture():
    f = load("paged_attention")
    kc, vc = f["k_cache"].copy(), f["v_cache"].copy()
    append_kv(kc, vc, f["k_new"], f["v_new"], f["block_tables"], f["context_lens"])
    lens = f["context_lens"] + 1
    d = f["q"].shape[-1]
    got = paged_attention_decode(f["q"], kc, vc, f["block_tables"], lens, 1.0 / np.sqrt(d))
    assert np.allclose(got, f["expected"], rtol=0, atol=1e-6)
    # independent route: dense K/V rebuilt by walking the table, torch SDPA in float64
    q = torch.from_numpy(bf16_bits_to_f32(f["q"])).double()
    hq, hkv = q.shape[1], kc.shape[1]
    for s in range(q.shape[0]):
        rows_k, rows_v = [], []
        for t in range(int(lens[s])):
            blk = int(f["block_tables"][s, t // 16])
            rows_k.append(bf16_bits_to_f32(kc[blk, :, t % 16, :]))
            rows_v.append(bf16_bits_to_f32(vc[blk, :, t % 16, :]))
        K = torch.from_numpy(np.stack(rows_k, 1)).double().repeat_interleave(hq // hkv, 0)
        V = torch.from_numpy(np.stack(rows_v, 1)).double().repeat_interleave(hq // hkv, 0)
        ref = torch.nn.functional.scaled_dot_product_attention(q[s][:, None, :], K, V)[:, 0, :]
        assert torch.allclose(torch.from_numpy(f["expected"][s]).double(), ref, atol=1e-5)


@pytest.mark.parametrize("name", ["nf4_dequant", "lora_linear_kv", "paged_attention"])
def test_fixtures_are_small_and_pickle_free(name):
    path = os.path.join(GOLDEN, f"{name}.npz")
    assert os.path.getsize(path) < 400_000
    load(name)  # allow_pickle=False
