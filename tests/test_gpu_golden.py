"""GPU parity against the committed golden fixtures, through the C ABI."""

import os

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from oracle.paged import append_kv

from conftest import ROOT, from_bf16, rel_err, to_dev_bf16

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(ROOT, "tests", "golden")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False))


def test_gpu_nf4_dequant_golden(dev):
    from grpo_mi355x.kernels import ops

    f = load("nf4_dequant")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    out = ops.nf4_dequant(t(f["packed"]), t(f["absmax"]), t(f["code"]), f["packed"].size * 2,
                          int(f["blocksize"]))
    torch.cuda.synchronize()
    assert np.array_equal(from_bf16(out), f["expected"])


def test_gpu_lora_linear_golden(dev):
    from grpo_mi355x.kernels import ops

    f = load("lora_linear_kv")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    code = torch.from_numpy(load("nf4_dequant")["code"]).to(dev)
    y = ops.nf4_lora_linear(to_dev_bf16(f["x"], dev), t(f["packed"]), t(f["absmax"]), code,
                            int(f["blocksize"]), int(f["n"]), bias=to_dev_bf16(f["bias"], dev),
                            lora_a=to_dev_bf16(f["lora_a"], dev),
                            lora_b=to_dev_bf16(f["lora_b"], dev), scaling=float(f["scaling"]))
    torch.cuda.synchronize()
    got = from_bf16(y)
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(f["expected"])) <= 1e-2
    assert np.mean(got == f["expected"]) >= 0.98


def test_gpu_paged_attention_golden(dev):
    from grpo_mi355x.kernels import ops

    f = load("paged_attention")
    kc, vc = to_dev_bf16(f["k_cache"], dev), to_dev_bf16(f["v_cache"], dev)
    tables = torch.from_numpy(f["block_tables"]).to(dev)
    lens = torch.from_numpy(f["context_lens"]).to(dev)
    ops.paged_kv_append(to_dev_bf16(f["k_new"], dev), to_dev_bf16(f["v_new"], dev), kc, vc,
                        tables, lens)
    out = ops.paged_attention_decode(to_dev_bf16(f["q"], dev), kc, vc, tables, lens + 1,
                                     1.0 / np.sqrt(f["q"].shape[-1]))
    torch.cuda.synchronize()
    k_ref, v_ref = f["k_cache"].copy(), f["v_cache"].copy()
    append_kv(k_ref, v_ref, f["k_new"], f["v_new"], f["block_tables"], f["context_lens"])
    assert np.array_equal(from_bf16(kc), k_ref) and np.array_equal(from_bf16(vc), v_ref)
    assert rel_err(out.cpu().numpy(), f["expected"]) <= 1e-2
