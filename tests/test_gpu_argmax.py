"""grpo_argmax_bf16 (the greedy token of rows whose logits were written by a
GEMM, the wide-batch lm_head path) against numpy's first-index argmax."""

import numpy as np
import pytest
import torch

from conftest import from_bf16, rng, to_dev_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,V,ld", [(64, 152064, 152064), (3, 151936, 151936), (5, 1001, 1001),
                                    (4, 7, 7), (6, 1000, 1003)])  # ld 1003: rows not 16-byte aligned
def test_argmax_bf16_first_index(dev, M, V, ld):
    from grpo_mi355x import _lib
    from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

    g = rng(M * 7 + V)
    x = (g.standard_normal((M, ld)) * 3).astype(np.float32)
    if V > 20:
        x[0, 5] = x[0, V - 3] = 50.0       # tie: the first index wins
        x[1, V - 1] = 60.0                 # maximum in the last column (tail / last chunk)
    x[-1, :V] = -np.inf                    # all -inf: index 0
    bits = f32_to_bf16_bits(x)
    t = to_dev_bf16(bits, dev)
    out = torch.full((M,), -5, dtype=torch.int64, device=dev)
    lib = _lib.device_library()
    rc = lib.grpo_argmax_bf16(t.data_ptr(), ld, V, M, out.data_ptr(), _lib.stream_handle(dev))
    assert rc == 0
    torch.cuda.synchronize()
    want = np.argmax(bf16_bits_to_f32(bits)[:, :V], axis=1)
    assert out.cpu().numpy().tolist() == want.tolist()
