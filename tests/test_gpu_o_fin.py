"""o_proj with its epilogue and the residual add in one launch, through the C ABI.

``grpo_nf4_linear_attn_residual`` (the K slice of each 64-column group that
arrives last finishes the group) is compared on the same attention split
partials with the oracle (``oracle.lora_linear.nf4_lora_linear`` of the merged
attention rows, which ``grpo_paged_attn_merge`` writes, plus the bf16 residual
add): bf16 tolerance 1e-2 and >= 97 % bit-identical outputs, as the other NF4
linear tests.  Against the two-launch path ``grpo_nf4_linear_partials_attn`` +
``grpo_linear_finish_residual`` (same partial sums and roundings; only the LoRA
product t . B runs on an MFMA instead of sequential FMAs) >= 99 % of the
outputs are bit-identical.  The per-64-column sums of squares are checked
against float64 sums of the kernel's own h (tolerance 1e-5).  Each case runs
the fused launch three times in a row (the arrival counters must come back to
zero, checked after the calls) and once more after the inputs changed.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.lora_linear import nf4_lora_linear
from oracle.nf4 import NF4_CODE, quantize_nf4

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _dev(arr, dev):
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dev)


def _dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def _attn_workspace(lib, g, dev, m, hq, hkv, bs, max_blocks, lens):
    """Split partials as grpo_paged_attn_decode_qkv leaves them: O [M][Hq][S][128]
    unnormalised, then (max in the log2 domain, sum) [M][Hq][S][2]."""
    from grpo_mi355x.kernels import ops

    s = int(lib.grpo_paged_attn_splits(m, hq, hkv, 128, bs, max_blocks))
    assert s >= 1
    nbytes = ops.paged_attention_workspace_bytes(m, hq, hkv, 128, bs, max_blocks)
    ws = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    o = g.standard_normal((m, hq, s, 128)).astype(np.float32) * 3.0
    ml = np.stack([g.uniform(-3, 3, (m, hq, s)), g.uniform(1, 8, (m, hq, s))], -1)
    ws[:o.size] = _dev(o.reshape(-1), dev)
    ws[o.size:o.size + ml.size] = _dev(ml.astype(np.float32).reshape(-1), dev)
    return ws, _dev(np.asarray(lens, np.int32), dev)


@pytest.mark.parametrize("m,hq,hkv,r,bias", [(8, 12, 2, 16, False), (5, 28, 4, 16, True),
                                              (16, 12, 2, 0, False), (1, 12, 2, 8, True)])
def test_attn_residual_matches_oracle_and_the_two_launch_path(dev, m, hq, hkv, r, bias):
    from grpo_mi355x import _lib
    from grpo_mi355x.kernels import ops

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    bs, block, max_blocks = 64, 16, 64
    k = n = hq * 128
    g = np.random.default_rng(m * 100 + hq + r)
    lens = g.integers(1, max_blocks * block + 1, m)
    lens[0] = max_blocks * block  # every split used
    if m > 2:
        lens[1] = 0  # an inactive row
    ws, len_d = _attn_workspace(lib, g, dev, m, hq, hkv, block, max_blocks, lens)
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    a = f32_to_bf16_bits((g.standard_normal((max(r, 1), k)) * 0.05).astype(np.float32))
    b = f32_to_bf16_bits((g.standard_normal((n, max(r, 1))) * 0.05).astype(np.float32))
    bias_bits = f32_to_bf16_bits((g.standard_normal(n) * 0.1).astype(np.float32))
    ld = n + 16  # columns past N must stay untouched
    res = f32_to_bf16_bits(g.standard_normal((m, ld)).astype(np.float32))
    splits, pbytes, tbytes = ops.nf4_linear_plan(m, n, k, r, 1, bs)
    a_d, b_d, bias_d = _dev_bf16(a, dev), _dev_bf16(b, dev), _dev_bf16(bias_bits, dev)
    pk_d, am_d, code_d = _dev(packed, dev), _dev(absmax, dev), _dev(NF4_CODE.astype(np.float32), dev)
    part = torch.empty(max(pbytes, 16) // 4, dtype=torch.float32, device=dev)
    tpart = torch.empty(max(tbytes, 16) // 4, dtype=torch.float32, device=dev)
    d = _lib.LinearParts()
    d.part, d.tpart = part.data_ptr(), tpart.data_ptr()
    d.splits, d.M, d.N, d.K, d.nseg, d.r = splits, m, n, k, 1, r
    d.seg_end[0] = n
    d.bias[0] = bias_d.data_ptr() if bias else None
    d.lora_b[0] = b_d.data_ptr() if r else None
    d.scaling = 2.0
    la = (ctypes.c_void_p * 1)(a_d.data_ptr() if r else None)
    args = (ws.data_ptr(), len_d.data_ptr(), hq, hkv, 128, block, max_blocks, pk_d.data_ptr(),
            am_d.data_ptr(), code_d.data_ptr(), bs, la, ctypes.byref(d))

    # two-launch path
    h2 = _dev_bf16(res, dev)
    ss2 = torch.zeros(m, n // 64, dtype=torch.float32, device=dev)
    print(f"attn_residual m={m} hq={hq} r={r} bias={bias}: two-launch path", flush=True)
    _lib.check(lib.grpo_nf4_linear_partials_attn(*args, st), "partials_attn")
    _lib.check(lib.grpo_linear_finish_residual(ctypes.byref(d), h2.data_ptr(), h2.data_ptr(), ld,
                                               ss2.data_ptr(), st), "finish_residual")
    # the oracle on the merged bf16 attention rows
    xm = torch.zeros(m, k, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_paged_attn_merge(ws.data_ptr(), len_d.data_ptr(), m, hq, hkv, 128, block,
                                         max_blocks, xm.data_ptr(), 1, st), "merge")
    torch.cuda.synchronize()
    want = _bits(h2)
    lin = nf4_lora_linear(_bits(xm), packed, absmax, n, k, bs,
                          bias_bits=bias_bits if bias else None, a_bits=a if r else None,
                          b_bits=b if r else None, scaling=2.0)
    ref = f32_to_bf16_bits(bf16_bits_to_f32(lin) + bf16_bits_to_f32(res[:, :n]))

    tb, cb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    groups = lib.grpo_nf4_linear_attn_residual_groups(m, n, k, r, bs, ctypes.byref(tb),
                                                      ctypes.byref(cb))
    assert groups == n // 64
    gt = torch.zeros(max(tb.value, 16) // 4, dtype=torch.float32, device=dev)
    cnt = torch.zeros(cb.value // 4, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    for call in range(3):
        h = _dev_bf16(res, dev)
        ss = torch.full((m, groups), -1.0, dtype=torch.float32, device=dev)
        print(f"  fused call {call}", flush=True)
        _lib.check(lib.grpo_nf4_linear_attn_residual(*args, gt.data_ptr(), cnt.data_ptr(),
                                                     err.data_ptr(), h.data_ptr(), h.data_ptr(),
                                                     ld, ss.data_ptr(), st), "attn_residual")
        torch.cuda.synchronize()
        got = _bits(h)
        assert np.array_equal(got[:, n:], res[:, n:])  # columns past N untouched
        gf = bf16_bits_to_f32(got[:, :n])
        assert rel_err(gf, bf16_bits_to_f32(ref)) <= 1e-2
        assert np.mean(got[:, :n] == ref) >= 0.97
        assert rel_err(gf, bf16_bits_to_f32(want[:, :n])) <= 1e-2
        assert np.mean(got == want) >= 0.99, f"call {call}: {np.mean(got != want):.4f} differ"
        if call > 0:
            assert np.array_equal(got, first)  # deterministic
        first = got
        assert np.count_nonzero(cnt.cpu().numpy()) == 0
        assert int(err.item()) == 0  # every group's K slices ran on one XCD
        hf = bf16_bits_to_f32(got[:, :n]).astype(np.float64)
        ref_ss = (hf ** 2).reshape(m, groups, 64).sum(-1)
        assert np.allclose(ss.cpu().numpy(), ref_ss, rtol=1e-5, atol=1e-30)

    # new inputs through the same counters: another residual and other splits
    res2 = f32_to_bf16_bits(g.standard_normal((m, ld)).astype(np.float32))
    ws.mul_(-0.5)
    h2 = _dev_bf16(res2, dev)
    _lib.check(lib.grpo_nf4_linear_partials_attn(*args, st), "partials_attn")
    _lib.check(lib.grpo_linear_finish_residual(ctypes.byref(d), h2.data_ptr(), h2.data_ptr(), ld,
                                               ss2.data_ptr(), st), "finish_residual")
    h = _dev_bf16(res2, dev)
    ss = torch.zeros(m, groups, dtype=torch.float32, device=dev)
    _lib.check(lib.grpo_nf4_linear_attn_residual(*args, gt.data_ptr(), cnt.data_ptr(),
                                                 err.data_ptr(), h.data_ptr(), h.data_ptr(), ld,
                                                 ss.data_ptr(), st), "attn_residual")
    torch.cuda.synchronize()
    got, want = _bits(h), _bits(h2)
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(want)) <= 1e-2
    assert np.mean(got == want) >= 0.99
    assert np.count_nonzero(cnt.cpu().numpy()) == 0
    assert int(err.item()) == 0


def test_attn_residual_rejects_unsupported(dev):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    tb, cb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.grpo_nf4_linear_attn_residual_groups(17, 1536, 1536, 16, 64, ctypes.byref(tb),
                                                    ctypes.byref(cb)) == 0  # M > 16
    assert lib.grpo_nf4_linear_attn_residual_groups(8, 1552, 1536, 16, 64, ctypes.byref(tb),
                                                    ctypes.byref(cb)) == 0  # N % 64
    assert lib.grpo_nf4_linear_attn_residual_groups(8, 1536, 1536, 16, 64, ctypes.byref(tb),
                                                    ctypes.byref(cb)) == 24
