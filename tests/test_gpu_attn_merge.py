"""The decode-step attention that merges its context splits in the kernel
(``grpo_paged_attn_decode_qkv_merged``), through the C ABI.

Against the two-launch form on the same inputs -- ``grpo_paged_attn_decode_qkv``
(split partials) followed by ``grpo_paged_attn_merge`` (bf16 rows) -- the merged
output and the K/V cache must be identical bit for bit: the last-arriving split
combines the same partials in the same order and with the same float32 formula
as the merge kernel, and a row whose context fits one split divides by the
same denominator.  The split partials themselves are pinned against the oracle
by ``tests/test_gpu_attention.py`` and the decode-step tests.  The LoRA-A product
the kernel leaves for o_proj (``o_lora_t[b][kvh][r]``: the row's bf16 output
over the pair's heads times A) is checked against a float64 product of the
kernel's own output (tolerance 1e-5 relative).  Every case runs three calls in
a row through the same counters, which must be zero afterwards, with the XCD
check word still zero (every pair's splits ran on one XCD).
"""

import math

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.decode import rope_tables

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _dev(arr, dev):
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dev)


def _dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def _case(dev, m, hq, hkv, lens, r, seed):
    """Random q|k|v partial sums (as the split-K linear leaves them), a shuffled
    paged cache with room for one more token per row, RoPE tables."""
    from grpo_mi355x import _lib

    g = np.random.default_rng(seed)
    D, BS, S = 128, 16, 6
    N = (hq + 2 * hkv) * D
    lens = [int(l) for l in lens]  # -1: a stopped row (no append, length 0)
    max_blocks = max(-(-(max(l, 0) + 1) // BS) for l in lens) + 1
    nblk = sum(-(-(max(l, 0) + 1) // BS) for l in lens) + 4
    perm = g.permutation(nblk).astype(np.int32)
    tables = np.full((m, max_blocks), -1, np.int32)
    cur = 0
    for b, l in enumerate(lens):
        nb = -(-(max(l, 0) + 1) // BS)
        tables[b, :nb] = perm[cur:cur + nb]
        cur += nb
    kc = f32_to_bf16_bits(g.standard_normal((nblk, hkv, BS, D)).astype(np.float32))
    vc = f32_to_bf16_bits(g.standard_normal((nblk, hkv, BS, D)).astype(np.float32))
    part = (g.standard_normal((S, m, N)) * 0.3).astype(np.float32)
    tpart = (g.standard_normal((S, 3, m, 16)) * 0.05).astype(np.float32)
    segs = [hq * D, hkv * D, hkv * D]
    bias = [f32_to_bf16_bits((g.standard_normal(n) * 0.1).astype(np.float32)) for n in segs]
    lb = [f32_to_bf16_bits((g.standard_normal((n, 16)) * 0.05).astype(np.float32)) for n in segs]
    pos = np.asarray(lens, np.int32)  # append slot = tokens already cached (-1: none)
    alen = np.where(pos < 0, 0, pos + 1).astype(np.int32)
    cos, sin = rope_tables(np.arange(max_blocks * BS), D, 10000.0)
    a_o = f32_to_bf16_bits((g.standard_normal((max(r, 1), hq * D)) * 0.05).astype(np.float32))
    keep = dict(part=_dev(part.reshape(-1), dev), tpart=_dev(tpart.reshape(-1), dev),
                bias=[_dev_bf16(x, dev) for x in bias], lb=[_dev_bf16(x, dev) for x in lb])
    d = _lib.LinearParts()
    d.part, d.tpart = keep["part"].data_ptr(), keep["tpart"].data_ptr()
    d.splits, d.M, d.N, d.K, d.nseg, d.r = S, m, N, 1536, 3, 16
    end = 0
    for i, n in enumerate(segs):
        end += n
        d.seg_end[i] = end
        d.bias[i] = keep["bias"][i].data_ptr()
        d.lora_b[i] = keep["lb"][i].data_ptr()
    d.scaling = 2.0
    return dict(d=d, keep=keep, kc=kc, vc=vc, tables=_dev(tables, dev), max_blocks=max_blocks,
                nblk=nblk, pos=_dev(pos, dev), alen=_dev(alen, dev), cos=_dev_bf16(cos, dev),
                sin=_dev_bf16(sin, dev), max_pos=max_blocks * BS, a_o=a_o,
                a_o_dev=_dev_bf16(a_o, dev))


@pytest.mark.parametrize("m,hq,hkv,lens,r", [
    (8, 12, 2, [576, 1023, 5, 300, -1, 1000, 64, 0], 16),  # config 3 shape, ragged, stopped row
    (8, 12, 2, [40, 17, 3, 90, 100, 120, 7, 1], 16),       # short: every pair one split
    (4, 28, 4, [2047, 1024, 1500, 33], 16),                # Qwen2-7B heads
    (3, 12, 2, [800, 200, 511], 8),                        # rank 8
    (2, 12, 2, [700, 9], 0),                               # no LoRA
])
def test_merged_attention_matches_split_plus_merge(dev, m, hq, hkv, lens, r):
    from grpo_mi355x import _lib
    from grpo_mi355x.kernels import ops

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    c = _case(dev, m, hq, hkv, lens, r, seed=m * 31 + hq + r)
    D, BS = 128, 16
    mb = c["max_blocks"]
    nbytes = ops.paged_attention_workspace_bytes(m, hq, hkv, D, BS, mb)
    ws1 = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    ws2 = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    cnt = torch.zeros(int(lib.grpo_paged_attn_merge_counter_bytes(m, hkv)) // 4,
                      dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(D)

    def common(kcd, vcd):
        return (ctypes_parts(c["d"]), hq, hkv, D, c["cos"].data_ptr(), c["sin"].data_ptr(),
                c["max_pos"], c["pos"].data_ptr(), c["alen"].data_ptr(), kcd.data_ptr(),
                vcd.data_ptr(), c["nblk"], c["tables"].data_ptr(), mb, BS, mb, scale)

    # two-launch reference
    kc1, vc1 = _dev_bf16(c["kc"], dev), _dev_bf16(c["vc"], dev)
    out1 = torch.zeros(m, hq * D, dtype=torch.bfloat16, device=dev)
    print(f"merged attention m={m} hq={hq} hkv={hkv} r={r}: split + merge", flush=True)
    _lib.check(lib.grpo_paged_attn_decode_qkv(*common(kc1, vc1), ws1.data_ptr(), nbytes * 1, None,
                                              st), "attn_qkv")
    _lib.check(lib.grpo_paged_attn_merge(ws1.data_ptr(), c["alen"].data_ptr(), m, hq, hkv, D, BS,
                                         mb, out1.data_ptr(), 1, st), "merge")
    torch.cuda.synchronize()
    want = _bits(out1)
    for call in range(3):
        kc2, vc2 = _dev_bf16(c["kc"], dev), _dev_bf16(c["vc"], dev)
        out2 = torch.full((m, hq * D), 7.0, dtype=torch.bfloat16, device=dev)
        lt = torch.full((m, hkv, 16), -9.0, dtype=torch.float32, device=dev)
        print(f"  merged call {call}", flush=True)
        _lib.check(lib.grpo_paged_attn_decode_qkv_merged(
            *common(kc2, vc2), ws2.data_ptr(), nbytes * 1, cnt.data_ptr(), err.data_ptr(),
            out2.data_ptr(), c["a_o_dev"].data_ptr() if r else None, r,
            lt.data_ptr() if r else None, st), "attn_qkv_merged")
        torch.cuda.synchronize()
        got = _bits(out2)
        assert np.array_equal(got, want), f"call {call}: {np.mean(got != want):.5f} differ"
        assert np.array_equal(_bits(kc2), _bits(kc1)) and np.array_equal(_bits(vc2), _bits(vc1))
        assert np.count_nonzero(cnt.cpu().numpy()) == 0
        assert int(err.item()) == 0
        if r:
            x = bf16_bits_to_f32(got).astype(np.float64).reshape(m, hkv, -1)
            a = bf16_bits_to_f32(c["a_o"]).astype(np.float64)[:r].reshape(r, hkv, -1)
            ref = np.einsum("bhk,rhk->bhr", x, a)
            t = lt.cpu().numpy()
            np.testing.assert_allclose(t[:, :, :r], ref, rtol=1e-5,
                                       atol=1e-5 * np.abs(ref).max())


def ctypes_parts(d):
    import ctypes

    return ctypes.byref(d)
