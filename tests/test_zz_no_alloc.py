"""The allocation-free attention entry (grpo_paged_attn_decode_noalloc) against
grpo_paged_attn_decode with a caller workspace, through the C ABI.

Both run the same kernels, so the outputs must be equal bit for bit.  Two calls
in a row, the second with a smaller input (fewer sequences, shorter contexts),
so the second reads the scratch array the first call left behind; a generic
path shape (head_dim 64, no partials); a shape whose partials exceed the array
is refused before anything is launched.
"""

import numpy as np
import pytest
import torch

from conftest import rng

pytestmark = pytest.mark.gpu


def _case(dev, seed, B, hq, hkv, d, ctx_lo, ctx_hi, bs=16):
    g = rng(seed)
    ctx = g.integers(ctx_lo, ctx_hi + 1, B).astype(np.int32)
    nblk = [-(-int(c) // bs) for c in ctx]
    nb = sum(nblk) + 4
    perm = g.permutation(nb).astype(np.int32)
    width = max(nblk)
    tab = np.full((B, width), -1, np.int32)
    o = 0
    for b in range(B):
        tab[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    gen = torch.Generator().manual_seed(seed)
    kc = torch.randn((nb, hkv, bs, d), generator=gen).to(torch.bfloat16).to(dev)
    vc = torch.randn((nb, hkv, bs, d), generator=gen).to(torch.bfloat16).to(dev)
    q = torch.randn((B, hq, d), generator=gen).to(torch.bfloat16).to(dev)
    return q, kc, vc, torch.from_numpy(tab).to(dev), torch.from_numpy(ctx).to(dev)


def _call(lib, q, kc, vc, tab, lens, out, ws=None):
    from grpo_mi355x import _lib

    B, hq, d = q.shape
    nb, hkv, bs, _ = kc.shape
    args = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), nb,
            tab.data_ptr(), tab.stride(0), lens.data_ptr(), out.data_ptr(), 0, B, hq, hkv, d, bs,
            tab.shape[1], float(d) ** -0.5)
    st = _lib.stream_handle(q.device)
    if ws is None:
        return lib.grpo_paged_attn_decode_noalloc(*args, st)
    return lib.grpo_paged_attn_decode(*args, ws.data_ptr() if ws.numel() else None, ws.numel(),
                                      st)


@pytest.mark.parametrize("shape", [
    [(8, 12, 2, 128, 512, 1024), (3, 12, 2, 128, 17, 200)],   # fast path, then smaller
    [(4, 28, 4, 128, 1024, 4096), (2, 28, 4, 128, 1, 40)],
    [(5, 8, 2, 64, 100, 300), (2, 8, 2, 64, 1, 30)],          # generic path (D = 64)
])
def test_noalloc_matches_workspace_entry_on_two_calls(dev, shape):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    assert lib.grpo_paged_attn_noalloc_max_bytes() == 8 << 20
    for i, (B, hq, hkv, d, lo, hi) in enumerate(shape):
        print(f"no-alloc attention call {i}: B={B} Hq={hq} Hkv={hkv} D={d} ctx U[{lo},{hi}]",
              flush=True)
        q, kc, vc, tab, lens = _case(dev, 100 + i, B, hq, hkv, d, lo, hi)
        need = lib.grpo_paged_attn_workspace_bytes(B, hq, hkv, d, 16, tab.shape[1])
        ws = torch.zeros(max(need, 0), dtype=torch.uint8, device=dev)
        want = torch.empty((B, hq, d), dtype=torch.float32, device=dev)
        got = torch.full((B, hq, d), float("nan"), dtype=torch.float32, device=dev)
        assert _call(lib, q, kc, vc, tab, lens, want, ws) == 0
        assert _call(lib, q, kc, vc, tab, lens, got) == 0, lib.grpo_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_noalloc_refuses_shapes_beyond_its_array(dev):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    # the largest partials the fast path plans: 8 splits while B * Hkv < 256
    B, hq, hkv, d, width = 255, 8, 1, 128, 512
    need = lib.grpo_paged_attn_workspace_bytes(B, hq, hkv, d, 16, width)
    assert need > lib.grpo_paged_attn_noalloc_max_bytes()
    q = torch.zeros((B, hq, d), dtype=torch.bfloat16, device=dev)
    kc = torch.zeros((4, hkv, 16, d), dtype=torch.bfloat16, device=dev)
    tab = torch.zeros((B, width), dtype=torch.int32, device=dev)
    lens = torch.ones(B, dtype=torch.int32, device=dev)
    out = torch.zeros((B, hq, d), dtype=torch.float32, device=dev)
    rc = _call(lib, q, kc, kc, tab, lens, out)
    assert rc == -3  # GRPO_EWORKSPACE, nothing launched
    assert b"allocation-free" in lib.grpo_last_error()
