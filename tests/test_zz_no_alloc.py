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


_CHILD = r"""
import sys
sys.path[:0] = sys.argv[1:3]
import torch
from grpo_mi355x import _lib

lib = _lib.library()  # loaded, grpo_init not called: nothing has resolved the scratch address
dev = torch.device("cuda:0")
gen = torch.Generator().manual_seed(7)
B, hq, hkv, d, bs, width = 6, 12, 2, 128, 16, 40
nb = B * width
kc = torch.randn((nb, hkv, bs, d), generator=gen).to(torch.bfloat16).to(dev)
vc = torch.randn((nb, hkv, bs, d), generator=gen).to(torch.bfloat16).to(dev)
q = torch.randn((B, hq, d), generator=gen).to(torch.bfloat16).to(dev)
tab = torch.randperm(nb, generator=gen).to(torch.int32).view(B, width).to(dev)
lens = torch.tensor([640, 17, 1, 333, 600, 129], dtype=torch.int32, device=dev)
got = torch.zeros((B, hq, d), dtype=torch.float32, device=dev)
want = torch.zeros((B, hq, d), dtype=torch.float32, device=dev)
need = lib.grpo_paged_attn_workspace_bytes(B, hq, hkv, d, bs, width)
ws = torch.zeros(need, dtype=torch.uint8, device=dev)

def args(out):
    return (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), nb,
            tab.data_ptr(), tab.stride(0), lens.data_ptr(), out.data_ptr(), 0, B, hq, hkv, d, bs,
            width, float(d) ** -0.5)

torch.cuda.synchronize()
side = torch.cuda.Stream(device=dev)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=side):
    rc = lib.grpo_paged_attn_decode_noalloc(*args(got), _lib.stream_handle(dev))
print("first call inside capture: rc", rc, flush=True)
assert rc == 0, lib.grpo_last_error()
assert lib.grpo_paged_attn_decode(*args(want), ws.data_ptr(), need,
                                  _lib.stream_handle(dev)) == 0
for i in range(3):
    got.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    same = torch.equal(got.view(torch.int32), want.view(torch.int32))
    print("replay", i, "bit-equal", same, flush=True)
    assert same
    lens.add_(1)  # the next replay reads the new lengths, as does the eager reference
    assert lib.grpo_paged_attn_decode(*args(want), ws.data_ptr(), need,
                                      _lib.stream_handle(dev)) == 0
    torch.cuda.synchronize()
print("ok", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(dev):
    """The entry's first call in a process (where it resolves its scratch
    array's device address) made inside a HIP graph capture: the capture
    succeeds and every replay equals the workspace entry bit for bit.  Run in
    a child process so that no earlier call has resolved the address."""
    import subprocess
    import sys

    from conftest import PKG, ROOT

    r = subprocess.run([sys.executable, "-c", _CHILD, ROOT, PKG], capture_output=True,
                       text=True, timeout=180)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert r.stdout.strip().endswith("ok")
