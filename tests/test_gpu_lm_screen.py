"""GPU tests of the screened greedy lm_head (grpo_lm_head_q8_tiles,
grpo_lm_head_screen[_norm], grpo_lm_head_exact_argmax /
grpo_lm_head_exact_advance_norm): the token must be the one the full bf16
pass gives (grpo_lm_head_argmax_tiles / _norm_tiles + grpo_decode_advance),
bit for bit, on random and adversarial inputs -- exact ties, an all-zero row,
near-ties below the int8 resolution, a dominant row, huge and tiny x, a
non-finite weight row -- and the screen's bounds must hold against the exact
logits.  The greedy rule is the reference's argmax of the bf16 logits
(paged_kv.py:444-445, 800-806)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
UB_OFF = 2048  # byte offset of the screen's bounds in the workspace (grpo_hip.h)


def _lib():
    from grpo_mi355x import _lib

    return _lib, _lib.device_library()


def _q8(lib, _l, w, dev):
    V, K = w.shape
    wq = torch.empty(V * K, dtype=torch.uint8, device=dev)
    scale = torch.empty(V, dtype=torch.float32, device=dev)
    rnorm = torch.empty(V, dtype=torch.float32, device=dev)
    _l.check(lib.grpo_lm_head_q8_tiles(w.data_ptr(), V, K, wq.data_ptr(), scale.data_ptr(),
                                       rnorm.data_ptr(), _l.stream_handle(dev)), "q8")
    return wq, scale, rnorm


def _tiles(lib, _l, w, dev):
    V, K = w.shape
    wt = torch.empty_like(w)
    _l.check(lib.grpo_lm_head_weight_tiles(w.data_ptr(), V, K, wt.data_ptr(),
                                           _l.stream_handle(dev)), "tiles")
    return wt


def _full(lib, _l, x, wt, V, K, dev, logits=None):
    M = x.shape[0]
    st = _l.stream_handle(dev)
    ws = torch.empty(int(lib.grpo_lm_head_workspace_bytes(M, V)), dtype=torch.uint8, device=dev)
    _l.check(lib.grpo_lm_head_argmax_tiles(x.data_ptr(), x.stride(0), wt.data_ptr(), V, K, M,
                                           None if logits is None else logits.data_ptr(), V,
                                           ws.data_ptr(), ws.numel(), st), "lm_head")
    nxt = torch.empty(M, dtype=torch.int64, device=dev)
    _l.check(lib.grpo_decode_advance(ws.data_ptr(), M, V, nxt.data_ptr(), None, None, None, None,
                                     None, None, None, 0, None, None, st), "advance")
    return nxt


def _screened(lib, _l, x, wq, scale, rnorm, wt, V, K, dev):
    M = x.shape[0]
    st = _l.stream_handle(dev)
    ws = torch.zeros(int(lib.grpo_lm_head_screen_workspace_bytes(M, V)), dtype=torch.uint8,
                     device=dev)
    _l.check(lib.grpo_lm_head_screen(x.data_ptr(), x.stride(0), wq.data_ptr(), scale.data_ptr(),
                                     rnorm.data_ptr(), V, K, M, ws.data_ptr(), ws.numel(), st),
             "screen")
    nxt = torch.full((M,), -7, dtype=torch.int64, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    _l.check(lib.grpo_lm_head_exact_argmax(x.data_ptr(), x.stride(0), wt.data_ptr(), V, K, M,
                                           ws.data_ptr(), ws.numel(), err.data_ptr(),
                                           nxt.data_ptr(), st),
             "exact")
    torch.cuda.synchronize()
    # the hand-over ran on one XCD per row and left its counters at zero
    assert int(err.item()) == 0
    assert bool((ws[:1024].view(torch.int32) == 0).all())
    return nxt, ws


def test_q8_layout_scale_and_residual_norm(dev):
    """The int8 copy: scale = fl(max|W[v]| / 127), q = rint(W / scale) stored as
    q + 128 in the screening order, and rnorm >= ||W - scale q||_2 (float64),
    within one float32 step of it."""
    _l, lib = _lib()
    g = torch.Generator().manual_seed(5)
    V, K = 64, 512
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16)
    w[3] = 0.0  # an all-zero row: scale 0, q 0, rnorm 0
    wd = w.to(dev)
    wq, scale, rnorm = _q8(lib, _l, wd, dev)
    torch.cuda.synchronize()
    wf = w.float()
    sc = wf.abs().amax(dim=1) / 127.0
    assert torch.equal(scale.cpu(), sc)
    q = torch.where(sc[:, None] > 0, torch.round(wf / torch.where(sc > 0, sc, 1)[:, None]),
                    torch.zeros_like(wf)).clamp(-127, 127)
    # order: byte (((t*KS + s)*4 + jj)*64 + lg*16 + ln)*16 + 8h + e holds
    # W[16t + ln][256s + 64jj + 32h + 8lg + e]
    KS = K // 256
    idx = torch.arange(V * K)
    e, h = idx % 8, (idx // 8) % 2
    ln, lg = (idx // 16) % 16, (idx // 256) % 4
    jj, rest = (idx // 1024) % 4, idx // 4096
    s_, t = rest % KS, rest // KS
    rows, cols = 16 * t + ln, 256 * s_ + 64 * jj + 32 * h + 8 * lg + e
    want = (q[rows, cols] + 128).to(torch.uint8)
    assert torch.equal(wq.cpu(), want)
    r = (w.double() - sc.double()[:, None] * q.double()).norm(dim=1)
    got = rnorm.cpu().double()
    assert torch.all(got >= r) and torch.all(got <= r * (1 + 2 ** -22) + 1e-45)
    assert float(got[3]) == 0.0


def _check_case(dev, x, w, expect_prune=True):
    _l, lib = _lib()
    V, K = w.shape
    wq, scale, rnorm = _q8(lib, _l, w, dev)
    wt = _tiles(lib, _l, w, dev)
    logits = torch.empty(x.shape[0], V, dtype=torch.bfloat16, device=dev)
    ref = _full(lib, _l, x, wt, V, K, dev, logits)
    got, ws = _screened(lib, _l, x, wq, scale, rnorm, wt, V, K, dev)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), (got.tolist(), ref.tolist())
    # the bounds hold against the exact logits (bf16 values of the full pass):
    # ub >= every logit of the tile, lb <= the largest logit of the workgroup
    M, NT = x.shape[0], V // 16
    ub = ws[UB_OFF:].view(torch.float32)[: M * NT].view(M, NT).cpu()
    zl = logits.float().cpu().view(M, NT, 16)
    fin = torch.isfinite(zl).all(dim=2)
    tile_max = zl.amax(dim=2)
    ok = torch.isnan(ub) | (ub >= tile_max - tile_max.abs() * 2 ** -8) | ~fin
    assert bool(ok.all())
    return ub, ref


@pytest.mark.parametrize("M,V,K,seed", [(8, 151936, 1536, 0), (1, 4096, 512, 1), (5, 8192, 256, 2),
                                        (8, 32768, 3584, 3)])
def test_screened_argmax_matches_full_random(dev, M, V, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    print(f"screened lm_head M={M} V={V} K={K} seed={seed}", flush=True)
    ub, _ = _check_case(dev, x, w)


def test_screened_argmax_adversarial(dev):
    """Exact ties (the first index wins), an all-zero row (every tile is a
    candidate; index 0), near-ties below the int8 resolution, a row that is a
    multiple of a weight row, huge and tiny x, negative logits and a NaN weight
    row (never wins)."""
    g = torch.Generator().manual_seed(9)
    M, V, K = 8, 16384, 1536
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16)
    w[4000:4004] = w[77]                   # exact ties with row 77
    w[9001] = w[9000]
    w[9001, :5] += 1e-4                    # a near-tie below the int8 step
    w[12345] = float("nan")                # a non-finite row
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    x[0] = w[77] * 3                       # the tied rows win; the first (77) must be chosen
    x[1] = 0.0                             # all-zero: index 0
    x[2] = w[9000] * 5                     # near-tie between 9000 and 9001
    x[3] = x[3] * 3e4                      # float16 range exceeded: every tile a candidate
    x[4] = x[4] * 1e-6                     # tiny x (float16 subnormals)
    x[5] = -w[500] * 4                     # a strongly negative direction
    print("screened lm_head adversarial rows", flush=True)
    _check_case(dev, x.to(dev), w.to(dev))


def test_screened_advance_norm_matches_full(dev):
    """The decode-step form: RMSNorm staged from h and the sums of squares, then
    the exact pass with grpo_decode_advance's bookkeeping; row state and tokens
    equal those of grpo_lm_head_argmax_norm_tiles + grpo_decode_advance, an
    inactive row keeps its token."""
    _l, lib = _lib()
    st = _l.stream_handle(dev)
    g = torch.Generator().manual_seed(21)
    M, V, K = 8, 151936, 1536
    h = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    nw = (torch.randn(K, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
    ss = (h.float() ** 2).reshape(M, K // 8, 8).sum(-1).contiguous()
    wq, scale, rnorm = _q8(lib, _l, w, dev)
    wt = _tiles(lib, _l, w, dev)

    def state():
        return dict(tokens=torch.arange(M, dtype=torch.int64, device=dev) + 1000,
                    pos=torch.arange(10, 10 + M, dtype=torch.int32, device=dev),
                    count=torch.arange(M, dtype=torch.int32, device=dev),
                    limit=torch.full((M,), 9, dtype=torch.int32, device=dev),
                    active=torch.tensor([1, 1, 0, 1, 1, 1, 1, 1], dtype=torch.uint8, device=dev),
                    eos=torch.tensor([-1], dtype=torch.int64, device=dev),
                    gen=torch.full((M, 9), -1, dtype=torch.int64, device=dev),
                    app=torch.zeros(M, dtype=torch.int32, device=dev),
                    alen=torch.zeros(M, dtype=torch.int32, device=dev),
                    nxt=torch.full((M,), -3, dtype=torch.int64, device=dev))

    a, b = state(), state()
    ws = torch.empty(int(lib.grpo_lm_head_workspace_bytes(M, V)), dtype=torch.uint8, device=dev)
    _l.check(lib.grpo_lm_head_argmax_norm_tiles(h.data_ptr(), K, ss.data_ptr(), K // 8,
                                                nw.data_ptr(), 1e-6, wt.data_ptr(), V, K, M, None,
                                                V, ws.data_ptr(), ws.numel(), st), "lm_head")
    _l.check(lib.grpo_decode_advance(ws.data_ptr(), M, V, a["nxt"].data_ptr(),
                                     a["tokens"].data_ptr(), a["pos"].data_ptr(),
                                     a["count"].data_ptr(), a["limit"].data_ptr(),
                                     a["active"].data_ptr(), a["eos"].data_ptr(),
                                     a["gen"].data_ptr(), 9, a["app"].data_ptr(),
                                     a["alen"].data_ptr(), st), "advance")
    sws = torch.zeros(int(lib.grpo_lm_head_screen_workspace_bytes(M, V)), dtype=torch.uint8,
                      device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    _l.check(lib.grpo_lm_head_screen_norm(h.data_ptr(), K, ss.data_ptr(), K // 8, nw.data_ptr(),
                                          1e-6, wq.data_ptr(), scale.data_ptr(), rnorm.data_ptr(),
                                          V, K, M, sws.data_ptr(), sws.numel(), st), "screen")
    _l.check(lib.grpo_lm_head_exact_advance_norm(
        h.data_ptr(), K, ss.data_ptr(), K // 8, nw.data_ptr(), 1e-6, wt.data_ptr(), V, K, M,
        sws.data_ptr(), sws.numel(), err.data_ptr(), b["nxt"].data_ptr(), b["tokens"].data_ptr(), b["pos"].data_ptr(),
        b["count"].data_ptr(), b["limit"].data_ptr(), b["active"].data_ptr(), b["eos"].data_ptr(),
        b["gen"].data_ptr(), 9, b["app"].data_ptr(), b["alen"].data_ptr(), st), "exact")
    torch.cuda.synchronize()
    for key in ("pos", "count", "active", "gen", "app", "alen"):
        assert torch.equal(a[key], b[key]), key
    act = a["active"].bool() | torch.tensor([1, 1, 0, 1, 1, 1, 1, 1], device=dev).bool()
    assert torch.equal(a["tokens"][act], b["tokens"][act])
    assert torch.equal(a["nxt"][act], b["nxt"][act])
    assert int(b["tokens"][2]) == 1002  # the inactive row keeps its token
    # the screen pruned: few candidate tiles per row
    NT = V // 16
    assert int(err.item()) == 0 and bool((sws[:1024].view(torch.int32) == 0).all())
    ub = sws[UB_OFF:].view(torch.float32)[: M * NT].view(M, NT)
    W = min(NT, 256)
    lbw = sws[UB_OFF:].view(torch.float32)[M * NT:M * NT + M * W].view(M, W)
    uv_off = (UB_OFF + 4 * (M * NT + M * W) + 15) // 16 * 16
    uv = sws[uv_off:uv_off + 16 * V].view(torch.bfloat16).view(V, 8)[:, :M].t().float()
    # the rows' bounds, rounded up to bf16: at least the tile bound's share of each row
    assert bool((uv.view(M, NT, 16).amax(dim=2) >= ub).all())
    assert bool((uv.view(M, NT, 16).amax(dim=2) <= ub + ub.abs() * 2 ** -7).all())
    thr = lbw.amax(dim=1)
    thr = thr - thr.abs() * 2 ** -6
    cand = (~(ub < thr[:, None])).sum(dim=1)
    rows = (~(uv < thr[:, None])).sum(dim=1)
    print("candidate tiles per row:", cand.tolist(), "candidate rows:", rows.tolist(), flush=True)
    assert int(cand.max()) <= NT // 50
