"""HIP top-p sampler (grpo_sample_top_p / grpo_sample_advance) against the
sampling oracle, bit for bit: the same bf16 logits and 64-bit draws give the
same token and the same number of kept tokens (the reference's rule,
src/triton_kernels/fused_ops.py:236-248, with every rounding point fixed as in
oracle/sampling.py)."""

import numpy as np
import pytest
import torch

from oracle import sampling as S
from oracle.bf16 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _lib_and_stream(dev):
    from grpo_mi355x import _lib

    return _lib, _lib.device_library(), _lib.stream_handle(dev)


def _logits(kind, M, V, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        x = rng.normal(0, 2.0, (M, V))
    elif kind == "flat":      # a random-init model: logits within a few hundredths
        x = rng.normal(0, 0.03, (M, V))
    elif kind == "peaked":
        x = rng.normal(0, 6.0, (M, V))
    elif kind == "ties":      # few distinct values: long runs of equal logits at the cut
        x = np.round(rng.normal(0, 1.0, (M, V)) * 2) / 2
    elif kind == "wide":      # values across zero up to ~40: the full LDS window
        x = rng.uniform(-60.0, 40.0, (M, V))
    elif kind == "spread":    # +-2^u over 105 binades: > 17408 distinct values in the
        # window, more than the compacted list holds (the bin-wise passes run)
        x = rng.choice([-1.0, 1.0], (M, V)) * np.exp2(rng.uniform(-100.0, 5.0, (M, V)))
    else:
        raise ValueError(kind)
    return f32_to_bf16_bits(x.astype(np.float32)).reshape(M, V)


def _draws(M, seed):
    rng = np.random.default_rng(seed)
    d = rng.integers(0, 2 ** 63, M, dtype=np.int64).astype(np.uint64) * np.uint64(2)
    d[0] = 0
    if M > 1:
        d[-1] = np.uint64(2 ** 64 - 1)
    return d


def _run(dev, bits, T, top_p, draws):
    _lib, lib, st = _lib_and_stream(dev)
    M, V = bits.shape
    lg = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)
    dr = torch.from_numpy(draws.view(np.int64)).to(dev)
    tok = torch.full((M,), -7, dtype=torch.int64, device=dev)
    kept = torch.full((M,), -7, dtype=torch.int32, device=dev)
    ws = _workspace(dev, lib, M, V)
    print(f"sample_top_p M={M} V={V} T={T} top_p={top_p}", flush=True)
    _lib.check(lib.grpo_sample_top_p(lg.data_ptr(), V, M, V, T, top_p, dr.data_ptr(),
                                     tok.data_ptr(), kept.data_ptr(), ws.data_ptr(), ws.numel(),
                                     st), "sample_top_p")
    torch.cuda.synchronize()
    # every call leaves the workspace zero-filled for the next one (bins cleared)
    assert not torch.any(ws.view(M, -1)[:, 288:]), "sampling bins not cleared"
    return tok.cpu().numpy(), kept.cpu().numpy()


def _workspace(dev, lib, M, V):
    return torch.zeros(int(lib.grpo_sample_workspace_bytes(M, V)), dtype=torch.uint8, device=dev)


@pytest.mark.parametrize("kind,M,V,T,top_p", [
    ("normal", 8, 151936, 0.7, 0.9),
    ("flat", 8, 151936, 0.7, 0.9),
    ("peaked", 8, 151936, 1.0, 0.5),
    ("ties", 8, 151936, 1.0, 0.9),
    ("wide", 4, 151936, 1.0, 0.999),
    ("spread", 4, 151936, 1.0, 0.9),
    ("spread", 2, 151936, 0.7, 1.0),
    ("normal", 64, 4096, 1.3, 0.95),
    ("normal", 8, 4096, 0.7, 1.0),
    ("normal", 8, 4096, 0.7, 0.0),
    ("peaked", 8, 4096, 1e-7, 0.9),
])
def test_sampler_matches_oracle_bit_for_bit(dev, kind, M, V, T, top_p):
    bits = _logits(kind, M, V, seed=sum(map(ord, kind)) + M + V)
    draws = _draws(M, seed=M + V)
    tok, kept = _run(dev, bits, T, top_p, draws)
    want_tok, want_kept = S.sample_rows(bits, T, top_p, draws)
    assert np.array_equal(kept, want_kept), (kept, want_kept)
    assert np.array_equal(tok, want_tok), (tok, want_tok)


def test_sampler_draw_sweep_and_non_finite_rows(dev):
    """One row under 256 evenly spaced draws (every kept token's share of the
    draws), and rows whose maximum is +inf or NaN (first index of it)."""
    V = 2048
    row = _logits("normal", 1, V, seed=5)[0]
    n = 256
    bits = np.repeat(row[None], n, axis=0)
    draws = np.array([int((i + 0.5) / n * 2 ** 64) for i in range(n)], dtype=np.uint64)
    tok, kept = _run(dev, bits, 0.7, 0.9, draws)
    want_tok, want_kept = S.sample_rows(bits, 0.7, 0.9, draws)
    assert np.array_equal(tok, want_tok) and np.array_equal(kept, want_kept)
    special = _logits("normal", 3, V, seed=6)
    special[0, 700] = 0x7F80          # +inf
    special[0, 900] = 0x7F80
    special[1, 33] = 0x7FC0           # NaN
    special[2, :] = 0x3F80            # every logit 1.0: all tied
    draws = np.array([5, 7, 2 ** 63], dtype=np.uint64)
    tok, kept = _run(dev, special, 1.0, 0.9, draws)
    want_tok, want_kept = S.sample_rows(special, 1.0, 0.9, draws)
    assert tok[0] == 700 and tok[1] == 33
    assert np.array_equal(tok, want_tok) and np.array_equal(kept, want_kept)


def test_torch_gpu_divides_by_a_scalar_as_reciprocal_multiply(dev):
    """The reference's `logits / T` on the GPU: bf16(logit * float32(1/T)), the
    scaling the oracle and the kernel use."""
    bits = _logits("normal", 4, 8192, seed=9)
    lg = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)
    for T in (0.7, 1.3, 0.3):
        got = (lg / max(T, 1e-6)).view(torch.int16).cpu().numpy().astype(np.uint16)
        assert np.array_equal(got, S.scaled_bits(bits, T))


def test_sample_advance_bookkeeping_and_draw_stream(dev):
    """grpo_sample_advance: row m draws SplitMix64(seed, m, count[m]); active
    rows record the token at generated[m, count[m]] and advance; stopped rows
    keep their token and state."""
    _lib, lib, st = _lib_and_stream(dev)
    M, V, seed = 6, 151936, 0xC0FFEE
    bits = _logits("normal", M, V, seed=12)
    lg = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)
    i32 = dict(dtype=torch.int32, device=dev)
    tokens = torch.arange(M, dtype=torch.int64, device=dev) + 100
    pos = torch.arange(M, **i32) + 20
    count = torch.tensor([0, 3, 5, 1, 0, 2], **i32)
    limit = torch.tensor([9, 4, 9, 9, 9, 9], **i32)
    active = torch.tensor([1, 1, 0, 1, 1, 1], dtype=torch.uint8, device=dev)
    gen = torch.full((M, 8), -1, dtype=torch.int64, device=dev)
    nxt = torch.full((M,), -9, dtype=torch.int64, device=dev)
    app = torch.zeros(M, **i32)
    alen = torch.zeros(M, **i32)
    c0, p0 = count.cpu().numpy().copy(), pos.cpu().numpy().copy()
    draws = np.array([S.step_draw(seed, m, int(c0[m])) for m in range(M)], dtype=np.uint64)
    want_tok, _ = S.sample_rows(bits, 0.7, 0.9, draws)
    eos = torch.tensor([int(want_tok[4])], dtype=torch.int64, device=dev)
    ws = _workspace(dev, lib, M, V)
    print("sample_advance M=6 V=151936", flush=True)
    _lib.check(lib.grpo_sample_advance(lg.data_ptr(), V, M, V, 0.7, 0.9, seed, nxt.data_ptr(),
                                       tokens.data_ptr(), pos.data_ptr(), count.data_ptr(),
                                       limit.data_ptr(), active.data_ptr(), eos.data_ptr(),
                                       gen.data_ptr(), 8, app.data_ptr(), alen.data_ptr(),
                                       ws.data_ptr(), ws.numel(), st), "sample_advance")
    torch.cuda.synchronize()
    was = [1, 1, 0, 1, 1, 1]
    for m in range(M):
        if was[m]:
            assert int(nxt[m]) == int(want_tok[m]) and int(tokens[m]) == int(want_tok[m])
            assert int(gen[m, c0[m]]) == int(want_tok[m])
            assert int(count[m]) == c0[m] + 1 and int(pos[m]) == p0[m] + 1
        else:
            assert int(tokens[m]) == 100 + m and int(nxt[m]) == 100 + m
            assert torch.all(gen[m] == -1) and int(count[m]) == c0[m] and int(pos[m]) == p0[m]
        still = bool(was[m]) and int(count[m]) < int(limit[m]) and int(tokens[m]) != int(eos[0])
        assert bool(active[m]) == still
        assert int(app[m]) == (int(pos[m]) if still else -1)
        assert int(alen[m]) == (int(pos[m]) + 1 if still else 0)
    assert not bool(active[1]) and not bool(active[4])  # limit reached / EOS drawn
