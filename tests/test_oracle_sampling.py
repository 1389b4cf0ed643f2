"""Pins of the sampling oracle (oracle/sampling.py), CPU only.

The oracle restates fused_logits_sampling (src/triton_kernels/fused_ops.py:236-248)
with every rounding point fixed.  These checks tie it to torch's own ops on the
same bf16 logits, to the closed forms of the rule's edge cases, and to the
mathematics of the draw, so that a dropped term, a flipped comparison, a wrong
tie order or an off-by-one in the cut fails one of them.
"""

import numpy as np
import pytest
import torch

from oracle import sampling as S
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits


def _bits(x):
    return f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def _torch_kept(s_bits, top_p):
    """The reference's keep mask, op for op with torch on the CPU (stable sort)."""
    s = torch.from_numpy(s_bits.astype(np.int16)).view(torch.bfloat16)
    srt, idx = torch.sort(s, descending=True, stable=True)
    cum = torch.softmax(srt, dim=-1).cumsum(dim=-1)
    cut = cum > top_p
    cut[0] = False
    keep = torch.zeros_like(cut)
    keep[idx] = ~cut
    return keep.numpy()


def test_exp_nonpos_accuracy_and_cutoff():
    x = np.linspace(-85.99, 0.0, 400001).astype(np.float32)
    e = S.exp_nonpos(x)
    ref = np.exp(x.astype(np.float64))
    assert np.max(np.abs(e - ref) / ref) < 3 * 2.0 ** -24
    assert S.exp_nonpos(np.float32(0.0)) == 1.0
    assert np.all(S.exp_nonpos(np.array([-86.0, -100.0, -np.inf], np.float32)) == 0.0)


def test_u64_to_f32_rounds_to_nearest_even():
    rng = np.random.default_rng(0)
    for v in [int(x) for x in rng.integers(0, 2 ** 62, 2000, dtype=np.int64)] + [2 ** 53 + 1]:
        f = S.u64_to_f32(v)
        ulp = 2.0 ** (int(np.floor(np.log2(float(f)))) - 23)
        err = abs(int(np.float64(f) * 1) - v) if float(f).is_integer() else None
        assert err is not None and err <= ulp / 2
    # exact halfway cases: 2^24 + 1 (halfway between 2^24 and 2^24 + 2) rounds to even
    assert S.u64_to_f32(2 ** 25 + 2) == np.float32(2 ** 25)      # tie -> even mantissa
    assert S.u64_to_f32(2 ** 25 + 6) == np.float32(2 ** 25 + 8)  # tie -> even mantissa
    assert S.u64_to_f32(2 ** 25 + 3) == np.float32(2 ** 25 + 4)


def test_scaled_bits_is_reciprocal_multiply_then_bf16():
    rng = np.random.default_rng(1)
    lb = _bits(rng.normal(0, 4, 5000))
    for T in (0.7, 1.0, 1.3, 1e-9):
        inv = np.float32(1.0) / np.float32(max(T, 1e-6))
        want = f32_to_bf16_bits(bf16_bits_to_f32(lb) * inv)
        assert np.array_equal(S.scaled_bits(lb, T), want)
    assert np.array_equal(S.scaled_bits(lb, 1.0), lb)


def test_keep_bound_is_the_bf16_comparison():
    """round_bf16(c) <= bf16(top_p) exactly when c <= keep_bound: the bound is
    the midpoint above bf16(top_p) (kept when bf16(top_p) is even, since torch
    rounds that tie down to it) or one unit below it; float32 values one step
    either side of the midpoint round to bf16(top_p) and above it in torch."""
    f32 = torch.float32
    for tp in (0.9, 0.5, 0.95, 0.3, 0.999, 0.1, 0.75, 0.898):
        b = S.keep_bound(tp)
        bp = torch.tensor(tp, dtype=f32).to(torch.bfloat16)
        odd = int(bp.view(torch.int16)) & 1
        mid = b + odd
        assert mid % (1 << 40) == 0  # a midpoint of bf16 values is a multiple of 2^-22
        m32 = torch.tensor(mid / 2.0 ** 62, dtype=torch.float64).to(f32)
        assert float(m32) == mid / 2.0 ** 62
        assert (float(m32.to(torch.bfloat16)) > float(bp)) == bool(odd)
        below = torch.nextafter(m32, torch.tensor(0.0, dtype=f32))
        above = torch.nextafter(m32, torch.tensor(2.0, dtype=f32))
        assert float(below.to(torch.bfloat16)) == float(bp)
        assert float(above.to(torch.bfloat16)) > float(bp)
        # the reference compares in bf16 (top_p becomes a bf16 scalar)
        assert bool(bp > tp) is False and bool(torch.tensor(float(above)).to(torch.bfloat16) > tp)
    assert S.keep_bound(1.0) is None and S.keep_bound(1.5) is None
    assert S.keep_bound(0.0) == -1 and S.keep_bound(-0.2) == -1


def test_known_answer_two_of_four_kept():
    """probs .5/.3/.15/.05, top_p 0.9: running sums .5, .8, .95 -> two kept,
    redrawn at .5/.8 and .3/.8 of the mass."""
    lb = _bits(np.log([0.5, 0.3, 0.15, 0.05]))
    toks = [S.sample_row(lb, 1.0, 0.9, d) for d in (0, 2 ** 63, 2 ** 64 - 1)]
    assert [t[1] for t in toks] == [2, 2, 2]
    assert [t[0] for t in toks] == [0, 0, 1]
    n = 4000
    draws = [int((i + 0.5) / n * 2 ** 64) for i in range(n)]
    counts = np.bincount([S.sample_row(lb, 1.0, 0.9, d)[0] for d in draws], minlength=4)
    p = bf16_bits_to_f32(f32_to_bf16_bits(np.float32(0.625)))  # bf16 of .5/.8
    assert abs(counts[0] - n * p) <= 8 and counts[2] == 0 and counts[3] == 0


def test_edge_cases_top_p_one_and_zero():
    rng = np.random.default_rng(2)
    lb = _bits(rng.normal(0, 3, 512))
    first = int(np.argmax(bf16_bits_to_f32(S.scaled_bits(lb, 0.7))))
    for d in (0, 2 ** 63, 2 ** 64 - 1, 12345):
        tok, kept = S.sample_row(lb, 0.7, 0.0, d)
        assert kept == 1 and tok == first
        tok, kept = S.sample_row(lb, 0.7, 1.0, d)
        assert kept == 512


def test_ties_are_kept_in_index_order():
    """64 equal logits, top_p 0.5: bf16(k/64) <= 0.5 for k <= 32, so the 32
    lowest indices are kept and draws spread evenly over them."""
    lb = _bits(np.full(64, 1.25))
    n = 64 * 50
    draws = [int((i + 0.5) / n * 2 ** 64) for i in range(n)]
    res = [S.sample_row(lb, 1.0, 0.5, d) for d in draws]
    assert {r[1] for r in res} == {32}
    counts = np.bincount([r[0] for r in res], minlength=64)
    assert np.all(counts[:32] == 100) and np.all(counts[32:] == 0)


@pytest.mark.parametrize("scale,T,top_p", [(2.0, 0.7, 0.9), (0.5, 0.7, 0.9), (4.0, 1.0, 0.5),
                                           (1.0, 1.3, 0.95), (8.0, 0.7, 0.2)])
def test_kept_set_matches_torch_ops(scale, T, top_p):
    """The kept set equals torch's sort/softmax/cumsum/compare on the same
    scaled bf16 logits, except where torch's float32 running sum and the exact
    one straddle the bound (checked: then the counts differ by one token)."""
    rng = np.random.default_rng(int(scale * 100 + T * 10))
    exact = 0
    for row in range(12):
        lb = _bits(rng.normal(0, scale, 4096))
        s_bits = S.scaled_bits(lb, T)
        keep_t = _torch_kept(s_bits, top_p)
        _, kept = S.sample_row(lb, T, top_p, 0)
        if int(keep_t.sum()) == kept:
            exact += 1
        else:
            assert abs(int(keep_t.sum()) - kept) <= 1
    assert exact >= 11


def test_draw_frequencies_follow_kept_probabilities():
    """Evenly spaced draws hit every kept token in proportion to its bf16
    probability renormalised over the kept set (up to one draw per token)."""
    rng = np.random.default_rng(3)
    lb = _bits(rng.normal(0, 2.0, 256))
    T, top_p, n = 0.7, 0.9, 20000
    draws = [int((i + 0.5) / n * 2 ** 64) for i in range(n)]
    res = [S.sample_row(lb, T, top_p, d) for d in draws]
    counts = np.bincount([r[0] for r in res], minlength=256)
    kept = res[0][1]
    s = bf16_bits_to_f32(S.scaled_bits(lb, T)).astype(np.float64)
    order = np.lexsort((np.arange(256), -s))
    keep = np.zeros(256, bool)
    keep[order[:kept]] = True
    q = np.where(keep, np.exp(s - s.max()), 0.0)
    q /= q.sum()
    assert np.all(counts[~keep] == 0)
    # bf16 rounding of each probability: 2^-8 relative, plus one draw
    assert np.all(np.abs(counts - n * q) <= n * q * 2.0 ** -7 + 1.5)


# ------------------------------------------------ oracle.decode (float64 rule)

from oracle import decode as Dec  # noqa: E402


def _torch_apply_top_p(logits, top_p):
    """``paged_kv.py:418-434`` op for op on float64 CPU tensors."""
    if top_p >= 1.0:
        return logits
    if top_p <= 0.0:
        return torch.full_like(logits, -float("inf"))
    srt, idx = torch.sort(logits, descending=True, dim=-1)
    cum = torch.softmax(srt, dim=-1).cumsum(dim=-1)
    cut = cum > top_p
    cut[..., 0] = False
    srt = srt.masked_fill(cut, -float("inf"))
    out = torch.full_like(logits, -float("inf"))
    out.scatter_(dim=-1, index=idx, src=srt)
    return out


@pytest.mark.parametrize("top_p", [1e-9, 0.3, 0.9, 0.999, 1.0, 0.0])
@pytest.mark.parametrize("T", [0.7, 1.0, 1e-7])
def test_decode_sampling_probs_match_torch_ops(T, top_p):
    g = np.random.default_rng(31)
    logits = g.standard_normal((6, 300)) * 3.0
    t = torch.from_numpy(logits)
    filt = _torch_apply_top_p(t / max(T, 1e-6), top_p)
    got = Dec.apply_top_p(logits / max(T, 1e-6), top_p)
    assert np.array_equal(np.isinf(got), torch.isinf(filt).numpy())
    fin = np.isfinite(got)
    assert np.array_equal(got[fin], filt.numpy()[fin])
    if top_p > 0.0:
        ref = torch.softmax(filt, dim=-1).numpy()
        p = Dec.sampling_probs(logits, T, top_p)
        assert np.allclose(p, ref, rtol=1e-12, atol=1e-15)
        kept = np.isfinite(got).sum(-1)
        if top_p < 1e-6:
            assert np.all(kept == 1)  # the first token is always kept
        if top_p >= 1.0:
            assert np.all(kept == logits.shape[-1])


def test_decode_top_p_cuts_the_crossing_token():
    """probs .5/.3/.15/.05 at top_p .75: cumulative .5, .8 -> the token that
    crosses the bound is cut (``cumulative > top_p``), so only one is kept."""
    logits = np.log(np.array([[0.5, 0.3, 0.15, 0.05]]))
    kept = np.isfinite(Dec.apply_top_p(logits, 0.75))
    assert kept.tolist() == [[True, False, False, False]]
    kept = np.isfinite(Dec.apply_top_p(logits, 0.85))
    assert kept.tolist() == [[True, True, False, False]]


def test_decode_sample_tokens_greedy_and_frequencies():
    g = np.random.default_rng(5)
    logits = g.standard_normal((3, 50))
    logits[1, 7] = logits[1, 9] = logits[1].max() + 1.0  # tie: first index wins
    want = torch.argmax(torch.from_numpy(logits), dim=-1).numpy()
    assert np.array_equal(Dec.sample_tokens(logits, False, 0.7, 0.9), want)
    assert np.array_equal(Dec.sample_tokens(logits, True, 0.0, 0.9), want)
    row = np.log(np.array([[0.4, 0.25, 0.2, 0.1, 0.05]]))
    p = Dec.sampling_probs(row, 1.0, 0.9)[0]   # cut after .4+.25+.2 = .85 < .9 < .95
    assert np.isclose(p[:4].sum(), 1.0) and p[4] == 0.0
    n = 20000
    r = np.random.default_rng(11)
    draws = np.array([Dec.sample_tokens(row, True, 1.0, 0.9, r)[0] for _ in range(n)])
    counts = np.bincount(draws, minlength=5)
    assert counts[4] == 0
    sigma = np.sqrt(n * p * (1 - p))
    assert np.all(np.abs(counts - n * p) <= 4.5 * sigma + 1)


def test_splitmix64_published_vectors():
    """Vigna's splitmix64.c: the generator's i-th output for seed s is the
    output function at s + (i-1)*0x9E3779B97F4A7C15.  Seed 1234567 gives the
    five values published with the Rosetta Code task "Pseudo-random
    numbers/Splitmix64"; seed 1477776061723855037 the first three of the
    rand_xoshiro crate's reference test."""
    gamma, m = 0x9E3779B97F4A7C15, (1 << 64) - 1
    got = [S.splitmix64((1234567 + i * gamma) & m) for i in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]
    got = [S.splitmix64((1477776061723855037 + i * gamma) & m) for i in range(3)]
    assert got == [1985237415132408290, 2979275885539914483, 13511426838097143398]
    # the same task's distribution check: floor(5 * next / 2^64), seed 987654321
    counts = [0] * 5
    s = 987654321
    for i in range(100000):
        counts[(S.splitmix64((s + i * gamma) & m) * 5) >> 64] += 1
    assert counts == [20027, 19892, 20073, 19978, 20030]
