"""Temperature / top-p sampling oracle -- TEST INFRASTRUCTURE ONLY.

Restates the reference's sampled-token rule on bf16 logits,
``fused_logits_sampling`` (``src/triton_kernels/fused_ops.py:236-248``):

1. ``scaled = logits / max(T, 1e-6)``: torch on the GPU multiplies a bf16 tensor
   by the float32 reciprocal of a scalar divisor and rounds to bf16
   (:func:`scaled_bits`);
2. sort descending, ``probs = softmax(sorted)`` in bf16 (float32 math, each
   probability rounded to bf16), ``cumulative = probs.cumsum()``;
3. ``cutoff = cumulative > top_p``: a bf16 comparison (``top_p`` becomes a bf16
   scalar), the first token is always kept; a token is kept while the bf16
   running sum is <= bf16(top_p) (:func:`keep_bound`);
4. ``softmax`` over the kept logits (others ``-inf``), one multinomial draw.

This restatement fixes every rounding point so that a kernel can reproduce it
bit for bit:

* ``exp`` is :func:`exp_nonpos` (Cody-Waite reduction + degree-7 Taylor
  polynomial, every operation rounded once; torch's ``expf`` differs by a few
  float32 ulps, far below the bf16 rounding of the probabilities);
* the softmax sums are exact fixed-point sums of the float32 exponentials
  (2^-44 units, converted to float32 once) instead of float32 sums in torch's
  reduction order;
* the running sum is exact (2^-62 units) and rounded to bf16 once per token,
  as torch's CPU ``cumsum`` does (float accumulation); torch's GPU ``cumsum``
  keeps a bf16 running total between blocks of the scan, which moves the cut
  by the rounding it accumulates -- an artifact of its scan blocking, not of
  the rule;
* ties in the sort are ordered by index (a stable sort), which decides which of
  several equal logits at the cut are kept;
* the draw is the inverse CDF of the kept bf16 probabilities, taken in sorted
  order (value descending, index ascending), at a 64-bit uniform ``r``:
  ``t = floor(r * W / 2^64)`` with ``W`` their 2^-62 fixed-point total; torch's
  ``multinomial`` picks ``argmax(p / E)`` with ``E ~ Exp(1)``, the same
  distribution.

Pins (tests/test_oracle_sampling.py): the kept set against torch's CPU ops
(sort, softmax, cumsum, compare) on the same bf16 logits, a known-answer case,
the closed forms of top_p >= 1 (no cut) and top_p <= 0 (first token only), tie
order against a stable sort, :func:`exp_nonpos` against float64 ``exp``, and the
draw's token frequencies under evenly spaced ``r`` against the kept
probabilities.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

F32 = np.float32
# exp: x = n*ln2 + r, ln2 = LN2_HI + LN2_LO with LN2_HI = 0x3F317200 (14
# significant bits, so n * LN2_HI is exact for |n| < 2^10).
L2E = F32(1.4426950408889634)
LN2_HI = F32(0.693145751953125)
LN2_LO = F32(1.4286068203094173e-06)
TAYLOR = [F32(1.0) / F32(d) for d in (5040.0, 720.0, 120.0, 24.0, 6.0, 2.0, 1.0, 1.0)]
EXP_MIN_X = F32(-86.0)  # exp(x) is returned as 0 for x <= -86 (below 2^-124)
Z_BITS = 44             # fixed-point fraction bits of the softmax sums
P_BITS = 62             # fixed-point fraction bits of the running sum and the draw


def exp_nonpos(x) -> np.ndarray:
    """exp(x) for float32 x <= 0, every operation rounded to float32 once."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        n = np.rint(x * L2E).astype(F32)
        r = (x - n * LN2_HI) - n * LN2_LO
        p = TAYLOR[0]
        for c in TAYLOR[1:]:
            p = (p * r).astype(F32) + c
        p = p.astype(F32)
        e = np.ldexp(p, np.where(x > EXP_MIN_X, n, 0).astype(np.int32)).astype(F32)
    return np.where(x > EXP_MIN_X, e, F32(0.0)).astype(F32)


def u64_to_f32(v: int) -> np.float32:
    """Nonnegative integer -> float32, round to nearest even (exact, no double step)."""
    v = int(v)
    if v == 0:
        return F32(0.0)
    nb = v.bit_length()
    if nb <= 24:
        return F32(v)
    sh = nb - 24
    q, rem = v >> sh, v & ((1 << sh) - 1)
    half = 1 << (sh - 1)
    if rem > half or (rem == half and (q & 1)):
        q += 1
    return F32(np.ldexp(np.float64(q), sh))


def scaled_bits(logit_bits, temperature: float) -> np.ndarray:
    """bf16(logits * float32(1 / max(T, 1e-6))) as bf16 bit patterns."""
    inv = F32(1.0) / F32(max(float(temperature), 1e-6))
    return f32_to_bf16_bits(bf16_bits_to_f32(logit_bits) * inv)


def keep_bound(top_p: float):
    """Largest running sum (2^-62 units) whose bf16 rounding is <= bf16(top_p);
    None when top_p >= 1 (no cut).  Negative when every token is cut but the first."""
    if top_p >= 1.0:
        return None
    b = int(f32_to_bf16_bits(np.array([top_p], dtype=F32))[0])
    bval = float(bf16_bits_to_f32(np.array([b], dtype=np.uint16))[0])
    if not bval > 0.0:
        return -1
    exp = int(np.floor(np.log2(bval)))
    while 2.0 ** exp > bval:
        exp -= 1
    while 2.0 ** (exp + 1) <= bval:
        exp += 1
    half_ulp = 2.0 ** (exp - 8)           # half the bf16 spacing above bval
    mid = int(round((bval + half_ulp) * 2.0 ** P_BITS))
    return mid if (b & 1) == 0 else mid - 1  # ties at the midpoint round to even


def _bf16_key(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32)
    return np.where(b & 0x8000, b ^ 0xFFFF, b ^ 0x8000)


def sample_row(logit_bits, temperature: float, top_p: float, draw: int):
    """One row: returns (token, number of kept tokens)."""
    s_bits = scaled_bits(np.asarray(logit_bits, dtype=np.uint16), temperature)
    V = s_bits.size
    key = _bf16_key(s_bits)
    s = bf16_bits_to_f32(s_bits)
    kmax = int(key.max())
    m = s[int(np.argmax(key == kmax))]
    if not np.isfinite(m):
        return int(np.argmax(key == kmax)), 1
    e = exp_nonpos((s - m).astype(F32))
    e44 = (e.astype(np.float64) * 2.0 ** Z_BITS).astype(np.uint64)
    z = u64_to_f32(sum(int(v) for v in e44[e44 > 0]))
    zf = F32(np.ldexp(np.float64(z), -Z_BITS))
    p = bf16_bits_to_f32(f32_to_bf16_bits(e / zf))
    p62 = [int(v) for v in (p.astype(np.float64) * 2.0 ** P_BITS).astype(np.uint64)]
    order = np.lexsort((np.arange(V), -key.astype(np.int64)))  # value desc, index asc
    bound = keep_bound(top_p)
    kept = np.ones(V, dtype=bool)
    nkept = V
    if bound is not None:
        cum = 0
        nkept = 0
        for j in order:
            cum += p62[j]
            if cum > bound:
                break
            nkept += 1
        nkept = max(1, nkept)
        kept[:] = False
        kept[order[:nkept]] = True
    zk = u64_to_f32(sum(int(v) for v in e44[kept]))
    zkf = F32(np.ldexp(np.float64(zk), -Z_BITS))
    q = np.where(kept, bf16_bits_to_f32(f32_to_bf16_bits(e / zkf)), F32(0.0))
    q62 = [int(v) for v in (q.astype(np.float64) * 2.0 ** P_BITS).astype(np.uint64)]
    W = sum(q62)
    t = (int(draw) * W) >> 64
    acc = 0
    for i in order:  # the kept tokens in sorted order (others have q = 0)
        acc += q62[i]
        if acc > t:
            return int(i), nkept
    return int(order[0]), nkept


def sample_rows(logit_bits, temperature: float, top_p: float, draws):
    """Every row of ``logit_bits`` [M, V]: (tokens [M], kept counts [M])."""
    lb = np.asarray(logit_bits, dtype=np.uint16)
    out = [sample_row(lb[i], temperature, top_p, int(draws[i])) for i in range(lb.shape[0])]
    return (np.array([o[0] for o in out], dtype=np.int64),
            np.array([o[1] for o in out], dtype=np.int64))


# SplitMix64 output function (Steele, Lea and Flood, "Fast splittable
# pseudorandom number generators", OOPSLA 2014).
_M64 = (1 << 64) - 1


def splitmix64(z: int) -> int:
    z = (z + 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def step_draw(seed: int, row: int, step: int) -> int:
    """The decode loop's 64-bit uniform for ``row`` at its ``step``-th token."""
    return splitmix64((int(seed) + splitmix64(((row & 0xFFFFFFFF) << 32) | (step & 0xFFFFFFFF)))
                      & _M64)
