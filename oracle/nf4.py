"""NF4 (4-bit NormalFloat) codebook, quantizer and dequantizer -- test oracle.

Storage format (the bitsandbytes ``Params4bit`` layout the reference reads in
``src/triton_kernels/lora_forward.py:171-206``):

* the weight ``W[N, K]`` is flattened row-major; element ``e = n*K + k``;
* two elements share one byte: ``byte = packed[e // 2]``; the EVEN element is
  the HIGH nibble (``byte >> 4``), the odd element the LOW nibble
  (``byte & 0xF``) -- ``lora_forward.py:173-181``;
* ``absmax`` holds one float32 scale per ``blocksize`` consecutive flat
  elements: ``a = absmax[e // blocksize]`` -- ``lora_forward.py:186, 201-202``;
* the dequantized value is ``bf16(code[q] * a)``: one float32 multiply, then
  round-to-nearest-even to bfloat16 -- ``lora_forward.py:183-184, 204-206``.

``dequantize_nf4`` is the bit-exact restatement of that.  ``quantize_nf4`` is
this repository's own input generator (nearest code by midpoint comparison,
ties to the lower code); the bitsandbytes quantizer's tie-breaking is not
reproduced and is not on any parity path (weights are generated, then only
dequantized).
"""

from __future__ import annotations

import numpy as np

from .bf16 import f32_to_bf16_bits, to_bits

# The 16 NF4 levels published with QLoRA (Dettmers et al. 2023, appendix E),
# identical to bitsandbytes' ``nf4`` map.  Pinned in tests against the closed
# form built from normal quantiles.
NF4_CODE = np.array(
    [
        -1.0,
        -0.6961928009986877,
        -0.5250730514526367,
        -0.39491748809814453,
        -0.28444138169288635,
        -0.18477343022823334,
        -0.09105003625154495,
        0.0,
        0.07958029955625534,
        0.16093020141124725,
        0.24611230194568634,
        0.33791524171829224,
        0.44070982933044434,
        0.5626170039176941,
        0.7229568362236023,
        1.0,
    ],
    dtype=np.float32,
)


def nf4_code_closed_form() -> np.ndarray:
    """NF4 levels from their definition: normal quantiles, normalised to [-1, 1].

    8 positive quantiles at ``linspace(offset, 0.5, 9)[:-1]``, 7 negative ones
    at ``linspace(offset, 0.5, 8)[:-1]``, plus an exact zero; ``offset`` is
    ``0.9677083`` (QLoRA appendix E).  Needs scipy.
    """
    from scipy.stats import norm

    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1]).tolist()
    neg = (-norm.ppf(np.linspace(offset, 0.5, 8)[:-1])).tolist()
    v = np.array(sorted(pos + [0.0] + neg), dtype=np.float64)
    return (v / np.abs(v).max()).astype(np.float32)


def quantize_nf4(w, blocksize: int = 64, code: np.ndarray = NF4_CODE):
    """Blockwise NF4 quantization of an array (flattened row-major).

    Returns ``(packed uint8 [ceil(n/2)], absmax float32 [ceil(n/blocksize)])``.
    Each block's scale is ``max|w|`` over the block (0 for an all-zero block);
    each element maps to the code nearest ``w / absmax``.
    """
    flat = np.asarray(w, dtype=np.float32).reshape(-1)
    n = flat.size
    nblocks = -(-n // blocksize)
    padded = np.zeros(nblocks * blocksize, dtype=np.float32)
    padded[:n] = flat
    blocks = padded.reshape(nblocks, blocksize)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    safe = np.where(absmax == 0, np.float32(1), absmax)
    scaled = blocks / safe[:, None]
    mids = (code[1:].astype(np.float64) + code[:-1].astype(np.float64)) / 2
    q = np.searchsorted(mids, scaled.astype(np.float64).reshape(-1), side="left")
    q = q[:n].astype(np.uint8)
    if n % 2:
        q = np.concatenate([q, np.zeros(1, np.uint8)])
    packed = ((q[0::2] << 4) | q[1::2]).astype(np.uint8)
    return packed, absmax


def nibbles(packed, numel: int) -> np.ndarray:
    """Code index of every flat element (``lora_forward.py:171-181``)."""
    e = np.arange(numel, dtype=np.int64)
    byte = np.asarray(packed, dtype=np.uint8).reshape(-1)[e >> 1]
    return np.where((e & 1) == 0, byte >> 4, byte & 0xF).astype(np.int64)


def nested_absmax(absmax_q, code2, absmax2, blocksize2: int, offset) -> np.ndarray:
    """Float32 absmax of a double-quantized state, per block
    (``lora_forward.py:187-199``): ``code2[q] * absmax2[blk // bs2] + offset``
    rounded once, as the fused multiply-add the reference kernel compiles to
    (Triton contracts the multiply and add by default).  The product of two
    float32 values is exact in float64; the float64 sum is rounded to float32
    (a double rounding only for a sum within 2^-53 of a float32 midpoint).
    bitsandbytes' own dequantize rounds the product first, then adds the
    offset (``nested_absmax_two_roundings``)."""
    q = np.asarray(absmax_q).reshape(-1).astype(np.int64)
    blk = np.arange(q.size, dtype=np.int64)
    c2 = np.asarray(code2, dtype=np.float32)[q].astype(np.float64)
    a2 = np.asarray(absmax2, dtype=np.float32).reshape(-1)[blk // int(blocksize2)]
    return (c2 * a2.astype(np.float64) + np.float64(np.float32(offset))).astype(np.float32)


def nested_absmax_two_roundings(absmax_q, code2, absmax2, blocksize2: int, offset) -> np.ndarray:
    """bitsandbytes' form of the same expansion: float32 product, then + offset."""
    q = np.asarray(absmax_q).reshape(-1).astype(np.int64)
    blk = np.arange(q.size, dtype=np.int64)
    c2 = np.asarray(code2, dtype=np.float32)[q]
    a2 = np.asarray(absmax2, dtype=np.float32).reshape(-1)[blk // int(blocksize2)]
    return ((c2 * a2).astype(np.float32) + np.float32(offset)).astype(np.float32)


def block_scales(absmax, numel: int, blocksize: int, nested: dict | None = None):
    """Per-element float32 scale (``lora_forward.py:186-202``).

    ``nested`` (bitsandbytes double quantization) is a dict with ``code``
    (float32 [256]), ``absmax`` (float32), ``blocksize`` and ``offset``; the
    block scales are then :func:`nested_absmax` of the uint8 ``absmax``.
    """
    blk = np.arange(numel, dtype=np.int64) // blocksize
    if nested is None:
        return np.asarray(absmax, dtype=np.float32).reshape(-1)[blk]
    full = nested_absmax(absmax, nested["code"], nested["absmax"], int(nested["blocksize"]),
                         nested["offset"])
    return full[blk]


def quantize_absmax_nested(absmax, blocksize2: int = 256, code2=None):
    """Double quantization of float32 block scales (test-data generator in the
    shape bitsandbytes produces: uint8 codes of ``absmax - mean`` per
    ``blocksize2`` blocks with a signed 256-entry codebook).  Returns
    ``(q uint8, code2 float32 [256], absmax2 float32, offset float32)``."""
    a = np.asarray(absmax, dtype=np.float32).reshape(-1)
    if code2 is None:
        code2 = np.linspace(-1.0, 1.0, 256, dtype=np.float32)
    code2 = np.asarray(code2, dtype=np.float32)
    offset = np.float32(a.astype(np.float64).mean())
    c = (a - offset).astype(np.float32)
    nb2 = -(-a.size // blocksize2)
    pad = np.zeros(nb2 * blocksize2, dtype=np.float32)
    pad[: a.size] = c
    a2 = np.abs(pad.reshape(nb2, blocksize2)).max(axis=1).astype(np.float32)
    a2 = np.where(a2 == 0, np.float32(1.0), a2).astype(np.float32)
    ratio = pad.reshape(nb2, blocksize2) / a2[:, None]
    q = np.abs(ratio[..., None] - code2[None, None, :]).argmin(axis=-1).astype(np.uint8)
    return q.reshape(-1)[: a.size], code2, a2, offset


def dequantize_nf4(packed, absmax, numel: int, blocksize: int,
                   code: np.ndarray = NF4_CODE, nested: dict | None = None,
                   dtype: str = "bf16") -> np.ndarray:
    """Bit-exact NF4 dequantization; returns bfloat16 bit patterns (uint16).

    ``w = bf16_rne(float32(code[q]) * float32(a))`` per element
    (``lora_forward.py:183-206``); ``dtype="f16"`` rounds to float16 instead
    (the reference's cast to a float16 LoRA / gradient dtype, ``:206, 343``).
    """
    if nested is None and numel % blocksize == 0 and blocksize % 2 == 0:
        return _dequantize_blocked(packed, absmax, numel, blocksize, code, dtype)
    q = nibbles(packed, numel)
    c = np.asarray(code, dtype=np.float32)[q]
    a = block_scales(absmax, numel, blocksize, nested)
    w = (c * a).astype(np.float32)
    return to_bits(w, dtype)


def _dequantize_blocked(packed, absmax, numel: int, blocksize: int, code,
                        dtype: str = "bf16") -> np.ndarray:
    """Same values as the element-wise path, computed per whole block.

    A 256-entry table gives (code[hi], code[lo]) per byte; each block of
    ``blocksize`` elements (``blocksize/2`` bytes) is multiplied by its absmax;
    identical float32 products, identical rounding.  Used to keep the CPU
    baseline of a full-model step within seconds.
    """
    c = np.asarray(code, dtype=np.float32)
    lut = np.stack([c[np.arange(256) >> 4], c[np.arange(256) & 15]], axis=1)  # [256, 2]
    nblk = numel // blocksize
    by = np.asarray(packed, dtype=np.uint8).reshape(-1)[: numel // 2].reshape(nblk, blocksize // 2)
    a = np.asarray(absmax, dtype=np.float32).reshape(-1)[:nblk]
    w = lut[by] * a[:, None, None]  # [nblk, bs/2, 2] float32
    return to_bits(w.reshape(-1), dtype)
