"""Paged KV cache addressing, append and decode attention -- test oracle.

Cache layout (``src/triton_kernels/paged_kv.py:378-415``): ``k_cache`` and
``v_cache`` are ``[num_blocks, H, block_size, D]``; sequence ``b``'s token at
position ``pos`` lives in physical block ``block_tables[b, pos // block_size]``
at offset ``pos % block_size`` (``paged_kv.py:97-107, 279-284``).

The reference caches ``H = Hq`` heads (``repeat_kv`` before caching,
``paged_kv.py:723-724``).  This oracle is GQA-native: the cache holds ``Hkv``
heads and query head ``h`` reads KV head ``h // (Hq // Hkv)``, which is exactly
``transformers``' ``repeat_kv`` mapping (``modeling_qwen2.py:repeat_kv``), so it
reduces to the reference when ``Hkv == Hq``.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32


def slot_of(block_tables: np.ndarray, b: int, pos, block_size: int):
    """(physical block, offset) of logical position(s) ``pos`` of sequence ``b``."""
    pos = np.asarray(pos, dtype=np.int64)
    return block_tables[b, pos // block_size].astype(np.int64), pos % block_size


def gather_kv(cache: np.ndarray, block_tables: np.ndarray, b: int, ctx_len: int) -> np.ndarray:
    """Dense ``[ctx_len, H, D]`` view of sequence ``b``'s cached rows."""
    bs = cache.shape[2]
    phys, off = slot_of(block_tables, b, np.arange(ctx_len), bs)
    return cache[phys, :, off, :]


def append_kv(k_cache: np.ndarray, v_cache: np.ndarray, k_new: np.ndarray, v_new: np.ndarray,
              block_tables: np.ndarray, context_lens: np.ndarray) -> None:
    """Write ``k_new[b]``/``v_new[b]`` (``[B, H, D]``) at slot ``context_lens[b]``.

    ``paged_kv.py:253-319``: the slot is the PRE-increment length; every head
    of the row is written.  Mutates the caches in place.
    """
    bs = k_cache.shape[2]
    for b in range(k_new.shape[0]):
        pos = int(context_lens[b])
        phys, off = slot_of(block_tables, b, pos, bs)
        k_cache[phys, :, off, :] = k_new[b]
        v_cache[phys, :, off, :] = v_new[b]


def paged_attention_decode(q_bits, k_cache_bits, v_cache_bits, block_tables, context_lens,
                           scale: float) -> np.ndarray:
    """Single-query attention per (sequence, query head) over the paged cache.

    ``paged_kv.py:63-251``: q/K/V are bf16 widened to float32 (``:120, :132,
    :240``); logits ``q.k * scale``; softmax over ``t < context_lens[b]``
    (``:99, :136, :181``); output ``sum_t w_t v_t / max(sum_t w_t, 1e-6)``
    (``:243-244``) in float32 (``:251``).  Computed in float64 here, then
    rounded to float32.  ``context_lens[b] == 0`` gives a zero row, as the
    reference's masked passes do.

    Shapes: q ``[B, Hq, D]``; caches ``[NB, Hkv, BS, D]`` (bf16 bits);
    returns float32 ``[B, Hq, D]``.
    """
    q = bf16_bits_to_f32(np.asarray(q_bits)).astype(np.float64)
    B, Hq, D = q.shape
    kc = np.asarray(k_cache_bits)
    vc = np.asarray(v_cache_bits)
    Hkv = kc.shape[1]
    rep = Hq // Hkv
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        K = bf16_bits_to_f32(gather_kv(kc, block_tables, b, ctx)).astype(np.float64)  # [ctx,Hkv,D]
        V = bf16_bits_to_f32(gather_kv(vc, block_tables, b, ctx)).astype(np.float64)
        for h in range(Hq):
            kh = h // rep
            logits = K[:, kh, :] @ q[b, h] * scale
            w = np.exp(logits - logits.max())
            out[b, h] = (w @ V[:, kh, :]) / max(w.sum(), 1e-6)
    return out.astype(np.float32)
