"""Decode-loop and decode-step oracle (test infrastructure only).

* ``sample_tokens``   -- ``src/triton_kernels/paged_kv.py:418-450``.
* ``paged_kv_decode`` -- the low-level paged decode loop,
                         ``paged_kv.py:840-985``.
* ``rmsnorm``         -- ``fused_ops.py:34-77`` (= transformers' Qwen2RMSNorm).
* ``rope_tables`` / ``apply_rope`` -- transformers' ``Qwen2RotaryEmbedding`` and
                         ``apply_rotary_pos_emb`` (``fused_ops.py:198-219``).
* ``silu_mul``        -- ``fused_ops.py:79-112``.
* ``Qwen2DecodeOracle.step`` -- one model-level decode step
                         (``paged_kv.py:690-820``) with a GQA-native cache and
                         per-sequence block tables (the intended semantics, not
                         the reference's shared ``arange`` table).
"""

from __future__ import annotations

from typing import Callable

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from .lora_linear import nf4_lora_linear, nf4_weight_bf16
from .paged import append_kv, paged_attention_decode


# ----------------------------------------------------------------- sampling

def apply_top_p(logits: np.ndarray, top_p: float) -> np.ndarray:
    """``paged_kv.py:418-434``: keep the smallest prefix whose mass exceeds top_p."""
    if top_p >= 1.0:
        return logits
    if top_p <= 0.0:
        return np.full_like(logits, -np.inf)
    order = np.argsort(-logits, axis=-1, kind="stable")
    srt = np.take_along_axis(logits, order, axis=-1).astype(np.float64)
    p = np.exp(srt - srt.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    cut = np.cumsum(p, axis=-1) > top_p
    cut[..., 0] = False
    srt = np.where(cut, -np.inf, srt)
    out = np.full(logits.shape, -np.inf)
    np.put_along_axis(out, order, srt, axis=-1)
    return out


def sampling_probs(logits: np.ndarray, temperature: float, top_p: float) -> np.ndarray:
    """``paged_kv.py:446-448``: ``softmax(_apply_top_p(logits / max(T, 1e-6), top_p))``
    in float64, the distribution the multinomial draw of ``:449`` samples."""
    scaled = apply_top_p(np.asarray(logits, dtype=np.float64) / max(temperature, 1e-6), top_p)
    p = np.exp(scaled - scaled.max(axis=-1, keepdims=True))
    return p / p.sum(axis=-1, keepdims=True)


def sample_tokens(logits: np.ndarray, do_sample: bool, temperature: float, top_p: float,
                  rng: np.random.Generator | None = None) -> np.ndarray:
    """``paged_kv.py:437-450``: greedy argmax (first max) unless sampling."""
    logits = np.asarray(logits, dtype=np.float64)
    if not do_sample or temperature <= 0.0:
        return np.argmax(logits, axis=-1)
    p = sampling_probs(logits, temperature, top_p)
    rng = rng or np.random.default_rng()
    return np.array([rng.choice(p.shape[-1], p=row) for row in p])


# ------------------------------------------------------ low-level decode loop

def paged_kv_decode(input_ids: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                    block_tables: np.ndarray, context_lens: np.ndarray,
                    qkv_proj_fn: Callable, logits_fn: Callable, max_new_tokens: int = 128,
                    temperature: float = 1.0, top_p: float = 1.0, do_sample: bool = True,
                    eos_token_id: int | None = None, pad_token_id: int | None = None,
                    rng: np.random.Generator | None = None) -> np.ndarray:
    """``paged_kv.py:840-985`` on numpy arrays.

    Per step: q,k,v = qkv_proj_fn(last_tokens) rounded to bf16 (``:906-912``);
    append at the pre-increment length (``:914-936``); ``context_lens +=
    ~finished`` (``:938``); attention (``:942-969``); logits_fn on the float32
    attention output (``:971``); sample (``:975``); finished rows emit
    ``input_ids[:, 0]`` (``:978``).  Caches (bf16 bits) are mutated in place.
    """
    if max_new_tokens <= 0:
        raise ValueError(f"max_new_tokens must be > 0, got {max_new_tokens}.")
    eos = -1 if eos_token_id is None else eos_token_id
    pad = 0 if pad_token_id is None else pad_token_id
    B = input_ids.shape[0]
    D = k_cache.shape[3]
    scale = 1.0 / np.sqrt(D)
    ctx = np.asarray(context_lens, dtype=np.int64).copy()
    generated = np.full((B, max_new_tokens), pad, dtype=np.int64)
    last = input_ids[:, -1].copy()
    finished = np.zeros(B, dtype=bool)
    for step in range(max_new_tokens):
        if finished.all():
            break
        q, k, v = qkv_proj_fn(last)
        qb = f32_to_bf16_bits(q)
        append_kv(k_cache, v_cache, f32_to_bf16_bits(k), f32_to_bf16_bits(v), block_tables, ctx)
        ctx = ctx + (~finished).astype(np.int64)
        attn = paged_attention_decode(qb, k_cache, v_cache, block_tables, ctx, scale)
        logits = logits_fn(attn)
        nxt = sample_tokens(logits, do_sample, temperature, top_p, rng)
        nxt = np.where(finished, input_ids[:, 0], nxt)
        generated[:, step] = nxt
        last = nxt
        if eos >= 0:
            finished = finished | (nxt == eos)
    return generated


# ------------------------------------------------------------- decode step

def rmsnorm(x_bits, w_bits, eps: float) -> np.ndarray:
    """``fused_ops.py:34-77``: float32 mean square, ``bf16(x*rsqrt(ms+eps)) * w``."""
    x = bf16_bits_to_f32(x_bits)
    ms = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    normed = round_bf16(x * inv)
    return f32_to_bf16_bits(normed * bf16_bits_to_f32(w_bits))


def rope_tables(positions, head_dim: int, theta: float):
    """cos/sin ``[len(positions), head_dim]`` as bf16 bits (Qwen2RotaryEmbedding).

    ``inv_freq = 1 / theta**(arange(0, D, 2)/D)`` in float32; ``freqs = inv_freq
    * pos`` in float32; ``emb = cat(freqs, freqs)``; cos/sin cast to bf16.
    """
    d = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    inv_freq = (1.0 / (np.float64(theta) ** d.astype(np.float64))).astype(np.float32)
    freqs = (np.asarray(positions, dtype=np.float32)[:, None] * inv_freq[None, :]).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1).astype(np.float64)
    return f32_to_bf16_bits(np.cos(emb)), f32_to_bf16_bits(np.sin(emb))


def apply_rope(x_bits, cos_bits, sin_bits) -> np.ndarray:
    """``x*cos + rotate_half(x)*sin`` in bf16 arithmetic; x ``[B, H, D]``, cos ``[B, D]``."""
    x = bf16_bits_to_f32(x_bits)
    c = bf16_bits_to_f32(cos_bits)[:, None, :]
    s = bf16_bits_to_f32(sin_bits)[:, None, :]
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return f32_to_bf16_bits(round_bf16(x * c) + round_bf16(rot * s))


def silu_mul(g_bits, u_bits) -> np.ndarray:
    """``fused_ops.py:79-112``: ``bf16(bf16(silu(g)) * u)``."""
    g = bf16_bits_to_f32(g_bits).astype(np.float64)
    silu = round_bf16((g / (1.0 + np.exp(-g))).astype(np.float32))
    return f32_to_bf16_bits(silu * bf16_bits_to_f32(u_bits))


def bf16_residual(a_bits, b_bits) -> np.ndarray:
    return f32_to_bf16_bits(bf16_bits_to_f32(a_bits) + bf16_bits_to_f32(b_bits))


class Qwen2DecodeOracle:
    """One decode step of a Qwen2-shaped model with NF4 weights and LoRA on q/k/v/o.

    ``weights`` (numpy, bf16 as uint16 bits):
      ``embed [V, H]``, ``norm [H]``, ``lm_head [V, H]``, ``layers``: list of dicts
      with ``input_norm``, ``post_norm`` and, for each of ``q k v o gate up down``,
      a dict ``{packed, absmax, n, k, bias?, A?, B?}``.
    ``cfg``: ``hidden, n_heads, n_kv, head_dim, eps, theta, blocksize, scaling``.
    """

    PROJ = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, weights: dict, cfg: dict, cache_dequant: bool = True):
        self.w = weights
        self.cfg = cfg
        self._deq = {}
        self.cache_dequant = cache_dequant

    def _linear(self, li: int, name: str, x_bits) -> np.ndarray:
        p = self.w["layers"][li][name]
        key = (li, name)
        wf = self._deq.get(key)
        if wf is None:
            wf = nf4_weight_bf16(p["packed"], p["absmax"], p["n"], p["k"], self.cfg["blocksize"])
            if self.cache_dequant:
                self._deq[key] = wf
        return nf4_lora_linear(x_bits, p["packed"], p["absmax"], p["n"], p["k"], self.cfg["blocksize"],
                               bias_bits=p.get("bias"), a_bits=p.get("A"), b_bits=p.get("B"),
                               scaling=self.cfg["scaling"], weight_f32=wf)

    def step(self, tokens, k_caches, v_caches, block_tables, context_lens,
             with_logits: bool = True):
        """Embed ``tokens`` at positions ``context_lens``; append; attend; return logits.

        Returns ``(logits bf16 bits [B, V], greedy next tokens [B])``, or
        ``(None, None)`` without ``with_logits`` (a prefill pass).  Every row's
        K/V of a layer is appended before that layer's attention, so rows at
        positions 0..n-1 sharing one block table compute a causal prefill.  The
        caches (lists of ``[NB, Hkv, BS, D]`` bf16 bits, one per layer) are
        appended to at ``context_lens[b]``; attention covers
        ``context_lens[b] + 1`` positions (``paged_kv.py:695-697, 731-761``).
        """
        c = self.cfg
        B = len(tokens)
        Hq, Hkv, D = c["n_heads"], c["n_kv"], c["head_dim"]
        pos = np.asarray(context_lens, dtype=np.int64)
        cos, sin = rope_tables(pos, D, c["theta"])
        h = self.w["embed"][np.asarray(tokens)]
        new_ctx = pos + 1
        scale = 1.0 / np.sqrt(D)
        for li, lw in enumerate(self.w["layers"]):
            res = h
            x = rmsnorm(h, lw["input_norm"], c["eps"])
            q = self._linear(li, "q", x).reshape(B, Hq, D)
            k = self._linear(li, "k", x).reshape(B, Hkv, D)
            v = self._linear(li, "v", x).reshape(B, Hkv, D)
            q = apply_rope(q, cos, sin)
            k = apply_rope(k, cos, sin)
            append_kv(k_caches[li], v_caches[li], k, v, block_tables, pos)
            attn = paged_attention_decode(q, k_caches[li], v_caches[li], block_tables, new_ctx, scale)
            attn_bits = f32_to_bf16_bits(attn).reshape(B, Hq * D)
            o = self._linear(li, "o", attn_bits)
            h = bf16_residual(res, o)
            res = h
            x = rmsnorm(h, lw["post_norm"], c["eps"])
            g = self._linear(li, "gate", x)
            u = self._linear(li, "up", x)
            d = self._linear(li, "down", silu_mul(g, u))
            h = bf16_residual(res, d)
        if not with_logits:
            return None, None
        h = rmsnorm(h, self.w["norm"], c["eps"])
        x = bf16_bits_to_f32(h).astype(np.float64)
        lm = self._deq.get("lm_head")
        if lm is None:
            lm = bf16_bits_to_f32(self.w["lm_head"]).astype(np.float64)
            if self.cache_dequant:
                self._deq["lm_head"] = lm
        logits = f32_to_bf16_bits((x @ lm.T).astype(np.float32))
        nxt = np.argmax(bf16_bits_to_f32(logits), axis=-1)
        return logits, nxt
