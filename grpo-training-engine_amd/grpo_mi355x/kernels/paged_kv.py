"""Paged-KV decode on the HIP kernels.

``paged_kv_decode`` keeps the signature and step semantics of the reference's
low-level entry (``src/triton_kernels/paged_kv.py:840-985``): per step,
``q, k, v = qkv_proj_fn(last_tokens)`` -> KV append at the pre-increment length
-> ``context_lens += ~finished`` -> attention (float32 output) ->
``logits_fn`` -> sampling -> finished rows emit ``input_ids[:, 0]``.

GQA extension: ``k_cache.shape[1]`` may be ``Hkv`` dividing the query head
count; ``qkv_proj_fn`` then returns ``q [B, Hq, D]`` and ``k, v [B, Hkv, D]``.
With ``Hkv == Hq`` this is exactly the reference contract.
"""

from __future__ import annotations

import math
from typing import Callable, Optional, Tuple

import torch

from . import ops


def _validate_inputs(input_ids, k_cache, v_cache, block_tables, context_lens):
    """``paged_kv.py:366-415`` (same checks, same ValueError messages)."""
    if input_ids.ndim != 2:
        raise ValueError(f"input_ids must be [batch, seq_len], got {input_ids.shape}.")
    if k_cache.ndim != 4 or v_cache.ndim != 4:
        raise ValueError("k_cache/v_cache must be [num_blocks, heads, block, head_dim].")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have identical shapes.")
    if block_tables.ndim != 2:
        raise ValueError(f"block_tables must be [batch, max_blocks], got {block_tables.shape}.")
    if context_lens.ndim != 1:
        raise ValueError(f"context_lens must be [batch], got {context_lens.shape}.")
    batch_size = input_ids.shape[0]
    if block_tables.shape[0] != batch_size:
        raise ValueError("block_tables batch dimension must match input_ids batch.")
    if context_lens.shape[0] != batch_size:
        raise ValueError("context_lens batch dimension must match input_ids batch.")
    if not (input_ids.is_cuda and k_cache.is_cuda and v_cache.is_cuda):
        raise ValueError("inputs and caches must be on CUDA device.")
    if not block_tables.is_cuda or not context_lens.is_cuda:
        raise ValueError("block_tables and context_lens must be on CUDA device.")
    if k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise ValueError("k_cache/v_cache must be bfloat16.")
    _, num_heads, block_size, head_dim = k_cache.shape
    max_context = block_tables.shape[1] * block_size
    return num_heads, block_size, head_dim, max_context


def _apply_top_p(logits: torch.Tensor, top_p: float) -> torch.Tensor:
    """``paged_kv.py:418-434``."""
    if top_p >= 1.0:
        return logits
    if top_p <= 0.0:
        return torch.full_like(logits, -float("inf"))
    sorted_logits, sorted_indices = torch.sort(logits, descending=True, dim=-1)
    probs = torch.softmax(sorted_logits, dim=-1)
    cutoff = probs.cumsum(dim=-1) > top_p
    cutoff[..., 0] = False
    sorted_logits = sorted_logits.masked_fill(cutoff, -float("inf"))
    filtered = torch.full_like(logits, -float("inf"))
    filtered.scatter_(dim=-1, index=sorted_indices, src=sorted_logits)
    return filtered


def _sample_tokens(logits: torch.Tensor, do_sample: bool, temperature: float, top_p: float,
                   generator: Optional[torch.Generator]) -> torch.Tensor:
    """``paged_kv.py:437-450``: greedy argmax unless sampling."""
    if not do_sample or temperature <= 0.0:
        return torch.argmax(logits, dim=-1)
    scaled = logits / max(temperature, 1e-6)
    probs = torch.softmax(_apply_top_p(scaled, top_p), dim=-1)
    return torch.multinomial(probs, num_samples=1, generator=generator).squeeze(-1)


@torch.no_grad()
def paged_kv_decode(
    input_ids: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    qkv_proj_fn: Callable[[torch.Tensor], Tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
    logits_fn: Callable[[torch.Tensor], torch.Tensor],
    max_new_tokens: int = 128,
    temperature: float = 1.0,
    top_p: float = 1.0,
    do_sample: bool = True,
    eos_token_id: Optional[int] = None,
    pad_token_id: Optional[int] = None,
    seed: Optional[int] = None,
    attention_mask: Optional[torch.Tensor] = None,
    use_cache: Optional[bool] = None,
) -> torch.Tensor:
    """Low-level paged decode loop; returns ``generated [B, max_new_tokens]``."""
    if max_new_tokens <= 0:
        raise ValueError(f"max_new_tokens must be > 0, got {max_new_tokens}.")
    num_kv_heads, block_size, head_dim, max_context = _validate_inputs(
        input_ids, k_cache, v_cache, block_tables, context_lens)
    if context_lens.max().item() >= max_context:
        raise ValueError("context_lens exceed block table capacity.")
    if eos_token_id is None:
        eos_token_id = -1
    if pad_token_id is None:
        pad_token_id = 0
    block_tables = block_tables.to(torch.int32).contiguous()
    context_lens = context_lens.to(torch.int32).contiguous()

    batch_size = input_ids.shape[0]
    generated = torch.full((batch_size, max_new_tokens), pad_token_id, device=input_ids.device,
                           dtype=input_ids.dtype)
    generator = None
    if seed is not None:
        generator = torch.Generator(device=input_ids.device)
        generator.manual_seed(seed)
    last_tokens = input_ids[:, -1]
    finished = torch.zeros(batch_size, device=input_ids.device, dtype=torch.bool)
    scale = 1.0 / math.sqrt(head_dim)

    for step in range(max_new_tokens):
        if finished.all():
            break
        q, k_new, v_new = qkv_proj_fn(last_tokens)
        if q.ndim != 3 or q.shape[0] != batch_size or q.shape[2] != head_dim \
                or q.shape[1] % num_kv_heads != 0:
            raise ValueError("qkv_proj_fn must return [B, H, D] tensors.")
        if k_new.shape != (batch_size, num_kv_heads, head_dim) or v_new.shape != k_new.shape:
            raise ValueError("qkv_proj_fn must return [B, H, D] tensors.")
        q = q.to(dtype=torch.bfloat16)
        ops.paged_kv_append(k_new.to(torch.bfloat16), v_new.to(torch.bfloat16), k_cache, v_cache,
                            block_tables, context_lens)
        context_lens = context_lens + (~finished).to(context_lens.dtype)
        attn_out = ops.paged_attention_decode(q, k_cache, v_cache, block_tables, context_lens,
                                              scale, out_dtype=torch.float32)
        logits = logits_fn(attn_out)
        if logits.ndim != 2 or logits.shape[0] != batch_size:
            raise ValueError("logits_fn must return [B, vocab] logits.")
        next_tokens = _sample_tokens(logits, do_sample, temperature, top_p, generator)
        next_tokens = torch.where(finished, input_ids[:, 0], next_tokens)
        generated[:, step] = next_tokens
        last_tokens = next_tokens
        if eos_token_id >= 0:
            finished = finished | (next_tokens == eos_token_id)
    # the one-launch attention's in-kernel merges ran on one XCD per pair
    ops.attention_handover_check(input_ids.device)
    return generated


__all__ = ["paged_kv_decode"]
