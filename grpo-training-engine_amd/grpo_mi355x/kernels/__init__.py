"""Operator registry of the rollout decode path (mirror of ``src/triton_kernels/__init__.py``).

Exports the reference's hot-path operator surface:

* ``paged_kv_decode(model, input_ids, attention_mask=None, max_new_tokens=128,
  **kwargs)`` -- routes to the low-level paged loop when all of ``k_cache,
  v_cache, block_tables, context_lens, qkv_proj_fn, logits_fn`` are given
  (``__init__.py:234-262``), else to the model-level decode
  (``__init__.py:264-296``);
* ``lora_fused_forward(...)`` (``__init__.py:323-354``);
* ``HIP_AVAILABLE`` (and ``TRITON_AVAILABLE``, the reference's flag name, as an
  alias so callers such as ``src/grpo/trainer.py:387`` keep working).

Unlike the reference, an unavailable backend never falls back to a PyTorch/CPU
implementation: the operators raise ``ImportError`` (the reference's own
signal for "no kernel backend", ``__init__.py:297``).
"""

from __future__ import annotations

from importlib import import_module
from typing import Callable

import torch

from .. import _lib

HIP_AVAILABLE: bool = _lib.available()
TRITON_AVAILABLE: bool = HIP_AVAILABLE  # name kept for drop-in callers

_kernel_cache: dict[str, Callable[..., object] | None] = {}

_EXPLICIT_MODULES = {
    "paged_kv_decode": "grpo_mi355x.kernels.paged_kv",
    "lora_fused_forward": "grpo_mi355x.kernels.lora_forward",
    "paged_kv_decode_model": "grpo_mi355x.rollout.decode",
}


def _get_hip_kernel(name: str) -> Callable[..., object] | None:
    """Name -> callable lookup (``__init__.py:98-127``), cached."""
    if not HIP_AVAILABLE:
        return None
    if name in _kernel_cache:
        return _kernel_cache[name]
    kernel = None
    module_name = _EXPLICIT_MODULES.get(name)
    if module_name is not None:
        kernel = getattr(import_module(module_name), name, None)
    _kernel_cache[name] = kernel
    return kernel


def _unavailable(name: str) -> ImportError:
    try:
        _lib.device_library()
        reason = "kernel not registered"
    except ImportError as exc:
        reason = str(exc)
    return ImportError(f"HIP kernels are not available for {name}: {reason}")


def paged_kv_decode(model: object, input_ids: object, attention_mask: object | None = None,
                    max_new_tokens: int = 128, **kwargs: object) -> object:
    kernel = _get_hip_kernel("paged_kv_decode")
    if kernel is None:
        raise _unavailable("paged_kv_decode")
    input_ids_t = input_ids
    low_level_args = ["k_cache", "v_cache", "block_tables", "context_lens", "qkv_proj_fn",
                      "logits_fn"]
    if all(arg in kwargs for arg in low_level_args):
        return kernel(
            input_ids_t,
            k_cache=kwargs["k_cache"],
            v_cache=kwargs["v_cache"],
            block_tables=kwargs["block_tables"],
            context_lens=kwargs["context_lens"],
            qkv_proj_fn=kwargs["qkv_proj_fn"],
            logits_fn=kwargs["logits_fn"],
            max_new_tokens=max_new_tokens,
            do_sample=kwargs.pop("do_sample", True),
            temperature=kwargs.pop("temperature", 1.0),
            top_p=kwargs.pop("top_p", 1.0),
            pad_token_id=kwargs.pop("pad_token_id", None),
            eos_token_id=kwargs.pop("eos_token_id", None),
            seed=kwargs.pop("seed", None),
            attention_mask=attention_mask,
            use_cache=kwargs.pop("use_cache", None),
        )
    model_kernel = _get_hip_kernel("paged_kv_decode_model")
    if model_kernel is None:
        raise _unavailable("paged_kv_decode_model")
    # the reference's model-path defaults (src/triton_kernels/__init__.py:283-296)
    return model_kernel(model, input_ids_t, attention_mask=attention_mask,
                        max_new_tokens=max_new_tokens,
                        do_sample=kwargs.pop("do_sample", True),
                        temperature=kwargs.pop("temperature", 1.0),
                        top_p=kwargs.pop("top_p", 1.0),
                        pad_token_id=kwargs.pop("pad_token_id", 0),
                        eos_token_id=kwargs.pop("eos_token_id", None),
                        seed=kwargs.pop("seed", None),
                        block_size=kwargs.pop("block_size", 16), **kwargs)


def lora_fused_forward(x: object, base_layer: object | None = None, lora_A: object | None = None,
                       lora_B: object | None = None, scaling: float | None = None,
                       dropout: object | None = None, lora_layer: object | None = None,
                       prefer_base_layer: bool = False) -> object:
    kernel = _get_hip_kernel("lora_fused_forward")
    if kernel is None:
        raise _unavailable("lora_fused_forward")
    return kernel(x, base_layer=base_layer, lora_A=lora_A, lora_B=lora_B, scaling=scaling,
                  dropout=dropout, lora_layer=lora_layer, prefer_base_layer=prefer_base_layer)


__all__ = ["HIP_AVAILABLE", "TRITON_AVAILABLE", "paged_kv_decode", "lora_fused_forward"]
