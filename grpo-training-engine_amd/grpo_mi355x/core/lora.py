"""Manual LoRA wrapper over an NF4 linear (mirror of ``src/core/lora.py``).

``ManualLoRALayer`` keeps the reference's constructor, attributes
(``base_layer, rank, alpha, scaling = alpha/rank, use_triton,
prefer_base_layer, lora_A, lora_B, lora_dropout``) and ``forward`` dispatch
(``lora.py:50-147``): try the fused kernel; on ``ImportError``,
``RuntimeError`` or ``ValueError`` run ``base_layer(x) + B(A(x)) * scaling``
(``lora.py:125-137``).  ``base_layer`` is a ``Linear4bitNF4`` (or a
bitsandbytes ``Linear4bit``); its own forward dequantizes on the GPU, so no
branch here computes on the CPU.
"""

from __future__ import annotations

from typing import List, cast

import torch
import torch.nn as nn

from ..kernels import lora_fused_forward
from .nf4 import Linear4bitNF4


def _linear4bit_types() -> tuple[type, ...]:
    types: list[type] = [Linear4bitNF4]
    try:  # bitsandbytes is optional; its Linear4bit has the same surface
        import bitsandbytes as bnb  # type: ignore

        lin = getattr(getattr(bnb, "nn", None), "Linear4bit", None)
        if lin is not None:
            types.append(lin)
    except Exception:
        pass
    return tuple(types)


def _is_linear4bit(module: nn.Module) -> bool:
    return isinstance(module, _linear4bit_types())


class ManualLoRALayer(nn.Module):
    """``Y = W_4bit(x) + B(A(x)) * (alpha / rank)`` (``lora.py:50-163``)."""

    def __init__(self, base_layer, rank: int = 16, alpha: int = 32, dropout: float = 0.0,
                 use_triton: bool = True, prefer_base_layer: bool = False):
        super().__init__()
        self.base_layer = base_layer
        self.rank = rank
        self.alpha = alpha
        self.scaling = alpha / rank
        self.use_triton = use_triton  # name kept: selects the fused (HIP) kernel
        self.prefer_base_layer = prefer_base_layer
        self.base_layer.weight.requires_grad = False
        in_features = base_layer.in_features
        out_features = base_layer.out_features
        self.lora_A = nn.Linear(in_features, rank, bias=False)
        self.lora_B = nn.Linear(rank, out_features, bias=False)
        self.lora_dropout = nn.Dropout(p=dropout) if dropout > 0 else nn.Identity()
        nn.init.kaiming_uniform_(self.lora_A.weight, a=5 ** 0.5)
        nn.init.zeros_(self.lora_B.weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.use_triton:
            try:
                return cast(torch.Tensor, lora_fused_forward(
                    x, lora_layer=self, prefer_base_layer=self.prefer_base_layer))
            except (ImportError, RuntimeError, ValueError):
                pass
        try:
            base_output = self.base_layer(x)
            if base_output.requires_grad:
                base_output = base_output.clone()
            x_adapt = x.to(self.lora_A.weight.dtype)
            lora_output = self.lora_B(self.lora_A(self.lora_dropout(x_adapt)))
            lora_output = lora_output * self.scaling
            if lora_output.dtype != base_output.dtype:
                lora_output = lora_output.to(base_output.dtype)
            return base_output + lora_output
        except Exception:
            if not self.use_triton:
                raise
            return cast(torch.Tensor, lora_fused_forward(x, lora_layer=self))

    def merge_weights(self) -> torch.Tensor:
        """``W_base + B A * scaling`` with the base dequantized on the GPU (``lora.py:149-163``)."""
        base_weight = self.base_layer.dequantize()
        lora_weight = self.lora_B.weight @ self.lora_A.weight * self.scaling
        return base_weight + lora_weight


def inject_lora_layers(model: nn.Module, target_modules: List[str], rank: int = 16,
                       alpha: int = 32, dropout: float = 0.0, use_triton: bool = True,
                       prefer_base_layer: bool = False, verbose: bool = True,
                       dtype: torch.dtype = torch.bfloat16) -> int:
    """Wrap every 4-bit linear whose short name is in ``target_modules`` (``lora.py:166-233``)."""
    injected = 0
    for name, module in list(model.named_modules()):
        short = name.split(".")[-1]
        if short in target_modules and _is_linear4bit(module):
            parent_name = ".".join(name.split(".")[:-1])
            parent = model.get_submodule(parent_name) if parent_name else model
            layer = ManualLoRALayer(module, rank=rank, alpha=alpha, dropout=dropout,
                                    use_triton=use_triton, prefer_base_layer=prefer_base_layer)
            layer = layer.to(device=module.weight.device, dtype=dtype)
            setattr(parent, short, layer)
            injected += 1
    return injected


def get_lora_parameters(model: nn.Module) -> List[nn.Parameter]:
    """Trainable LoRA parameters (``lora.py:236-250``)."""
    return [p for n, p in model.named_parameters()
            if p.requires_grad and ("lora_A" in n or "lora_B" in n)]
