"""``lora_fused_forward`` -- the NF4 + LoRA linear on the HIP kernel.

Same call surface and dispatch as the reference's
``src/triton_kernels/lora_forward.py:933-1037``:

* ``lora_layer`` (a ``ManualLoRALayer``-like object) or explicit
  ``base_layer/lora_A/lora_B/scaling/dropout``;
* dropout p > 0 -> ``ValueError`` (``:958-960``);
* a base weight with ``quant_state`` and ``prefer_base_layer=False`` -> the
  fused kernel (``FusedLoRAFunction``, ``:966-984``); otherwise the adapter
  branch ``base_layer(x) + B(A(x)) * scaling`` (``:986-1037``);
* shape/dtype/device problems -> ``ValueError`` (``_validate_inputs``,
  ``:435-487``); rank <= 0 -> ``ValueError`` (``:670-671``).

The fused forward is ``grpo_nf4_lora_linear``: the split-K kernel up to 64
rows, the NF4 GEMM (weight decoded in the kernel, epilogue fused) beyond, and
for the largest training batches (``fused_forward_rows``) the weight
dequantized once (bit-exact) plus bf16 GEMMs with the same rounding points.
float16 x with float16 adapters (the reference's float16 X_DTYPE / LORA_DTYPE,
``:141-143, 745-749``) runs the NF4 GEMM's float16 form at any M, every
rounding point float16; mixed dtypes raise ``ValueError`` (the caller's torch
branch then serves them, as for any shape the kernels do not take).  The backward (``:761-930``) keeps the
reference's gradients and rounding points: grad_x's NF4 product on the fused
``grpo_nf4_grad_x`` kernel (LoRA part added in its store) below
``GRAD_X_GEMM_MIN_ROWS`` rows for the shapes it tiles, otherwise dequantize +
bf16 GEMM; the rank-r products and the weight gradients are bf16 GEMMs.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import ops


def _validate_inputs(x: torch.Tensor, weight_4bit: torch.Tensor, quant_state,
                     lora_A: torch.Tensor, lora_B: torch.Tensor):
    """``lora_forward.py:435-487`` (same messages, same ValueError)."""
    if x.ndim != 3:
        raise ValueError(f"x must be [batch, seq_len, hidden], got {x.shape}.")
    if lora_A.ndim != 2 or lora_B.ndim != 2:
        raise ValueError("lora_A and lora_B must be 2D weight matrices.")
    if not x.is_cuda:
        raise ValueError("x must be on CUDA device.")
    if not weight_4bit.is_cuda:
        raise ValueError("weight_4bit must be on CUDA device.")
    if not lora_A.is_cuda or not lora_B.is_cuda:
        raise ValueError("lora_A and lora_B must be on CUDA device.")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"x must be float16/bfloat16, got {x.dtype}.")
    if lora_A.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"lora_A must be float16/bfloat16, got {lora_A.dtype}.")
    if lora_B.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"lora_B must be float16/bfloat16, got {lora_B.dtype}.")
    if lora_A.dtype != lora_B.dtype:
        raise ValueError(
            f"lora_A and lora_B must have the same dtype, got {lora_A.dtype} and {lora_B.dtype}.")
    batch, seq_len, in_features = x.shape
    out_features, in_features_w = tuple(quant_state.shape)
    if in_features != in_features_w:
        raise ValueError("Input hidden size does not match quantized weight shape: "
                         f"{in_features} vs {in_features_w}.")
    rank, in_features_a = lora_A.shape
    out_features_b, rank_b = lora_B.shape
    if in_features_a != in_features:
        raise ValueError(f"lora_A input features mismatch: {in_features_a} vs {in_features}.")
    if out_features_b != out_features or rank_b != rank:
        raise ValueError("lora_B shape mismatch: expected "
                         f"[{out_features}, {rank}], got {lora_B.shape}.")
    return batch * seq_len, out_features, in_features, rank


def _extract_quant_state(weight_4bit: torch.Tensor, quant_state):
    """``lora_forward.py:527-576``: the float32 absmax, codebook and blocksize.

    A double-quantized (nested) state's absmax is expanded to float32 once
    (``lora_forward.py:187-199``, see ``core.nf4.float_absmax``) and cached on
    the state: the base weights are frozen."""
    from ..core.nf4 import float_absmax

    device = weight_4bit.device
    if bool(getattr(quant_state, "nested", False)) and quant_state.absmax.device != device:
        raise ValueError("nested quant_state must be on the weight's device.")
    absmax = float_absmax(quant_state).to(device=device).contiguous()
    code = quant_state.code.to(device=device, dtype=torch.float32).contiguous()
    if absmax.dtype != torch.float32:
        raise ValueError(f"absmax must be float32 for a non-nested state, got {absmax.dtype}.")
    if code.numel() != 16:
        raise ValueError("quant_state.code must have 16 entries (a 4-bit codebook).")
    return absmax, code, int(quant_state.blocksize)


def _scalar_as(v: float, dtype: torch.dtype) -> float:
    """``v`` rounded to ``dtype`` (bf16 or float16), as a Python float:
    ``t * _scalar_as(v, t.dtype)`` is dtype(float(t) * dtype(v)), the
    reference's product with a 0-dim tensor of the LoRA dtype
    (lora_forward.py:836-837), without a host-to-device copy."""
    return float(torch.tensor(float(v), dtype=dtype))


def _bf16_scalar(v: float) -> float:
    """``_scalar_as(v, torch.bfloat16)``."""
    return _scalar_as(v, torch.bfloat16)


# Rows of grad_out from which grad_x's NF4 product runs as dequantize + bf16
# GEMM instead of the fused nf4_grad_x kernel.  Measured on MI355X at M = 4096
# over the Qwen2-1.5B projection shapes: the GEMM path is 1.8x (q, o) to 4.2x
# (gate, up) faster.  Below 1024 rows the fused kernel avoids writing and
# re-reading the whole dequantized weight for few rows.
GRAD_X_GEMM_MIN_ROWS = 1024


def fused_forward_rows(k: int) -> int:
    """Most rows for which the forward runs the fused NF4 GEMM rather than the
    dequantized weight + hipBLASLt.  Measured on MI355X over the Qwen2-1.5B
    projection shapes (r = 16): the fused GEMM is faster up to 4096 rows for
    K = 1536 (e.g. gate at 4096 rows: 217 us against 257 us) and up to 1024
    rows for down_proj's K = 8960 (96 against 84 us at 1024 rows with LoRA, 73
    against 84 without); from 8192 rows hipBLASLt's GEMM wins for every shape.
    """
    return 4096 if k <= 4096 else 1024


class FusedLoRAFunction(torch.autograd.Function):
    """Forward = one fused NF4+LoRA kernel launch (``lora_forward.py:653-759``);
    backward = the reference's gradients (``:761-930``): grad_x from the NF4
    weight on the HIP kernel with the LoRA part added in its store, the
    rank-r products as plain bf16 GEMMs (float32 accumulation)."""

    @staticmethod
    def forward(ctx, x, weight_4bit, quant_state, lora_A, lora_B, scaling, bias):
        m, n, k, r = _validate_inputs(x, weight_4bit, quant_state, lora_A, lora_B)
        if r <= 0:
            raise ValueError(f"LoRA rank must be > 0, got {r}.")
        if lora_A.dtype != x.dtype:
            raise ValueError("the HIP NF4+LoRA kernels take x and the adapters in one dtype "
                             f"(bfloat16 or float16); got x {x.dtype}, lora {lora_A.dtype}.")
        dt = x.dtype
        absmax, code, blocksize = _extract_quant_state(weight_4bit, quant_state)
        w = weight_4bit.contiguous().view(-1)
        if w.dtype != torch.uint8:
            w = w.view(torch.uint8)
        x_flat = x.contiguous().view(m, k)
        out = torch.empty((m, n), device=x.device, dtype=x.dtype)
        gemm_ok = m <= fused_forward_rows(k) and ops.nf4_gemm_supported(m, n, k, r, blocksize)
        fused = gemm_ok or (dt == torch.bfloat16
                            and ops.nf4_linear_plan(m, n, k, r, 1, blocksize) is not None)
        if m > 0 and n > 0 and not fused:
            # the largest batches: W dequantized once (bit-exact), then GEMMs
            # with the kernel's rounding points (lora_forward.py:246-257):
            # dt(x W^T), + bias, t = dt(x A^T), u = dt(dt(t B^T) * dt(scaling)),
            # y = dt(acc + u), dt = bf16 or float16
            wb = ops.nf4_dequant(w, absmax, code, n * k, blocksize, dtype=dt).view(n, k)
            acc = F.linear(x_flat, wb)
            if bias is not None:
                acc = acc + bias.to(acc.dtype)
            u = F.linear(F.linear(x_flat, lora_A), lora_B)
            out = torch.add(acc, u * _scalar_as(scaling, dt))
        elif m > 0 and n > 0:
            ops.nf4_lora_linear(x_flat, w, absmax, code, blocksize, n, bias=bias,
                                lora_a=lora_A, lora_b=lora_B, scaling=float(scaling), out=out)
        ctx.save_for_backward(x_flat, lora_A, lora_B, w, absmax, code)
        ctx.blocksize, ctx.scaling, ctx.has_bias = blocksize, float(scaling), bias is not None
        ctx.x_shape = x.shape
        return out.view(x.shape[:-1] + (n,))

    @staticmethod
    def backward(ctx, grad_out):
        x_flat, lora_A, lora_B, w, absmax, code = ctx.saved_tensors
        m, k = x_flat.shape
        n = lora_B.shape[0]
        dt = x_flat.dtype  # the adapters' dtype too (checked in forward)
        g = grad_out.contiguous().view(m, n)
        if g.dtype != dt:
            g = g.to(dt)
        grad_bias = g.sum(dim=0) if ctx.has_bias else None  # lora_forward.py:790
        # scaled_grad = dt(g * dt(scaling)) (:836-837); grad_intermediate,
        # grad_x_lora, xA, grad_B, grad_A: dt GEMMs, float32 accumulation (:839-928)
        sg = g * _scalar_as(ctx.scaling, dt)
        gi = torch.matmul(sg, lora_B)
        gxl = torch.matmul(gi, lora_A)
        if (dt != torch.bfloat16 or m >= GRAD_X_GEMM_MIN_ROWS
                or not ops.nf4_grad_x_supported(n, k, ctx.blocksize)):
            # float16, many rows, or a shape the fused bf16 kernel does not
            # tile (the reference's masked kernel takes any shape, :262-348): W
            # dequantized once to the gradient's dtype (bit-exact HIP kernel,
            # the reference's cast of W to grad_block.dtype, :343), then a
            # plain GEMM -- the same rounding points as the fused kernel
            wb = ops.nf4_dequant(w, absmax, code, n * k, ctx.blocksize, dtype=dt).view(n, k)
            grad_x = torch.add(torch.matmul(g, wb), gxl)
        else:
            grad_x = ops.nf4_grad_x(g, w, absmax, code, ctx.blocksize, n, k, addend=gxl)
        xa = torch.matmul(x_flat, lora_A.t().contiguous())
        grad_B = torch.matmul(sg.t().contiguous(), xa)
        grad_A = torch.matmul(gi.t().contiguous(), x_flat)
        return grad_x.view(ctx.x_shape), None, None, grad_A, grad_B, None, grad_bias


def lora_fused_forward(x: torch.Tensor, base_layer=None, lora_A=None, lora_B=None,
                       scaling: Optional[float] = None, dropout=None, lora_layer=None,
                       prefer_base_layer: bool = False) -> torch.Tensor:
    """Drop-in for ``src.triton_kernels.lora_forward.lora_fused_forward``."""
    if lora_layer is not None:
        base_layer = getattr(lora_layer, "base_layer", None)
        lora_A = getattr(lora_layer, "lora_A", None)
        lora_B = getattr(lora_layer, "lora_B", None)
        scaling = getattr(lora_layer, "scaling", None)
        dropout = getattr(lora_layer, "lora_dropout", None)
    if base_layer is None or lora_A is None or lora_B is None or scaling is None:
        raise ValueError("Provide lora_layer or base_layer/lora_A/lora_B/scaling for fused LoRA.")
    dropout_p = getattr(dropout, "p", 0.0) if dropout is not None else 0.0
    if dropout_p and dropout_p > 0.0:
        raise ValueError("Dropout is not supported in lora_fused_forward.")

    weight_4bit = getattr(base_layer, "weight", None)
    lora_A_weight = getattr(lora_A, "weight", lora_A)
    lora_B_weight = getattr(lora_B, "weight", lora_B)

    if (not prefer_base_layer and weight_4bit is not None
            and getattr(weight_4bit, "quant_state", None) is not None):
        return FusedLoRAFunction.apply(x, weight_4bit, weight_4bit.quant_state, lora_A_weight,
                                       lora_B_weight, float(scaling),
                                       getattr(base_layer, "bias", None))

    # Adapter branch (lora_forward.py:986-1037): base layer + the two adapter
    # products, each rounded to the adapter dtype, scaled, cast, added.
    if x.ndim != 3:
        raise ValueError(f"x must be [batch, seq_len, hidden], got {x.shape}.")
    if lora_A_weight.ndim != 2 or lora_B_weight.ndim != 2:
        raise ValueError("lora_A and lora_B must be 2D weight matrices.")
    if not x.is_cuda or not lora_A_weight.is_cuda or not lora_B_weight.is_cuda:
        raise ValueError("x, lora_A and lora_B must be on CUDA device.")
    r = lora_A_weight.shape[0]
    if r <= 0:
        raise ValueError(f"LoRA rank must be > 0, got {r}.")
    if lora_A_weight.shape[1] != x.shape[-1] or lora_B_weight.shape[1] != r:
        raise ValueError("lora_A/lora_B shape mismatch.")
    base_output = base_layer(x.contiguous())
    if getattr(base_output, "requires_grad", False):
        base_output = base_output.clone()
    x_lora = x.reshape(-1, x.shape[-1]).to(lora_A_weight.dtype)
    t = (x_lora.float() @ lora_A_weight.float().t()).to(lora_A_weight.dtype)
    u = (t.float() @ lora_B_weight.float().t()).to(lora_A_weight.dtype)
    u = u * float(scaling)
    if u.dtype != base_output.dtype:
        u = u.to(base_output.dtype)
    return base_output + u.view(base_output.shape)


__all__ = ["lora_fused_forward", "FusedLoRAFunction"]
