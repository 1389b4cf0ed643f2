"""NF4-dequant linear with the fused LoRA term -- test oracle.

Restates ``_lora_forward_kernel`` (``src/triton_kernels/lora_forward.py:107-260``)
with its rounding points (bf16; float16 throughout with ``dtype="f16"``):

1. ``acc = sum_k bf16(x[m,k]) * bf16(w[n,k])`` accumulated in float32
   (``:204-208``; here accumulated in float64, then rounded to float32);
2. ``acc = bf16(acc)`` (``:246``), then ``acc = bf16(acc + bf16(bias))``
   (``:247-251``);
3. ``t = bf16(sum_k x[m,k] * A[r,k])`` (``:217-243``);
4. ``u = bf16(sum_r t[m,r] * B[n,r])`` (``:244, 253``);
5. ``u = bf16(u * bf16(scaling))`` (``:211, 254``);
6. ``y = bf16(acc + u)`` (``:255-257``).

The reference's PyTorch branch (``src/core/lora.py:125-137``) rounds at the same
points except that bitsandbytes adds the bias inside ``F.linear``; both agree
to within one bf16 ulp, far inside the 1e-2 tolerance used for this op.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, from_bits, round_bf16, round_to, to_bits
from .nf4 import NF4_CODE, dequantize_nf4


def _mm(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """float64 matmul rounded to float32 (the 'fp32 accumulate' of the kernel)."""
    return (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)


def nf4_weight_bf16(packed, absmax, n: int, k: int, blocksize: int,
                    code: np.ndarray = NF4_CODE, nested: dict | None = None,
                    dtype: str = "bf16") -> np.ndarray:
    """Dequantized weight ``[N, K]`` as float32 holding exact bf16 values
    (float16 values with ``dtype="f16"``)."""
    bits = dequantize_nf4(packed, absmax, n * k, blocksize, code, nested, dtype)
    return from_bits(bits, dtype).reshape(n, k)


def nf4_lora_linear(x_bits, packed, absmax, n: int, k: int, blocksize: int,
                    bias_bits=None, a_bits=None, b_bits=None, scaling: float = 1.0,
                    code: np.ndarray = NF4_CODE, nested: dict | None = None,
                    weight_f32: np.ndarray | None = None, dtype: str = "bf16") -> np.ndarray:
    """``y = W_nf4(x) + bias + B(A(x)) * scaling``; bf16 bits in, bf16 bits out.

    ``x_bits`` is ``[M, K]`` bf16 bits; ``a_bits`` ``[r, K]``; ``b_bits``
    ``[N, r]``.  ``a_bits=None`` (or r = 0) drops the LoRA term, which is the
    plain NF4 linear of the MLP projections.  ``weight_f32`` may pass a
    pre-dequantized weight (from ``nf4_weight_bf16``) to skip that step.
    ``dtype="f16"``: every operand, the weight values and every rounding point
    in float16 (the reference kernel with X_DTYPE = LORA_DTYPE = float16).
    """
    rd = lambda v: round_to(v, dtype)
    x = from_bits(np.asarray(x_bits), dtype).reshape(-1, k)
    w = weight_f32 if weight_f32 is not None else nf4_weight_bf16(
        packed, absmax, n, k, blocksize, code, nested, dtype)
    acc = rd(_mm(x, w.T))
    if bias_bits is not None:
        acc = rd(acc + from_bits(bias_bits, dtype).reshape(1, n))
    if a_bits is not None and np.asarray(a_bits).size > 0:
        a = from_bits(a_bits, dtype).reshape(-1, k)
        b = from_bits(b_bits, dtype).reshape(n, -1)
        t = rd(_mm(x, a.T))
        u = rd(_mm(t, b.T))
        s = rd(np.float32(scaling))
        u = rd(u * s)
        acc = rd(acc + u)
    return to_bits(acc, dtype)


def nf4_lora_backward(g_bits, x_bits, packed, absmax, n: int, k: int, blocksize: int,
                      a_bits, b_bits, scaling: float, has_bias: bool = False,
                      code: np.ndarray = NF4_CODE, nested: dict | None = None,
                      exact: bool = False, dtype: str = "bf16"):
    """Gradients of ``nf4_lora_linear`` as ``FusedLoRAFunction.backward`` computes
    them (``src/triton_kernels/lora_forward.py:761-930``), each product
    accumulated in float64, rounded to float32, then to bf16 where the reference
    stores a bf16 tensor:

    1. ``base = bf16(g @ W)`` with W = bf16(code[q] * absmax), the reduction
       over the N output features (``_lora_grad_x_base_kernel``, ``:262-348``);
    2. ``sg = bf16(g * bf16(scaling))`` (``:836-837``);
    3. ``gi = bf16(sg @ B)`` [M, r]; ``gxl = bf16(gi @ A)`` [M, K];
       ``grad_x = bf16(base + gxl)`` (``:839-873``);
    4. ``xA = bf16(x @ A^T)``; ``grad_B = bf16(sg^T @ xA)`` [N, r];
       ``grad_A = bf16(gi^T @ x)`` [r, K] (``:882-928``);
    5. ``grad_bias = bf16(sum_m g)`` when the layer has a bias (``:790``).

    ``exact=True`` returns the same four products in float64 with no rounding
    at all (the linear map's true adjoint, used to pin the formulas).  Returns
    float arrays ``(grad_x [M, K], grad_A [r, K], grad_B [N, r], grad_bias or
    None)``.  ``dtype="f16"``: float16 inputs, weight values and roundings.
    """
    g = from_bits(np.asarray(g_bits), dtype).reshape(-1, n).astype(np.float64)
    x = from_bits(np.asarray(x_bits), dtype).reshape(-1, k).astype(np.float64)
    w = nf4_weight_bf16(packed, absmax, n, k, blocksize, code, nested,
                        dtype).astype(np.float64)
    a = from_bits(a_bits, dtype).reshape(-1, k).astype(np.float64)
    b = from_bits(b_bits, dtype).reshape(n, -1).astype(np.float64)
    if exact:
        sg = g * float(scaling)
        gi = sg @ b
        return g @ w + gi @ a, gi.T @ x, sg.T @ (x @ a.T), (g.sum(0) if has_bias else None)
    rb = lambda v: round_to(np.asarray(v).astype(np.float32), dtype)
    base = rb(g @ w)
    sg = rb(g * float(np.ravel(round_to(np.float32(scaling), dtype))[0]))
    gi = rb(sg.astype(np.float64) @ b)
    gxl = rb(gi.astype(np.float64) @ a)
    grad_x = rb(base + gxl)
    xa = rb(x @ a.T)
    grad_b = rb(sg.astype(np.float64).T @ xa.astype(np.float64))
    grad_a = rb(gi.astype(np.float64).T @ x)
    grad_bias = rb(g.sum(0)) if has_bias else None
    return grad_x, grad_a, grad_b, grad_bias
