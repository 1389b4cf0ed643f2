"""NF4 weight container with the bitsandbytes ``Linear4bit`` surface the reference reads.

The reference's fused path reads, from ``base_layer.weight``: the packed uint8
data and ``weight.quant_state.{absmax, code, blocksize, shape, nested, offset,
state2}`` (``src/triton_kernels/lora_forward.py:25-32, 527-576``), and from
``base_layer``: ``bias``, ``in_features``, ``out_features`` (``src/core/lora.py:84-85``).
``Linear4bitNF4`` provides exactly those, so ``ManualLoRALayer`` and
``lora_fused_forward`` work unchanged on it.  A real bitsandbytes
``Linear4bit`` is accepted by the same code, with a plain or a double-quantized
(nested) state (``float_absmax``).

Storage: ``weight`` is ``uint8 [ceil(N*K/2), 1]`` (bitsandbytes' packed
shape), element ``e = n*K + k`` in byte ``e // 2``, even ``e`` = high nibble;
``absmax`` float32 per ``blocksize`` flat elements; ``code`` float32 [16].
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

# QLoRA's NF4 levels (Dettmers et al. 2023, appendix E) = bitsandbytes' nf4 map.
NF4_CODE_VALUES = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)


def nf4_code(device=None) -> torch.Tensor:
    return torch.tensor(NF4_CODE_VALUES, dtype=torch.float32, device=device)


class QuantState:
    """The fields of ``bitsandbytes.functional.QuantState`` used on the hot path."""

    def __init__(self, absmax: torch.Tensor, shape, code: torch.Tensor, blocksize: int = 64,
                 dtype: torch.dtype = torch.bfloat16, quant_type: str = "nf4",
                 offset=None, state2: "QuantState | None" = None):
        self.absmax = absmax
        self.shape = torch.Size(shape)
        self.code = code
        self.blocksize = int(blocksize)
        self.dtype = dtype
        self.quant_type = quant_type
        self.offset = offset
        self.state2 = state2
        self.nested = state2 is not None

    def to(self, device) -> "QuantState":
        self.absmax = self.absmax.to(device)
        self.code = self.code.to(device)
        if self.state2 is not None:
            self.state2.to(device)
        if isinstance(self.offset, torch.Tensor):
            self.offset = self.offset.to(device)
        return self


def float_absmax(qs) -> torch.Tensor:
    """The float32 per-block absmax the kernels read.

    A non-nested state's ``absmax`` as is.  A double-quantized state
    (bitsandbytes ``compress_statistics=True``, the reference's
    ``bnb_4bit_use_double_quant=True``, ``src/core/model_loader.py:19``) holds
    uint8 ``absmax`` with ``state2.{code, absmax, blocksize}`` and ``offset``:
    it is expanded once on the device (``grpo_nf4_absmax_expand``, the
    reference kernel's ``code2[q] * absmax2 + offset``, ``lora_forward.py:
    187-199``) and kept on the state, since NF4 base weights are frozen.
    """
    if not getattr(qs, "nested", False) and getattr(qs, "state2", None) is None:
        return qs.absmax
    cached = getattr(qs, "_grpo_absmax_f32", None)
    key = (qs.absmax.data_ptr(), qs.absmax.device)
    if cached is not None and cached[0] == key:
        return cached[1]
    from ..kernels.ops import nf4_absmax_expand

    s2 = qs.state2
    off = qs.offset
    off = float(off.item()) if isinstance(off, torch.Tensor) else float(off or 0.0)
    out = nf4_absmax_expand(qs.absmax.reshape(-1), s2.code.float(), s2.absmax.float().reshape(-1),
                            int(s2.blocksize), off)
    qs._grpo_absmax_f32 = (key, out)
    return out


def quantize_nf4(weight: torch.Tensor, blocksize: int = 64):
    """Blockwise NF4 quantization (this repository's quantizer; runs on weight's device).

    Per block of ``blocksize`` flat elements: ``absmax = max|w|``; each element
    maps to the code nearest ``w / absmax`` (midpoint comparison in float64,
    ties to the lower code).  Returns ``(packed uint8 [ceil(n/2), 1], QuantState)``.
    """
    if weight.ndim != 2:
        raise ValueError("quantize_nf4 expects a 2-D weight [out_features, in_features].")
    n_out, n_in = weight.shape
    flat = weight.detach().to(torch.float32).reshape(-1)
    n = flat.numel()
    nblocks = -(-n // blocksize)
    padded = torch.zeros(nblocks * blocksize, dtype=torch.float32, device=weight.device)
    padded[:n] = flat
    blocks = padded.view(nblocks, blocksize)
    absmax = blocks.abs().amax(dim=1)
    safe = torch.where(absmax == 0, torch.ones_like(absmax), absmax)
    scaled = (blocks / safe[:, None]).reshape(-1)[:n]
    code = nf4_code(weight.device)
    mids = (code[1:].double() + code[:-1].double()) / 2
    q = torch.bucketize(scaled.double(), mids, right=False).to(torch.uint8)
    if n % 2:
        q = torch.cat([q, torch.zeros(1, dtype=torch.uint8, device=q.device)])
    packed = ((q[0::2] << 4) | q[1::2]).to(torch.uint8).reshape(-1, 1)
    state = QuantState(absmax=absmax.contiguous(), shape=(n_out, n_in), code=code,
                       blocksize=blocksize, dtype=torch.bfloat16)
    return packed, state


class Params4bit(nn.Parameter):
    """uint8 parameter carrying a ``quant_state`` (as bitsandbytes' Params4bit does)."""

    def __new__(cls, data: torch.Tensor, quant_state: QuantState | None = None,
                requires_grad: bool = False):
        self = torch.Tensor._make_subclass(cls, data, requires_grad)
        self.quant_state = quant_state
        return self

    def __deepcopy__(self, memo):
        qs = self.quant_state
        new = type(self)(self.data.clone(), qs, self.requires_grad)
        memo[id(self)] = new
        return new


class Linear4bitNF4(nn.Module):
    """NF4 linear layer: ``y = x W^T + b`` with ``W`` dequantized on the GPU.

    ``forward`` follows bitsandbytes' ``matmul_4bit`` for bf16 compute: the
    weight is dequantized to bf16 (bit-exact HIP kernel) and multiplied with
    ``F.linear``.  The fused NF4+LoRA path does not call this; it is the
    ``prefer_base_layer`` / fallback branch of ``ManualLoRALayer``
    (``src/core/lora.py:125-137``).
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 blocksize: int = 64, device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.blocksize = blocksize
        nbytes = -(-(in_features * out_features) // 2)
        data = torch.zeros(nbytes, 1, dtype=torch.uint8, device=device)
        nblocks = -(-(in_features * out_features) // blocksize)
        state = QuantState(torch.zeros(nblocks, dtype=torch.float32, device=device),
                           (out_features, in_features), nf4_code(device), blocksize)
        self.weight = Params4bit(data, state)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16, device=device),
                                     requires_grad=False)
        else:
            self.register_parameter("bias", None)

    @classmethod
    def from_weight(cls, weight: torch.Tensor, bias: torch.Tensor | None = None,
                    blocksize: int = 64) -> "Linear4bitNF4":
        out_f, in_f = weight.shape
        layer = cls(in_f, out_f, bias=bias is not None, blocksize=blocksize, device=weight.device)
        packed, state = quantize_nf4(weight, blocksize)
        layer.weight = Params4bit(packed, state)
        if bias is not None:
            layer.bias = nn.Parameter(bias.detach().to(torch.bfloat16).clone(), requires_grad=False)
        return layer

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        qs = getattr(self.weight, "quant_state", None)
        if qs is not None:
            # Follow device moves only: a dtype cast (module.to(bf16)) must not
            # touch the float32 scales or the codebook.
            target = fn(torch.empty(0, dtype=torch.float32, device=qs.absmax.device)).device
            qs.to(target)
        return self

    def dequantize(self, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """``[out_features, in_features]`` in bf16 (or float16): bit-exact NF4
        dequantization."""
        from ..kernels.ops import nf4_dequant

        qs = self.weight.quant_state
        n = self.out_features * self.in_features
        w = nf4_dequant(self.weight.data.view(-1), float_absmax(qs), qs.code, n, qs.blocksize,
                        dtype=dtype)
        return w.view(self.out_features, self.in_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # computes in x's dtype when that is float16 (bitsandbytes' Linear4bit
        # returns the input's dtype), in bf16 otherwise
        w = self.dequantize(torch.float16 if x.dtype == torch.float16 else torch.bfloat16)
        bias = None if self.bias is None else self.bias.to(w.dtype)
        return F.linear(x.to(w.dtype), w, bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, nf4 blocksize={self.blocksize}")


def nf4_bytes(n_out: int, n_in: int, blocksize: int = 64) -> int:
    """Packed weight + absmax bytes of an NF4 [n_out, n_in] matrix."""
    n = n_out * n_in
    return math.ceil(n / 2) + math.ceil(n / blocksize) * 4
