"""Tensor-level wrappers of the C ABI (one call = one or two kernel launches).

These validate shapes/dtypes on the host (``ValueError``, like the reference's
``_validate_inputs``), pass raw device pointers and torch's current stream to
``libgrpo_hip.so``, and manage the per-device workspaces the kernels need.
"""

from __future__ import annotations

import torch

from .. import _lib

# ----------------------------------------------------------- workspaces --

_workspaces: dict[tuple[str, int], torch.Tensor] = {}


def workspace(kind: str, nbytes: int, device: torch.device) -> torch.Tensor | None:
    """A zero-initialised uint8 scratch tensor of at least ``nbytes`` per (kind, device).

    Used for the attention's split-context partials and the NF4 linear's
    split-K partial sums (no initialisation needed).  Calls on different
    streams must not run concurrently with the same workspace.
    """
    if nbytes <= 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (kind, idx)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 1 << 20)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def reserve_workspace(kind: str, nbytes: int, device: torch.device) -> None:
    """Pre-size a workspace (call before HIP-graph capture)."""
    workspace(kind, nbytes, device)


# ------------------------------------------------------------- helpers --

def _need_cuda(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("all tensors must be on the ROCm/HIP device.")


def _need_dtype(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}.")


# --------------------------------------------------------------- NF4 ---

def nf4_absmax_expand(absmax_q: torch.Tensor, code2: torch.Tensor, absmax2: torch.Tensor,
                      blocksize2: int, offset: float) -> torch.Tensor:
    """Float32 absmax of a double-quantized NF4 state (``lora_forward.py:187-199``):
    ``fma(code2[absmax_q[i]], absmax2[i // blocksize2], offset)`` per block."""
    lib = _lib.device_library()
    _need_cuda(absmax_q, code2, absmax2)
    _need_dtype(absmax_q, torch.uint8, "nested absmax")
    _need_dtype(code2, torch.float32, "state2 code")
    _need_dtype(absmax2, torch.float32, "state2 absmax")
    n = absmax_q.numel()
    if code2.numel() != 256:
        raise ValueError("state2 code must have 256 entries.")
    if absmax2.numel() * blocksize2 < n:
        raise ValueError("state2 absmax too short for the nested absmax.")
    q, c2, a2 = absmax_q.contiguous(), code2.contiguous(), absmax2.contiguous()
    out = torch.empty(n, dtype=torch.float32, device=absmax_q.device)
    rc = lib.grpo_nf4_absmax_expand(q.data_ptr(), c2.data_ptr(), a2.data_ptr(), int(blocksize2),
                                    float(offset), n, out.data_ptr(),
                                    _lib.stream_handle(absmax_q.device))
    _lib.check(rc, "grpo_nf4_absmax_expand")
    return out


def nf4_dequant(packed: torch.Tensor, absmax: torch.Tensor, code: torch.Tensor, numel: int,
                blocksize: int, out: torch.Tensor | None = None,
                dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Bit-exact NF4 dequantization to a flat tensor of ``numel`` elements:
    ``dtype(code[q] * absmax)``, bf16 or float16 (round to nearest even)."""
    if dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"dequantization to bfloat16 or float16, got {dtype}.")
    lib = _lib.device_library()
    _need_cuda(packed, absmax, code)
    _need_dtype(packed, torch.uint8, "packed weight")
    _need_dtype(absmax, torch.float32, "absmax")
    _need_dtype(code, torch.float32, "code")
    if packed.numel() * 2 < numel:
        raise ValueError(f"packed weight holds {packed.numel() * 2} nibbles, need {numel}.")
    if absmax.numel() * blocksize < numel:
        raise ValueError("absmax too short for numel/blocksize.")
    if code.numel() != 16:
        raise ValueError("code must have 16 entries.")
    packed, absmax, code = packed.contiguous(), absmax.contiguous(), code.contiguous()
    if out is None:
        out = torch.empty(numel, dtype=dtype, device=packed.device)
    elif out.dtype != dtype:
        raise ValueError(f"out must be {dtype}.")
    fn = lib.grpo_nf4_dequant_f16 if dtype == torch.float16 else lib.grpo_nf4_dequant
    rc = fn(packed.data_ptr(), absmax.data_ptr(), code.data_ptr(), out.data_ptr(), numel,
            blocksize, _lib.stream_handle(packed.device))
    _lib.check(rc, "grpo_nf4_dequant")
    return out


def nf4_grad_x_supported(n: int, k: int, blocksize: int) -> bool:
    """Shapes ``grpo_nf4_grad_x`` takes: N a multiple of 32, K of 128, blocksize of 8."""
    return n > 0 and k > 0 and n % 32 == 0 and k % 128 == 0 and blocksize > 0 \
        and blocksize % 8 == 0


def nf4_grad_x(grad: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor,
               code: torch.Tensor, blocksize: int, n: int, k: int,
               addend: torch.Tensor | None = None) -> torch.Tensor:
    """``bf16(grad [M, n] @ W_nf4 [n, k])`` (+ ``addend`` [M, k], rounded once more)."""
    lib = _lib.device_library()
    _need_cuda(grad, packed, absmax, code, addend)
    _need_dtype(grad, torch.bfloat16, "grad")
    _need_dtype(packed, torch.uint8, "packed weight")
    _need_dtype(absmax, torch.float32, "absmax")
    if grad.ndim != 2 or grad.shape[1] != n:
        raise ValueError(f"grad must be [M, {n}], got {tuple(grad.shape)}.")
    if packed.numel() * 2 < n * k or absmax.numel() * blocksize < n * k:
        raise ValueError("packed weight or absmax too short for [n, k].")
    if code.numel() != 16:
        raise ValueError("code must have 16 entries.")
    m = grad.shape[0]
    grad = grad.contiguous()
    if addend is not None:
        _need_dtype(addend, torch.bfloat16, "addend")
        if tuple(addend.shape) != (m, k):
            raise ValueError(f"addend must be [{m}, {k}], got {tuple(addend.shape)}.")
        addend = addend.contiguous()
    out = torch.empty((m, k), dtype=torch.bfloat16, device=grad.device)
    rc = lib.grpo_nf4_grad_x(grad.data_ptr(), n, packed.data_ptr(), absmax.data_ptr(),
                             code.contiguous().data_ptr(), blocksize, m, n, k,
                             None if addend is None else addend.data_ptr(), k, out.data_ptr(), k,
                             _lib.stream_handle(grad.device))
    _lib.check(rc, "grpo_nf4_grad_x")
    return out


def nf4_lora_linear(x2d: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor,
                    code: torch.Tensor, blocksize: int, n: int, bias: torch.Tensor | None = None,
                    lora_a: torch.Tensor | None = None, lora_b: torch.Tensor | None = None,
                    scaling: float = 1.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """``y[M, N] = W_nf4(x) + bias + B(A(x)) * scaling`` (bf16).

    Up to 32 rows: the one-launch tile kernel (``grpo_nf4_tile_linear``, LoRA A
    packed once per tensor version); up to 64 rows split-K partial sums +
    finish (two launches); beyond, the NF4 GEMM (one launch, or K slices +
    finish when the tiles are few); one generic launch for other shapes.
    float16 x (with float16 LoRA and bias) runs the NF4 GEMM's float16 form for
    any M (``y`` float16).
    """
    lib = _lib.device_library()
    _need_cuda(x2d, packed, absmax, code, bias, lora_a, lora_b)
    if x2d.ndim != 2:
        raise ValueError(f"x must be 2-D [M, K], got {tuple(x2d.shape)}.")
    if x2d.dtype == torch.float16:
        return _nf4_lora_linear_f16(lib, x2d, packed, absmax, code, blocksize, n, bias, lora_a,
                                    lora_b, scaling, out)
    _need_dtype(x2d, torch.bfloat16, "x")
    m, k = x2d.shape
    if x2d.stride(1) != 1:
        x2d = x2d.contiguous()
    r = 0
    if lora_a is not None:
        r = lora_a.shape[0]
        if lora_a.shape != (r, k) or lora_b is None or lora_b.shape != (n, r):
            raise ValueError("lora_A must be [r, K] and lora_B [N, r].")
        _need_dtype(lora_a, torch.bfloat16, "lora_A")
        _need_dtype(lora_b, torch.bfloat16, "lora_B")
        lora_a, lora_b = lora_a.contiguous(), lora_b.contiguous()
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias must have {n} elements.")
        bias = bias.to(torch.bfloat16).contiguous()
    if packed.numel() * 2 < n * k:
        raise ValueError("packed weight smaller than N*K/2 bytes.")
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=x2d.device)
    elif out.shape != (m, n) or out.stride(1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError("out must be a bf16 [M, N] tensor with unit column stride.")
    if (m <= TILE_MAX_ROWS and x2d.stride(0) % 8 == 0 and x2d.data_ptr() % 16 == 0
            and packed.data_ptr() % 16 == 0 and out.data_ptr() % 2 == 0
            and lib.grpo_nf4_tile_supported(m, n, k, r, 1, int(blocksize))):
        # decode batches: the one-launch tile linear (LoRA A in its packed
        # order, built once per A version)
        d = _lib.TileLinear()
        d.M, d.N, d.K, d.nseg, d.r = m, n, k, 1, r
        d.seg_end[0] = n
        d.bias[0] = _lib.ptr(bias)
        if r > 0:
            d.lora_a[0] = packed_lora_a(lora_a).data_ptr()
            d.lora_b[0] = lora_b.data_ptr()
        d.scaling = float(scaling)
        rc = lib.grpo_nf4_tile_linear(x2d.data_ptr(), x2d.stride(0), packed.data_ptr(),
                                      absmax.data_ptr(), code.data_ptr(), int(blocksize),
                                      ctypes_byref(d), out.data_ptr(), out.stride(0),
                                      _lib.stream_handle(x2d.device))
        _lib.check(rc, "grpo_nf4_tile_linear")
        return out
    nbytes = int(lib.grpo_nf4_lora_linear_workspace_bytes(m, n, k, r, 1, int(blocksize)))
    ws = workspace("nf4_linear", nbytes, x2d.device)
    rc = lib.grpo_nf4_lora_linear(
        x2d.data_ptr(), x2d.stride(0), packed.data_ptr(), absmax.data_ptr(), code.data_ptr(),
        int(blocksize), _lib.ptr(bias), _lib.ptr(lora_a), _lib.ptr(lora_b), r, float(scaling),
        out.data_ptr(), out.stride(0), m, n, k, _lib.ptr(ws), 0 if ws is None else ws.numel(),
        _lib.stream_handle(x2d.device))
    _lib.check(rc, "grpo_nf4_lora_linear")
    return out


TILE_MAX_ROWS = 32  # rows up to which nf4_lora_linear runs the one-launch tile kernel

# Packed LoRA A per live A tensor: id(A) -> (weakref to A, A._version, packed).
# An entry is valid while A is the same object at the same version (an
# optimizer step updates A in place and bumps the version) and is dropped
# when A is freed.
_packed_a: dict[int, tuple] = {}


def packed_lora_a(a: torch.Tensor) -> torch.Tensor:
    """``pack_lora_a(a)``, cached per A tensor and version."""
    import weakref

    key = id(a)
    e = _packed_a.get(key)
    if e is not None and e[0]() is a and e[1] == a._version:
        return e[2]
    p = pack_lora_a(a)
    _packed_a[key] = (weakref.ref(a, lambda _r, k=key: _packed_a.pop(k, None)), a._version, p)
    return p


def pack_lora_a(a: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """LoRA A [r, K] bf16 in the MFMA order the one-launch linear reads
    (``grpo_nf4_tile_pack_lora_a``); valid until A changes."""
    lib = _lib.device_library()
    _need_cuda(a)
    _need_dtype(a, torch.bfloat16, "lora_A")
    r, k = a.shape
    a = a.contiguous()
    nbytes = int(lib.grpo_nf4_tile_packed_lora_a_bytes(k))
    if out is None:
        out = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=a.device)
    elif out.numel() * out.element_size() < nbytes:
        raise ValueError(f"packed LoRA A needs {nbytes} bytes.")
    _lib.check(lib.grpo_nf4_tile_pack_lora_a(a.data_ptr(), r, k, k, out.data_ptr(),
                                             _lib.stream_handle(a.device)), "pack_lora_a")
    return out


def tile_linear_desc(m: int, k: int, seg_rows, biases=None, lora_a=None, lora_b=None,
                     scaling: float = 1.0):
    """``grpo_tile_linear_t`` of an [M, K] x [N = sum(seg_rows), K] NF4 linear:
    per segment an optional bf16 bias and LoRA A [r, K] / B [rows, r] (device
    tensors, kept referenced by the returned descriptor)."""
    d = _lib.TileLinear()
    d.M, d.K, d.nseg = m, k, len(seg_rows)
    if not 1 <= d.nseg <= _lib.MAX_SEGMENTS:
        raise ValueError(f"1..{_lib.MAX_SEGMENTS} segments, got {d.nseg}.")
    keep = []
    end, r = 0, 0
    for i, rows in enumerate(seg_rows):
        end += int(rows)
        d.seg_end[i] = end
        if biases is not None and biases[i] is not None:
            b = biases[i].to(torch.bfloat16).contiguous()
            if b.numel() != rows:
                raise ValueError(f"bias {i} must have {rows} elements.")
            keep.append(b)
            d.bias[i] = b.data_ptr()
        if lora_a is not None:
            a, bb = lora_a[i].contiguous(), lora_b[i].contiguous()
            r = a.shape[0]
            if a.shape != (r, k) or bb.shape != (rows, r):
                raise ValueError("lora_A must be [r, K] and lora_B [rows, r] per segment.")
            _need_dtype(a, torch.bfloat16, "lora_A")
            _need_dtype(bb, torch.bfloat16, "lora_B")
            ap = pack_lora_a(a)
            keep += [ap, bb]
            d.lora_a[i], d.lora_b[i] = ap.data_ptr(), bb.data_ptr()
    d.N, d.r, d.scaling = end, r, float(scaling)
    d._keep = keep
    return d


def nf4_tile_linear(x: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor,
                    code: torch.Tensor, blocksize: int, desc, out: torch.Tensor | None = None,
                    norm: tuple | None = None, residual: torch.Tensor | None = None,
                    sumsq: torch.Tensor | None = None) -> torch.Tensor:
    """The one-launch NF4 (+ LoRA) linear (``grpo_nf4_tile_linear*``) for a
    ``tile_linear_desc`` descriptor.

    ``norm = (sumsq [M, G] float32, weight [K] bf16, eps)``: ``x`` is h and the
    kernel stages RMSNorm(h).  ``residual`` ([M, N] bf16, may be ``out``):
    ``out = bf16(residual + y)`` and ``sumsq`` ([M, G] float32, G =
    ``grpo_nf4_tile_sumsq_groups``) receives the per-group sums of ``out**2``."""
    lib = _lib.device_library()
    _need_cuda(x, packed, absmax, code, out, residual, sumsq)
    _need_dtype(x, torch.bfloat16, "x")
    m, n, k = desc.M, desc.N, desc.K
    if x.ndim != 2 or x.shape != (m, k) or x.stride(1) != 1:
        raise ValueError(f"x must be [{m}, {k}] with unit column stride.")
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    if out.shape != (m, n) or out.stride(1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError("out must be a bf16 [M, N] tensor with unit column stride.")
    st = _lib.stream_handle(x.device)
    args = (packed.data_ptr(), absmax.data_ptr(), code.data_ptr(), int(blocksize),
            ctypes_byref(desc))
    if norm is not None:
        ss, w, eps = norm
        rc = lib.grpo_nf4_tile_linear_norm(x.data_ptr(), x.stride(0), ss.data_ptr(), ss.shape[1],
                                           w.data_ptr(), float(eps), *args, out.data_ptr(),
                                           out.stride(0), st)
    elif residual is not None:
        if sumsq is None or residual.stride() != out.stride():
            raise ValueError("residual needs sumsq and the row stride of out.")
        rc = lib.grpo_nf4_tile_linear_residual(x.data_ptr(), x.stride(0), *args,
                                               residual.data_ptr(), out.data_ptr(), out.stride(0),
                                               sumsq.data_ptr(), st)
    else:
        rc = lib.grpo_nf4_tile_linear(x.data_ptr(), x.stride(0), *args, out.data_ptr(),
                                      out.stride(0), st)
    _lib.check(rc, "grpo_nf4_tile_linear")
    return out


def ctypes_byref(obj):
    import ctypes

    return ctypes.byref(obj)


def _nf4_lora_linear_f16(lib, x2d, packed, absmax, code, blocksize, n, bias, lora_a, lora_b,
                         scaling, out):
    """float16 x and adapters: the NF4 GEMM's float16 form (``grpo_nf4_gemm_f16``,
    every rounding point float16, any M)."""
    m, k = x2d.shape
    if x2d.stride(1) != 1 or x2d.stride(0) % 8 or x2d.data_ptr() % 16:
        x2d = x2d.contiguous()
    r = 0
    if lora_a is not None:
        r = lora_a.shape[0]
        if lora_a.shape != (r, k) or lora_b is None or lora_b.shape != (n, r):
            raise ValueError("lora_A must be [r, K] and lora_B [N, r].")
        _need_dtype(lora_a, torch.float16, "lora_A")
        _need_dtype(lora_b, torch.float16, "lora_B")
        lora_a, lora_b = lora_a.contiguous(), lora_b.contiguous()
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias must have {n} elements.")
        bias = bias.to(torch.float16).contiguous()
    if packed.numel() * 2 < n * k:
        raise ValueError("packed weight smaller than N*K/2 bytes.")
    if not nf4_gemm_supported(m, n, k, r, blocksize):
        raise ValueError(f"float16 NF4 linear: shape M={m} N={n} K={k} r={r} blocksize="
                         f"{blocksize} is outside the NF4 GEMM (K % 32, r <= 32).")
    if out is None:
        out = torch.empty((m, n), dtype=torch.float16, device=x2d.device)
    elif out.shape != (m, n) or out.stride(1) != 1 or out.dtype != torch.float16:
        raise ValueError("out must be a float16 [M, N] tensor with unit column stride.")
    if m == 0 or n == 0:
        return out
    rc = lib.grpo_nf4_gemm_f16(
        x2d.data_ptr(), x2d.stride(0), packed.data_ptr(), absmax.data_ptr(), code.data_ptr(),
        int(blocksize), _lib.ptr(bias), _lib.ptr(lora_a), _lib.ptr(lora_b), r, float(scaling),
        out.data_ptr(), out.stride(0), m, n, k, _lib.stream_handle(x2d.device))
    _lib.check(rc, "grpo_nf4_gemm_f16")
    return out


def nf4_gemm_supported(m: int, n: int, k: int, r: int, blocksize: int) -> bool:
    """True if the NF4 GEMM (``grpo_nf4_gemm``; more than 64 rows) takes this
    shape (alignment aside)."""
    return bool(_lib.library().grpo_nf4_gemm_supported(m, n, k, r, int(blocksize)))


def nf4_linear_plan(m: int, n: int, k: int, r: int, nseg: int,
                    blocksize: int) -> tuple[int, int, int] | None:
    """(splits, part_bytes, tpart_bytes) of the split-K path, or None if the
    shape takes the generic kernel."""
    import ctypes

    s, pb, tb = ctypes.c_int(0), ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = _lib.library().grpo_nf4_linear_plan(m, n, k, r, nseg, blocksize, ctypes.byref(s),
                                             ctypes.byref(pb), ctypes.byref(tb))
    if rc != 0:
        return None
    return s.value, pb.value, tb.value


# ----------------------------------------------------------- paged KV ---

def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if k_cache.ndim != 4 or v_cache.ndim != 4:
        raise ValueError("k_cache/v_cache must be [num_blocks, heads, block, head_dim].")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have identical shapes.")
    _need_dtype(k_cache, torch.bfloat16, "k_cache")
    _need_dtype(v_cache, torch.bfloat16, "v_cache")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous.")


def _check_tables(block_tables: torch.Tensor, context_lens: torch.Tensor, b: int) -> None:
    if block_tables.ndim != 2 or block_tables.shape[0] != b:
        raise ValueError("block_tables must be [batch, max_blocks].")
    if context_lens.ndim != 1 or context_lens.shape[0] != b:
        raise ValueError("context_lens must be [batch].")
    _need_dtype(block_tables, torch.int32, "block_tables")
    _need_dtype(context_lens, torch.int32, "context_lens")
    if block_tables.stride(1) != 1 or not context_lens.is_contiguous():
        raise ValueError("block_tables rows and context_lens must be contiguous.")


def paged_kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                    v_cache: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor) -> None:
    """Write ``k_new/v_new [B, Hkv, D]`` at slot ``context_lens[b]`` of each sequence."""
    lib = _lib.device_library()
    _need_cuda(k_new, v_new, k_cache, v_cache, block_tables, context_lens)
    _check_cache(k_cache, v_cache)
    nb, hkv, bs, d = k_cache.shape
    if k_new.shape != v_new.shape or k_new.ndim != 3 or k_new.shape[1:] != (hkv, d):
        raise ValueError(f"k_new/v_new must be [B, {hkv}, {d}].")
    b = k_new.shape[0]
    _check_tables(block_tables, context_lens, b)
    k_new = k_new.to(torch.bfloat16)
    v_new = v_new.to(torch.bfloat16)
    if k_new.stride(2) != 1 or k_new.stride() != v_new.stride():
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    rc = lib.grpo_paged_kv_append(
        k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), k_cache.data_ptr(),
        v_cache.data_ptr(), nb, block_tables.data_ptr(), block_tables.stride(0),
        context_lens.data_ptr(), b, hkv, d, bs, block_tables.shape[1],
        _lib.stream_handle(k_cache.device))
    _lib.check(rc, "grpo_paged_kv_append")


def paged_attention_workspace_bytes(b: int, hq: int, hkv: int, d: int, bs: int,
                                    max_blocks: int) -> int:
    return int(_lib.library().grpo_paged_attn_workspace_bytes(b, hq, hkv, d, bs, max_blocks))


# One-launch attention (grpo_paged_attn_decode_merged): per device, the int32
# arrival counters of the in-kernel merge (zero, left zero by every call) and
# the XCD error word.  Calls on one device share them, as they share the
# workspace: calls that overlap on two streams must be ordered by the caller.
_attn_merge: dict = {}
ATTN_ONE_LAUNCH = True


def _attn_merge_state(lib, device, b: int, hkv: int):
    need = max(int(lib.grpo_paged_attn_merge_counter_bytes(b, hkv)) // 4, 1)
    key = device if isinstance(device, torch.device) else torch.device(device)
    st = _attn_merge.get(key)
    if st is None or st[0].numel() < need:
        err = st[1] if st is not None else torch.zeros(1, dtype=torch.int32, device=key)
        st = (torch.zeros(need, dtype=torch.int32, device=key), err)
        _attn_merge[key] = st
    return st


def attention_handover_check(device=None) -> None:
    """Check the one-launch attention calls made so far on ``device`` (host
    sync): their in-kernel merge hands each (sequence, KV head)'s split
    partials to the last-arriving split through an L2 counter, which is
    correct only when the pair's splits ran on one XCD.  The kernel flags a
    pair that did not, and such a pair leaves its counter non-zero; either
    raises ``RuntimeError`` (those calls' outputs are not valid), clears the
    state and turns the one-launch form off (``ATTN_ONE_LAUNCH``) for later
    calls, which then take the split launch + merge launch."""
    global ATTN_ONE_LAUNCH
    keys = [torch.device(device)] if device is not None else list(_attn_merge)
    for key in keys:
        st = _attn_merge.get(key)
        if st is None:
            continue
        if int(st[1].item()) != 0 or bool((st[0] != 0).any()):
            st[0].zero_()
            st[1].zero_()
            ATTN_ONE_LAUNCH = False
            raise RuntimeError("paged attention: the context splits of a (sequence, KV head) "
                               "pair did not run on one XCD; outputs of the one-launch calls "
                               "since the last check are not valid (one-launch form now off)")


def paged_attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                           out_dtype: torch.dtype = torch.float32,
                           out: torch.Tensor | None = None,
                           no_alloc: bool = False) -> torch.Tensor:
    """GQA paged decode attention; ``q [B, Hq, D]`` bf16 -> ``[B, Hq, D]`` out_dtype.

    One launch (``grpo_paged_attn_decode_merged``: the last-arriving context
    split of each (sequence, KV head) merges the pair's splits) while
    ``ATTN_ONE_LAUNCH``; ``attention_handover_check`` verifies those calls.
    ``no_alloc`` calls ``grpo_paged_attn_decode_noalloc`` (split partials in the
    library's per-GPU scratch array, no workspace, split + merge launches);
    ``out`` must then be given for the call to allocate nothing at all."""
    lib = _lib.device_library()
    _need_cuda(q, k_cache, v_cache, block_tables, context_lens)
    _check_cache(k_cache, v_cache)
    nb, hkv, bs, d = k_cache.shape
    if q.ndim != 3 or q.shape[2] != d:
        raise ValueError(f"q must be [B, Hq, {d}].")
    b, hq, _ = q.shape
    if hq % hkv != 0:
        raise ValueError(f"query heads ({hq}) must be a multiple of KV heads ({hkv}).")
    _check_tables(block_tables, context_lens, b)
    q = q.to(torch.bfloat16)
    if q.stride(2) != 1:
        q = q.contiguous()
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out_dtype must be float32 or bfloat16.")
    if out is None:
        out = torch.empty((b, hq, d), dtype=out_dtype, device=q.device)
    elif out.shape != (b, hq, d) or not out.is_contiguous() or out.dtype != out_dtype:
        raise ValueError("out must be a contiguous [B, Hq, D] tensor of out_dtype.")
    max_blocks = block_tables.shape[1]
    if no_alloc:
        rc = lib.grpo_paged_attn_decode_noalloc(
            q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), nb,
            block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(),
            out.data_ptr(), 1 if out_dtype == torch.bfloat16 else 0, b, hq, hkv, d, bs,
            max_blocks, float(scale), _lib.stream_handle(q.device))
        _lib.check(rc, "grpo_paged_attn_decode_noalloc")
        return out
    nbytes = int(lib.grpo_paged_attn_workspace_bytes(b, hq, hkv, d, bs, max_blocks))
    ws = workspace("paged_attn", nbytes, q.device)
    args = (q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), nb,
            block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(),
            out.data_ptr(), 1 if out_dtype == torch.bfloat16 else 0, b, hq, hkv, d, bs,
            max_blocks, float(scale), _lib.ptr(ws), 0 if ws is None else ws.numel())
    if ATTN_ONE_LAUNCH:
        cnt, err = _attn_merge_state(lib, q.device, b, hkv)
        rc = lib.grpo_paged_attn_decode_merged(*args, cnt.data_ptr(), err.data_ptr(),
                                               _lib.stream_handle(q.device))
        _lib.check(rc, "grpo_paged_attn_decode_merged")
    else:
        rc = lib.grpo_paged_attn_decode(*args, _lib.stream_handle(q.device))
        _lib.check(rc, "grpo_paged_attn_decode")
    return out
