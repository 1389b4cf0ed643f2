"""ctypes binding of libgrpo_hip.so (the C ABI declared in include/grpo_hip.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already loaded.  A missing library or a missing gfx950 device raises
``ImportError`` -- the reference's convention for an unavailable kernel backend
(``src/triton_kernels/__init__.py:297``, caught by ``src/core/lora.py:122`` and
``src/grpo/trainer.py:401``).  There is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

from ._build import LIB_PATH

_c = ctypes
_VP, _I64, _I32, _F32, _SZ = _c.c_void_p, _c.c_int64, _c.c_int, _c.c_float, _c.c_size_t
MAX_SEGMENTS = 4


class LinearParts(ctypes.Structure):
    """``grpo_linear_parts_t``: split-K partial sums of one NF4 (+ LoRA) linear
    and the epilogue parameters its consumer applies."""

    _fields_ = [
        ("part", _VP),
        ("tpart", _VP),
        ("splits", _I32),
        ("M", _I32),
        ("N", _I32),
        ("K", _I32),
        ("nseg", _I32),
        ("r", _I32),
        ("seg_end", _I32 * MAX_SEGMENTS),
        ("bias", _VP * MAX_SEGMENTS),
        ("lora_b", _VP * MAX_SEGMENTS),
        ("scaling", _F32),
    ]


_PARTS = ctypes.POINTER(LinearParts)


class TileLinear(ctypes.Structure):
    """``grpo_tile_linear_t``: one NF4 (+ LoRA, + bias) linear finished in one
    launch (device pointers for lora_a, lora_b and bias)."""

    _fields_ = [
        ("M", _I32),
        ("N", _I32),
        ("K", _I32),
        ("nseg", _I32),
        ("r", _I32),
        ("seg_end", _I32 * MAX_SEGMENTS),
        ("lora_a", _VP * MAX_SEGMENTS),
        ("lora_b", _VP * MAX_SEGMENTS),
        ("bias", _VP * MAX_SEGMENTS),
        ("scaling", _F32),
        ("lora_t", _VP),
        ("lora_t_parts", _I32),
    ]


_TILE = ctypes.POINTER(TileLinear)

# name -> (restype, argtypes); mirrors include/grpo_hip.h one to one.
SIGNATURES = {
    "grpo_version": (_I32, []),
    "grpo_init": (_I32, []),
    "grpo_last_error": (_c.c_char_p, []),
    "grpo_nf4_dequant": (_I32, [_VP, _VP, _VP, _VP, _I64, _I32, _VP]),
    "grpo_nf4_dequant_f16": (_I32, [_VP, _VP, _VP, _VP, _I64, _I32, _VP]),
    "grpo_nf4_absmax_expand": (_I32, [_VP, _VP, _VP, _I32, _F32, _I64, _VP, _VP]),
    "grpo_nf4_grad_x": (_I32, [_VP, _I64, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _I64, _VP,
                                _I64, _VP]),
    "grpo_nf4_linear_plan": (
        _I32,
        [_I32, _I32, _I32, _I32, _I32, _I32, _c.POINTER(_I32), _c.POINTER(_SZ),
         _c.POINTER(_SZ)],
    ),
    "grpo_nf4_linear_partials": (_I32, [_VP, _I64, _VP, _VP, _VP, _I32, _VP, _PARTS, _VP]),
    "grpo_nf4_linear_finish": (_I32, [_PARTS, _VP, _I64, _VP]),
    "grpo_nf4_lora_linear_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "grpo_nf4_lora_linear": (
        _I32,
        [_VP, _I64, _VP, _VP, _VP, _I32, _VP, _VP, _VP, _I32, _F32, _VP, _I64, _I32, _I32, _I32,
         _VP, _SZ, _VP],
    ),
    "grpo_nf4_gemm_supported": (_I32, [_I32, _I32, _I32, _I32, _I32]),
    "grpo_nf4_gemm": (
        _I32,
        [_VP, _I64, _VP, _VP, _VP, _I32, _VP, _VP, _VP, _I32, _F32, _VP, _I64, _I32, _I32, _I32,
         _VP],
    ),
    "grpo_nf4_gemm_f16": (
        _I32,
        [_VP, _I64, _VP, _VP, _VP, _I32, _VP, _VP, _VP, _I32, _F32, _VP, _I64, _I32, _I32, _I32,
         _VP],
    ),
    "grpo_nf4_lora_linear_grouped": (
        _I32,
        [_VP, _I64, _VP, _VP, _VP, _I32, _I32, _VP, _VP, _VP, _VP, _I32, _F32, _VP, _I64, _I32,
         _I32, _VP, _SZ, _VP],
    ),
    "grpo_embedding": (_I32, [_VP, _VP, _I64, _I32, _VP, _I32, _VP]),
    "grpo_add_rmsnorm": (_I32, [_VP, _VP, _VP, _VP, _VP, _I32, _I32, _F32, _VP]),
    "grpo_rope_append": (
        _I32,
        [_VP, _I64, _I32, _I32, _I32, _VP, _VP, _I32, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I32,
         _I32, _I32, _VP],
    ),
    "grpo_silu_mul": (_I32, [_VP, _I64, _I32, _VP, _I64, _I32, _VP]),
    "grpo_add_rmsnorm_parts": (_I32, [_PARTS, _VP, _VP, _VP, _VP, _F32, _VP]),
    "grpo_qkv_rope_append_parts": (
        _I32,
        [_PARTS, _I32, _I32, _I32, _VP, _VP, _I32, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I32,
         _I32, _VP],
    ),
    "grpo_silu_mul_parts": (_I32, [_PARTS, _VP, _I64, _VP]),
    "grpo_argmax_bf16": (_I32, [_VP, _I64, _I32, _I32, _VP, _VP]),
    "grpo_lm_head_workspace_bytes": (_SZ, [_I32, _I32]),
    "grpo_lm_head_argmax": (
        _I32, [_VP, _I64, _VP, _I32, _I32, _I32, _VP, _I64, _VP, _SZ, _VP]),
    "grpo_decode_advance": (
        _I32,
        [_VP, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _VP, _VP, _VP],
    ),
    "grpo_sample_workspace_bytes": (_SZ, [_I32, _I32]),
    "grpo_sample_top_p": (
        _I32, [_VP, _I64, _I32, _I32, _F32, _c.c_double, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "grpo_sample_advance": (
        _I32,
        [_VP, _I64, _I32, _I32, _F32, _c.c_double, _c.c_uint64, _VP, _VP, _VP, _VP, _VP, _VP,
         _VP, _VP, _I64, _VP, _VP, _VP, _SZ, _VP],
    ),
    "grpo_paged_kv_append": (
        _I32,
        [_VP, _VP, _I64, _I64, _VP, _VP, _I64, _VP, _I64, _VP, _I32, _I32, _I32, _I32, _I32, _VP],
    ),
    "grpo_paged_attn_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "grpo_paged_attn_decode_qkv": (
        _I32,
        [_PARTS, _I32, _I32, _I32, _VP, _VP, _I32, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I32,
         _I32, _F32, _VP, _SZ, _VP, _VP],
    ),
    "grpo_paged_attn_splits": (_I32, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "grpo_paged_attn_qkv_max_slices": (_I32, []),
    "grpo_paged_attn_merge_counter_bytes": (_SZ, [_I32, _I32]),
    "grpo_paged_attn_decode_qkv_merged": (
        _I32,
        [_PARTS, _I32, _I32, _I32, _VP, _VP, _I32, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I32,
         _I32, _F32, _VP, _SZ, _VP, _VP, _VP, _VP, _I32, _VP, _VP],
    ),
    "grpo_nf4_linear_partials_silu": (_I32, [_PARTS, _VP, _VP, _VP, _I32, _PARTS, _VP]),
    "grpo_nf4_gate_up_silu": (
        _I32, [_VP, _I64, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _I64, _VP]),
    "grpo_nf4_gate_up_silu_supported": (_I32, [_I32, _I32, _I32, _I32]),
    "grpo_nf4_gate_up_silu_tiles": (
        _I32, [_VP, _I64, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _VP]),
    "grpo_fold_tiles_elements": (_SZ, [_I32]),
    "grpo_nf4_gate_up_silu_tiles_norm": (
        _I32, [_VP, _I64, _VP, _I32, _VP, _F32, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _VP]),
    "grpo_nf4_gate_up_silu_tiles_norm_supported": (_I32, [_I32, _I32, _I32, _I32]),
    "grpo_linear_finish_residual": (_I32, [_PARTS, _VP, _VP, _I64, _VP, _VP]),
    "grpo_embedding_sumsq": (_I32, [_VP, _VP, _I64, _I32, _VP, _I32, _VP, _VP]),
    "grpo_embedding_sumsq_groups": (_I32, []),
    "grpo_lm_head_argmax_norm": (
        _I32, [_VP, _I64, _VP, _I32, _VP, _F32, _VP, _I32, _I32, _I32, _VP, _I64, _VP, _SZ, _VP]),
    "grpo_lm_head_argmax_norm_tiles": (
        _I32, [_VP, _I64, _VP, _I32, _VP, _F32, _VP, _I32, _I32, _I32, _VP, _I64, _VP, _SZ, _VP]),
    "grpo_lm_head_argmax_tiles": (
        _I32, [_VP, _I64, _VP, _I32, _I32, _I32, _VP, _I64, _VP, _SZ, _VP]),
    "grpo_lm_head_weight_tiles": (_I32, [_VP, _I32, _I32, _VP, _VP]),
    "grpo_lm_head_q8_tiles": (_I32, [_VP, _I32, _I32, _VP, _VP, _VP, _VP]),
    "grpo_lm_head_screen_workspace_bytes": (_SZ, [_I32, _I32]),
    "grpo_lm_head_screen": (
        _I32, [_VP, _I64, _VP, _VP, _VP, _I32, _I32, _I32, _VP, _SZ, _VP]),
    "grpo_lm_head_screen_norm": (
        _I32, [_VP, _I64, _VP, _I32, _VP, _F32, _VP, _VP, _VP, _I32, _I32, _I32, _VP, _SZ, _VP]),
    "grpo_lm_head_exact_argmax": (
        _I32, [_VP, _I64, _VP, _I32, _I32, _I32, _VP, _SZ, _VP, _VP, _VP]),
    "grpo_lm_head_exact_advance_norm": (
        _I32, [_VP, _I64, _VP, _I32, _VP, _F32, _VP, _I32, _I32, _I32, _VP, _SZ, _VP, _VP, _VP,
               _VP, _VP, _VP, _VP, _VP, _VP, _I64, _VP, _VP, _VP]),
    "grpo_nf4_linear_residual": (
        _I32, [_VP, _I64, _I32, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _I64, _VP, _I64,
               _VP, _VP]),
    "grpo_nf4_linear_residual_supported": (_I32, [_I32, _I32, _I32, _I32]),
    "grpo_nf4_linear_partials_norm": (
        _I32, [_VP, _I64, _VP, _I32, _VP, _F32, _VP, _VP, _VP, _I32, _VP, _PARTS, _VP]),
    "grpo_nf4_linear_partials_attn": (
        _I32,
        [_VP, _VP, _I32, _I32, _I32, _I32, _I32, _VP, _VP, _VP, _I32, _VP, _PARTS, _VP],
    ),
    "grpo_nf4_linear_attn_residual": (
        _I32,
        [_VP, _VP, _I32, _I32, _I32, _I32, _I32, _VP, _VP, _VP, _I32, _VP, _PARTS, _VP, _VP,
         _VP, _VP, _VP, _I64, _VP, _VP],
    ),
    "grpo_nf4_linear_attn_residual_groups": (
        _I32, [_I32, _I32, _I32, _I32, _I32, _VP, _VP]),
    "grpo_paged_attn_decode": (
        _I32,
        [_VP, _I64, _I64, _VP, _VP, _I64, _VP, _I64, _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32,
         _I32, _F32, _VP, _SZ, _VP],
    ),
    "grpo_paged_attn_decode_merged": (
        _I32,
        [_VP, _I64, _I64, _VP, _VP, _I64, _VP, _I64, _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32,
         _I32, _F32, _VP, _SZ, _VP, _VP, _VP],
    ),
    "grpo_paged_attn_merge": (_I32, [_VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32, _VP, _I32,
                                     _VP]),
    "grpo_nf4_tile_supported": (_I32, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "grpo_nf4_tile_norm_supported": (_I32, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "grpo_nf4_tile_sumsq_groups": (_I32, [_I32, _I32, _I32, _I32, _I32]),
    "grpo_nf4_tile_packed_lora_a_bytes": (_SZ, [_I32]),
    "grpo_nf4_tile_pack_lora_a": (_I32, [_VP, _I32, _I32, _I64, _VP, _VP]),
    "grpo_nf4_tile_linear": (_I32, [_VP, _I64, _VP, _VP, _VP, _I32, _TILE, _VP, _I64, _VP]),
    "grpo_nf4_tile_linear_norm": (
        _I32, [_VP, _I64, _VP, _I32, _VP, _F32, _VP, _VP, _VP, _I32, _TILE, _VP, _I64, _VP]),
    "grpo_nf4_tile_linear_residual": (
        _I32, [_VP, _I64, _VP, _VP, _VP, _I32, _TILE, _VP, _VP, _I64, _VP, _VP]),
    "grpo_paged_attn_noalloc_max_bytes": (_SZ, []),
    "grpo_paged_attn_decode_noalloc": (
        _I32,
        [_VP, _I64, _I64, _VP, _VP, _I64, _VP, _I64, _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I32,
         _I32, _F32, _VP],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None
_device_ok: bool | None = None
_device_error: str | None = None


def library_path() -> Path:
    return LIB_PATH


def _load() -> ctypes.CDLL:
    global _lib, _load_error
    with _lock:
        if _lib is not None:
            return _lib
        if _load_error is not None:
            raise ImportError(_load_error)
        if not LIB_PATH.exists():
            _load_error = (f"libgrpo_hip.so not built ({LIB_PATH}); run "
                           "__graft_entry__.build() or python -m grpo_mi355x._build")
            raise ImportError(_load_error)
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - depends on the host
            _load_error = f"cannot load {LIB_PATH}: {exc}"
            raise ImportError(_load_error) from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def library() -> ctypes.CDLL:
    """The loaded library (no device needed); ImportError if it is not built."""
    return _load()


def device_library() -> ctypes.CDLL:
    """The library after checking that a gfx950 device is usable.

    Raises ImportError when there is no device, so callers that follow the
    reference's ``except ImportError`` fallback chain behave as they do there.
    """
    global _device_ok, _device_error
    lib = _load()
    if _device_ok is None:
        if not torch.cuda.is_available():
            _device_ok, _device_error = False, "no ROCm/HIP device visible to torch"
        else:
            rc = lib.grpo_init()
            _device_ok = rc == 0
            if not _device_ok:
                _device_error = lib.grpo_last_error().decode(errors="replace")
    if not _device_ok:
        raise ImportError(f"libgrpo_hip unavailable: {_device_error}")
    return lib


def available() -> bool:
    """True when the library is built and a gfx950 device is usable."""
    try:
        device_library()
        return True
    except ImportError:
        return False


def check(rc: int, what: str) -> None:
    """Map a C-ABI return code to the reference's exception types."""
    if rc == 0:
        return
    msg = _load().grpo_last_error().decode(errors="replace")
    if rc < 0:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {rc}: {msg}")


def stream_handle(device: torch.device | None = None) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an integer)."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
