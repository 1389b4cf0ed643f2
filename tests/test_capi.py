"""CPU checks of the C ABI: the library loads, exports every function declared in
include/grpo_hip.h, and its host-only functions behave (no kernel is launched)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "grpo_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(grpo_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from grpo_mi355x import _lib

    if not _lib.library_path().exists():
        pytest.fail("libgrpo_hip.so is not built: run __graft_entry__.build()")
    return _lib.library()


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("grpo_nf4_dequant", "grpo_nf4_lora_linear", "grpo_paged_kv_append",
              "grpo_paged_attn_decode", "grpo_last_error", "grpo_init"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_python_signatures_cover_the_header():
    from grpo_mi355x import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_version_and_workspace_sizes(lib):
    assert lib.grpo_version() == 100
    assert lib.grpo_paged_attn_workspace_bytes(8, 12, 2, 128, 16, 64) > 0
    assert lib.grpo_paged_attn_workspace_bytes(8, 12, 2, 8, 4, 64) == 0  # generic path


def test_argument_errors_return_negative_codes(lib):
    rc = lib.grpo_nf4_dequant(None, None, None, None, -1, 64, None)
    assert rc < 0 and b"numel" in lib.grpo_last_error()
    rc = lib.grpo_nf4_lora_linear(None, 0, None, None, None, 64, None, None, None, 0, 1.0, None,
                                  0, 1, 1, 1, None)
    assert rc < 0 and b"null" in lib.grpo_last_error()
    rc = lib.grpo_paged_attn_decode(None, 0, 0, None, None, 1, None, 0, None, None, 0, 1, 12, 5,
                                    128, 16, 4, 1.0, None, 0, None)
    assert rc < 0 and b"multiple" in lib.grpo_last_error()
    # empty problems are no-ops
    assert lib.grpo_nf4_dequant(None, None, None, None, 0, 64, None) == 0


def test_check_maps_codes_to_reference_exceptions(lib):
    from grpo_mi355x import _lib

    lib.grpo_nf4_dequant(None, None, None, None, -1, 64, None)
    with pytest.raises(ValueError):
        _lib.check(-1, "x")
    with pytest.raises(RuntimeError):
        _lib.check(7, "x")


def test_no_device_means_import_error():
    import torch

    from grpo_mi355x import _lib

    if torch.cuda.is_available():
        pytest.skip("a device is present")
    with pytest.raises(ImportError):
        _lib.device_library()
    from grpo_mi355x import kernels

    assert kernels.HIP_AVAILABLE is False
    with pytest.raises(ImportError):
        kernels.lora_fused_forward(torch.zeros(1, 1, 4))
    with pytest.raises(ImportError):
        kernels.paged_kv_decode(None, torch.zeros(1, 1, dtype=torch.long))
