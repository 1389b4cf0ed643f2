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
    # split-K linear: partial sums [splits, M, N] float32 (+ LoRA [splits, nseg, M, 16])
    assert lib.grpo_nf4_lora_linear_workspace_bytes(8, 1536, 8960, 0, 1, 64) >= 8 * 1536 * 4
    assert lib.grpo_nf4_lora_linear_workspace_bytes(8, 48, 100, 4, 1, 64) == 0  # generic
    assert lib.grpo_nf4_lora_linear_workspace_bytes(8, 256, 512, 16, 1, 96) == 0  # blocksize


def test_split_k_plan_covers_k_exactly():
    """Every plan's slices cover K: splits * kpw >= K/256 > (splits - 1) * kpw for a
    k-steps-per-slice value kpw in {1, 2, 3, 4, 5, 6, 8} (5 only for more than 16
    rows); partial bytes match the layout."""
    from grpo_mi355x.kernels import ops

    for m, n, k, r, nseg in [(8, 2048, 1536, 16, 3), (8, 1536, 1536, 16, 1), (8, 17920, 1536, 0, 1),
                             (8, 1536, 8960, 0, 1), (64, 512, 3584, 16, 3), (1, 256, 512, 16, 1),
                             (33, 256, 768, 16, 1), (8, 3584, 18944, 0, 1),
                             (64, 3584, 18944, 0, 1), (64, 4608, 3584, 16, 3)]:
        splits, pb, tb = ops.nf4_linear_plan(m, n, k, r, nseg, 64)
        ks = k // 256
        kpws = (1, 2, 3, 4, 5, 6, 8) if m > 16 else (1, 2, 3, 4, 6, 8)
        assert any(splits * kpw >= ks > (splits - 1) * kpw for kpw in kpws)
        assert pb == splits * m * n * 4
        assert tb == (splits * nseg * m * 16 * 4 if r else 0)
    # Qwen2-7B's down_proj at 64 rows: 15 slices of 5 k-steps (one workgroup round)
    assert ops.nf4_linear_plan(64, 3584, 18944, 0, 1, 64)[0] == 15
    assert ops.nf4_linear_plan(8, 40, 512, 0, 1, 64) is None  # N % 16
    assert ops.nf4_linear_plan(65, 256, 512, 0, 1, 64) is None  # M > 64
    # 16 slices of 8 k-steps: even 16 staged rows of x exceed LDS
    assert ops.nf4_linear_plan(16, 256, 32768, 0, 1, 64) is None


def test_argument_errors_return_negative_codes(lib):
    rc = lib.grpo_nf4_dequant(None, None, None, None, -1, 64, None)
    assert rc < 0 and b"numel" in lib.grpo_last_error()
    rc = lib.grpo_nf4_lora_linear(None, 0, None, None, None, 64, None, None, None, 0, 1.0, None,
                                  0, 1, 1, 1, None, 0, None)
    assert rc < 0 and b"null" in lib.grpo_last_error()
    rc = lib.grpo_paged_attn_decode(None, 0, 0, None, None, 1, None, 0, None, None, 0, 1, 12, 5,
                                    128, 16, 4, 1.0, None, 0, None)
    assert rc < 0 and b"multiple" in lib.grpo_last_error()
    # empty problems are no-ops
    assert lib.grpo_nf4_dequant(None, None, None, None, 0, 64, None) == 0
    # split-K descriptors are validated before anything is launched
    from grpo_mi355x import _lib

    d = _lib.LinearParts()
    d.splits, d.M, d.N, d.K, d.nseg = 1, 8, 256, 512, 1
    d.seg_end[0] = 256
    assert lib.grpo_nf4_linear_finish(d, None, 256, None) < 0  # null part buffer
    d.part = 16
    d.seg_end[0] = 128
    assert lib.grpo_nf4_linear_finish(d, None, 256, None) < 0
    assert b"segment" in lib.grpo_last_error()
    d.seg_end[0] = 256
    d.r = 16
    assert lib.grpo_add_rmsnorm_parts(d, None, None, None, None, 1e-6, None) < 0  # no tpart
    # the screened lm_head's passes check the workspace against its size (before
    # any launch: the addresses below are never dereferenced)
    V, K, M, fake = 4096, 512, 4, 1 << 20
    need = lib.grpo_lm_head_screen_workspace_bytes(M, V)
    assert need > 2048
    assert lib.grpo_lm_head_screen(fake, K, fake, fake, fake, V, K, M, fake, need - 1,
                                   None) == -3  # GRPO_EWORKSPACE
    assert lib.grpo_lm_head_exact_argmax(fake, K, fake, V, K, M, fake, need - 1, None, fake,
                                         None) == -3
    assert b"workspace" in lib.grpo_last_error()
    assert lib.grpo_lm_head_exact_argmax(fake, K, fake, V, K, 9, fake, need, None, fake,
                                         None) < 0  # rows


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


def test_build_compiles_every_source_with_its_flags():
    """Every HIP source in csrc/ is built, each per-source flag set names a
    built source, and the per-source flags are machine-scheduler strategies
    only (they change instruction order, not results)."""
    from grpo_mi355x import _build

    csrc = {p.name for p in _build.CSRC.glob("*.hip")}
    assert csrc == set(_build.SOURCES)
    assert set(_build.SOURCE_FLAGS) <= set(_build.SOURCES)
    for flags in _build.SOURCE_FLAGS.values():
        assert flags[0] == "-mllvm" and flags[1].startswith("-amdgpu-sched-strategy=")
