"""Shared pytest setup.

* ``gpu`` marker: tests that need the MI355X (run with ``-m gpu``); everything
  else runs on CPU.
* Paths: the repository root (for ``oracle``) and ``grpo-training-engine_amd``
  (for the ``grpo_mi355x`` package) go on ``sys.path``.
* Inputs are generated on the CPU from seeded generators and then moved to the
  device, so seeds mean the same thing on every host.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
PKG = os.path.join(ROOT, "grpo-training-engine_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libgrpo_hip.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from grpo_mi355x import _lib

    _lib.device_library()  # raises ImportError (test error) if the HIP library is unusable
    return torch.device("cuda:0")


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def bf16_bits(a) -> np.ndarray:
    from oracle.bf16 import f32_to_bf16_bits

    return f32_to_bf16_bits(np.asarray(a, dtype=np.float32))


def to_dev_bf16(bits: np.ndarray, device):
    """uint16 bf16 bit patterns (numpy) -> torch bf16 tensor on device."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16)
    return t.to(device)


def from_bf16(t) -> np.ndarray:
    """torch bf16 tensor -> uint16 bit patterns (numpy)."""
    import torch

    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """max|a - b| / max|b| (float64)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    denom = max(np.abs(b).max(), 1e-30)
    return float(np.abs(a - b).max() / denom)
