"""Build libgrpo_hip.so in-tree with hipcc for gfx950.

``python -m grpo_mi355x._build`` (with ``grpo-training-engine_amd`` on
``sys.path``) or ``build_library()`` compiles ``csrc/*.hip`` into
``grpo_mi355x/_native/libgrpo_hip.so``.  The library is built in the source
tree so that it travels with the repository snapshot to the GPU host.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
PROJECT_DIR = PKG_DIR.parent
CSRC = PROJECT_DIR / "csrc"
NATIVE_DIR = PKG_DIR / "_native"
LIB_PATH = NATIVE_DIR / "libgrpo_hip.so"
ARCH = "gfx950"

SOURCES = ("capi.hip", "nf4_linear.hip", "paged_attention.hip", "decode_ops.hip", "lm_head.hip",
           "sampling.hip", "nf4_backward.hip")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libgrpo_hip)")


def build_command(out: Path) -> list[str]:
    srcs = [str(CSRC / s) for s in SOURCES if (CSRC / s).exists()]
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Keep the compiler from emitting packed-FP32 VALU ops (v_pk_*_f32).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-o", str(out),
        *srcs,
    ]


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source into ``_native/libgrpo_hip.so`` (always rebuilds)."""
    NATIVE_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = build_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        msg = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{msg}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    p = build_library(verbose=True)
    print(p)
    sys.exit(0)
