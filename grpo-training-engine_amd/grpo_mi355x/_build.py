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

SOURCES = ("capi.hip", "nf4_linear.hip", "nf4_fold.hip", "nf4_tile.hip", "nf4_gemm.hip",
           "paged_attention.hip", "decode_ops.hip", "lm_head.hip", "sampling.hip",
           "nf4_backward.hip")

# Flags of one source only (machine-scheduler strategies measured per source
# on the decode step): the folded down_proj kernel is scheduled for
# instruction-level parallelism (it runs two waves per SIMD; nf4_fold.hip), the
# attention kernels for clauses of memory operations (same registers; config 3
# 3637 -> 3670 tok/s).
SOURCE_FLAGS = {"nf4_fold.hip": ("-mllvm", "-amdgpu-sched-strategy=max-ilp"),
                "paged_attention.hip": ("-mllvm", "-amdgpu-sched-strategy=max-memory-clause")}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libgrpo_hip)")


COMPILE_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Keep the compiler from emitting packed-FP32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        msg = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{msg}")


def build_library(verbose: bool = False, jobs: int = 0, incremental: bool = False) -> Path:
    """Compile every HIP source into ``_native/libgrpo_hip.so`` (always rebuilds).

    Each source is compiled to an object of its own, in parallel (``jobs``
    processes, default: one per source up to the CPU count), and the objects
    are linked into the library.  ``incremental`` keeps the objects and
    recompiles only sources newer than their object (or any header newer)."""
    from concurrent.futures import ThreadPoolExecutor

    NATIVE_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = NATIVE_DIR / "_obj"
    obj_dir.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES if (CSRC / s).exists()]
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    cc = hipcc()
    hdr = max((h.stat().st_mtime for h in CSRC.glob("*.hpp")), default=0.0)
    hdr = max(hdr, (PROJECT_DIR.parent / "include" / "grpo_hip.h").stat().st_mtime
              if (PROJECT_DIR.parent / "include" / "grpo_hip.h").exists() else 0.0)

    def stale(s: Path, o: Path) -> bool:
        return (not incremental or not o.exists()
                or o.stat().st_mtime < max(s.stat().st_mtime, hdr))

    cmds = [[cc, *COMPILE_FLAGS, *SOURCE_FLAGS.get(s.name, ()), "-c", "-o", str(o), str(s)]
            for s, o in zip(srcs, objs) if stale(s, o)]
    jobs = jobs or max(1, min(len(cmds), os.cpu_count() or 1))
    if verbose:
        for c in cmds:
            print(" ".join(c), flush=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, c) for c in cmds]:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-fPIC", "-shared", "-o", str(tmp),
            *[str(o) for o in objs]]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    if not incremental:
        for o in objs:
            o.unlink()
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    p = build_library(verbose=True, incremental="--incremental" in sys.argv)
    print(p)
    sys.exit(0)
