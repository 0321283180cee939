"""Builds libqwen3_attn.so, the gfx950 HIP kernels behind the C ABI in
include/qwen3_attn.h, in-tree next to this file.

    python -m qwen3_engine_from_scratch_amd.build

Every .hip file under csrc/ is compiled to an object in parallel with hipcc
(cross-compiling for gfx950 works without a GPU), then linked into one shared
library.  The library is loaded with ctypes by _lib.py.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = REPO_DIR / "_build" / "qwen3_attn"
LIB_NAME = "libqwen3_attn.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for every device pass; the host pass
# prints a harmless "not a recognized feature" warning for it.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP kernels)")
    return found


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # Keep warnings visible, minus the known host-pass feature notice.
    noise = "is not a recognized feature for this target"
    lines = [ln for ln in (res.stderr or "").splitlines() if noise not in ln]
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def build(verbose: bool = True) -> Path:
    """Compiles all kernels and links LIB_PATH; returns its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, sources, objs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build()
