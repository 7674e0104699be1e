"""Compile the gfx950 HIP sources into the in-tree C-ABI library librlt_kv.so.

Every call recompiles (no up-to-date check): the caller decides when to build.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
PROJECT_DIR = PACKAGE_DIR.parent
REPO_DIR = PROJECT_DIR.parent
CSRC_DIR = PROJECT_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = PROJECT_DIR / "_build"
LIBRARY = PACKAGE_DIR / "librlt_kv.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for all device code; -O3 would otherwise
# emit v_pk_{add,mul,fma}_f32 from ordinary float code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build librlt_kv.so")
    return path


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def _compile(source: Path) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [hipcc(), *DEVICE_FLAGS, f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{result.stderr}")
    return obj


def build(jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link librlt_kv.so in the package."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2) // 2), 8)
    with ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking librlt_kv.so failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
