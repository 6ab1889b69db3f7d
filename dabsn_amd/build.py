"""Build the gfx950 HIP library ``dabsn_amd/_build/libdabsn_hip.so``.

Each ``csrc/*.hip`` translation unit is compiled with hipcc for gfx950 (objects in
parallel), then linked into one shared library exposing the C ABI declared in
``include/dabsn_hip.h``. ``python -m dabsn_amd.build`` rebuilds unconditionally.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "_build"
LIB = OUT / "libdabsn_hip.so"
ARCH = os.environ.get("DABSN_HIP_ARCH", "gfx950")

FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    # Match the reference CPU backend's strict evaluation (no implicit FMA contraction).
    "-ffp-contract=off",
    # Packed fp32 ops are kept off on this target.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the DABSN HIP library needs ROCm")
    return exe


def _compile(src: Path) -> Path:
    obj = OUT / (src.stem + ".o")
    cmd = [_hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    for o in objs:
        o.unlink(missing_ok=True)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
