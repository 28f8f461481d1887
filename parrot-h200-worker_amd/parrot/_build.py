"""Compile the gfx950 HIP kernels into ``parrot/_lib/libparrot_hip.so``.

Usage: ``python -m parrot._build`` (with ``parrot-h200-worker_amd`` on
``sys.path``) or ``parrot._build.build()``.  Cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
KERNELS = PACKAGE / "kernels"
LIB_DIR = PACKAGE / "_lib"
LIBRARY = LIB_DIR / "libparrot_hip.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU instructions.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP kernels cannot be built")
    return path


def sources() -> list[Path]:
    return sorted(KERNELS.glob("*.hip"))


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that the device-only feature is unknown: harmless.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(jobs: int | None = None) -> Path:
    """Compile every kernel source and link the C-ABI shared library."""
    hipcc = _hipcc()
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda so: _compile(hipcc, *so), zip(srcs, objs)))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
