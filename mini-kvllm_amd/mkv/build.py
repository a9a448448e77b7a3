"""Build recipe for libmkv.so (the HIP/gfx950 KV-cache kernels + C ABI).

Compiles every ``csrc/*.hip`` / ``csrc/*.cpp`` file with hipcc for gfx950 in
parallel and links them into ``mkv/libmkv.so`` next to this file.  No GPU is
needed: hipcc cross-compiles.  Run ``python -m mkv.build`` from
``mini-kvllm_amd/`` or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_DIR = PKG_DIR.parent / "csrc"
REPO_DIR = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libmkv.so"
BUILD_DIR = PKG_DIR.parent / "_build"

ARCH = "gfx950"
# Packed fp32 VALU ops are disabled for every device compile: some of their
# forms have produced wrong results on this hardware without any error.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libmkv")


def sources() -> list[Path]:
    return sorted(list(SRC_DIR.glob("*.hip")) + list(SRC_DIR.glob("*.cpp")))


def _compile(hipcc: str, src: Path, obj: Path) -> str:
    cmd = [hipcc, *DEVICE_FLAGS, f"-I{INCLUDE_DIR}", f"-I{SRC_DIR}", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")
    return msg


def build(verbose: bool = False) -> Path:
    """Compile all sources and link libmkv.so; returns the library path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    objs = [BUILD_DIR / (s.name + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, msg in zip(srcs, ex.map(lambda so: _compile(hipcc, *so), zip(srcs, objs))):
            if verbose and msg.strip():
                print(f"[mkv.build] {src.name}:\n{msg}", file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
