"""Build recipe for libmkv.so (the HIP/gfx950 KV-cache kernels + C ABI).

Compiles every ``csrc/*.hip`` / ``csrc/*.cpp`` file with hipcc for gfx950 in
parallel and links them into ``mkv/libmkv.so`` next to this file.  No GPU is
needed: hipcc cross-compiles.  Run ``python -m mkv.build`` from
``mini-kvllm_amd/`` or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
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


# The compiler's per-kernel resource report (registers, spills, scratch,
# occupancy) for each source, kept beside its object file.
RESOURCE_FLAG = "-Rpass-analysis=kernel-resource-usage"


def _resource_path(obj: Path) -> Path:
    return obj.with_suffix(obj.suffix + ".resources.txt")


def _compile(hipcc: str, src: Path, obj: Path) -> str:
    cmd = [hipcc, *DEVICE_FLAGS, RESOURCE_FLAG, f"-I{INCLUDE_DIR}", f"-I{SRC_DIR}", "-c", str(src), "-o",
           str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    lines = [l for l in (r.stdout + r.stderr).splitlines() if noise not in l]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(lines))
    _resource_path(obj).write_text("\n".join(l for l in lines if "remark:" in l) + "\n")
    return "\n".join(l for l in lines if "remark:" not in l and l.strip() and not l.lstrip()[:1].isdigit()
                     and not l.lstrip().startswith("|"))


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


def parse_resources(text: str) -> dict[str, dict[str, int]]:
    """Per-kernel figures of a -Rpass-analysis=kernel-resource-usage report:
    {mangled kernel name: {"VGPRs", "AGPRs", "SGPRs", "VGPRs Spill", "SGPRs
    Spill", "ScratchSize", "Occupancy", ...}}."""
    out: dict[str, dict[str, int]] = {}
    cur = None
    for line in text.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\d+) \[-Rpass", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = int(m.group(2))
    return out


def kernel_resources() -> dict[str, dict[str, int]]:
    """The resource report of every kernel in csrc/: from the last build's
    reports when they are newer than every source and header, else by
    compiling the sources' device code again (no link)."""
    hipcc = _hipcc()
    headers = list(SRC_DIR.glob("*.hpp")) + list(INCLUDE_DIR.glob("*.h"))
    newest_header = max((h.stat().st_mtime for h in headers), default=0.0)
    res: dict[str, dict[str, int]] = {}
    for src in sources():
        if src.suffix != ".hip":
            continue
        rep = _resource_path(BUILD_DIR / (src.name + ".o"))
        if not (rep.exists() and rep.stat().st_mtime >= max(src.stat().st_mtime, newest_header)):
            BUILD_DIR.mkdir(parents=True, exist_ok=True)
            _compile(hipcc, src, BUILD_DIR / (src.name + ".o"))
        res.update(parse_resources(rep.read_text()))
    return res


if __name__ == "__main__":
    print(build(verbose=True))
