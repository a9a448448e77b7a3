"""CPU check of the compiler's per-kernel resource report for the decode and
prefill kernels (hipcc -Rpass-analysis=kernel-resource-usage, gfx950): no
VGPR spills and no scratch memory in any of them.  A spilled register is
reloaded from scratch memory, and a reload inside a key loop waits behind
the tile prefetches in flight.  The report comes from the last build when it
is newer than the sources (mkv.build writes it beside each object file),
else the sources' device code is compiled here.  SGPR spills go to VGPR
lanes (v_writelane / v_readlane, no memory), so they are reported, not
failed."""
from __future__ import annotations

import shutil
import subprocess

import pytest

from mkv import build


def _demangle(names):
    tool = shutil.which("c++filt") or shutil.which("llvm-cxxfilt")
    if not tool:
        return {n: n for n in names}
    out = subprocess.run([tool], input="\n".join(names), capture_output=True, text=True).stdout.splitlines()
    return dict(zip(names, out)) if len(out) == len(names) else {n: n for n in names}


@pytest.fixture(scope="module")
def resources():
    try:
        build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    return build.kernel_resources()


def test_decode_and_prefill_kernels_do_not_spill(resources):
    hot = {k: v for k, v in resources.items() if "paged_decode" in k or "prefill" in k}
    names = _demangle(list(hot))
    assert len(hot) >= 60, f"expected every decode / prefill instantiation, found {len(hot)}"
    bad = {names[k]: (v.get("VGPRs Spill"), v.get("ScratchSize")) for k, v in hot.items()
           if v.get("VGPRs Spill", 0) or v.get("ScratchSize", 0)}
    assert not bad, f"VGPR spills / scratch bytes per lane: {bad}"
    missing = [names[k] for k, v in hot.items() if "VGPRs Spill" not in v or "ScratchSize" not in v]
    assert not missing, f"no resource figures for {missing}"
    sgpr = {names[k]: v["SGPRs Spill"] for k, v in hot.items() if v.get("SGPRs Spill", 0)}
    print(f"{len(hot)} decode / prefill kernels: no VGPR spills, no scratch; SGPR spills to VGPR lanes "
          f"in {len(sgpr)}")


def test_headline_decode_kernel_residency(resources):
    """The batch-256 FP8 decode kernel (stream-K, groups of up to 4 query
    heads) holds two waves per SIMD: its persistent grid is sized for that."""
    names = _demangle(list(resources))
    k = [n for n in resources if "paged_decode_stream_kernelILi3ELb1ELb0E" in n]
    assert len(k) == 1, names
    r = resources[k[0]]
    assert r["Occupancy"] >= 2 and r["VGPRs"] + r["AGPRs"] <= 256, r
