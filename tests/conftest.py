"""Shared pytest setup: import paths, the `gpu` marker, device fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
PKG_ROOT = REPO / "mini-kvllm_amd"
for p in (str(PKG_ROOT), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmkv.so")


@pytest.fixture(scope="session")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from mkv import _lib

    _lib.load()  # raise now (not skip) if the native library is missing
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Name the GPU case on stdout before it runs (flushed), so a run that
    dies inside a kernel still says which case it was."""
    print(f"[case] {msg}", flush=True)


def assert_close_out(got: torch.Tensor, want: torch.Tensor, out_dtype: torch.dtype,
                     abs_tol: float) -> None:
    """|got - want| <= abs_tol + half an ulp of out_dtype at |want|.

    The kernels, like the reference, compute in fp32 and round the result to
    the query dtype on store; abs_tol bounds the error before that rounding
    and the half-ulp term is the rounding itself (0 for fp32 outputs)."""
    got = got.double().cpu()
    want = want.double().cpu()
    if out_dtype == torch.float32:
        tol = torch.full_like(want, abs_tol)
    else:
        mant = {torch.bfloat16: 8, torch.float16: 11}[out_dtype]
        e = torch.floor(torch.log2(want.abs().clamp(min=2.0 ** -14)))
        tol = abs_tol + 0.5 * torch.exp2(e - (mant - 1))
    err = (got - want).abs()
    # a NaN (or inf - inf) difference is a failure unless both sides are NaN
    # there; `err > tol` alone is False for NaN and would let it pass
    both_nan = torch.isnan(got) & torch.isnan(want)
    bad = ~(err <= tol) & ~both_nan
    assert not bool(bad.any()), (
        f"{int(bad.sum())} of {err.numel()} elements out of tolerance; max abs err "
        f"{float(err.max()):.3e}, max excess {float((err - tol).max()):.3e} (abs_tol {abs_tol})")


def compact_pool(k_cache, v_cache, block_tables, context_lens):
    """The blocks that the given sequences use, gathered on the device and
    copied to the host as a small pool, with their block tables renumbered
    into it (absent entries stay -1): the float64 oracle then checks sampled
    rows of a full-size workload without copying the whole pool."""
    bs = k_cache.shape[1]
    bt = block_tables.cpu().clone()
    used = sorted({int(x) for s in range(bt.shape[0])
                   for x in bt[s, :(int(context_lens[s]) + bs - 1) // bs] if int(x) >= 0})
    remap = {p: i for i, p in enumerate(used)}
    nb = bt.shape[1]
    for s in range(bt.shape[0]):
        need = (int(context_lens[s]) + bs - 1) // bs
        for j in range(nb):
            x = int(bt[s, j])
            bt[s, j] = remap[x] if (j < need and x >= 0) else -1
    idx = torch.tensor(used if used else [0], dtype=torch.int64, device=k_cache.device)
    return k_cache.index_select(0, idx).cpu(), v_cache.index_select(0, idx).cpu(), bt
