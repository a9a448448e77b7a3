"""GPU tests of the engine's fused row kernels (mkv_rmsnorm, mkv_silu_mul)
against float64 references of LayerNorm.rms_forward / residual_rms_forward
(layernorm.py:16-33) and SiluAndMul (activation.py:16-19).

The kernels compute in fp32 and round once, so the bound is half an ulp of
the output dtype at the reference value plus a 2e-6 relative margin for the
fp32 arithmetic; the updated residual (x + residual rounded to the dtype) is
bit-exact against torch's own add."""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from mkv import engine as E

pytestmark = pytest.mark.gpu

MANT = {torch.float32: 24, torch.bfloat16: 8, torch.float16: 11}
EMIN = {torch.float32: -126, torch.bfloat16: -126, torch.float16: -14}  # below: subnormal spacing


def _check(got, want, dtype):
    got, want = got.double().cpu(), want.double().cpu()
    e = torch.floor(torch.log2(want.abs().clamp(min=2.0 ** -149))).clamp(min=EMIN[dtype])
    tol = 0.5 * torch.exp2(e - (MANT[dtype] - 1)) + 2e-6 * want.abs() + 1e-30
    # (a NaN difference fails unless both sides are NaN; `> tol` alone passes it)
    bad = ~((got - want).abs() <= tol) & ~(torch.isnan(got) & torch.isnan(want))
    assert not bool(bad.any()), f"{int(bad.sum())} elements off; max err {float((got - want).abs().max()):.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,hidden", [(1, 1024), (64, 1024), (1000, 1024), (7, 2048), (33, 520)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm(dev, dtype, rows, hidden, with_residual):
    announce(f"rmsnorm {dtype} {rows}x{hidden} residual={with_residual}")
    g = torch.Generator().manual_seed(rows + hidden)
    x = (torch.randn(rows, hidden, generator=g) * 3).to(dtype)
    w = (1 + 0.5 * torch.randn(hidden, generator=g)).to(dtype)
    r = torch.randn(rows, hidden, generator=g).to(dtype) if with_residual else None
    xd, wd = x.to(dev), w.to(dev)
    rd = r.to(dev) if with_residual else None
    out = E.rms_norm(xd, wd, 1e-5, rd)
    h = (x + r) if with_residual else x  # torch's add: fp32 then one rounding
    if with_residual:
        assert torch.equal(rd.cpu(), h)
    hd = h.double()
    want = hd * w.double() / torch.sqrt(hd.pow(2).mean(-1, keepdim=True) + 1e-5)
    _check(out, want, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,inter", [(1, 3072), (64, 3072), (1024, 3072), (5, 24)])
def test_silu_mul(dev, dtype, rows, inter):
    announce(f"silu_mul {dtype} {rows}x{inter}")
    g = torch.Generator().manual_seed(rows + inter)
    x = (torch.randn(rows, 2 * inter, generator=g) * 4).to(dtype)
    x[0, :4] = torch.tensor([-100.0, 100.0, 0.0, -0.0]).to(dtype)
    out = E.silu_and_mul(x.to(dev))
    a, b = x[:, :inter].double(), x[:, inter:].double()
    _check(out, a / (1 + torch.exp(-a)) * b, dtype)


def test_silu_mul_strided_rows(dev):
    announce("silu_mul on a strided row view")
    g = torch.Generator().manual_seed(3)
    big = torch.randn(16, 2 * 64 + 32, generator=g).to(torch.bfloat16).to(dev)
    x = big[:, :128]
    out = E.silu_and_mul(x)
    a, b = x[:, :64].double().cpu(), x[:, 64:].double().cpu()
    _check(out, a / (1 + torch.exp(-a)) * b, torch.bfloat16)
