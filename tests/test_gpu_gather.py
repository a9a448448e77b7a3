"""GPU parity of K4 (block-table gather): bit-exact against the oracle."""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from mkv import attention as A
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("bs", [16, 256])
def test_gather_bit_exact(dev, dtype, bs):
    announce(f"gather {dtype} bs={bs}")
    g = torch.Generator().manual_seed(bs)
    B, H, D, N = 5, 8, 128, 40
    ctx = torch.tensor([1, bs - 1, bs, 3 * bs + 5, 0], dtype=torch.int64)
    bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=5)
    bt[3, 1] = -1  # an absent block inside the context reads as zeros
    cache = torch.randn(N, bs, H, D, generator=g).to(dtype)
    max_len = 5 * bs
    got = A.gather_kv(cache.to(dev), bt.to(dev), ctx.to(dev), max_len)
    want = R.gather_kv_ref(cache, bt, ctx, max_len)
    assert torch.equal(got.cpu().view(torch.uint8), want.view(torch.uint8))
    got32 = A.gather_kv(cache.to(dev), bt.to(dev), ctx.to(torch.int32).to(dev), max_len)
    assert torch.equal(got32.cpu().view(torch.uint8), want.view(torch.uint8))
