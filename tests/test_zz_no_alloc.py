"""GPU test of mkv_paged_decode_noalloc, the decode entry point that takes no
workspace (its partials live in the library's static per-device scratch).

It must give the same bytes as mkv_paged_decode with a caller workspace (the
same kernels and schedule) on consecutive calls that reuse the scratch, the
second with a smaller batch, for the stream-K route (FP8 per tensor, bf16,
per-token-head FP8) and the split-K route (fp32 cache, explicit splits); and
refuse an explicit route larger than the scratch before launching anything.
With the library's choice of route, a call whose stream-K slots do not fit
(16 query heads per KV head on 256 CUs) takes the workgroup route instead:
the same result within rounding.
"""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

from conftest import announce, assert_close_out
from mkv import _lib
from mkv import attention as A
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu

D = 128


def _pools(dev, fmt, N, bs, Hkv, g):
    x = torch.randn(N, bs, Hkv, D, generator=g)
    y = torch.randn(N, bs, Hkv, D, generator=g)
    if fmt == "fp8":
        ks = float(x.abs().amax() / 448)
        vs = float(y.abs().amax() / 448)
        kc = (x / ks).to(torch.float8_e4m3fn).to(dev)
        vc = (y / vs).to(torch.float8_e4m3fn).to(dev)
        return kc, vc, torch.tensor([ks], device=dev), torch.tensor([vs], device=dev), _lib.SCALE_PER_TENSOR
    if fmt == "fp8_token":
        kc = torch.empty(N, bs, Hkv, D, dtype=torch.float8_e4m3fn, device=dev)
        vc = torch.empty_like(kc)
        kst = torch.empty(N, bs, Hkv, device=dev)
        vst = torch.empty_like(kst)
        slots = torch.arange(N * bs, device=dev)
        A.store_kvcache_fp8(x.to(dev).reshape(-1, Hkv, D), y.to(dev).reshape(-1, Hkv, D), kc, vc,
                            kst, vst, slots, bs, "fp8_per_token_head")
        return kc, vc, kst, vst, _lib.SCALE_PER_TOKEN_HEAD
    dt = {"bf16": torch.bfloat16, "f32": torch.float32}[fmt]
    return x.to(dt).to(dev), y.to(dt).to(dev), None, None, _lib.SCALE_PER_TENSOR


def _call(name, out, q, kc, vc, ks, vs, mode, bt, ctx, Hq, Hkv, bs, split, ws=None):
    dev = q.device
    args = [out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), A._dtype_code(q, "q"),
            kc.data_ptr(), vc.data_ptr(), A._dtype_code(kc, "k"), kc.shape[0],
            ks.data_ptr() if ks is not None else None, vs.data_ptr() if vs is not None else None,
            mode, bt.data_ptr(), bt.stride(0), bt.shape[1], ctx.data_ptr(), _lib.INDEX_I64,
            q.shape[0], Hq, Hkv, D, bs, 1.0 / math.sqrt(D), split]
    if name == "mkv_paged_decode":
        args += [ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0]
    args.append(torch.cuda.current_stream(dev).cuda_stream)
    _lib.call(name, *args)


CASES = [  # (kv format, Hq, Hkv, bs, split_tokens, batches)
    ("fp8", 32, 8, 256, 0, (256, 40)),
    ("bf16", 16, 8, 16, 0, (96, 7)),
    ("fp8_token", 32, 8, 256, 0, (64, 5)),
    ("f32", 16, 8, 256, 0, (4, 2)),
    ("bf16", 32, 4, 64, 256, (48, 9)),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-g{c[1] // c[2]}-bs{c[3]}-split{c[4]}" for c in CASES])
def test_noalloc_decode_matches_workspace_decode(dev, case):
    fmt, Hq, Hkv, bs, split, batches = case
    announce(f"noalloc decode vs workspace decode: {case}")
    g = torch.Generator().manual_seed(900 + len(fmt) + Hq + bs + split)
    N = 160
    kc, vc, ks, vs, mode = _pools(dev, fmt, N, bs, Hkv, g)
    mb = max(1, 2048 // bs)
    for call, B in enumerate(batches):
        ctx = torch.randint(0, mb * bs + 1, (B,), generator=g)
        ctx[0] = 0  # a padded row: zeros
        if int(((ctx + bs - 1) // bs).sum()) <= N:
            bt = W.fragmented_block_tables(ctx, bs, N, g)
        else:  # blocks shared between sequences: fine for reads
            bt = torch.randint(0, N, (B, mb), generator=g, dtype=torch.int32)
        if bt.shape[1] < mb:
            bt = torch.cat([bt, torch.full((B, mb - bt.shape[1]), -1, dtype=torch.int32)], 1)
        q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(dev)
        bt_d, ctx_d = bt.to(dev).contiguous(), ctx.to(dev)
        need = _lib.query("mkv_paged_decode_workspace_size", B, Hq, Hkv, mb, bs, D,
                          A._dtype_code(kc, "k"), split)
        assert need <= _lib.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        want = torch.full_like(q, float("nan"))
        got = torch.full_like(q, float("nan"))
        _call("mkv_paged_decode", want, q, kc, vc, ks, vs, mode, bt_d, ctx_d, Hq, Hkv, bs, split, ws)
        _call("mkv_paged_decode_noalloc", got, q, kc, vc, ks, vs, mode, bt_d, ctx_d, Hq, Hkv, bs, split)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {call} (batch {B})"
        assert torch.count_nonzero(got[0].float()) == 0
        assert bool(torch.isfinite(got.float()).all())


def test_noalloc_decode_refuses_oversized_requests(dev):
    announce("noalloc decode: request beyond the static scratch")
    B, Hq, Hkv, bs, mb = 1024, 32, 8, 256, 32
    q = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev)
    out = torch.full_like(q, 3.0)
    kc = torch.zeros(8, bs, Hkv, D, dtype=torch.float32, device=dev)
    bt = torch.zeros(B, mb, dtype=torch.int32, device=dev)
    ctx = torch.ones(B, dtype=torch.int64, device=dev)
    with pytest.raises(_lib.MkvError) as e:
        _call("mkv_paged_decode_noalloc", out, q, kc, kc, None, None, 0, bt, ctx, Hq, Hkv, bs, 32)
    assert e.value.status == -10
    torch.cuda.synchronize()
    assert bool((out == 3.0).all()), "a refused call must not launch"


@pytest.mark.parametrize("fmt", ["bf16", "fp8"])
def test_noalloc_default_route_falls_back_when_stream_slots_do_not_fit(dev, fmt):
    """16 query heads per KV head: stream-K's partial slots for the whole
    persistent grid (2048 waves x 2 slots x 16 heads x 130 fp32 on 256 CUs,
    34 MB) exceed the 32 MiB scratch.  The library's choice (split_tokens
    0) then runs the workgroup route, which needs no workspace: within
    rounding of the workspace call and of the oracle, on two calls in a row
    (the second smaller).  Where the slots fit (fewer CUs), the two calls
    take the same route and agree bit for bit."""
    Hq, Hkv, bs = 32, 2, 64
    announce(f"noalloc decode, {fmt}, group 16, library route")
    g = torch.Generator().manual_seed(1616)
    N, mb = 96, 24
    kc, vc, ks, vs, mode = _pools(dev, fmt, N, bs, Hkv, g)
    tol = 2e-2 if fmt == "fp8" else 2e-3
    for B in (12, 3):
        ctx = torch.randint(1, mb * bs + 1, (B,), generator=g)
        ctx[0] = 0
        bt = torch.randint(0, N, (B, mb), generator=g, dtype=torch.int32)
        q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(dev)
        bt_d, ctx_d = bt.to(dev), ctx.to(dev)
        need = _lib.query("mkv_paged_decode_workspace_size", B, Hq, Hkv, mb, bs, D, A._dtype_code(kc, "k"), 0)
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        want = torch.full_like(q, float("nan"))
        got = torch.full_like(q, float("nan"))
        _call("mkv_paged_decode", want, q, kc, vc, ks, vs, mode, bt_d, ctx_d, Hq, Hkv, bs, 0, ws)
        _call("mkv_paged_decode_noalloc", got, q, kc, vc, ks, vs, mode, bt_d, ctx_d, Hq, Hkv, bs, 0)
        torch.cuda.synchronize()
        print(f"batch {B}: workspace route needs {need} bytes (scratch {_lib.NOALLOC_SCRATCH_BYTES})")
        if need <= _lib.NOALLOC_SCRATCH_BYTES:
            assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        else:
            assert_close_out(got.cpu(), want.cpu().double(), got.dtype, tol)
        ksf = float(ks) if ks is not None else None
        vsf = float(vs) if vs is not None else None
        ref = R.paged_decode_ref(q.cpu().double(), kc.cpu(), vc.cpu(), bt, ctx, 1.0 / math.sqrt(D), Hq, Hkv,
                                 ksf, vsf)
        assert_close_out(got.cpu(), ref, got.dtype, tol)
        assert torch.count_nonzero(got[0].float()) == 0
