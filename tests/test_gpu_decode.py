"""GPU parity of K2 (paged decode attention).

Tolerances (absolute, on the attention output): 2e-3 for fp32 / bf16 / fp16
KV and 2e-2 for FP8 KV, against the float64 oracle (small cases) or a float32
torch reference computed on the GPU (batch-256 sizes).
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import announce, assert_close_out, compact_pool
from mkv import attention as A
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 2e-3, torch.bfloat16: 2e-3, torch.float16: 2e-3, torch.float8_e4m3fn: 2e-2}


def _run(dev, q, k, v, bt, ctx, scale, Hq, Hkv, ks=None, vs=None, split_tokens=0):
    ksd = None if ks is None else torch.tensor([ks], dtype=torch.float32, device=dev)
    vsd = None if vs is None else torch.tensor([vs], dtype=torch.float32, device=dev)
    out = A._decode(q.to(dev), k.to(dev), v.to(dev), bt.to(dev), ctx.to(dev), scale, Hq, Hkv, 128,
                    ksd, vsd, split_tokens=split_tokens)
    return out.cpu()


def _oracle(q, k, v, bt, ctx, scale, Hq, Hkv, ks=None, vs=None):
    return R.paged_decode_ref(q.double(), k, v, bt, ctx, scale, Hq, Hkv, ks, vs)


@pytest.mark.parametrize("route", [0, -1])
def test_decode_small_fp32(dev, route):
    announce(f"decode: batch 4, 16/8 heads, fp32, bs 256, pool 64, route {route}")
    w = W.decode_small(seed=1)
    args = (w["q"], w["k_cache"], w["v_cache"], w["block_tables"], w["context_lens"], w["scale"],
            w["num_heads"], w["num_kv_heads"])
    got = _run(dev, *args, split_tokens=route)
    want = _oracle(*args)
    assert_close_out(got, want, got.dtype, 2e-3)


def test_decode_fp8_batch32_over_appended_pool(dev):
    announce("decode fp8: batch 32, 32/8 heads over the appended 1024-block pool")
    w = W.decode_fp8_b32(seed=2)
    N, bs, H = w["num_blocks"], w["block_size"], w["num_kv_heads"]
    kc = torch.zeros(N, bs, H, 128, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1, device=dev)
    vs = torch.ones(1, device=dev)
    # the per-tensor scales are calibrated on the 4096-token append (outliers
    # included), then every slot is filled and the append applied with them
    A.calibrate_fp8_per_tensor(w["key"].to(dev), w["value"].to(dev), ks, vs)
    A.store_kvcache_fp8(w["fill_key"].to(dev), w["fill_value"].to(dev), kc, vc, ks, vs,
                        w["fill_slots"].to(dev), bs, "fp8_per_tensor")
    A.store_kvcache_fp8(w["key"].to(dev), w["value"].to(dev), kc, vc, ks, vs,
                        w["slot_mapping"].to(dev), bs, "fp8_per_tensor")
    assert float(ks) == R.calibrate_scale_ref(w["key"])
    out = A.paged_attention_decode_quantized(
        w["q"].to(dev), kc, vc, ks, vs, w["block_tables"].to(dev), w["context_lens"].to(dev),
        w["scale"], w["num_heads"], H, 128, bs, "fp8_per_tensor").cpu()
    kcc, vcc = kc.cpu(), vc.cpu()
    want = _oracle(w["q"], kcc, vcc, w["block_tables"], w["context_lens"], w["scale"],
                   w["num_heads"], H, float(ks), float(vs))
    assert_close_out(out, want, out.dtype, 2e-2)
    # against the unquantised bf16 values (information: FP8 storage error)
    kb = torch.zeros(N * bs, H, 128, dtype=torch.bfloat16)
    vb = torch.zeros_like(kb)
    kb[w["fill_slots"]] = w["fill_key"]
    vb[w["fill_slots"]] = w["fill_value"]
    ok = w["slot_mapping"] >= 0
    kb[w["slot_mapping"][ok]] = w["key"][ok]
    vb[w["slot_mapping"][ok]] = w["value"][ok]
    exact = _oracle(w["q"], kb.view(N, bs, H, 128), vb.view(N, bs, H, 128), w["block_tables"],
                    w["context_lens"], w["scale"], w["num_heads"], H)
    err = (out.double() - exact).abs().max().item()
    print(f"fp8 decode vs unquantised bf16 cache: max abs err {err:.3e}")


def _case(seed, B, Hq, Hkv, bs, N, max_blocks, dtype, ctx=None):
    g = torch.Generator().manual_seed(seed)
    if ctx is None:
        ctx = torch.randint(1, max_blocks * bs + 1, (B,), generator=g)
    bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=max_blocks)
    q = torch.randn(B, Hq, 128, generator=g)
    k = torch.randn(N, bs, Hkv, 128, generator=g)
    v = torch.randn(N, bs, Hkv, 128, generator=g)
    ks = vs = None
    if dtype == torch.float8_e4m3fn:
        ks, vs = R.calibrate_scale_ref(k.to(torch.bfloat16)), R.calibrate_scale_ref(v.to(torch.bfloat16))
        k, v = R.fp8_quantize_ref(k.to(torch.bfloat16), ks), R.fp8_quantize_ref(v.to(torch.bfloat16), vs)
        q = q.to(torch.bfloat16)
    else:
        k, v = k.to(dtype), v.to(dtype)
        q = q.to(dtype if dtype != torch.float32 else torch.float32)
    return q, k, v, bt, ctx.to(torch.int64), ks, vs


WG = A.DECODE_WORKGROUP
SK = A.DECODE_STREAM


@pytest.mark.parametrize("route", [0, SK, WG])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float32])
@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
def test_decode_group_sizes(dev, dtype, group, route):
    announce(f"decode {dtype} group {group} route {route}")
    Hkv = 2
    q, k, v, bt, ctx, ks, vs = _case(100 + group, 6, Hkv * group, Hkv, 32, 64, 10, dtype)
    got = _run(dev, q, k, v, bt, ctx, 1 / math.sqrt(128), Hkv * group, Hkv, ks, vs, split_tokens=route)
    want = _oracle(q, k, v, bt, ctx, 1 / math.sqrt(128), Hkv * group, Hkv, ks, vs)
    assert_close_out(got, want, got.dtype, TOL[dtype])


@pytest.mark.parametrize("route", [0, WG])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.float32])
@pytest.mark.parametrize("bs", [16, 32, 128])
def test_decode_block_sizes_and_edges(dev, dtype, bs, route):
    announce(f"decode {dtype} bs {bs} with ctx 0/1/holes, route {route}")
    ctx = torch.tensor([0, 1, 2, bs - 1, bs, bs + 1, 5 * bs + 7, 31], dtype=torch.int64)
    q, k, v, bt, ctx, ks, vs = _case(7 * bs, 8, 8, 2, bs, 80, 6, dtype, ctx=ctx)
    bt[6, 2] = -1  # an absent block inside a context: its tokens are skipped
    got = _run(dev, q, k, v, bt, ctx, 0.09, 8, 2, ks, vs, split_tokens=route)
    want = _oracle(q, k, v, bt, ctx, 0.09, 8, 2, ks, vs)
    assert_close_out(got, want, got.dtype, TOL[dtype])
    assert torch.count_nonzero(got[0]) == 0  # context 0 -> zeros
    got32 = _run(dev, q, k, v, bt, ctx.to(torch.int32), 0.09, 8, 2, ks, vs, split_tokens=route)
    assert torch.equal(got, got32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_decode_split_count_independence(dev, dtype):
    announce(f"decode {dtype} split-K sizes")
    q, k, v, bt, ctx, ks, vs = _case(55, 4, 32, 8, 256, 64, 16, dtype)
    want = _oracle(q, k, v, bt, ctx, 0.088, 32, 8, ks, vs)
    outs = []
    for st in (32, 64, 256, 512, 4096):
        got = _run(dev, q, k, v, bt, ctx, 0.088, 32, 8, ks, vs, split_tokens=st)
        assert_close_out(got, want, got.dtype, TOL[dtype])
        outs.append(got)
    # deterministic run to run
    again = _run(dev, q, k, v, bt, ctx, 0.088, 32, 8, ks, vs, split_tokens=256)
    assert torch.equal(again, outs[2])


def test_decode_query_dtypes_over_bf16_and_fp8(dev):
    announce("decode: fp32 / fp16 queries over bf16 and fp8 caches")
    for dtype in (torch.bfloat16, torch.float8_e4m3fn):
        q, k, v, bt, ctx, ks, vs = _case(77, 3, 8, 2, 64, 40, 8, dtype)
        want = _oracle(q, k, v, bt, ctx, 0.1, 8, 2, ks, vs)
        for qd in (torch.float32, torch.float16):
            got = _run(dev, q.to(qd), k, v, bt, ctx, 0.1, 8, 2, ks, vs)
            # an fp32 query is rounded to the MFMA input type for a bf16 cache
            assert_close_out(got, want, got.dtype, TOL[dtype] + 2e-3)


def _torch_gpu_reference(q, kc, vc, bt, ctx, scale, Hq, Hkv, ks=None, vs=None):
    """float32 torch reference on the GPU, one sequence at a time."""
    bs = kc.shape[1]
    G = Hq // Hkv
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for b in range(q.shape[0]):
        L = int(ctx[b])
        nb = (L + bs - 1) // bs
        blocks = bt[b, :nb].long()
        kk = kc[blocks].float().reshape(-1, Hkv, 128)[:L]
        vv = vc[blocks].float().reshape(-1, Hkv, 128)[:L]
        if ks is not None:
            kk = kk * ks
            vv = vv * vs
        qq = q[b].float().reshape(Hkv, G, 128)
        s = torch.matmul(qq, kk.permute(1, 2, 0).contiguous()) * scale  # (Hkv, G, L)
        p = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(p, vv.permute(1, 0, 2).contiguous()).reshape(Hq, 128)
    return out


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_decode_batch256_full_size(dev, kv):
    announce(f"decode batch 256, 32/8 heads, ctx log-U[512, 8192], {kv} KV")
    m = W.decode_b256_metadata(seed=3)
    N, bs = m["num_blocks"], m["block_size"]
    dtype = torch.bfloat16 if kv == "bf16" else torch.float8_e4m3fn
    kc = torch.empty(N, bs, 8, 128, dtype=dtype, device=dev)
    vc = torch.empty_like(kc)
    ks = vs = None
    if kv == "fp8":
        ks, vs = 4.5 / 448, 4.4 / 448
    W.fill_pool_on_device(kc, 31, ks)
    W.fill_pool_on_device(vc, 32, vs)
    g = torch.Generator().manual_seed(33)
    q = torch.randn(256, 32, 128, generator=g).to(torch.bfloat16).to(dev)
    bt, ctx = m["block_tables"].to(dev), m["context_lens"].to(dev)
    ksd = None if ks is None else torch.tensor([ks], device=dev)
    vsd = None if vs is None else torch.tensor([vs], device=dev)
    got = A._decode(q, kc, vc, bt, ctx, 1 / math.sqrt(128), 32, 8, 128, ksd, vsd)
    want = _torch_gpu_reference(q, kc, vc, bt, ctx, 1 / math.sqrt(128), 32, 8, ks, vs)
    assert_close_out(got, want, got.dtype, 2e-2 if kv == "fp8" else 2e-3)
    # 8 sampled sequences (shortest, longest and spread) against the float64 oracle
    lens = m["context_lens"]
    idx = torch.tensor(sorted({int(lens.argmin()), int(lens.argmax())} | set(range(5, 256, 43))))[:8]
    kcs, vcs, bts = compact_pool(kc, vc, m["block_tables"][idx], lens[idx])
    ref = R.paged_decode_ref(q[idx].cpu().double(), kcs, vcs, bts, lens[idx], 1 / math.sqrt(128), 32, 8, ks, vs)
    assert_close_out(got[idx].cpu(), ref, got.dtype, 2e-2 if kv == "fp8" else 2e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.float16])
def test_decode_stream_k_vs_split_k_and_empty_rows(dev, dtype):
    """The default stream-K decomposition and explicit split-K agree; rows
    with context 0 anywhere in the batch come out as zeros."""
    announce(f"decode {dtype} stream-K vs split-K with empty rows")
    g = torch.Generator().manual_seed(71)
    B = 40
    ctx = torch.randint(1, 16 * 64 + 1, (B,), generator=g)
    ctx[[0, 7, 8, 39]] = 0
    q, k, v, bt, ctx, ks, vs = _case(72, B, 16, 4, 64, 400, 16, dtype, ctx=ctx)
    want = _oracle(q, k, v, bt, ctx, 0.11, 16, 4, ks, vs)
    sk = _run(dev, q, k, v, bt, ctx, 0.11, 16, 4, ks, vs, split_tokens=SK)
    sp = _run(dev, q, k, v, bt, ctx, 0.11, 16, 4, ks, vs, split_tokens=128)
    assert_close_out(sk, want, sk.dtype, TOL[dtype])
    assert_close_out(sp, want, sp.dtype, TOL[dtype])
    assert torch.count_nonzero(sk[[0, 7, 8, 39]]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("Hkv", [1, 3, 5, 12, 40])
def test_decode_stream_k_kv_head_counts(dev, dtype, Hkv):
    """The stream-K grid forms groups of Hkv waves (one KV head each) and
    leaves the waves past the last whole group idle: KV head counts that do
    not divide the grid, and large ones, give the oracle's result."""
    announce(f"decode {dtype} stream-K with {Hkv} KV heads")
    g = torch.Generator().manual_seed(93 + Hkv)
    ctx = torch.randint(1, 2049, (5,), generator=g)
    ctx[2] = 0
    q, k, v, bt, ctx, ks, vs = _case(94 + Hkv, 5, 2 * Hkv, Hkv, 128, 96, 16, dtype, ctx=ctx)
    want = _oracle(q, k, v, bt, ctx, 0.09, 2 * Hkv, Hkv, ks, vs)
    got = _run(dev, q, k, v, bt, ctx, 0.09, 2 * Hkv, Hkv, ks, vs, split_tokens=SK)
    assert_close_out(got, want, got.dtype, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_decode_stream_k_item_over_many_groups(dev, dtype):
    """One long sequence beside a short one, 8 KV heads: the long sequence's
    columns are cut over ~190 wave groups, so its items take the merge
    kernel's general path (more than 64 contributors); the short one's take
    the one-round-trip path."""
    announce(f"decode {dtype} stream-K, one item over ~190 wave groups")
    ctx = torch.tensor([6000, 300])
    q, k, v, bt, ctx, ks, vs = _case(91, 2, 32, 8, 256, 64, 24, dtype, ctx=ctx)
    want = _oracle(q, k, v, bt, ctx, 0.08, 32, 8, ks, vs)
    got = _run(dev, q, k, v, bt, ctx, 0.08, 32, 8, ks, vs, split_tokens=SK)
    assert_close_out(got, want, got.dtype, TOL[dtype])


@pytest.mark.parametrize("B,dtype", [(2048, torch.float8_e4m3fn), (4096, torch.bfloat16),
                                     (8192, torch.float8_e4m3fn)])
def test_decode_stream_k_large_batches(dev, B, dtype):
    """Batches of 2048-8192 take the stream-K route with the larger
    per-sequence prefix in LDS (above 2047 sequences the launch is sized for
    up to 8192); short contexts with some empty rows, checked against the
    oracle on every 61st row, and the empty rows exactly zero."""
    announce(f"decode {dtype} stream-K batch {B}")
    g = torch.Generator().manual_seed(75 + B)
    ctx = torch.randint(0, 70, (B,), generator=g)
    ctx[::37] = 0
    q, k, v, bt, ctx, ks, vs = _case(76 + B, B, 8, 2, 16, 3 * B, 5, dtype, ctx=ctx)
    got = _run(dev, q, k, v, bt, ctx, 0.1, 8, 2, ks, vs, split_tokens=SK)
    idx = torch.arange(0, B, 61)
    want = _oracle(q[idx], k, v, bt[idx], ctx[idx], 0.1, 8, 2, ks, vs)
    assert_close_out(got[idx], want, got.dtype, TOL[dtype])
    assert torch.count_nonzero(got[ctx == 0].float()) == 0


def test_decode_large_batch_uses_split_k_fallback(dev):
    announce("decode batch 9000 (beyond the stream-K batch cap)")
    g = torch.Generator().manual_seed(73)
    B = 9000
    ctx = torch.randint(0, 40, (B,), generator=g)
    q, k, v, bt, ctx, ks, vs = _case(74, B, 8, 2, 16, 4 * B, 3, torch.bfloat16, ctx=ctx)
    got = _run(dev, q, k, v, bt, ctx, 0.1, 8, 2)
    idx = torch.arange(0, B, 97)
    want = _oracle(q[idx], k, v, bt[idx], ctx[idx], 0.1, 8, 2)
    assert_close_out(got[idx], want, got.dtype, 2e-3)


@pytest.mark.parametrize("kv,qdt", [(torch.bfloat16, torch.float32), (torch.bfloat16, torch.float16),
                                    (torch.float16, torch.float32), (torch.float16, torch.bfloat16),
                                    (torch.float8_e4m3fn, torch.float32)])
@pytest.mark.parametrize("group", [4, 8])
def test_decode_q_dtype_differs_from_cache(dev, kv, qdt, group):
    """q in another dtype than the cache (the reference computes in fp32): a
    bf16 cache with an fp32 / fp16 q takes the split (hi + lo) q path."""
    announce(f"decode kv {kv} q {qdt} group {group}")
    Hkv = 4
    q, k, v, bt, ctx, ks, vs = _case(81, 12, group * Hkv, Hkv, 16, 160, 12, kv)
    q = torch.randn(q.shape, generator=torch.Generator().manual_seed(82)).to(qdt)
    want = _oracle(q, k, v, bt, ctx, 0.09, group * Hkv, Hkv, ks, vs)
    for st in (0, SK, 64, WG):
        got = _run(dev, q, k, v, bt, ctx, 0.09, group * Hkv, Hkv, ks, vs, split_tokens=st)
        assert got.dtype == qdt
        assert_close_out(got, want, got.dtype, TOL[kv])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.float32])
def test_decode_workgroup_route_small_batches(dev, dtype):
    """The workgroup route (one workgroup per sequence and KV head, waves
    merged in LDS) on the shapes it serves: 32 sequences of up to 4096 tokens
    (8 waves per workgroup) and 60 of 300-800 (4 waves), with empty rows, each
    against the oracle and against stream-K."""
    for B, Hq, lo, hi in ((32, 32, 256, 4096), (60, 16, 300, 800)):
        announce(f"decode {dtype} workgroup route, batch {B}, contexts [{lo}, {hi}]")
        g = torch.Generator().manual_seed(500 + B)
        ctx = torch.randint(lo, hi + 1, (B,), generator=g)
        ctx[[1, B - 1]] = 0
        mb = (hi + 255) // 256
        q, k, v, bt, ctx, ks, vs = _case(501 + B, B, Hq, 8, 256, B * mb + 8, mb, dtype, ctx=ctx)
        want = _oracle(q, k, v, bt, ctx, 0.088, Hq, 8, ks, vs)
        got = _run(dev, q, k, v, bt, ctx, 0.088, Hq, 8, ks, vs, split_tokens=WG)
        assert_close_out(got, want, got.dtype, TOL[dtype])
        assert torch.count_nonzero(got[[1, B - 1]].float()) == 0
        sk = _run(dev, q, k, v, bt, ctx, 0.088, Hq, 8, ks, vs, split_tokens=SK)
        assert_close_out(got, sk.double(), got.dtype, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.float32])
def test_decode_long_block_spans_on_every_route(dev, dtype):
    """Block-table entries are looked up tile by tile on every route, so a
    wave's range may span any number of blocks: one sequence of up to 9600
    tokens in 16-token blocks (600 blocks) through the workgroup route (one
    wave spans ~75 blocks), split-K with 4096-token splits (256 blocks per
    split), stream-K and the library's choice, each against the oracle."""
    announce(f"decode {dtype} long block spans (600 blocks of 16) on every route")
    g = torch.Generator().manual_seed(10)
    ctx = torch.tensor([9600, 5000, 17])
    q, k, v, bt, ctx, ks, vs = _case(10, 3, 8, 2, 16, 1300, 600, dtype, ctx=ctx)
    bt[0, 300] = -1  # an absent block deep inside the long context
    want = _oracle(q, k, v, bt, ctx, 0.1, 8, 2, ks, vs)
    for st in (WG, 4096, SK, 0):
        got = _run(dev, q, k, v, bt, ctx, 0.1, 8, 2, ks, vs, split_tokens=st)
        assert_close_out(got, want, got.dtype, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.bfloat16])
def test_decode_default_route_block16_long_contexts(dev, dtype):
    """60 sequences x 8 KV heads with 16-token blocks and contexts of
    4000-5000 tokens (320-block tables) through the library's choice
    (stream-K: a workgroup wave would take up to 1280 tokens) and through
    the workgroup route, whose waves then span ~80 blocks each (the route
    refused such tables before its block-table entries were looked up tile
    by tile).  Checked on every 7th row."""
    announce(f"decode {dtype} default route, batch 60, block 16, contexts 4000-5000")
    from mkv import _lib
    g = torch.Generator().manual_seed(4000)
    B, mb, N = 60, 320, 400
    # one 400-block pool; the tables share its blocks between sequences (reads only)
    q, k, v, _, _, ks, vs = _case(4001, B, 16, 8, 16, N, 8, dtype)
    ctx = torch.randint(4000, 5001, (B,), generator=g)
    bt = torch.randint(0, N, (B, mb), generator=g, dtype=torch.int32)
    dt = {torch.float8_e4m3fn: _lib.DTYPE_FP8E4M3, torch.bfloat16: _lib.DTYPE_BF16}[dtype]
    route = _lib.query("mkv_paged_decode_route", B, 16, 8, mb, 16, 128, dt, 0, 0)
    assert route == _lib.ROUTE_STREAM
    idx = torch.arange(0, B, 7)
    want = _oracle(q[idx], k, v, bt[idx], ctx[idx], 0.088, 16, 8, ks, vs)
    for st in (0, WG):
        got = _run(dev, q, k, v, bt, ctx, 0.088, 16, 8, ks, vs, split_tokens=st)
        assert_close_out(got[idx], want, got.dtype, TOL[dtype])
