"""GPU parity at head_dim 64, the Llama-3.2-1B attention shape (32 query /
8 KV heads, head_dim 64; reference main_llama32.py:29-34, models/llama.py:31).
Every reference kernel takes head_dim as a parameter (attention.py:528, :717,
:343, :966, :1137); here decode and prefill read the KV heads of a
head_dim-64 cache in pairs (two adjacent 64-element head segments as one
128-element one).

Decode: every route (library choice, stream-K, split-K, workgroup) and every
KV format (fp32, bf16, fp16, FP8 per tensor, FP8 / INT8 per token and head)
against the float64 oracle on the cache's own values (dequantised codes for
the quantised formats), with group sizes 1-8, empty rows and absent blocks.
Chunked prefill over the paged cache and full prefill over fresh K/V,
likewise.  The Attention layer runs full prefill -> chunked prefill ->
decode at head_dim 64.

Tolerances (absolute, before the output's own rounding): 2e-3 for fp32 /
bf16 / fp16 KV and for decode over per-token-head codes (the oracle reads
the same codes and scales), 2e-2 for FP8 per tensor and for prefill over
per-token-head codes (as at head_dim 128: their prefill takes P times the V
scale as one fp16 MFMA operand, 11 bits).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import announce, assert_close_out
import mkv
from mkv import attention as A
from mkv import context as C
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu
D = 64
FORMATS = ["f32", "bf16", "f16", "fp8", "fp8_token", "int8_token"]
TOL = {"f32": 2e-3, "bf16": 2e-3, "f16": 2e-3, "fp8": 2e-2, "fp8_token": 2e-3, "int8_token": 2e-3}
PREFILL_TOL = {**TOL, "fp8_token": 2e-2, "int8_token": 2e-2}
ROUTES = [0, A.DECODE_STREAM, 64, A.DECODE_WORKGROUP]
MODE = {"fp8": "fp8_per_tensor", "fp8_token": "fp8_per_token_head", "int8_token": "int8_per_token_head"}


def _pools(dev, fmt, N, bs, Hkv, g):
    """Device pools of format fmt filled with seeded values, and what the
    oracle reads: (kc, vc, ks, vs) on the device and (kc, vc, ks, vs) on the
    host (scales: None, a float, or per-token-head tensors)."""
    x = torch.randn(N * bs, Hkv, D, generator=g)
    y = torch.randn(N * bs, Hkv, D, generator=g)
    if fmt in ("f32", "bf16", "f16"):
        dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[fmt]
        kc, vc = x.to(dt).view(N, bs, Hkv, D), y.to(dt).view(N, bs, Hkv, D)
        return (kc.to(dev), vc.to(dev), None, None), (kc, vc, None, None)
    if fmt == "fp8":
        xb, yb = x.to(torch.bfloat16), y.to(torch.bfloat16)
        ks, vs = R.calibrate_scale_ref(xb), R.calibrate_scale_ref(yb)
        kc = R.fp8_quantize_ref(xb, ks).view(N, bs, Hkv, D)
        vc = R.fp8_quantize_ref(yb, vs).view(N, bs, Hkv, D)
        return ((kc.to(dev), vc.to(dev), torch.tensor([ks], device=dev), torch.tensor([vs], device=dev)),
                (kc, vc, ks, vs))
    # per token and head: the append writes codes and scales on the device
    cdt = torch.float8_e4m3fn if fmt == "fp8_token" else torch.int8
    kc = torch.zeros(N, bs, Hkv, D, dtype=cdt, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(N, bs, Hkv, device=dev)
    vs = torch.zeros_like(ks)
    slots = torch.arange(N * bs, device=dev)
    xd, yd = x.to(torch.bfloat16).to(dev), y.to(torch.bfloat16).to(dev)
    if fmt == "int8_token":
        A.store_kvcache_int8(xd, yd, kc, vc, ks, vs, slots, bs)
    else:
        A.store_kvcache_fp8(xd, yd, kc, vc, ks, vs, slots, bs, "fp8_per_token_head")
    return (kc, vc, ks, vs), (kc.cpu(), vc.cpu(), ks.cpu(), vs.cpu())


def _decode(dev, fmt, q, dpools, bt, ctx, scale, Hq, Hkv, route):
    kc, vc, ks, vs = dpools
    if fmt in ("f32", "bf16", "f16"):
        return A.paged_attention_decode(q.to(dev), kc, vc, bt.to(dev), ctx.to(dev), scale, Hq, Hkv, D,
                                        kc.shape[1], split_tokens=route).cpu()
    return A.paged_attention_decode_quantized(q.to(dev), kc, vc, ks, vs, bt.to(dev), ctx.to(dev), scale,
                                              Hq, Hkv, D, kc.shape[1], MODE[fmt], split_tokens=route).cpu()


def _qdtype(fmt):
    return torch.float32 if fmt == "f32" else (torch.float16 if fmt == "f16" else torch.bfloat16)


@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("group", [1, 2, 4, 8])
@pytest.mark.parametrize("fmt", FORMATS)
def test_decode_head_dim64_groups_routes_formats(dev, fmt, group, route):
    announce(f"decode head_dim 64: {fmt}, group {group}, route {route}")
    g = torch.Generator().manual_seed(6400 + 10 * group + FORMATS.index(fmt))
    Hkv, bs, N, mb = 4, 32, 96, 10
    B = 9
    ctx = torch.randint(1, mb * bs + 1, (B,), generator=g)
    ctx[[0, 5]] = torch.tensor([0, 1])
    ctx[3] = bs  # exactly one block
    bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=mb)
    bt[4, 1] = -1  # an absent block inside a context: its tokens are skipped
    dpools, hpools = _pools(dev, fmt, N, bs, Hkv, g)
    Hq = Hkv * group
    q = torch.randn(B, Hq, D, generator=g).to(_qdtype(fmt))
    got = _decode(dev, fmt, q, dpools, bt, ctx, 0.125, Hq, Hkv, route)
    want = R.paged_decode_ref(q.double(), hpools[0], hpools[1], bt, ctx, 0.125, Hq, Hkv, hpools[2], hpools[3])
    assert got.shape == (B, Hq, D) and got.dtype == q.dtype
    assert_close_out(got, want, got.dtype, TOL[fmt])
    assert torch.count_nonzero(got[0].float()) == 0  # context 0 -> zeros


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "fp8_token"])
def test_decode_head_dim64_llama_shape(dev, fmt):
    """Llama-3.2-1B decode: 32 query / 8 KV heads, block 256, a batch of 48
    sequences of up to 3000 tokens; the library's schedule and each explicit
    one against the oracle."""
    announce(f"decode head_dim 64, Llama-3.2-1B shape, {fmt}")
    g = torch.Generator().manual_seed(3201)
    Hq, Hkv, bs, B = 32, 8, 256, 48
    ctx = torch.randint(1, 3001, (B,), generator=g)
    mb = 12
    N = int(((ctx + bs - 1) // bs).sum()) + 4
    bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=mb)
    dpools, hpools = _pools(dev, fmt, N, bs, Hkv, g)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    sm = 1.0 / math.sqrt(D)
    idx = torch.arange(0, B, 5)
    want = R.paged_decode_ref(q[idx].double(), hpools[0], hpools[1], bt[idx], ctx[idx], sm, Hq, Hkv,
                              hpools[2], hpools[3])
    for route in ROUTES:
        got = _decode(dev, fmt, q, dpools, bt, ctx, sm, Hq, Hkv, route)
        assert_close_out(got[idx], want, got.dtype, TOL[fmt])


def test_decode_head_dim64_pairs_keep_heads_apart(dev):
    """Head pairing must not mix the two KV heads of a pair: with KV head 2v
    all zeros and KV head 2v + 1 large, the query heads of 2v see uniform
    attention over zero values (output 0) and those of 2v + 1 their own
    values; the same with the roles swapped."""
    announce("decode head_dim 64: paired heads kept apart")
    g = torch.Generator().manual_seed(77)
    Hkv, group, bs, N, B = 2, 4, 16, 16, 2
    for zero_head in (0, 1):
        k = torch.randn(N, bs, Hkv, D, generator=g) * 5
        v = torch.randn(N, bs, Hkv, D, generator=g) * 5
        k[:, :, zero_head] = 0
        v[:, :, zero_head] = 0
        ctx = torch.tensor([37, 100])
        bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=7)
        q = torch.randn(B, Hkv * group, D, generator=g)
        for route in ROUTES:
            got = A.paged_attention_decode(q.to(dev), k.to(dev), v.to(dev), bt.to(dev), ctx.to(dev), 0.2,
                                           Hkv * group, Hkv, D, bs, split_tokens=route).cpu()
            zq = slice(zero_head * group, (zero_head + 1) * group)
            assert torch.count_nonzero(got[:, zq]) == 0
            want = R.paged_decode_ref(q.double(), k, v, bt, ctx, 0.2, Hkv * group, Hkv)
            assert_close_out(got, want, torch.float32, 2e-3)


def test_decode_head_dim64_rejects_unpairable_shapes(dev):
    from mkv._lib import MkvError
    q = torch.zeros(2, 6, D, device=dev)
    kc = torch.zeros(4, 16, 3, D, device=dev)  # 3 KV heads do not pair up
    bt = torch.zeros(2, 1, dtype=torch.int32, device=dev)
    ctx = torch.ones(2, dtype=torch.int64, device=dev)
    with pytest.raises(MkvError):
        A.paged_attention_decode(q, kc, kc, bt, ctx, 0.1, 6, 3, D, 16)


def _prefill_case(seed, fmt, Hq, Hkv, bs, prior, qlen, dev, holes=()):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.tensor([p + n for p, n in zip(prior, qlen)], dtype=torch.int64)
    N = sum((int(c) + bs - 1) // bs for c in ctx) + 3
    bt = W.fragmented_block_tables(ctx, bs, N, g)
    for s, j in holes:
        bt[s, j] = -1
    cu = torch.zeros(len(qlen) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(qlen), 0).to(torch.int32)
    pos = torch.tensor([p + j for p, n in zip(prior, qlen) for j in range(n)], dtype=torch.int64)
    dpools, hpools = _pools(dev, fmt, N, bs, Hkv, g)
    q = torch.randn(int(cu[-1]), Hq, D, generator=g).to(_qdtype(fmt))
    return q, dpools, hpools, bt, ctx, cu, pos


@pytest.mark.parametrize("fmt", ["fp8_token", "int8_token"])
@pytest.mark.parametrize("qdt", [torch.bfloat16, torch.float32])
def test_prefill_head_dim64_large_v_scales(dev, fmt, qdt):
    """Paired KV heads with V scales 2^20 times the usual: the prefill's
    running-max lift takes the larger of the two heads' largest V scales of
    a tile.  Divided back by 2^20 (exact), the output meets the oracle on
    the unscaled caches within the prefill bound."""
    announce(f"chunked prefill head_dim 64: {fmt}, q {qdt}, V scales x 2^20")
    Hkv, group = 4, 4
    Hq = Hkv * group
    prior, qlen = [0, 300, 70], [130, 64, 150]
    q, dp, hp, bt, ctx, cu, pos = _prefill_case(6400, fmt, Hq, Hkv, 16, prior, qlen, dev)
    q = q.to(qdt)
    S = float(2 ** 20)
    sc = 1 / math.sqrt(D)
    got = A.paged_attention_prefill_triton(
        q.to(dev), dp[0], dp[1], bt.to(dev), ctx.to(dev), cu.to(dev), pos.to(dev), sc, Hq, Hkv, D, 16,
        k_scale=dp[2], v_scale=dp[3] * S, kv_cache_dtype=MODE[fmt]).cpu()
    assert torch.isfinite(got.float()).all()
    want = R.paged_prefill_ref(q.double(), hp[0], hp[1], bt, ctx, cu, pos, sc, Hq, Hkv, hp[2], hp[3])
    assert_close_out(got / S, want, got.dtype, PREFILL_TOL[fmt])


@pytest.mark.parametrize("group", [1, 2, 4, 8])
@pytest.mark.parametrize("fmt", FORMATS)
def test_prefill_head_dim64_groups_formats(dev, fmt, group):
    announce(f"chunked prefill head_dim 64: {fmt}, group {group}")
    Hkv = 2
    Hq = Hkv * group
    prior, qlen = [0, 37, 130, 5, 0], [70, 33, 1, 200, 1]
    q, dp, hp, bt, ctx, cu, pos = _prefill_case(640 + group, fmt, Hq, Hkv, 32, prior, qlen, dev,
                                                holes=[(3, 2)])
    sc = 1 / math.sqrt(D)
    mode = MODE.get(fmt, "auto")
    got = A.paged_attention_prefill_triton(
        q.to(dev), dp[0], dp[1], bt.to(dev), ctx.to(dev), cu.to(dev), pos.to(dev), sc, Hq, Hkv, D, 32,
        k_scale=dp[2], v_scale=dp[3], kv_cache_dtype=mode).cpu()
    want = R.paged_prefill_ref(q.double(), hp[0], hp[1], bt, ctx, cu, pos, sc, Hq, Hkv, hp[2], hp[3])
    assert got.shape == q.shape and got.dtype == q.dtype
    assert_close_out(got, want, got.dtype, PREFILL_TOL[fmt])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("group", [1, 4, 8])
def test_flash_prefill_head_dim64(dev, dtype, group):
    announce(f"full prefill head_dim 64: {dtype}, group {group}")
    g = torch.Generator().manual_seed(650 + group)
    lens = [1, 77, 130, 5, 300, 0, 64]
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    T, Hkv = int(cu[-1]), 4
    q = torch.randn(T, Hkv * group, D, generator=g).to(dtype)
    k = torch.randn(T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(T, Hkv, D, generator=g).to(dtype)
    got = mkv.flash_attention_prefill(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), 0.11,
                                      Hkv * group, Hkv, D).cpu()
    want = R.flash_prefill_ref(q.double(), k.double(), v.double(), cu, 0.11, Hkv * group, Hkv)
    assert_close_out(got, want, got.dtype, 2e-3)


@pytest.mark.parametrize("mode", ["auto", "fp8_per_tensor", "fp8_per_token_head"])
def test_attention_layer_head_dim64_full_then_chunked_then_decode(dev, mode):
    """The Llama-3.2-1B attention shape through Attention.forward: three
    sequences go through a full prefill, a chunked prefill of further tokens
    over the cache, then decode steps; every step's output and the cache are
    checked against the oracle on the oracle's own cache."""
    announce(f"Attention layer head_dim 64 (32/8 heads), {mode}: full -> chunked -> decode")
    g = torch.Generator().manual_seed(3202)
    Hq, Hkv, bs, N = 32, 8, 16, 64
    sm = 1.0 / math.sqrt(D)
    layer = A.Attention(Hq, D, scale=1.0, num_kv_heads=Hkv, block_size=bs)
    cdt = torch.bfloat16 if mode == "auto" else torch.float8_e4m3fn
    layer.k_cache = torch.zeros(N, bs, Hkv, D, dtype=cdt, device=dev)
    layer.v_cache = torch.zeros_like(layer.k_cache)
    layer.kv_cache_dtype = mode
    if mode == "fp8_per_tensor":
        layer.k_scale = torch.ones(1, device=dev)
        layer.v_scale = torch.ones(1, device=dev)
    elif mode == "fp8_per_token_head":
        layer.k_scale = torch.zeros(N, bs, Hkv, device=dev)
        layer.v_scale = torch.zeros(N, bs, Hkv, device=dev)
    perm = torch.randperm(N, generator=g)
    tables = [perm[i * 20:(i + 1) * 20].tolist() for i in range(3)]  # disjoint blocks
    bt = torch.tensor(tables, dtype=torch.int32)
    lens = [0, 0, 0]
    tol = TOL["fp8"] if mode == "fp8_per_tensor" else 2e-3
    tol_prefill = TOL["fp8"] if mode != "auto" else 2e-3

    def step(new_tokens, full):
        seqs = [s for s in range(3) if new_tokens[s] > 0]
        qlen = [new_tokens[s] for s in seqs]
        pos = torch.tensor([lens[s] + j for s in seqs for j in range(new_tokens[s])], dtype=torch.int64)
        slots = torch.tensor([tables[s][(lens[s] + j) // bs] * bs + (lens[s] + j) % bs
                              for s in seqs for j in range(new_tokens[s])], dtype=torch.int64)
        for s in seqs:
            lens[s] += new_tokens[s]
        ctx = torch.tensor([lens[s] for s in seqs], dtype=torch.int64)
        cu = torch.zeros(len(seqs) + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(torch.tensor(qlen), 0).to(torch.int32)
        T = int(cu[-1])
        q = torch.randn(T, Hq, D, generator=g).to(torch.bfloat16)
        k = torch.randn(T, Hkv, D, generator=g).to(torch.bfloat16)
        v = torch.randn(T, Hkv, D, generator=g).to(torch.bfloat16)
        btd = bt[seqs]
        decode = all(n == 1 for n in qlen) and not full
        if decode:
            C.set_context(False, slot_mapping=slots.to(dev), context_lens=ctx.to(dev),
                          block_tables=btd.to(dev))
        else:
            C.set_context(True, cu_seqlens_q=cu.to(dev), max_seqlen_q=max(qlen),
                          slot_mapping=slots.to(dev), context_lens=ctx.to(dev),
                          block_tables=btd.to(dev), positions=pos.to(dev), is_full_prefill=full)
        try:
            out = layer(q.to(dev), k.to(dev), v.to(dev)).cpu()
        finally:
            C.reset_context()
        # the oracle reads the layer's own cache (codes and scales as written)
        kc, vc = layer.k_cache.cpu(), layer.v_cache.cpu()
        ks = vs = None
        if mode == "fp8_per_tensor":
            ks, vs = float(layer.k_scale), float(layer.v_scale)
        elif mode == "fp8_per_token_head":
            ks, vs = layer.k_scale.cpu(), layer.v_scale.cpu()
        # the step's rows landed in the cache exactly as the append's oracle writes them
        if mode == "auto":
            assert torch.equal(kc.view(-1, Hkv, D)[slots], k) and torch.equal(vc.view(-1, Hkv, D)[slots], v)
        if decode:
            want = R.paged_decode_ref(q.double(), kc, vc, btd, ctx, sm, Hq, Hkv, ks, vs)
        elif full:
            want = R.flash_prefill_ref(q.double(), k.double(), v.double(), cu, sm, Hq, Hkv)
        else:
            want = R.paged_prefill_ref(q.double(), kc, vc, btd, ctx, cu, pos, sm, Hq, Hkv, ks, vs)
        assert_close_out(out.reshape(T, Hq, D), want, torch.bfloat16, tol if decode or full else tol_prefill)

    step([37, 100, 5], full=True)
    step([20, 1, 64], full=False)
    step([1, 1, 1], full=False)
    step([1, 0, 1], full=False)
