"""GPU parity of K3 (chunked-prefill attention over the paged cache and full
prefill over contiguous K/V), and of the Attention layer's dispatch.

Tolerances (absolute): 2e-3 for bf16 / fp16 KV, 2e-2 for FP8 KV, against the
float64 oracle (small cases) or a float32 torch reference on the GPU (the
512-row chunk workload).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import announce, assert_close_out, compact_pool
import mkv
from mkv import attention as A
from mkv import context as C
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 2e-3, torch.bfloat16: 2e-3, torch.float16: 2e-3, torch.float8_e4m3fn: 2e-2}


def _make(seed, prior, qlen, Hq, Hkv, bs, dtype, N=None, holes=()):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.tensor([p + n for p, n in zip(prior, qlen)], dtype=torch.int64)
    need = sum((int(c) + bs - 1) // bs for c in ctx)
    N = N or need + 3
    bt = W.fragmented_block_tables(ctx, bs, N, g)
    for s, j in holes:
        bt[s, j] = -1
    cu = torch.zeros(len(qlen) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(qlen), 0).to(torch.int32)
    pos = torch.tensor([p + j for p, n in zip(prior, qlen) for j in range(n)], dtype=torch.int64)
    q = torch.randn(int(cu[-1]), Hq, 128, generator=g)
    k = torch.randn(N, bs, Hkv, 128, generator=g)
    v = torch.randn(N, bs, Hkv, 128, generator=g)
    ks = vs = None
    if dtype == torch.float8_e4m3fn:
        kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)
        ks, vs = R.calibrate_scale_ref(kb), R.calibrate_scale_ref(vb)
        k, v = R.fp8_quantize_ref(kb, ks), R.fp8_quantize_ref(vb, vs)
        q = q.to(torch.bfloat16)
    else:
        k, v, q = k.to(dtype), v.to(dtype), q.to(dtype)
    return q, k, v, bt, ctx, cu, pos, ks, vs


def _gpu(dev, q, k, v, bt, ctx, cu, pos, scale, Hq, Hkv, ks, vs):
    fp8 = k.dtype == torch.float8_e4m3fn
    ksd = torch.tensor([ks], device=dev) if fp8 else None
    vsd = torch.tensor([vs], device=dev) if fp8 else None
    out = A.paged_attention_prefill_triton(
        q.to(dev), k.to(dev), v.to(dev), bt.to(dev), ctx.to(dev), cu.to(dev), pos.to(dev), scale,
        Hq, Hkv, 128, k.shape[1], k_scale=ksd, v_scale=vsd,
        kv_cache_dtype="fp8_per_tensor" if fp8 else "auto")
    return out.cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn])
@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
def test_prefill_small_groups(dev, dtype, group):
    announce(f"prefill {dtype} group {group}")
    Hkv = 2
    prior = [0, 37, 130, 5, 0]
    qlen = [70, 33, 1, 200, 1]
    q, k, v, bt, ctx, cu, pos, ks, vs = _make(group, prior, qlen, Hkv * group, Hkv, 32, dtype)
    sc = 1 / math.sqrt(128)
    got = _gpu(dev, q, k, v, bt, ctx, cu, pos, sc, Hkv * group, Hkv, ks, vs)
    want = R.paged_prefill_ref(q.double(), k, v, bt, ctx, cu, pos, sc, Hkv * group, Hkv, ks, vs)
    assert_close_out(got, want, got.dtype, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn])
@pytest.mark.parametrize("scale", [0.0, -0.09])
def test_prefill_zero_and_negative_scale(dev, dtype, scale):
    """The kernel keeps raw scores and scales them once: a zero scale (every
    visible key weighs the same) and a negative one (the softmax of the
    negated scores) must still match the oracle."""
    announce(f"prefill {dtype} scale {scale}")
    prior = [0, 40, 3]
    qlen = [90, 24, 70]
    q, k, v, bt, ctx, cu, pos, ks, vs = _make(7, prior, qlen, 8, 2, 16, dtype)
    got = _gpu(dev, q, k, v, bt, ctx, cu, pos, scale, 8, 2, ks, vs)
    want = R.paged_prefill_ref(q.double(), k, v, bt, ctx, cu, pos, scale, 8, 2, ks, vs)
    assert_close_out(got, want, got.dtype, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("nseq,Hkv", [(40, 2), (40, 8), (64, 2), (65, 8), (100, 2), (193, 8), (256, 2),
                                      (300, 2)])
def test_prefill_visit_order_many_tied_and_empty_sequences(dev, nseq, Hkv, dtype):
    """The tile list visits sequences longest first (ranked on the device for
    up to 256 sequences, one to four waves of them, in batch order beyond)
    and each sequence's tiles last first; ties, empty sequences and both grid
    mappings (KV heads a multiple of 8 or not) must leave every row's result
    unchanged."""
    announce(f"prefill visit order: {nseq} sequences, {Hkv} kv heads, {dtype}")
    g = torch.Generator().manual_seed(500 + nseq + Hkv)
    prior = [int(x) for x in torch.tensor([0, 16, 50, 97])[torch.randint(0, 4, (nseq,), generator=g)]]
    qlen = [int(x) for x in torch.randint(0, 7, (nseq,), generator=g)]
    qlen[3] = 70  # one sequence of several tiles
    q, k, v, bt, ctx, cu, pos, ks, vs = _make(nseq, prior, qlen, 2 * Hkv, Hkv, 16, dtype)
    got = _gpu(dev, q, k, v, bt, ctx, cu, pos, 0.09, 2 * Hkv, Hkv, ks, vs)
    want = R.paged_prefill_ref(q.double(), k, v, bt, ctx, cu, pos, 0.09, 2 * Hkv, Hkv, ks, vs)
    assert_close_out(got, want, got.dtype, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("bs", [16, 64, 256])
def test_prefill_block_sizes_holes_and_context_caps(dev, dtype, bs):
    announce(f"prefill {dtype} bs {bs} holes")
    prior = [3, 0, 300]
    qlen = [129, 64, 17]
    q, k, v, bt, ctx, cu, pos, ks, vs = _make(bs, prior, qlen, 8, 2, bs, dtype, holes=[(2, 0)])
    ctx2 = ctx.clone()
    ctx2[0] = 50  # context shorter than some positions: visible = min(ctx, pos + 1)
    got = _gpu(dev, q, k, v, bt, ctx2, cu, pos, 0.1, 8, 2, ks, vs)
    want = R.paged_prefill_ref(q.double(), k, v, bt, ctx2, cu, pos, 0.1, 8, 2, ks, vs)
    assert_close_out(got, want, got.dtype, TOL[dtype])


def _torch_prefill_gpu(q, kc, vc, bt, ctx, cu, pos, scale, Hq, Hkv, ks=None, vs=None):
    """float32 torch reference on the GPU, one sequence at a time."""
    bs = kc.shape[1]
    G = Hq // Hkv
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    cuh = cu.tolist()
    for s in range(len(cuh) - 1):
        a, b = cuh[s], cuh[s + 1]
        L = int(ctx[s])
        nb = (L + bs - 1) // bs
        blocks = bt[s, :nb].long()
        kk = kc[blocks].float().reshape(-1, Hkv, 128)[:L]
        vv = vc[blocks].float().reshape(-1, Hkv, 128)[:L]
        if ks is not None:
            kk, vv = kk * ks, vv * vs
        qq = q[a:b].float().reshape(b - a, Hkv, G, 128).permute(1, 0, 2, 3).reshape(Hkv, (b - a) * G, 128)
        sc = torch.matmul(qq.contiguous(), kk.permute(1, 2, 0).contiguous()) * scale  # (Hkv, rows*G, L)
        vis = torch.minimum(pos[a:b] + 1, torch.full_like(pos[a:b], L)).repeat_interleave(G)
        mask = torch.arange(L, device=q.device)[None, :] < vis[:, None]
        sc = sc.masked_fill(~mask[None], float("-inf"))
        o = torch.matmul(torch.softmax(sc, -1), vv.permute(1, 0, 2).contiguous())
        out[a:b] = o.reshape(Hkv, b - a, G, 128).permute(1, 0, 2, 3).reshape(b - a, Hq, 128)
    return out


@pytest.mark.parametrize("kv", ["bf16", "fp8", "f32"])
def test_prefill_chunk_workload_full_size(dev, kv):
    announce(f"prefill 8 x 512-row chunks, prior U[0,4096], 32/8 heads, {kv} KV")
    m = W.prefill_mixed(seed=4, num_decode=0)
    N, bs = m["num_blocks"], m["block_size"]
    dtype = {"bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn, "f32": torch.float32}[kv]
    kc = torch.empty(N, bs, 8, 128, dtype=dtype, device=dev)
    vc = torch.empty_like(kc)
    ks = W.fill_pool_on_device(kc, 41)
    vs = W.fill_pool_on_device(vc, 42)
    g = torch.Generator().manual_seed(43)
    T = int(m["cu_seqlens_q"][-1])
    q = torch.randn(T, 32, 128, generator=g).to(torch.bfloat16).to(dev)
    args = (m["block_tables"].to(dev), m["context_lens"].to(dev), m["cu_seqlens_q"].to(dev),
            m["positions"].to(dev))
    sc = 1 / math.sqrt(128)
    ksd = torch.tensor([ks], device=dev) if ks else None
    vsd = torch.tensor([vs], device=dev) if vs else None
    got = A.paged_attention_prefill_triton(q, kc, vc, *args, sc, 32, 8, 128, bs, k_scale=ksd,
                                           v_scale=vsd, kv_cache_dtype="fp8_per_tensor" if ks else "auto")
    want = _torch_prefill_gpu(q, kc, vc, *args, sc, 32, 8, ks, vs)
    assert_close_out(got, want, got.dtype, 2e-2 if ks else 2e-3)


@pytest.mark.parametrize("scale", [0.3, 1.0])
def test_prefill_peaked_attention_long_context(dev, scale):
    """Peaked softmaxes (scale 0.3 and 1.0 on N(0,1) q and k: a row's weight
    sits on two or three keys, where a P rounded once to bf16 would miss 2e-3)
    over 290-1500 keys, paged and contiguous, bf16, within 2e-3 of the float64
    oracle."""
    announce(f"prefill peaked attention, long context, scale {scale}")
    q, k, v, bt, ctx, cu, pos, _, _ = _make(77, [250, 700, 1400], [64, 40, 100], 8, 2, 64,
                                            torch.bfloat16)
    got = _gpu(dev, q, k, v, bt, ctx, cu, pos, scale, 8, 2, None, None)
    want = R.paged_prefill_ref(q.double(), k, v, bt, ctx, cu, pos, scale, 8, 2)
    assert_close_out(got, want, got.dtype, 2e-3)
    g = torch.Generator().manual_seed(78)
    lens = [600, 1100, 300]
    cuf = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    T = int(cuf[-1])
    qf = torch.randn(T, 8, 128, generator=g).to(torch.bfloat16)
    kf = torch.randn(T, 2, 128, generator=g).to(torch.bfloat16)
    vf = torch.randn(T, 2, 128, generator=g).to(torch.bfloat16)
    gotf = mkv.flash_attention_prefill(qf.to(dev), kf.to(dev), vf.to(dev), cuf.to(dev), scale, 8, 2,
                                       128).cpu()
    wantf = R.flash_prefill_ref(qf.double(), kf.double(), vf.double(), cuf, scale, 8, 2)
    assert_close_out(gotf, wantf, gotf.dtype, 2e-3)


@pytest.mark.parametrize("paged", [True, False])
def test_prefill_bf16_values_beyond_fp16_range(dev, paged):
    """V values beyond the fp16 range in a bf16 cache (7e4, -3e5 and 2e9
    inside sequence 0's context, none in sequence 1, one launch) stay exact
    through the PV products: against the float64 oracle, whose half-ulp term
    scales with the large outputs, paged and contiguous."""
    announce(f"prefill bf16 V beyond fp16, paged={paged}")
    prior, qlen = [300, 90], [70, 130]
    q, k, v, bt, ctx, cu, pos, _, _ = _make(505, prior, qlen, 8, 2, 64, torch.bfloat16)
    sc = 0.3
    if paged:
        blk = int(bt[0, 1])
        v[blk, 5, 0, 17] = 7e4
        v[blk, 40, 1, 100] = -3e5
        v[int(bt[0, 0]), 3, 0, 0] = 2e9
        got = _gpu(dev, q, k, v, bt, ctx, cu, pos, sc, 8, 2, None, None)
        want = R.paged_prefill_ref(q.double(), k, v, bt, ctx, cu, pos, sc, 8, 2)
    else:
        lens = [370, 220]
        cuf = torch.tensor([0, 370, 590], dtype=torch.int32)
        g = torch.Generator().manual_seed(506)
        qf = torch.randn(590, 8, 128, generator=g).to(torch.bfloat16)
        kf = torch.randn(590, 2, 128, generator=g).to(torch.bfloat16)
        vf = torch.randn(590, 2, 128, generator=g).to(torch.bfloat16)
        vf[69, 0, 17] = 7e4
        vf[200, 1, 100] = -3e5
        vf[3, 0, 0] = 2e9
        got = mkv.flash_attention_prefill(qf.to(dev), kf.to(dev), vf.to(dev), cuf.to(dev), sc, 8, 2,
                                          128).cpu()
        want = R.flash_prefill_ref(qf.double(), kf.double(), vf.double(), cuf, sc, 8, 2)
        assert lens[0] + lens[1] == 590
    assert float(want.abs().max()) > 1e4  # the large values reach the output
    assert_close_out(got, want, got.dtype, 2e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("group", [1, 4, 16])
def test_flash_prefill_contiguous(dev, dtype, group):
    announce(f"flash prefill contiguous {dtype} group {group}")
    g = torch.Generator().manual_seed(90 + group)
    lens = [1, 77, 130, 5, 300]
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    T, Hkv = int(cu[-1]), 2
    q = torch.randn(T, Hkv * group, 128, generator=g).to(dtype)
    k = torch.randn(T, Hkv, 128, generator=g).to(dtype)
    v = torch.randn(T, Hkv, 128, generator=g).to(dtype)
    got = mkv.flash_attention_prefill(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), 0.08,
                                      Hkv * group, Hkv, 128).cpu()
    want = R.flash_prefill_ref(q.double(), k.double(), v.double(), cu, 0.08, Hkv * group, Hkv)
    assert_close_out(got, want, got.dtype, 2e-3)


@pytest.mark.parametrize("nseq", [60, 64, 65, 120, 256])
def test_flash_prefill_many_ragged_prompts(dev, nseq):
    """Full prefill of many short prompts (the end-to-end workload's shape:
    prompt lengths 0-200 with ties on a tile boundary and an empty prompt),
    each row's visibility taken from its token's position."""
    announce(f"flash prefill {nseq} ragged prompts")
    g = torch.Generator().manual_seed(700 + nseq)
    lens = [int(x) for x in torch.randint(0, 201, (nseq,), generator=g)]
    lens[1] = 0
    lens[2] = lens[5] = lens[7] = 64  # ties on a tile boundary
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    T, Hkv, group = int(cu[-1]), 2, 2
    q = torch.randn(T, Hkv * group, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    got = mkv.flash_attention_prefill(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), 0.08,
                                      Hkv * group, Hkv, 128).cpu()
    want = R.flash_prefill_ref(q.double(), k.double(), v.double(), cu, 0.08, Hkv * group, Hkv)
    assert_close_out(got, want, got.dtype, 2e-3)


def test_chunked_equals_one_shot_and_append_path(dev):
    announce("prefill: two chunks == one shot; paged(prior 0) == flash prefill")
    g = torch.Generator().manual_seed(5)
    n, Hq, Hkv, bs, N = 300, 8, 2, 16, 40
    q = torch.randn(n, Hq, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(n, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(n, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    ctx = torch.tensor([n])
    bt = W.fragmented_block_tables(ctx, bs, N, g).to(dev)
    slots = torch.cat([bt[0, t // bs:t // bs + 1].long() * bs + t % bs for t in range(n)])
    kc = torch.zeros(N, bs, Hkv, 128, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    mkv.store_kvcache(k, v, kc, vc, slots, bs)
    pos = torch.arange(n, device=dev)
    one = A.paged_attention_prefill_triton(q, kc, vc, bt, ctx.to(dev), torch.tensor([0, n], dtype=torch.int32, device=dev),
                                           pos, 0.1, Hq, Hkv, 128, bs)
    # two chunks of the same sequence as two "sequences" sharing the table
    cu2 = torch.tensor([0, 123, n], dtype=torch.int32, device=dev)
    ctx2 = torch.tensor([123, n], device=dev)
    two = A.paged_attention_prefill_triton(q, kc, vc, bt.repeat(2, 1), ctx2, cu2, pos, 0.1, Hq, Hkv, 128, bs)
    assert torch.equal(one, two)
    flash = mkv.flash_attention_prefill(q, k, v, torch.tensor([0, n], dtype=torch.int32, device=dev),
                                        0.1, Hq, Hkv, 128)
    want = R.flash_prefill_ref(q.cpu().double(), k.cpu().double(), v.cpu().double(),
                               torch.tensor([0, n]), 0.1, Hq, Hkv)
    assert_close_out(one, want, one.dtype, 2e-3)
    assert_close_out(flash, want, flash.dtype, 2e-3)


@pytest.mark.parametrize("mode", ["auto", "fp8_per_tensor"])
@pytest.mark.parametrize("route", ["unified", "split", "overlap"])
def test_attention_layer_mixed_batch(dev, mode, route):
    """The Attention layer stores the step's K/V, then attends: all rows in
    one prefill launch ("unified"), or decode rows to the decode kernel and
    prefill rows to the prefill kernel ("split", the reference's route)."""
    announce(f"Attention layer mixed batch {mode} {route}")
    g = torch.Generator().manual_seed(17)
    Hq, Hkv, bs, N = 8, 2, 16, 64
    prior = [40, 0, 99, 7]
    qlen = [1, 50, 1, 20]
    is_dec = [True, False, True, False]
    ctx = torch.tensor([p + n for p, n in zip(prior, qlen)])
    bt = W.fragmented_block_tables(ctx, bs, N, g)
    cu = torch.zeros(5, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(qlen), 0).to(torch.int32)
    pos = torch.tensor([p + j for p, n in zip(prior, qlen) for j in range(n)], dtype=torch.int64)
    seq_of_row = torch.repeat_interleave(torch.arange(4), torch.tensor(qlen))
    slots = torch.tensor([int(bt[s, int(p) // bs]) * bs + int(p) % bs for s, p in zip(seq_of_row, pos)])
    T = int(cu[-1])
    q = torch.randn(T, Hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    hist_k = torch.randn(N, bs, Hkv, 128, generator=g).to(torch.bfloat16)
    hist_v = torch.randn(N, bs, Hkv, 128, generator=g).to(torch.bfloat16)
    layer = A.Attention(Hq, 128, scale=1.0, num_kv_heads=Hkv, block_size=bs)
    layer.kv_cache_dtype = mode
    layer.mixed_batch = route
    fp8 = mode == "fp8_per_tensor"
    cdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    kcr = torch.zeros(N, bs, Hkv, 128, dtype=cdt)
    vcr = torch.zeros_like(kcr)
    ksr, vsr = torch.ones(1), torch.ones(1)
    all_slots = torch.arange(N * bs)
    if fp8:
        R.store_kvcache_fp8_ref(hist_k.view(-1, Hkv, 128), hist_v.view(-1, Hkv, 128), kcr, vcr, ksr, vsr, all_slots)
        R.store_kvcache_fp8_ref(k, v, kcr, vcr, ksr, vsr, slots)
    else:
        R.store_kvcache_ref(hist_k.view(-1, Hkv, 128), hist_v.view(-1, Hkv, 128), kcr, vcr, all_slots)
        R.store_kvcache_ref(k, v, kcr, vcr, slots)
    layer.k_cache = torch.zeros(N, bs, Hkv, 128, dtype=cdt, device=dev)
    layer.v_cache = torch.zeros_like(layer.k_cache)
    if fp8:
        layer.k_scale = torch.ones(1, device=dev)
        layer.v_scale = torch.ones(1, device=dev)
        A.store_kvcache_fp8(hist_k.view(-1, Hkv, 128).to(dev), hist_v.view(-1, Hkv, 128).to(dev),
                            layer.k_cache, layer.v_cache, layer.k_scale, layer.v_scale,
                            all_slots.to(dev), bs, mode)
    else:
        A.store_kvcache(hist_k.view(-1, Hkv, 128).to(dev), hist_v.view(-1, Hkv, 128).to(dev),
                        layer.k_cache, layer.v_cache, all_slots.to(dev), bs)
    split = C.split_mixed_decode_prefill_metadata(cu.tolist(), qlen, is_dec)
    split.decode_token_indices_tensor = torch.tensor(split.decode_token_indices, device=dev)
    split.decode_seq_indices_tensor = torch.tensor(split.decode_seq_indices, device=dev)
    split.prefill_token_indices_tensor = torch.tensor(split.prefill_token_indices, device=dev)
    split.prefill_seq_indices_tensor = torch.tensor(split.prefill_seq_indices, device=dev)
    split.prefill_cu_seqlens_q_tensor = torch.tensor(split.prefill_cu_seqlens_q, dtype=torch.int32, device=dev)
    C.set_context(True, cu_seqlens_q=cu.to(dev), max_seqlen_q=max(qlen), slot_mapping=slots.to(dev),
                  context_lens=ctx.to(dev), block_tables=bt.to(dev), positions=pos.to(dev),
                  mixed_attention_split=split, is_full_prefill=False)
    try:
        out = layer(q.to(dev), k.to(dev), v.to(dev)).cpu()
    finally:
        C.reset_context()
    assert torch.equal(layer.k_cache.cpu().view(torch.uint8), kcr.view(torch.uint8))
    ks = float(ksr) if fp8 else None
    vs = float(vsr) if fp8 else None
    want = R.paged_prefill_ref(q.double(), kcr, vcr, bt, ctx, cu, pos, 1 / math.sqrt(128), Hq, Hkv, ks, vs)
    assert_close_out(out, want.reshape(T, Hq * 128), out.dtype, 2e-2 if fp8 else 2e-3)


@pytest.mark.parametrize("kv,qdt", [(torch.bfloat16, torch.float32), (torch.bfloat16, torch.float16),
                                    (torch.float16, torch.float32), (torch.float32, torch.bfloat16),
                                    (torch.float32, torch.float16)])
def test_prefill_q_dtype_differs_from_cache(dev, kv, qdt):
    """q in another dtype than the cache: a bf16 cache with an fp32 / fp16 q
    takes the split (hi + lo) q path."""
    announce(f"prefill kv {kv} q {qdt}")
    q, k, v, bt, ctx, cu, pos, ks, vs = _make(91, [40, 0, 300], [33, 70, 5], 16, 4, 16, kv)
    q = torch.randn(q.shape, generator=torch.Generator().manual_seed(92)).to(qdt)
    sc = 1.0 / math.sqrt(128)
    got = _gpu(dev, q, k, v, bt, ctx, cu, pos, sc, 16, 4, ks, vs)
    want = R.paged_prefill_ref(q.double(), k, v, bt, ctx, cu, pos, sc, 16, 4)
    assert got.dtype == qdt
    assert_close_out(got, want, got.dtype, 2e-3)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("route", ["unified", "split", "overlap"])
def test_attention_layer_mixed_batch_full_size(dev, kv, route):
    """The chunked-prefill mixed batch at full size through Attention.forward:
    8 chunks of 512 rows after priors U[0, 4096] plus 120 decode rows with
    contexts U[256, 4096], shuffled, 32 q / 8 kv heads, block 256.  The
    layer appends every row's own K/V (store, then attend, as the reference's
    forward does, attention.py:1654-1760) and the output is checked against a
    float32 torch reference over the appended cache; the appended rows are
    checked byte for byte against the oracle's append."""
    announce(f"Attention layer mixed batch, full size (8x512 + 120 decode), {kv} KV, {route}")
    m = W.prefill_mixed(seed=4)
    N, bs, Hq, Hkv = m["num_blocks"], m["block_size"], 32, 8
    cu, pos, ctx, bt = m["cu_seqlens_q"], m["positions"], m["context_lens"], m["block_tables"]
    qlen, is_dec = m["query_lens"], m["is_decode"]
    T = int(cu[-1])
    seq_of_row = torch.repeat_interleave(torch.arange(len(qlen)), torch.tensor(qlen))
    slots = bt[seq_of_row, pos // bs].long() * bs + pos % bs
    fp8 = kv == "fp8"
    cdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    layer = A.Attention(Hq, 128, scale=1.0, num_kv_heads=Hkv, block_size=bs)
    layer.kv_cache_dtype = "fp8_per_tensor" if fp8 else "auto"
    layer.mixed_batch = route
    layer.k_cache = torch.empty(N, bs, Hkv, 128, dtype=cdt, device=dev)
    layer.v_cache = torch.empty_like(layer.k_cache)
    ks = W.fill_pool_on_device(layer.k_cache, 51)
    vs = W.fill_pool_on_device(layer.v_cache, 52)
    if fp8:
        layer.k_scale = torch.tensor([ks], device=dev)
        layer.v_scale = torch.tensor([vs], device=dev)
    g = torch.Generator().manual_seed(53)
    q = torch.randn(T, Hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    split = C.split_mixed_decode_prefill_metadata(cu.tolist(), qlen, is_dec)
    split.decode_token_indices_tensor = torch.tensor(split.decode_token_indices, device=dev)
    split.decode_seq_indices_tensor = torch.tensor(split.decode_seq_indices, device=dev)
    split.prefill_token_indices_tensor = torch.tensor(split.prefill_token_indices, device=dev)
    split.prefill_seq_indices_tensor = torch.tensor(split.prefill_seq_indices, device=dev)
    split.prefill_cu_seqlens_q_tensor = torch.tensor(split.prefill_cu_seqlens_q, dtype=torch.int32,
                                                     device=dev)
    assert len(split.decode_token_indices) == 120 and len(split.prefill_token_indices) == 8 * 512
    C.set_context(True, cu_seqlens_q=cu.to(dev), max_seqlen_q=max(qlen), slot_mapping=slots.to(dev),
                  context_lens=ctx.to(dev), block_tables=bt.to(dev), positions=pos.to(dev),
                  mixed_attention_split=split, is_full_prefill=False)
    try:
        out = layer(q.to(dev), k.to(dev), v.to(dev))
    finally:
        C.reset_context()
    torch.cuda.synchronize()
    # the step's own rows landed in their slots, bytes as the oracle's append
    sd = slots.to(dev)
    got_k = layer.k_cache.view(-1, Hkv, 128).index_select(0, sd).cpu()
    got_v = layer.v_cache.view(-1, Hkv, 128).index_select(0, sd).cpu()
    if fp8:
        assert torch.equal(got_k.view(torch.uint8), R.fp8_quantize_ref(k, ks).view(torch.uint8))
        assert torch.equal(got_v.view(torch.uint8), R.fp8_quantize_ref(v, vs).view(torch.uint8))
    else:
        assert torch.equal(got_k.view(torch.int16), k.view(torch.int16))
        assert torch.equal(got_v.view(torch.int16), v.view(torch.int16))
    want = _torch_prefill_gpu(q.to(dev), layer.k_cache, layer.v_cache, bt.to(dev), ctx.to(dev), cu,
                              pos.to(dev), 1 / math.sqrt(128), Hq, Hkv, ks, vs)
    assert out.shape == (T, Hq * 128)
    assert_close_out(out.reshape(T, Hq, 128), want, out.dtype, 2e-2 if fp8 else 2e-3)
    # sampled rows against the float64 oracle over the appended cache: the
    # first, middle and last rows of 4 prefill chunks and 4 decode rows
    cuh = cu.tolist()
    pre = [s_ for s_ in range(len(qlen)) if not is_dec[s_]][:4]
    dec = [s_ for s_ in range(len(qlen)) if is_dec[s_]][:4]
    seqs, rows = [], []
    for s_ in pre + dec:
        a, b = cuh[s_], cuh[s_ + 1]
        r = sorted({a, (a + b) // 2, b - 1})
        seqs.append(s_)
        rows.append(r)
    sel = torch.tensor([r for rr in rows for r in rr])
    cu_s = torch.tensor([0] + list(np.cumsum([len(rr) for rr in rows])), dtype=torch.int32)
    kcs, vcs, bts = compact_pool(layer.k_cache, layer.v_cache, bt[seqs], ctx[seqs])
    ref = R.paged_prefill_ref(q[sel].double(), kcs, vcs, bts, ctx[seqs], cu_s, pos[sel], 1 / math.sqrt(128),
                              Hq, Hkv, ks, vs)
    assert_close_out(out.reshape(T, Hq, 128)[sel].cpu(), ref, out.dtype, 2e-2 if fp8 else 2e-3)


def test_attention_layer_fp32_auto_full_then_chunked_then_decode(dev):
    """The reference engine's default precision: an fp32 model with 'auto'
    (fp32) caches (model_runner.py:87, :249).  Three sequences go through a
    full prefill (flash_attention_prefill on the fresh k/v, after the
    append), a chunked prefill of further tokens over the cache, then two
    decode steps, all through Attention.forward; each step's output is
    checked against the float64 oracle on the oracle's own cache."""
    announce("Attention layer, fp32 'auto' caches: full prefill -> chunked prefill -> decode")
    g = torch.Generator().manual_seed(71)
    Hq, Hkv, bs, N = 8, 2, 16, 64
    sm = 1.0 / math.sqrt(128)
    layer = A.Attention(Hq, 128, scale=1.0, num_kv_heads=Hkv, block_size=bs)
    layer.k_cache = torch.zeros(N, bs, Hkv, 128, dtype=torch.float32, device=dev)
    layer.v_cache = torch.zeros_like(layer.k_cache)
    kcr = torch.zeros(N, bs, Hkv, 128, dtype=torch.float32)
    vcr = torch.zeros_like(kcr)
    tables = [torch.randperm(N, generator=g)[i * 20:(i + 1) * 20].tolist() for i in range(3)]
    bt = torch.tensor(tables, dtype=torch.int32)
    lens = [0, 0, 0]

    def step(new_tokens, full):
        """new_tokens[s] rows for sequence s (0 = not scheduled)."""
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
        q = torch.randn(T, Hq, 128, generator=g)
        k = torch.randn(T, Hkv, 128, generator=g)
        v = torch.randn(T, Hkv, 128, generator=g)
        R.store_kvcache_ref(k, v, kcr, vcr, slots)
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
        assert out.dtype == torch.float32
        assert torch.equal(layer.k_cache.cpu(), kcr) and torch.equal(layer.v_cache.cpu(), vcr)
        if decode:
            want = R.paged_decode_ref(q.double(), kcr, vcr, btd, ctx, sm, Hq, Hkv)
        elif full:
            want = R.flash_prefill_ref(q.double(), k.double(), v.double(), cu, sm, Hq, Hkv)
        else:
            want = R.paged_prefill_ref(q.double(), kcr, vcr, btd, ctx, cu, pos, sm, Hq, Hkv)
        assert_close_out(out.reshape(T, Hq, 128), want, torch.float32, 2e-3)

    step([37, 100, 5], full=True)
    step([20, 1, 64], full=False)
    step([1, 1, 1], full=False)
    step([1, 0, 1], full=False)
