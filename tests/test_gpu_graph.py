"""The decode-step capture contract (reference: model_runner.py:681-813).

The reference engine captures decode steps in a graph and replays them with
padded rows: slot_mapping -1, context_len 0 and block-table rows of 0 (not -1)
beyond the real rows (model_runner.py:697-701, :773).  The operators here do
no host synchronisation and, after one warm-up call, no allocation, so FP8
append + decode can be captured once and replayed.  Every replay is checked
bit for bit against the same operators run eagerly on a parallel copy of the
caches (the kernels are deterministic), with eager work and synchronisations
between replays.
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import announce
from mkv import attention as A
from mkv.decode_state import graph_capture

pytestmark = pytest.mark.gpu


def test_fp8_append_and_decode_replay_in_a_graph(dev):
    announce("graph: fp8 append + stream-K decode, 4 replays, 2 padded rows")
    g = torch.Generator().manual_seed(11)
    B, real, Hq, Hkv, D, bs, N = 8, 6, 32, 8, 128, 16, 96
    kc = torch.zeros(N, bs, Hkv, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1, device=dev)
    vs = torch.ones(1, device=dev)
    # block tables: real rows own disjoint blocks; padded rows are all 0
    max_blocks = 8
    perm = torch.randperm(N, generator=g)
    bt = torch.zeros(B, max_blocks, dtype=torch.int32)
    for b in range(real):
        bt[b] = perm[b * max_blocks:(b + 1) * max_blocks].to(torch.int32)
    ctx = torch.zeros(B, dtype=torch.int64)
    ctx[:real] = torch.randint(1, max_blocks * bs, (real,), generator=g)
    # one new token per real row, at position ctx - 1; padded rows skip (-1)
    slots = torch.full((B,), -1, dtype=torch.int64)
    for b in range(real):
        t = int(ctx[b]) - 1
        slots[b] = int(bt[b, t // bs]) * bs + t % bs
    bt_d, ctx_d, slots_d = bt.to(dev), ctx.to(dev), slots.to(dev)
    key = torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    value = torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(dev)
    # prior context: fill every slot once so that all visible tokens exist
    prior_k = torch.randn(N * bs, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    prior_v = torch.randn(N * bs, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    all_slots = torch.arange(N * bs, dtype=torch.int64, device=dev)
    A.store_kvcache_fp8(prior_k, prior_v, kc, vc, ks, vs, all_slots, bs, "fp8_per_tensor")
    scale = 1.0 / math.sqrt(D)

    def step(kc_, vc_):
        A.store_kvcache_fp8(key, value, kc_, vc_, ks, vs, slots_d, bs, "fp8_per_tensor")
        return A.paged_attention_decode_quantized(q, kc_, vc_, ks, vs, bt_d, ctx_d, scale, Hq, Hkv,
                                                  D, bs, "fp8_per_tensor")

    kc_e, vc_e = kc.clone(), vc.clone()
    step(kc.clone(), vc.clone())  # warm-up: workspaces allocated outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(kc.clone(), vc.clone())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with graph_capture(graph):
        out_g = step(kc, vc)
    torch.cuda.synchronize()
    # capturing does not execute: the graph's caches are still the prior state
    assert torch.equal(kc.view(torch.uint8), kc_e.view(torch.uint8))

    for rep in range(4):
        key.copy_(torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16))
        value.copy_(torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16))
        q.copy_(torch.randn(B, Hq, D, generator=g).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        out_e = step(kc_e, vc_e)
        _ = (q.float() * 2).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(kc.view(torch.uint8), kc_e.view(torch.uint8)), f"replay {rep}: cache"
        assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16)), f"replay {rep}: out"
        assert torch.all(out_g[real:] == 0), "padded rows (context_len 0) must be zero"
        assert torch.isfinite(out_g[:real].float()).all()
