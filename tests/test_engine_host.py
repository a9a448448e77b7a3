"""Host-side tests of the engine slice (mkv.engine): the scheduler's
continuous batching with chunked prefill, block accounting and preemption,
and the per-step metadata, with the model replaced by a stub that returns
fixed tokens.  Reference behaviour: scheduler.py:113-233 (running first,
then FCFS admission into the remaining token budget, chunks of long
prompts), model_runner.py:530-671 (slots, positions, context lengths)."""
from __future__ import annotations

import random

import pytest

from mkv import engine as E


def _run(sched, reqs, bs, max_steps=10000, token=7):
    """Drive the scheduler with a stub model; check every step's invariants."""
    steps = []
    owner = {}
    for _ in range(max_steps):
        if sched.done():
            break
        items = sched.schedule()
        assert items, "a non-empty scheduler must schedule something"
        assert sum(s.num_tokens for s in items) <= sched.max_num_batched_tokens
        assert len(items) <= sched.max_num_seqs
        assert len({id(s.req) for s in items}) == len(items)
        owner.clear()
        for s in sched.running:  # blocks are never shared between requests
            for b in s.blocks:
                assert b not in owner, "block owned twice"
                owner[b] = s
        for s in items:
            r = s.req
            assert s.start == r.num_cached, "a step continues where the cache ends"
            assert len(r.blocks) * bs >= s.start + s.num_tokens
        m = E.mixed_metadata(items, bs)
        assert len(m["input_ids"]) == len(m["positions"]) == len(m["slot_mapping"]) == m["cu_seqlens_q"][-1]
        for s, ctx in zip(items, m["context_lens"]):
            assert ctx == s.start + s.num_tokens
        for p, slot, s in zip(m["positions"], m["slot_mapping"],
                              [s for s in items for _ in range(s.num_tokens)]):
            assert slot == s.req.blocks[p // bs] * bs + p % bs
        sampled = [token] * len(m["sample_rows"])
        steps.append(items)
        sched.finish_step(items, sampled)
    assert sched.done()
    return steps


def test_continuous_batching_with_chunked_prefill_generates_every_token():
    rng = random.Random(0)
    bs = 16
    sched = E.Scheduler(num_blocks=400, block_size=bs, max_num_seqs=8, max_num_batched_tokens=64)
    reqs = []
    for i in range(20):
        n = rng.randint(1, 150)
        r = E.Request(i, n, [rng.randint(0, 999) for _ in range(n)], max_tokens=rng.randint(1, 30))
        sched.add(r)
        reqs.append(r)
    steps = _run(sched, reqs, bs)
    for r in reqs:
        assert r.finished and r.num_generated == r.max_tokens and r.tokens[r.prompt_len:] == [7] * r.max_tokens
        assert r.blocks == []
    assert sorted(sched.pool.free) == list(range(400)), "every block returned"
    # a prompt longer than the budget is cut into chunks across steps
    long_req = max(reqs, key=lambda r: r.prompt_len)
    chunks = [s for items in steps for s in items if s.req is long_req and s.start < long_req.prompt_len]
    assert len(chunks) >= 2 and sum(c.num_tokens for c in chunks) == long_req.prompt_len
    # FCFS: requests are admitted (first scheduled) in arrival order
    first = {}
    for k, items in enumerate(steps):
        for s in items:
            first.setdefault(s.req.req_id, k)
    order = sorted(first, key=lambda i: (first[i], i))
    assert order == sorted(order)


def test_decode_rows_run_before_new_prompts_and_budget_is_filled():
    bs = 16
    sched = E.Scheduler(num_blocks=100, block_size=bs, max_num_seqs=4, max_num_batched_tokens=32)
    a = E.Request(0, 10, list(range(10)), max_tokens=5)
    sched.add(a)
    items = sched.schedule()
    assert [(s.req.req_id, s.start, s.num_tokens) for s in items] == [(0, 0, 10)]
    sched.finish_step(items, [1])
    b = E.Request(1, 100, list(range(100)), max_tokens=3)
    sched.add(b)
    items = sched.schedule()
    # the decode row first (one token at position 10), then b's first chunk fills the budget
    assert [(s.req.req_id, s.start, s.num_tokens) for s in items] == [(0, 10, 1), (1, 0, 31)]
    assert items[0].samples and not items[1].samples
    m = E.mixed_metadata(items, bs)
    assert m["sample_rows"] == [0] and not m["is_full_prefill"]
    assert m["positions"][:2] == [10, 0]


def test_preemption_when_the_pool_runs_out_recomputes_and_finishes():
    bs = 16
    # 6 blocks: two requests of 40-token prompts that grow to 80 tokens cannot
    # both hold their blocks at the end
    sched = E.Scheduler(num_blocks=6, block_size=bs, max_num_seqs=4, max_num_batched_tokens=128)
    reqs = [E.Request(i, 40, [i] * 40, max_tokens=40) for i in range(2)]
    for r in reqs:
        sched.add(r)
    _run(sched, reqs, bs)
    assert sched.num_preemptions >= 1
    for r in reqs:
        assert r.finished and r.num_generated == 40
    assert sorted(sched.pool.free) == list(range(6))


def test_sequence_cap_limits_running_requests():
    sched = E.Scheduler(num_blocks=100, block_size=16, max_num_seqs=3, max_num_batched_tokens=1000)
    for i in range(5):
        sched.add(E.Request(i, 5, [0] * 5, max_tokens=2))
    items = sched.schedule()
    assert len(items) == 3 and len(sched.running) == 3 and len(sched.waiting) == 2


def test_request_larger_than_the_pool_is_refused():
    """A request whose prompt + max_tokens needs more blocks than the pool
    holds would preempt itself and be re-admitted forever; it is refused
    when it is added, and one that fits exactly still completes."""
    bs = 16
    sched = E.Scheduler(num_blocks=4, block_size=bs, max_num_seqs=4, max_num_batched_tokens=64)
    with pytest.raises(ValueError, match="KV blocks"):
        sched.add(E.Request(0, 60, list(range(60)), max_tokens=5))  # 65 tokens: 5 blocks
    assert sched.done()
    fits = E.Request(1, 60, list(range(60)), max_tokens=4)  # 64 tokens: 4 blocks
    sched.add(fits)
    _run(sched, [fits], bs)
    assert fits.num_generated == 4
