"""GPU tests of the device-side decode metadata and the captured decode step
(mkv.decode_state; reference ModelRunner.prepare_decode / run_model /
capture_cudagraph, model_runner.py:621-640, :681-813).

* The metadata kernel is compared, step by step and bit for bit, with the
  oracle (decode_metadata_ref) over a simulated run in which sequences join,
  grow across block boundaries, get new blocks and leave.
* Captured steps (metadata advance + two layers of FP8 append + decode) are
  replayed over a run whose batch grows and shrinks inside and across
  buckets, and compared bit for bit with the same operators run eagerly on a
  shadow copy of the state: outputs, KV pools and scales.
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import announce
from mkv import attention as A
from mkv import decode_state as DS
from oracle import reference as R

pytestmark = pytest.mark.gpu


class _Blocks:
    """A tiny block allocator standing in for the engine's block manager."""

    def __init__(self, n, g):
        self.free = torch.randperm(n, generator=g).tolist()

    def take(self):
        return self.free.pop()

    def give(self, ids):
        self.free.extend(ids)


def test_decode_metadata_matches_oracle_over_a_run(dev):
    announce("decode metadata: 80 steps, joins/leaves/new blocks, bs 16, 24 rows")
    g = torch.Generator().manual_seed(61)
    bs, max_rows, max_blocks, N = 16, 24, 12, 400
    meta = DS.DecodeMetadata(max_rows, max_blocks, bs, N, dev)
    blocks = _Blocks(N, g)
    rows: list[dict] = []  # active rows 0..len-1: {"bt": [...], "L": next-step length}

    def join():
        L0 = int(torch.randint(2, 100, (1,), generator=g))
        bt = [blocks.take() for _ in range((L0 + bs - 1) // bs)]
        meta.set_row(len(rows), bt, L0)
        rows.append({"bt": bt, "L": L0, "new": True})

    for _ in range(10):
        join()
    for step in range(80):
        # sequences that already ran a step grow by one token (and may need a block)
        for r, s in enumerate(rows):
            if s.pop("new", False):
                continue
            s["L"] += 1
            if (s["L"] - 1) % bs == 0:
                if len(s["bt"]) >= max_blocks:
                    continue
                b = blocks.take()
                meta.append_block(r, len(s["bt"]), b)
                s["bt"].append(b)
        slot, ctx, _ = meta.step(max_rows, 1)
        ok = [s["L"] <= len(s["bt"]) * bs for s in rows]
        want_ctx, want_slot = R.decode_metadata_ref(
            [s["bt"] for s in rows] + [[0]] * (max_rows - len(rows)),
            [s["L"] for s in rows] + [0] * (max_rows - len(rows)), bs)
        got_ctx, got_slot = ctx.cpu().tolist(), slot.cpu().tolist()
        for r in range(max_rows):
            if r < len(rows) and not ok[r]:
                continue  # ran out of max_blocks: not a case the runner produces
            assert (got_ctx[r], got_slot[r]) == (want_ctx[r], want_slot[r]), f"step {step} row {r}"
        # leave: the last-but-one row finishes, the last row moves into its place
        if step % 7 == 3 and len(rows) > 2:
            victim = len(rows) - 2
            blocks.give(rows[victim]["bt"])
            meta.move_row(len(rows) - 1, victim)
            rows[victim] = rows.pop()
        # rows that ran out of table capacity leave as well
        for r in reversed(range(len(rows))):
            if rows[r]["L"] >= max_blocks * bs - 1:
                blocks.give(rows[r]["bt"])
                last = len(rows) - 1
                if r != last:
                    meta.move_row(last, r)
                    rows[r] = rows.pop()
                else:
                    meta.clear_row(r)
                    rows.pop()
        if step % 5 == 0 and len(rows) < max_rows:
            join()


def _make_layers(dev, n_layers, N, bs, Hkv, scale=0.02):
    layers = []
    for _ in range(n_layers):
        kc = torch.zeros(N, bs, Hkv, 128, dtype=torch.float8_e4m3fn, device=dev)
        layers.append((kc, torch.zeros_like(kc), torch.full((1,), scale, device=dev),
                       torch.full((1,), scale, device=dev)))
    return layers


@pytest.mark.parametrize("sentinel", [False, True], ids=["calibrated", "sentinel"])
def test_captured_decode_steps_match_eager(dev, sentinel):
    """sentinel: the scales start at the runner's 1.0 "not yet calibrated"
    value (model_runner.py:327).  The capture must leave them at 1.0, and the
    first replay must calibrate them from its own K/V exactly as the eager
    store_kvcache_fp8 does."""
    announce(f"decode graphs: buckets 1/2/4/8/16, 2 layers fp8 append+decode, 30 steps, "
             f"scales {'1.0 sentinel' if sentinel else 'preset'}")
    g = torch.Generator().manual_seed(62)
    bs, max_rows, max_blocks, N, Hq, Hkv, L = 16, 16, 16, 300, 16, 4, 2
    sm = 1.0 / math.sqrt(128)
    # graph side and eager shadow side: same state, separate buffers
    sides = []
    for _ in range(2):
        meta = DS.DecodeMetadata(max_rows, max_blocks, bs, N, dev)
        q = torch.zeros(L, max_rows, Hq, 128, dtype=torch.bfloat16, device=dev)
        k = torch.zeros(L, max_rows, Hkv, 128, dtype=torch.bfloat16, device=dev)
        v = torch.zeros_like(k)
        out = torch.zeros(L, max_rows, Hq, 128, dtype=torch.bfloat16, device=dev)
        sides.append(dict(meta=meta, q=q, k=k, v=v, out=out,
                          layers=_make_layers(dev, L, N, bs, Hkv, 1.0 if sentinel else 0.02)))

    def make_step(sd):
        def step_fn(rows, slot, ctx, bt):
            for li, (kc, vc, ks, vs) in enumerate(sd["layers"]):
                A.store_kvcache_fp8(sd["k"][li, :rows], sd["v"][li, :rows], kc, vc, ks, vs, slot,
                                    bs, "fp8_per_tensor")
                A._decode(sd["q"][li, :rows], kc, vc, bt, ctx, sm, Hq, Hkv, 128, ks, vs,
                          out=sd["out"][li, :rows])
        return step_fn

    graphs = DS.DecodeGraphs(sides[0]["meta"], make_step(sides[0]), buckets=[1, 2, 4, 8, 16])
    scales = [x for lay in sides[0]["layers"] for x in lay[2:]]
    graphs.capture(scales=scales)
    for sd in sides:  # capture wrote nothing: pools still zero
        for kc, vc, _, _ in sd["layers"]:
            assert torch.count_nonzero(kc.view(torch.uint8)) == 0
    for x in scales:  # and left the scales (and their calibration state) alone
        assert float(x) == float(torch.tensor(1.0 if sentinel else 0.02, dtype=torch.float32))
        assert not getattr(x, "_mkv_calibrated", False)
    eager_step = make_step(sides[1])
    blocks = _Blocks(N, g)
    rows: list[dict] = []

    def join():
        L0 = int(torch.randint(2, 60, (1,), generator=g))
        bt = [blocks.take() for _ in range((L0 + bs - 1) // bs)]
        for sd in sides:
            sd["meta"].set_row(len(rows), bt, L0)
        rows.append({"bt": bt, "L": L0, "new": True})

    for _ in range(3):
        join()
    batches = []
    for step in range(30):
        for r, s in enumerate(rows):
            if s.pop("new", False):
                continue
            s["L"] += 1
            if (s["L"] - 1) % bs == 0:
                b = blocks.take()
                for sd in sides:
                    sd["meta"].append_block(r, len(s["bt"]), b)
                s["bt"].append(b)
        n = len(rows)
        batches.append(n)
        for name, shape in (("q", (L, n, Hq, 128)), ("k", (L, n, Hkv, 128)), ("v", (L, n, Hkv, 128))):
            x = torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)
            for sd in sides:
                sd[name][:, :n].copy_(x)
        rows_run = graphs.run(n)
        ev = sides[1]
        eager_step(rows_run, *ev["meta"].step(rows_run, 1))
        torch.cuda.synchronize()
        ga, eb = sides[0], sides[1]
        assert torch.equal(ga["out"][:, :n].view(torch.int16), eb["out"][:, :n].view(torch.int16)), \
            f"step {step} (batch {n}, bucket {rows_run}): outputs"
        assert torch.count_nonzero(ga["out"][:, n:rows_run].float()) == 0, "padded rows must be zero"
        for (kc, vc, ks, vs), (kc2, vc2, ks2, vs2) in zip(ga["layers"], eb["layers"]):
            assert torch.equal(ks, ks2) and torch.equal(vs, vs2), f"step {step}: scales"
            if sentinel:
                assert float(ks) != 1.0 and float(vs) != 1.0, f"step {step}: scale not calibrated"
            assert torch.equal(kc.view(torch.uint8), kc2.view(torch.uint8)), f"step {step}: K pool"
            assert torch.equal(vc.view(torch.uint8), vc2.view(torch.uint8)), f"step {step}: V pool"
        # grow to 11, shrink to 2, grow again: buckets change in both directions
        if step < 10 or 20 <= step:
            if len(rows) < 11:
                join()
        elif len(rows) > 2:
            victim = len(rows) - 2
            blocks.give(rows[victim]["bt"])
            for sd in sides:
                sd["meta"].move_row(len(rows) - 1, victim)
            rows[victim] = rows.pop()
    assert max(batches) == 11 and min(batches) == 2


def test_replay_after_workspace_growth(dev):
    """A captured decode keeps the device address of the decode workspace.
    A later eager decode that needs a larger workspace must not hand the
    captured one back to the allocator: tensors allocated afterwards would
    share its memory and the replay would write partials into them."""
    announce("decode graph replay after a larger eager decode grew the workspace")
    g = torch.Generator().manual_seed(63)
    bs, rows, max_blocks, N, Hq, Hkv = 16, 4, 8, 200, 16, 4
    sm = 1.0 / math.sqrt(128)
    kc = (torch.randn(N, bs, Hkv, 128, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    vc = torch.randn(N, bs, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    meta = DS.DecodeMetadata(rows, max_blocks, bs, N, dev)
    perm = torch.randperm(N, generator=g).tolist()
    for r in range(rows):
        meta.set_row(r, perm[r * max_blocks:(r + 1) * max_blocks], 40 + 17 * r)
    q = torch.randn(rows, Hq, 128, generator=g).to(torch.bfloat16).to(dev)
    out = torch.zeros(rows, Hq, 128, dtype=torch.bfloat16, device=dev)

    def step_fn(n, slot, ctx, bt):
        A._decode(q[:n], kc, vc, bt, ctx, sm, Hq, Hkv, 128, out=out[:n])

    graphs = DS.DecodeGraphs(meta, step_fn, buckets=[rows])
    graphs.capture()
    # an eager decode with a much larger batch and table: its workspace is larger
    B2, mb2 = 2048, 12
    ctx2 = torch.randint(1, mb2 * bs, (B2,), generator=g)
    bt2 = torch.randint(0, N, (B2, mb2), generator=g, dtype=torch.int32)
    q2 = torch.randn(B2, Hq, 128, generator=g).to(torch.bfloat16).to(dev)
    A.paged_attention_decode(q2, kc, vc, bt2.to(dev), ctx2.to(dev), sm, Hq, Hkv, 128, bs)
    # tensors allocated now may take any memory the allocator got back
    fillers = [torch.full((n,), 7, dtype=torch.uint8, device=dev) for n in (1 << 20, 4 << 20, 8 << 20)]
    torch.cuda.synchronize()
    for step in range(3):
        graphs.run(rows)
        torch.cuda.synchronize()
        slot, ctx, bt = meta.slot_mapping, meta.context_lens, meta.block_tables
        want = A.paged_attention_decode(q, kc, vc, bt, ctx, sm, Hq, Hkv, 128, bs)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {step}"
        for f in fillers:
            assert int((f != 7).sum()) == 0, f"replay {step} wrote into memory it does not own"
