"""Persistent decode-step metadata and captured decode steps.

The reference runner rebuilds the decode metadata on the host for every step
(ModelRunner.prepare_decode, model_runner.py:621-640: Python lists of
context lengths, slots and padded block tables, four host-to-device copies)
and its graph path copies them again into the captured buffers
(run_model, :681-706).  Its capture (capture_cudagraph, :760-813) reads
config['max_num_seqs'] where the config names it 'max_num_sequences' (:762,
:363), runs its warm-up forward with a zero-filled slot_mapping, so every
capture writes dummy K/V into slot 0 (:769, :794), and its replay writes -1
only into the real rows (:697), so the padded rows of a bucket keep the
slots of an earlier, larger batch and write K/V there.

:class:`DecodeMetadata` keeps the per-row sequence lengths and block tables
resident on the device; one kernel (``mkv_decode_metadata``) advances the
lengths and derives ``context_lens`` and ``slot_mapping`` for the step, so a
steady decode step sends nothing from the host.  The host writes a table row
when a sequence joins and one entry when it gets a new block.
:class:`DecodeGraphs` captures a user step function (metadata advance +
the layers' append/decode) once per batch bucket and block-table width over
these buffers and replays the smallest bucket and narrowest width that hold
the batch; captures run with every row inactive, so they write no K/V and
leave the state untouched.
"""
from __future__ import annotations

import contextlib
import gc
from typing import Callable, Iterable

import torch

from . import _lib


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


class DecodeMetadata:
    """Device-resident decode metadata for up to ``max_rows`` sequences.

    Row b holds one running sequence: ``seq_lens[b]`` is its length after the
    last advanced step (0 = inactive) and ``block_tables[b]`` its block table
    (unused entries are 0, as in the reference's graph buffers,
    model_runner.py:773).  ``step()`` produces the context views
    (``slot_mapping``, ``context_lens``, ``block_tables``) that
    :class:`mkv.Attention` and the operators read.
    """

    def __init__(self, max_rows: int, max_blocks: int, block_size: int, num_blocks: int,
                 device: torch.device | str):
        if block_size <= 0 or block_size & (block_size - 1):
            raise ValueError("block_size must be a power of two")
        self.device = torch.device(device)
        self.max_rows = max_rows
        self.max_blocks = max_blocks
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.seq_lens = torch.zeros(max_rows, dtype=torch.int64, device=self.device)
        self.context_lens = torch.zeros(max_rows, dtype=torch.int64, device=self.device)
        self.slot_mapping = torch.full((max_rows,), -1, dtype=torch.int64, device=self.device)
        self.block_tables = torch.zeros(max_rows, max_blocks, dtype=torch.int32, device=self.device)

    # -- host edits (rare: a sequence joins, leaves or gets a new block) ----
    def set_row(self, row: int, block_table: Iterable[int], num_tokens: int) -> None:
        """Put a sequence in ``row``: its block table and ``num_tokens`` =
        len(seq) at its next decode step (the count that includes the token
        that step decodes, as prepare_decode's context_lens).  A decoding
        sequence holds its prompt and at least one sampled token, so
        num_tokens >= 2; the row stores num_tokens - 1 and the next
        ``step()`` advances it."""
        bt = torch.tensor(list(block_table), dtype=torch.int32)
        if bt.numel() > self.max_blocks:
            raise ValueError(f"block table of {bt.numel()} blocks > max_blocks {self.max_blocks}")
        if num_tokens < 2 or num_tokens > bt.numel() * self.block_size:
            raise ValueError("num_tokens must be in 2 .. len(block_table) * block_size")
        row_t = torch.zeros(self.max_blocks, dtype=torch.int32)
        row_t[:bt.numel()] = bt
        self.block_tables[row].copy_(row_t)
        self.seq_lens[row] = num_tokens - 1

    def append_block(self, row: int, block_index: int, block_id: int) -> None:
        """Record that the sequence in ``row`` got block ``block_id`` as its
        ``block_index``-th block (the block manager's may_append)."""
        if not 0 <= block_index < self.max_blocks:
            raise ValueError(f"block_index {block_index} outside max_blocks {self.max_blocks}")
        self.block_tables[row, block_index] = block_id

    def clear_row(self, row: int) -> None:
        """Deactivate ``row`` (its sequence finished or was preempted)."""
        self.seq_lens[row] = 0
        self.block_tables[row].zero_()

    def move_row(self, src: int, dst: int) -> None:
        """Move the sequence in row ``src`` to row ``dst`` (to keep the
        active rows contiguous) and deactivate ``src``."""
        self.block_tables[dst].copy_(self.block_tables[src])
        self.seq_lens[dst].copy_(self.seq_lens[src])
        self.clear_row(src)

    # -- per step (device only, capturable) ---------------------------------
    def step(self, rows: int, increment: int = 1, width: int | None = None):
        """Advance the active rows among the first ``rows`` by ``increment``
        tokens and derive the step's metadata (one kernel, no host sync).
        Returns (slot_mapping, context_lens, block_tables) views of ``rows``
        rows; the block-table view has ``width`` columns (default: all
        ``max_blocks``), which must cover every active row's blocks, as the
        reference pads each decode step's tables to its longest sequence
        (model_runner.py:640-644)."""
        if not 0 <= rows <= self.max_rows:
            raise ValueError(f"rows {rows} outside 0..{self.max_rows}")
        width = self.max_blocks if width is None else width
        if not 1 <= width <= self.max_blocks:
            raise ValueError(f"width {width} outside 1..{self.max_blocks}")
        _lib.call("mkv_decode_metadata", self.seq_lens.data_ptr(), self.context_lens.data_ptr(),
                  self.slot_mapping.data_ptr(), self.block_tables.data_ptr(),
                  self.block_tables.stride(0), self.max_blocks, self.num_blocks, self.block_size,
                  rows, increment, _stream(self.device))
        return (self.slot_mapping[:rows], self.context_lens[:rows], self.block_tables[:rows, :width])


@contextlib.contextmanager
def graph_capture(graph: torch.cuda.CUDAGraph, pool=None):
    """``torch.cuda.graph(graph, pool)`` with Python's cyclic garbage
    collector run first and held off until the capture ends.  An object
    freed by a collection inside the capture frees what it owns there (a
    dead engine's graphs and their memory pool, a workspace), and those
    calls are not allowed while a stream captures: the process aborts.
    torch (2.10) no longer collects before a capture by itself."""
    gc.collect()
    enabled = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph, pool):
            yield
    finally:
        if enabled:
            gc.enable()


class DecodeGraphs:
    """Decode steps captured per (batch bucket, table width) over one
    :class:`DecodeMetadata`.

    ``step_fn(rows, slot_mapping, context_lens, block_tables)`` runs one
    decode step's device work for ``rows`` rows (e.g. every layer's append
    and decode over persistent input/output buffers); it must not allocate
    after its first call and must not synchronise.  Each graph holds the
    metadata advance followed by ``step_fn``.  Batch buckets follow the
    reference (1, 2, 4, 8, then multiples of 16 up to max_rows,
    model_runner.py:783), and ``run(batch, blocks)`` replays the smallest
    bucket that holds ``batch`` (the reference picks it the same way, :689)
    with the narrowest of ``widths`` that holds ``blocks`` block-table
    columns (default: one width, all ``max_blocks`` columns); rows past
    ``batch`` must be inactive.  A (bucket, width) pair that ``capture``
    left out is captured on its first ``run``.
    """

    def __init__(self, meta: DecodeMetadata, step_fn: Callable, buckets: Iterable[int] | None = None,
                 widths: Iterable[int] | None = None):
        self.meta = meta
        self.step_fn = step_fn
        if buckets is None:
            buckets = [b for b in (1, 2, 4, 8) if b <= meta.max_rows] + \
                list(range(16, meta.max_rows + 1, 16))
        self.buckets = sorted(set(buckets))
        if not self.buckets or self.buckets[-1] > meta.max_rows:
            raise ValueError("buckets must be non-empty and <= max_rows")
        self.widths = sorted(set(widths)) if widths is not None else [meta.max_blocks]
        if not self.widths or self.widths[0] < 1 or self.widths[-1] > meta.max_blocks:
            raise ValueError("widths must be non-empty and in 1..max_blocks")
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        self.pool = None
        self.scales: list[torch.Tensor] = []

    def capture(self, scales: Iterable[torch.Tensor] = (),
                keys: Iterable[tuple[int, int]] | None = None) -> None:
        """Capture one graph per (bucket, width) key (default: every bucket
        at the widest width), largest first, sharing one memory pool.  The
        state is saved, every row deactivated for the warm-up and the
        capture (so no K/V is written anywhere), and then restored.

        ``scales``: the per-tensor FP8 scale tensors that ``step_fn``'s
        appends use (kept for the captures that ``run`` makes later).  The
        warm-up runs the appends eagerly on the inactive rows, and a scale
        that still holds the 1.0 "not yet calibrated" sentinel would be
        calibrated there from those rows' dummy K/V and then frozen (the
        reference's capture has the same hazard, model_runner.py:769-794).
        Their values and calibration flags are saved before the warm-up and
        restored after the capture, so a scale that held 1.0 is calibrated by
        the first real step (eager, or a replay: the captured append keeps
        the sentinel test)."""
        m = self.meta
        scales = list(scales)
        if scales:
            self.scales = scales
        keys = sorted(keys if keys is not None else [(b, self.widths[-1]) for b in self.buckets],
                      reverse=True)
        saved_scales = [(s, s.clone(), getattr(s, "_mkv_calibrated", None)) for s in self.scales]
        saved = (m.seq_lens.clone(), m.context_lens.clone(), m.slot_mapping.clone())
        m.seq_lens.zero_()
        side = torch.cuda.Stream(m.device)
        side.wait_stream(torch.cuda.current_stream(m.device))
        with torch.cuda.stream(side):
            for rows, width in keys:  # warm-up: workspaces allocated here
                self.step_fn(rows, *m.step(rows, 0, width))
        torch.cuda.current_stream(m.device).wait_stream(side)
        torch.cuda.synchronize(m.device)
        for rows, width in keys:
            g = torch.cuda.CUDAGraph()
            with graph_capture(g, self.pool):
                self.step_fn(rows, *m.step(rows, 1, width))
            if self.pool is None:
                self.pool = g.pool()
            self.graphs[(rows, width)] = g
            torch.cuda.synchronize(m.device)
        m.seq_lens.copy_(saved[0])
        m.context_lens.copy_(saved[1])
        m.slot_mapping.copy_(saved[2])
        for s, value, flag in saved_scales:
            s.copy_(value)
            if flag is None:
                if hasattr(s, "_mkv_calibrated"):
                    del s._mkv_calibrated
            else:
                s._mkv_calibrated = flag
        torch.cuda.synchronize(m.device)

    def bucket(self, batch: int) -> int:
        for b in self.buckets:
            if b >= batch:
                return b
        raise ValueError(f"batch {batch} exceeds the largest bucket {self.buckets[-1]}")

    def width(self, blocks: int | None = None) -> int:
        """The narrowest table width that holds ``blocks`` columns (None: the
        widest)."""
        if blocks is None:
            return self.widths[-1]
        for w in self.widths:
            if w >= blocks:
                return w
        raise ValueError(f"{blocks} blocks exceed the widest table width {self.widths[-1]}")

    def run(self, batch: int, blocks: int | None = None) -> int:
        """Replay one decode step for ``batch`` active rows whose block
        tables hold at most ``blocks`` entries; returns the bucket replayed
        (rows of the step's outputs that are meaningful: the first
        ``batch``)."""
        key = (self.bucket(batch), self.width(blocks))
        if key not in self.graphs:
            self.capture(keys=[key])
        self.graphs[key].replay()
        return key[0]
