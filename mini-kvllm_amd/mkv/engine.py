"""A minimal serving engine over the mkv KV-cache path: continuous batching
with chunked prefill, FP8 (or bf16 / fp32) paged KV, captured decode steps.

It exists to run the path end to end the way the reference engine drives it
(LLMEngine.generate -> Scheduler.schedule -> ModelRunner.run,
llm_engine.py:106-123, model_runner.py:503-752) and to measure generated
tokens per second; it is not a port of the reference's runner.  The pieces:

* :class:`Scheduler` (host only): FCFS admission under a token budget per
  step (``max_num_batched_tokens``) and a sequence cap
  (``max_num_seqs``).  Running sequences go first, each taking one decode
  token or its next prompt chunk; waiting requests are admitted into what
  is left of the budget, a long prompt being cut into chunks across steps
  (the reference's chunked prefill, scheduler.py:113-233).  Blocks are
  handed out as the tokens that need them are scheduled; a running sequence
  that cannot get a block preempts the newest running sequence, which
  starts again from its prompt (recompute).
* :class:`Qwen3Model`: the Qwen3 decoder (qwen3.py:73-284) in bf16 on torch
  GEMMs, with the attention layer's producer fused
  (:func:`mkv.producer.qkv_norm_rope_append`: q/k RMSNorm + RoPE + the FP8
  append) and :class:`mkv.Attention` for the paged attention; embeddings tied
  to the LM head.
* :class:`Engine`: runs a mixed / prefill step eagerly (host-built metadata,
  the Context the attention layers read) and a decode-only step as one
  replay of a captured HIP graph over device-resident metadata
  (:class:`mkv.decode_state.DecodeGraphs`); samples with the reference's
  rule (softmax(logits / T) / Exp(1), argmax; sampler.py:13-18).
"""
from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import _lib
from . import context as C
from .attention import DECODE_STREAM, DECODE_WORKGROUP, Attention, _dtype_code, _stream
from .decode_state import DecodeGraphs, DecodeMetadata
from .producer import qkv_norm_rope_append, qkv_norm_rope_append_decode


# ---------------------------------------------------------------------------
# Requests and scheduling (host only)
# ---------------------------------------------------------------------------
@dataclass(eq=False)
class Request:
    """One generation request.  ``tokens`` holds the prompt followed by the
    generated tokens; ``num_cached`` of them have their K/V in the cache.
    Requests compare by identity (membership tests on the running list must
    not compare token lists)."""

    req_id: int
    prompt_len: int
    tokens: list[int]
    max_tokens: int
    ignore_eos: bool = True
    temperature: float = 1.0
    num_cached: int = 0
    blocks: list[int] = field(default_factory=list)
    finished: bool = False

    @property
    def num_generated(self) -> int:
        return len(self.tokens) - self.prompt_len

    @property
    def in_prefill(self) -> bool:
        """True while prompt tokens (or, after a preemption, earlier output
        tokens) are still to be computed; a decode step feeds exactly the last
        token."""
        return self.num_cached < len(self.tokens) - 1


@dataclass(frozen=True)
class Scheduled:
    """A request's share of one step: ``num_tokens`` tokens starting at
    position ``start`` (a prompt chunk, or one decode token)."""

    req: Request
    start: int
    num_tokens: int

    @property
    def samples(self) -> bool:
        """The step produces a token for this request: its last scheduled
        token is the last known token."""
        return self.start + self.num_tokens == len(self.req.tokens)


class BlockPool:
    """Free list of KV-cache blocks (one block id covers ``block_size``
    slots in every layer's pool)."""

    def __init__(self, num_blocks: int):
        self.free = deque(range(num_blocks))

    def take(self) -> int | None:
        return self.free.popleft() if self.free else None

    def give(self, blocks: list[int]) -> None:
        self.free.extend(blocks)


class Scheduler:
    """Continuous batching with chunked prefill (see the module docstring)."""

    def __init__(self, num_blocks: int, block_size: int, max_num_seqs: int,
                 max_num_batched_tokens: int, eos: int | None = None):
        self.pool = BlockPool(num_blocks)
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.eos = eos
        self.waiting: deque[Request] = deque()
        self.running: list[Request] = []
        self.num_preemptions = 0

    def add(self, req: Request) -> None:
        """Queue a request.  One that needs more blocks than the whole pool
        (prompt + max_tokens) is refused here: admitted, it would preempt
        itself and be re-admitted forever."""
        need = (req.prompt_len + req.max_tokens + self.block_size - 1) // self.block_size
        if need > self.num_blocks:
            raise ValueError(f"request {req.req_id} needs {need} KV blocks (prompt {req.prompt_len} + "
                             f"max_tokens {req.max_tokens}) but the pool holds {self.num_blocks}")
        self.waiting.append(req)

    def done(self) -> bool:
        return not self.waiting and not self.running

    def _grow(self, req: Request, upto: int) -> bool:
        """Give req enough blocks for positions [0, upto)."""
        need = (upto + self.block_size - 1) // self.block_size
        while len(req.blocks) < need:
            b = self.pool.take()
            if b is None:
                return False
            req.blocks.append(b)
        return True

    def _preempt(self, req: Request) -> None:
        self.running.remove(req)
        self.pool.give(req.blocks)
        req.blocks = []
        req.num_cached = 0
        self.waiting.appendleft(req)
        self.num_preemptions += 1

    def schedule(self) -> list[Scheduled]:
        budget = self.max_num_batched_tokens
        out: list[Scheduled] = []
        preemptions = self.num_preemptions
        i = 0
        while i < len(self.running) and budget > 0:
            req = self.running[i]
            n = min(len(req.tokens) - req.num_cached, budget) if req.in_prefill else 1
            while not self._grow(req, req.num_cached + n):
                victim = self.running[-1]
                self._preempt(victim)
                if victim is req:
                    break
            if req not in self.running:
                break
            out.append(Scheduled(req, req.num_cached, n))
            budget -= n
            i += 1
        # after a preemption the pool is short: admit nothing this step
        preempted = self.num_preemptions != preemptions
        while self.waiting and budget > 0 and len(self.running) < self.max_num_seqs and not preempted:
            req = self.waiting[0]
            n = min(len(req.tokens) - req.num_cached, budget)
            if not self._grow(req, req.num_cached + n):
                self.pool.give(req.blocks)
                req.blocks = []
                break
            self.waiting.popleft()
            self.running.append(req)
            out.append(Scheduled(req, req.num_cached, n))
            budget -= n
        return out

    def finish_step(self, items: list[Scheduled], sampled: list[int]) -> list[Request]:
        """Record the step: advance each request's cached count, append the
        sampled tokens (one per item that samples, in item order) and retire
        finished requests.  Returns the requests that finished."""
        it = iter(sampled)
        done = []
        for s in items:
            req = s.req
            req.num_cached = s.start + s.num_tokens
            if not s.samples:
                continue
            tok = next(it)
            req.tokens.append(tok)
            if req.num_generated >= req.max_tokens or (
                    not req.ignore_eos and self.eos is not None and tok == self.eos):
                req.finished = True
                self.running.remove(req)
                self.pool.give(req.blocks)
                req.blocks = []
                done.append(req)
        return done


# ---------------------------------------------------------------------------
# Model
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class ModelConfig:
    """Qwen3 decoder shape.  Defaults: Qwen3-0.6B as the reference's
    benchmark configures it (benchmark_chunk_prefill.py:27-42): tied
    embeddings, RoPE base 1e6, no biases; every RMSNorm has eps 1e-5, the
    LayerNorm default the reference's modules are built with (qwen3.py:50-51,
    :192, :199; layernorm.py:5)."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    num_layers: int = 28
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    rope_base: float = 1e6
    max_position: int = 32768
    eps: float = 1e-5


def rope_cos_sin(base: float, head_dim: int, max_position: int, device) -> torch.Tensor:
    """(max_position, head_dim) fp32 table [cos | sin] of the NeoX rotary
    embedding (rotary_embedding.py:60-101)."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    f = torch.outer(torch.arange(max_position, dtype=torch.float32), inv)
    return torch.cat([f.cos(), f.sin()], dim=-1).to(device)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm of the rows of x (layernorm.py:16-24); with residual, the
    residual stream is first updated in place to x + residual and that sum
    is normalised (residual_rms_forward, :31-33).  One kernel
    (mkv_rmsnorm)."""
    out = torch.empty_like(x)
    _lib.call("mkv_rmsnorm", out.data_ptr(), residual.data_ptr() if residual is not None else None,
              x.data_ptr(), weight.data_ptr(), x.shape[0], x.shape[1], float(eps),
              _dtype_code(x, "x"), _stream(x.device))
    return out


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """silu(x[:, :I]) * x[:, I:] for rows of 2I (activation.py:16-19), one
    kernel (mkv_silu_mul)."""
    inter = x.shape[1] // 2
    out = torch.empty(x.shape[0], inter, dtype=x.dtype, device=x.device)
    _lib.call("mkv_silu_mul", out.data_ptr(), x.data_ptr(), x.stride(0), x.shape[0], inter,
              _dtype_code(x, "x"), _stream(x.device))
    return out


class Qwen3Model(torch.nn.Module):
    """Random-init Qwen3 decoder (weights N(0, std), norm weights 1) whose
    attention layers run on the mkv operators.  A decode step runs each
    layer's producer step and attention as one call
    (:func:`mkv.producer.qkv_norm_rope_append_decode`) unless
    fuse_decode_step is False (then through :meth:`attention`, which a
    subclass may replace)."""

    fuse_decode_step = True

    def __init__(self, cfg: ModelConfig, device, dtype=torch.bfloat16, seed: int = 5,
                 std: float = 0.02, block_size: int = 256):
        super().__init__()
        self.cfg = cfg
        self.block_size = block_size
        g = torch.Generator(device=device).manual_seed(seed)
        H, D, Hq, Hkv, I = cfg.hidden_size, cfg.head_dim, cfg.num_heads, cfg.num_kv_heads, cfg.intermediate_size

        def rnd(*shape):
            return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(dtype)

        self.embed = rnd(cfg.vocab_size, H)  # tied LM head
        self.layers = []
        for _ in range(cfg.num_layers):
            att = Attention(Hq, D, scale=1.0, num_kv_heads=Hkv, block_size=block_size)
            self.layers.append(dict(
                in_norm=torch.ones(H, dtype=dtype, device=device),
                qkv=rnd((Hq + 2 * Hkv) * D, H),
                q_norm=torch.ones(D, dtype=dtype, device=device),
                k_norm=torch.ones(D, dtype=dtype, device=device),
                o=rnd(H, Hq * D),
                post_norm=torch.ones(H, dtype=dtype, device=device),
                gate_up=rnd(2 * I, H),
                down=rnd(H, I),
                attn=att,
            ))
        self.final_norm = torch.ones(H, dtype=dtype, device=device)
        self.cos_sin = rope_cos_sin(cfg.rope_base, D, cfg.max_position, device)
        self.kv_cache_dtype = "auto"

    def attach_kv_cache(self, num_blocks: int, kv_cache_dtype: str = "fp8_per_tensor",
                        cache_dtype: torch.dtype | None = None) -> None:
        """Allocate every layer's pools (num_blocks, block_size, Hkv, D) and
        scales and inject them into the attention layers (:376-395):
        per-tensor scales hold the 1.0 sentinel (model_runner.py:311-329);
        the per-token-head modes ('fp8_per_token_head', 'int8_per_token_head')
        keep one fp32 K and one V scale per slot and KV head,
        (num_blocks, block_size, Hkv) (:330-338), written by the append."""
        cfg = self.cfg
        dev = self.embed.device
        cdt = {"fp8_per_tensor": torch.float8_e4m3fn, "fp8_per_token_head": torch.float8_e4m3fn,
               "int8_per_token_head": torch.int8}.get(kv_cache_dtype)
        if kv_cache_dtype == "auto":
            cdt = cache_dtype or self.embed.dtype
        elif cdt is None:
            raise ValueError(f"kv_cache_dtype {kv_cache_dtype!r}: the engine runs 'auto', 'fp8_per_tensor', "
                             "'fp8_per_token_head' or 'int8_per_token_head'")
        self.kv_cache_dtype = kv_cache_dtype
        for lay in self.layers:
            att = lay["attn"]
            att.k_cache = torch.zeros(num_blocks, self.block_size, cfg.num_kv_heads, cfg.head_dim,
                                      dtype=cdt, device=dev)
            att.v_cache = torch.zeros_like(att.k_cache)
            att.kv_cache_dtype = kv_cache_dtype
            if kv_cache_dtype == "fp8_per_tensor":
                att.k_scale = torch.ones(1, device=dev)
                att.v_scale = torch.ones(1, device=dev)
            elif kv_cache_dtype != "auto":
                att.k_scale = torch.zeros(num_blocks, self.block_size, cfg.num_kv_heads, device=dev)
                att.v_scale = torch.zeros_like(att.k_scale)

    def scales(self) -> list[torch.Tensor]:
        """The per-tensor FP8 scales (what a decode graph's capture must
        leave as it found them); per-token-head scales are written only by
        appends to real slots."""
        if self.kv_cache_dtype != "fp8_per_tensor":
            return []
        return [s for lay in self.layers for s in (lay["attn"].k_scale, lay["attn"].v_scale)
                if s is not None]

    def attention(self, li: int, q, k, v):
        """The attention of layer li on the producer's q (and, for a full
        prefill, the rotated k and v): the step's K/V are already in the
        cache."""
        return self.layers[li]["attn"](q, k, v, kv_appended=True)

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor,
                slot_mapping: torch.Tensor, full_prefill: bool = False) -> torch.Tensor:
        """Hidden states (tokens, hidden) after the final norm.  The
        attention metadata is the current mkv Context."""
        cfg = self.cfg
        Hq, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        x = F.embedding(input_ids, self.embed)
        residual = None
        for li, lay in enumerate(self.layers):
            if residual is None:
                residual = x
                h = rms_norm(x, lay["in_norm"], cfg.eps)
            else:
                h = rms_norm(x, lay["in_norm"], cfg.eps, residual)
            qkv = F.linear(h, lay["qkv"])
            att = lay["attn"]
            ctx = C.current_context()
            if self.fuse_decode_step and not ctx.is_prefill:
                # a decode step: the producer step and the attention in one
                # launch where the decode schedule allows it
                o = qkv_norm_rope_append_decode(
                    qkv, positions, Hq, Hkv, D, self.cos_sin, att.k_cache, att.v_cache, slot_mapping,
                    self.block_size, ctx.block_tables, ctx.context_lens,
                    att.scale / (D ** 0.5), q_norm_weight=lay["q_norm"], k_norm_weight=lay["k_norm"],
                    eps=cfg.eps, kv_cache_dtype=att.kv_cache_dtype, k_scale=att.k_scale,
                    v_scale=att.v_scale, split_tokens=att.decode_split_tokens).reshape(-1, Hq * D)
            else:
                q, k, v = qkv_norm_rope_append(
                    qkv, positions, Hq, Hkv, D, self.cos_sin, att.k_cache, att.v_cache, slot_mapping,
                    self.block_size, q_norm_weight=lay["q_norm"], k_norm_weight=lay["k_norm"],
                    eps=cfg.eps, kv_cache_dtype=att.kv_cache_dtype, k_scale=att.k_scale,
                    v_scale=att.v_scale, return_k=full_prefill)
                o = self.attention(li, q, k, v)
            x = F.linear(o, lay["o"])
            h = rms_norm(x, lay["post_norm"], cfg.eps, residual)
            x = F.linear(silu_and_mul(F.linear(h, lay["gate_up"])), lay["down"])
        return rms_norm(x, self.final_norm, cfg.eps, residual)

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden, self.embed)


def sample(logits: torch.Tensor, temperature: torch.Tensor, gen: torch.Generator) -> torch.Tensor:
    """The reference's sampler (sampler.py:13-18) draws
    argmax(softmax(logits / T) / E) with E ~ Exp(1) per entry.  The
    softmax's normaliser is the same for every entry of a row, so that
    argmax equals argmax(logits / T - log E), which needs no softmax pass
    over the vocabulary."""
    noise = torch.empty(logits.shape, dtype=torch.float32, device=logits.device)
    noise.exponential_(1.0, generator=gen).clamp_min_(1e-10)
    return (logits.float() / temperature[:, None] - noise.log_()).argmax(dim=-1)


# ---------------------------------------------------------------------------
# Engine
# ---------------------------------------------------------------------------
def mixed_metadata(items: list[Scheduled], block_size: int) -> dict:
    """Host lists of one eager step (the fields prepare_mixed builds,
    model_runner.py:530-671): the scheduled tokens with their absolute
    positions and cache slots (slot of position p = blocks[p // bs] * bs +
    p % bs), cu_seqlens_q, the context length each item sees after the step,
    block tables padded with -1, the rows whose logits are sampled (each
    sampling item's last row) and whether every item starts at position 0
    (then attention may run on the fresh contiguous k / v)."""
    bs = block_size
    ids, pos, slots, cu, ctx, qlens = [], [], [], [0], [], []
    for s in items:
        r = s.req
        ids.extend(r.tokens[s.start:s.start + s.num_tokens])
        for p in range(s.start, s.start + s.num_tokens):
            pos.append(p)
            slots.append(r.blocks[p // bs] * bs + p % bs)
        cu.append(cu[-1] + s.num_tokens)
        ctx.append(s.start + s.num_tokens)
        qlens.append(s.num_tokens)
    nb = max(len(s.req.blocks) for s in items)
    return dict(
        input_ids=ids, positions=pos, slot_mapping=slots, cu_seqlens_q=cu, context_lens=ctx,
        max_seqlen_q=max(qlens),
        block_tables=[s.req.blocks + [-1] * (nb - len(s.req.blocks)) for s in items],
        sample_rows=[cu[i + 1] - 1 for i, s in enumerate(items) if s.samples],
        temperatures=[s.req.temperature for s in items if s.samples],
        is_full_prefill=all(s.start == 0 for s in items))

@dataclass
class StepStats:
    kind: str        # "decode" (captured replay) or "mixed" (eager)
    tokens: int      # tokens fed to the model
    sampled: int     # tokens generated
    seconds: float


class Engine:
    """Generation over a :class:`Qwen3Model` with the scheduler above.

    Decode-only steps replay a graph captured per batch bucket and table
    width (each captured on its first use, after the prefills have
    calibrated the FP8 scales); a step with any prompt chunk runs eagerly
    through the paged-prefill path (a decode row is a one-token chunk
    there)."""

    def __init__(self, model: Qwen3Model, num_blocks: int, max_num_seqs: int = 64,
                 max_num_batched_tokens: int = 1024, kv_cache_dtype: str = "fp8_per_tensor",
                 max_model_len: int = 4096, eos: int | None = None, seed: int = 0,
                 use_graphs: bool = True, decode_split_tokens: int = 0):
        self.model = model
        for layer in model.layers:
            layer["attn"].decode_split_tokens = decode_split_tokens
        self.dev = model.embed.device
        self.bs = model.block_size
        model.attach_kv_cache(num_blocks, kv_cache_dtype)
        self.sched = Scheduler(num_blocks, self.bs, max_num_seqs, max_num_batched_tokens, eos)
        self.max_rows = max_num_seqs
        self.max_blocks = (max_model_len + self.bs - 1) // self.bs
        self.num_blocks = num_blocks
        self.gen = torch.Generator(device=self.dev).manual_seed(seed)
        self.use_graphs = use_graphs
        self.stats: list[StepStats] = []
        self._next_id = 0
        # decode-step state on the device
        self.meta = DecodeMetadata(self.max_rows, self.max_blocks, self.bs, num_blocks, self.dev)
        self.ids_buf = torch.zeros(self.max_rows, dtype=torch.int64, device=self.dev)
        self.temp_buf = torch.ones(self.max_rows, dtype=torch.float32, device=self.dev)
        self.logits_buf = None
        self.last_logits = None  # logits of the last step's sampled rows
        self.last_sampled: list[int] = []
        self.graphs: DecodeGraphs | None = None
        self._rows: list[Request] = []   # decode row -> request, as last loaded
        self._loaded_lens: list[int] = []
        self._loaded_nblocks: list[int] = []
        self._pin_lens = torch.zeros(self.max_rows, dtype=torch.int64).pin_memory()
        self._pin_bt = torch.zeros(self.max_rows, self.max_blocks, dtype=torch.int32).pin_memory()
        self._pin_ids = torch.zeros(self.max_rows, dtype=torch.int64).pin_memory()
        self._pin_temp = torch.ones(self.max_rows, dtype=torch.float32).pin_memory()

    def add_request(self, prompt: list[int], max_tokens: int, ignore_eos: bool = True,
                    temperature: float = 1.0) -> Request:
        if len(prompt) + max_tokens > self.max_blocks * self.bs:
            raise ValueError("prompt + max_tokens exceeds max_model_len")
        req = Request(self._next_id, len(prompt), list(prompt), max_tokens, ignore_eos, temperature)
        self._next_id += 1
        self.sched.add(req)
        return req

    # -- mixed / prefill step (eager) ---------------------------------------
    def _run_mixed(self, items: list[Scheduled]) -> torch.Tensor:
        m = mixed_metadata(items, self.bs)
        d = self.dev

        def dt(x, dtype):
            return torch.tensor(x, dtype=dtype).pin_memory().to(d, non_blocking=True)

        input_ids, positions = dt(m["input_ids"], torch.int64), dt(m["positions"], torch.int64)
        slot_mapping = dt(m["slot_mapping"], torch.int64)
        C.set_context(True, cu_seqlens_q=dt(m["cu_seqlens_q"], torch.int32),
                      max_seqlen_q=m["max_seqlen_q"], slot_mapping=slot_mapping,
                      context_lens=dt(m["context_lens"], torch.int64),
                      block_tables=dt(m["block_tables"], torch.int32), positions=positions,
                      is_full_prefill=m["is_full_prefill"])
        try:
            hidden = self.model(input_ids, positions, slot_mapping, full_prefill=m["is_full_prefill"])
        finally:
            C.reset_context()
        if not m["sample_rows"]:
            return torch.empty(0, dtype=torch.int64, device=d)
        logits = self.model.logits(hidden[dt(m["sample_rows"], torch.int64)])
        self.last_logits = logits
        return sample(logits, dt(m["temperatures"], torch.float32), self.gen)

    # -- decode-only step (captured) ----------------------------------------
    def _decode_step_fn(self, rows, slot, ctx, bt):
        C.set_context(False, slot_mapping=slot, context_lens=ctx, block_tables=bt)
        try:
            positions = (ctx - 1).clamp_(min=0)
            hidden = self.model(self.ids_buf[:rows], positions, slot)
            self.logits_buf[:rows].copy_(self.model.logits(hidden))
        finally:
            C.reset_context()

    def _load_rows(self, reqs: list[Request]) -> None:
        """Upload the decode rows' lengths, block tables, last tokens and
        temperatures (only when the set of rows or a table changed since the
        last decode step: a steady decode step sends nothing)."""
        lens = [len(r.tokens) - 1 for r in reqs]  # K/V cached before this step
        if (reqs == self._rows and lens == self._loaded_lens
                and all(len(r.blocks) == n for r, n in zip(reqs, self._loaded_nblocks))):
            return
        self._pin_lens.zero_()
        self._pin_bt.zero_()
        for i, r in enumerate(reqs):
            self._pin_lens[i] = lens[i]
            self._pin_bt[i, :len(r.blocks)] = torch.tensor(r.blocks, dtype=torch.int32)
            self._pin_ids[i] = r.tokens[-1]
            self._pin_temp[i] = r.temperature
        n = len(reqs)
        self.meta.seq_lens.copy_(self._pin_lens, non_blocking=True)
        self.meta.block_tables.copy_(self._pin_bt, non_blocking=True)
        self.ids_buf[:n].copy_(self._pin_ids[:n], non_blocking=True)
        self.temp_buf[:n].copy_(self._pin_temp[:n], non_blocking=True)
        self._rows = list(reqs)
        self._loaded_nblocks = [len(r.blocks) for r in reqs]

    def _run_decode(self, items: list[Scheduled]) -> torch.Tensor:
        reqs = [s.req for s in items]
        n = len(reqs)
        if self.logits_buf is None:
            self.logits_buf = torch.empty(self.max_rows, self.model.cfg.vocab_size,
                                          dtype=self.model.embed.dtype, device=self.dev)
        self._load_rows(reqs)
        if self.graphs is None:
            # decode tables as wide as the batch's longest sequence, rounded up
            # to a power of two (the reference pads each decode step's tables to
            # its longest sequence, model_runner.py:640-644); the decode
            # kernels' schedule follows the width.  Graphs are captured per
            # (batch bucket, width) on first use.
            widths = sorted({min(1 << i, self.max_blocks) for i in range(self.max_blocks.bit_length() + 1)})
            self.graphs = DecodeGraphs(self.meta, self._decode_step_fn, widths=widths)
            if self.use_graphs:
                self.graphs.capture(scales=self.model.scales(), keys=[])
        blocks = max(len(r.blocks) for r in reqs)
        if self.use_graphs:
            self.graphs.run(n, blocks)
        else:  # the same work eagerly, on the bucket's rows (the same GEMM shapes)
            rows = self.graphs.bucket(n)
            self._decode_step_fn(rows, *self.meta.step(rows, 1, self.graphs.width(blocks)))
        self.last_logits = self.logits_buf[:n]
        tok = sample(self.logits_buf[:n], self.temp_buf[:n], self.gen)
        self.ids_buf[:n].copy_(tok)
        # the rows advanced by one token on the device
        self._loaded_lens = [len(r.tokens) for r in reqs]
        return tok

    def step(self) -> list[Request]:
        items = self.sched.schedule()
        if not items:
            return []
        t0 = time.perf_counter()
        decode_only = all(not s.req.in_prefill and s.num_tokens == 1 for s in items)
        if decode_only:
            tok = self._run_decode(items)
        else:
            tok = self._run_mixed(items)
            self._rows = []  # decode rows must be reloaded before the next captured step
        sampled = tok.cpu().tolist()
        self.last_sampled = sampled
        dt = time.perf_counter() - t0
        done = self.sched.finish_step(items, sampled)
        self.stats.append(StepStats("decode" if decode_only else "mixed",
                                    sum(s.num_tokens for s in items), len(sampled), dt))
        return done

    def generate(self, prompts: list[list[int]], max_tokens: int, ignore_eos: bool = True,
                 temperature: float = 1.0) -> list[list[int]]:
        """Generate for every prompt; returns the generated tokens in prompt
        order."""
        reqs = [self.add_request(p, max_tokens, ignore_eos, temperature) for p in prompts]
        while not self.sched.done():
            self.step()
        return [r.tokens[r.prompt_len:] for r in reqs]

    def summary(self, wall_s: float) -> dict:
        gen = sum(s.sampled for s in self.stats)
        dec = [s for s in self.stats if s.kind == "decode"]
        mix = [s for s in self.stats if s.kind == "mixed"]
        dec_s = sum(s.seconds for s in dec)
        return {
            "generated_tokens": gen,
            "wall_s": round(wall_s, 4),
            "e2e_decode_tok_s": round(gen / wall_s, 1),
            "decode_steps": len(dec),
            "decode_only_tok_s": round(sum(s.sampled for s in dec) / dec_s, 1) if dec_s else None,
            "decode_step_ms_mean": round(1e3 * dec_s / len(dec), 3) if dec else None,
            "mixed_steps": len(mix),
            "mixed_tokens": sum(s.tokens for s in mix),
            "mixed_s": round(sum(s.seconds for s in mix), 4),
            "preemptions": self.sched.num_preemptions,
        }
