"""Seeded synthetic workloads for the KV-cache hot path.

Each generator draws from ``torch.Generator(device='cpu').manual_seed(seed)``
in a fixed, documented order, so the oracle, a CPU baseline and the GPU
kernels can all see identical bytes.  Large KV pools (the batch-256 decode
workload) are filled on the GPU with a seeded CUDA generator instead, which
keeps setup time to seconds; their parity is checked through properties
rather than against a CPU copy.

Workloads (all head_dim 128):

* decode_small       batch 4, 16/8 heads, fp32, block 256, pool 64 blocks,
                     context U[64, 2048]
* append_fp8         4096 tokens, 8 kv heads, bf16 with 1% x20 outliers,
                     slots in a 1024 x 256 pool, 5% slots = -1
* decode_fp8_b32     batch 32, 32/8 heads over the pool written by append_fp8
* decode_b256        batch 256, 32/8 heads, block 256, context
                     log-uniform [512, 8192], pool 4096 blocks, bf16 or fp8
* prefill_mixed      8 prefill chunks of 512 rows (prior U[0, 4096]) plus
                     120 decode rows (context U[256, 4096]), 32/8 heads
"""
from __future__ import annotations

import math

import torch

HEAD_DIM = 128


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def fragmented_block_tables(ctx_lens: torch.Tensor, block_size: int, num_blocks: int,
                            gen: torch.Generator, max_blocks: int | None = None) -> torch.Tensor:
    """Give sequence i the next ceil(ctx_i / block_size) entries of one random
    permutation of the pool; pad rows with -1 to max_blocks columns."""
    nb = [(int(c) + block_size - 1) // block_size for c in ctx_lens]
    if max_blocks is None:
        max_blocks = max(max(nb), 1)
    if sum(nb) > num_blocks:
        raise ValueError(f"pool of {num_blocks} blocks cannot hold {sum(nb)} blocks")
    perm = torch.randperm(num_blocks, generator=gen)
    bt = torch.full((len(nb), max_blocks), -1, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(nb):
        bt[i, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    return bt


def decode_small(seed: int = 1) -> dict:
    """Batch 4, 16 q / 8 kv heads, fp32, block 256, pool of 64 blocks, context
    U[64, 2048]; draw order: ctx, perm, q, K pool, V pool."""
    g = _gen(seed)
    B, Hq, Hkv, bs, N = 4, 16, 8, 256, 64
    ctx = torch.randint(64, 2049, (B,), generator=g)
    bt = fragmented_block_tables(ctx, bs, N, g, max_blocks=8)
    q = torch.randn(B, Hq, HEAD_DIM, generator=g)
    k = torch.randn(N, bs, Hkv, HEAD_DIM, generator=g)
    v = torch.randn(N, bs, Hkv, HEAD_DIM, generator=g)
    return dict(q=q, k_cache=k, v_cache=v, block_tables=bt, context_lens=ctx.to(torch.int64),
                scale=1.0 / math.sqrt(HEAD_DIM), num_heads=Hq, num_kv_heads=Hkv, block_size=bs)


def append_fp8(seed: int = 2, num_tokens: int = 4096) -> dict:
    """num_tokens x 8 x 128 bf16 K/V with 1% outliers x20; distinct slots in a
    1024 x 256 pool with 5% = -1.  Draw order: K, V, K outlier mask, V outlier
    mask, slot permutation, padding mask."""
    g = _gen(seed)
    Hkv, N, bs = 8, 1024, 256
    k = torch.randn(num_tokens, Hkv, HEAD_DIM, generator=g)
    v = torch.randn(num_tokens, Hkv, HEAD_DIM, generator=g)
    k = torch.where(torch.rand(k.shape, generator=g) < 0.01, k * 20, k).to(torch.bfloat16)
    v = torch.where(torch.rand(v.shape, generator=g) < 0.01, v * 20, v).to(torch.bfloat16)
    slots = torch.randperm(N * bs, generator=g)[:num_tokens].to(torch.int64)
    slots = torch.where(torch.rand(num_tokens, generator=g) < 0.05, torch.full_like(slots, -1), slots)
    return dict(key=k, value=v, slot_mapping=slots, num_blocks=N, block_size=bs, num_kv_heads=Hkv)


def decode_fp8_b32(seed: int = 2) -> dict:
    """Decode step over the fp8 pool of append_fp8: every slot pre-filled with
    seeded bf16 values, then the 4096-token append applied; batch 32, 32 q /
    8 kv heads, context U[256, 4096].  Returns the bf16 pool contents and the
    decode metadata; the caller quantises (on the device or in the oracle)."""
    base = append_fp8(seed)
    g = _gen(seed + 1000)
    N, bs, Hkv = base["num_blocks"], base["block_size"], base["num_kv_heads"]
    fill_k = torch.randn(N * bs, Hkv, HEAD_DIM, generator=g).to(torch.bfloat16)
    fill_v = torch.randn(N * bs, Hkv, HEAD_DIM, generator=g).to(torch.bfloat16)
    B, Hq = 32, 32
    ctx = torch.randint(256, 4097, (B,), generator=g)
    bt = fragmented_block_tables(ctx, bs, N, g)
    q = torch.randn(B, Hq, HEAD_DIM, generator=g).to(torch.bfloat16)
    base.update(fill_key=fill_k, fill_value=fill_v, fill_slots=torch.arange(N * bs),
                q=q, block_tables=bt, context_lens=ctx.to(torch.int64),
                scale=1.0 / math.sqrt(HEAD_DIM), num_heads=Hq)
    return base


def decode_b256_metadata(seed: int = 3, batch: int = 256, num_blocks: int = 4096,
                         block_size: int = 256, max_blocks: int = 32) -> dict:
    """Context lengths floor(exp(U(ln 512, ln 8192))) and fragmented block
    tables for the batch-256 decode workload (draw order: ctx, perm)."""
    g = _gen(seed)
    u = torch.rand(batch, generator=g, dtype=torch.float64)
    ctx = torch.floor(torch.exp(math.log(512) + u * (math.log(8192) - math.log(512)))).to(torch.int64)
    ctx = ctx.clamp(max=max_blocks * block_size)
    bt = fragmented_block_tables(ctx, block_size, num_blocks, g, max_blocks=max_blocks)
    return dict(context_lens=ctx, block_tables=bt, num_blocks=num_blocks, block_size=block_size,
                max_blocks=max_blocks)


def fill_pool_on_device(pool: torch.Tensor, seed: int, scale: float | None = None) -> float | None:
    """Fill a (N, bs, H, D) pool on its device with seeded N(0, 1) values
    rounded to bf16.  An fp8 pool stores clamp(x / scale, +-448) in e4m3fn;
    with scale=None the per-tensor scale is calibrated first from the same
    values (bf16(amax) / 448 rounded to bf16, the reference's rule) and
    returned."""
    N = pool.shape[0]
    step = max(1, (1 << 27) // max(1, pool[0].numel()))  # ~128M elements per chunk

    def chunks():
        g = torch.Generator(device=pool.device).manual_seed(seed)
        for i in range(0, N, step):
            x = torch.randn(pool[i:i + step].shape, generator=g, device=pool.device,
                            dtype=torch.float32)
            yield i, x.to(torch.bfloat16)

    if pool.dtype == torch.float8_e4m3fn and scale is None:
        amax = torch.zeros((), dtype=torch.bfloat16, device=pool.device)
        for _, x in chunks():
            amax = torch.maximum(amax, x.abs().amax())
        scale = float((amax.clamp(min=1e-8) / 448.0).item())
    for i, x in chunks():
        if pool.dtype == torch.float8_e4m3fn:
            s = torch.tensor(scale, dtype=torch.float32, device=pool.device)
            pool[i:i + step] = torch.clamp(x.float() / s, -448.0, 448.0).to(pool.dtype)
        else:
            pool[i:i + step] = x.to(pool.dtype)
    return scale if pool.dtype == torch.float8_e4m3fn else None


def fill_pools_per_token_head_on_device(k_pool: torch.Tensor, v_pool: torch.Tensor,
                                        k_scale: torch.Tensor, v_scale: torch.Tensor, seed: int,
                                        mode: str) -> None:
    """Fill (N, bs, H, D) FP8 / INT8 K and V pools and their (N, bs, H) fp32
    scales on their device: seeded N(0, 1) bf16 rows, each (token, head)
    scaled by 2^U(-2, 2), quantised by the per-token-head append kernel into
    every slot in order (mode 'fp8_per_token_head' or 'int8_per_token_head')."""
    from . import attention as A

    N, bs, H, D = k_pool.shape
    rows = N * bs
    step = max(1, (1 << 26) // (H * D))  # ~64M elements per chunk
    g = torch.Generator(device=k_pool.device).manual_seed(seed)

    def rand_rows(n):
        x = torch.randn(n, H, D, generator=g, device=k_pool.device)
        x = x * torch.exp2(torch.rand(n, H, 1, generator=g, device=k_pool.device) * 4 - 2)
        return x.to(torch.bfloat16)

    for i in range(0, rows, step):
        n = min(step, rows - i)
        kx, vx = rand_rows(n), rand_rows(n)
        slots = torch.arange(i, i + n, dtype=torch.int64, device=k_pool.device)
        if mode == "int8_per_token_head":
            A.store_kvcache_int8(kx, vx, k_pool, v_pool, k_scale, v_scale, slots, bs)
        else:
            A.store_kvcache_fp8(kx, vx, k_pool, v_pool, k_scale, v_scale, slots, bs, mode)


def prefill_mixed(seed: int = 4, num_prefill: int = 8, chunk: int = 512, num_decode: int = 120,
                  block_size: int = 256, num_blocks: int = 4096) -> dict:
    """Chunked-prefill mixed batch metadata: prefill sequence s has prior
    context P_s ~ U[0, 4096] and a chunk of `chunk` rows at positions
    P_s .. P_s + chunk - 1; decode sequences have context U[256, 4096] and
    one row at position ctx - 1.  Item order is a seeded shuffle.  Draw
    order: P, decode ctx, shuffle, perm."""
    g = _gen(seed)
    P = torch.randint(0, 4097, (num_prefill,), generator=g)
    dctx = torch.randint(256, 4097, (num_decode,), generator=g)
    items = [("prefill", int(p)) for p in P] + [("decode", int(c)) for c in dctx]
    order = torch.randperm(len(items), generator=g).tolist()
    items = [items[i] for i in order]
    ctx, qlens, positions, is_decode = [], [], [], []
    for kind, x in items:
        if kind == "prefill":
            ctx.append(x + chunk)
            qlens.append(chunk)
            positions.extend(range(x, x + chunk))
            is_decode.append(False)
        else:
            ctx.append(x)
            qlens.append(1)
            positions.append(x - 1)
            is_decode.append(True)
    ctx_t = torch.tensor(ctx, dtype=torch.int64)
    bt = fragmented_block_tables(ctx_t, block_size, num_blocks, g)
    cu = torch.zeros(len(items) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(qlens), 0).to(torch.int32)
    return dict(context_lens=ctx_t, block_tables=bt, cu_seqlens_q=cu,
                positions=torch.tensor(positions, dtype=torch.int64), query_lens=qlens,
                is_decode=is_decode, block_size=block_size, num_blocks=num_blocks)


def alg_bytes_decode(context_lens: torch.Tensor, block_size: int, num_heads: int,
                     num_kv_heads: int, kv_bytes: int, q_bytes: int = 2,
                     ctx_bytes: int = 8, scale_bytes: int = 0, head_dim: int = HEAD_DIM) -> int:
    """Algorithmic HBM bytes of one decode step: every visible K and V element
    once (plus its K and V scales for per-token-head caches, scale_bytes = 4),
    q and out once, the used block-table entries and context_lens."""
    L = context_lens.to(torch.int64)
    kv = int(L.sum()) * num_kv_heads * (head_dim * kv_bytes + scale_bytes) * 2
    qo = int(L.numel()) * num_heads * head_dim * 2 * q_bytes
    bt = int(((L + block_size - 1) // block_size).sum()) * 4
    return kv + qo + bt + int(L.numel()) * ctx_bytes


def alg_flops_prefill(context_lens: torch.Tensor, cu_seqlens_q: torch.Tensor,
                      positions: torch.Tensor, num_heads: int) -> int:
    """Algorithmic FLOPs of one causal paged prefill: every (query row, head)
    attends to visible = min(context_len, position + 1) keys, 2*D for
    S = q.K and 2*D for O += p.V per key."""
    cu = cu_seqlens_q.to(torch.int64)
    seq_of_row = torch.repeat_interleave(torch.arange(cu.numel() - 1), cu[1:] - cu[:-1])
    vis = torch.minimum(context_lens.to(torch.int64)[seq_of_row], positions.to(torch.int64) + 1)
    return int(vis.clamp(min=0).sum()) * num_heads * 4 * HEAD_DIM


def alg_bytes_append(slot_mapping: torch.Tensor, num_kv_heads: int, in_bytes: int,
                     out_bytes: int) -> int:
    """Algorithmic bytes of one append: each valid K and V row read once and
    written once, plus the slot mapping."""
    valid = int((slot_mapping >= 0).sum())
    return valid * num_kv_heads * HEAD_DIM * 2 * (in_bytes + out_bytes) + slot_mapping.numel() * 8
