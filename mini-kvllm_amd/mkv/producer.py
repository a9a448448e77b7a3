"""Fused producer: q/k RMSNorm + rotary embedding + KV append in one kernel.

Reference: between its qkv projection and its attention kernels, one
attention layer of the reference engine runs the q/k/v split, q_norm and
k_norm (Qwen3Attention.forward, qwen3.py:73-118; LayerNorm.rms_forward,
layernorm.py:16-24), the rotary embedding (rotary_embedding.py:100-109) and
Attention.forward's contiguous copies and append (attention.py:1654-1691).
:func:`qkv_norm_rope_append` does all of it in one pass over the qkv rows
(``mkv_qkv_norm_rope_append``) and returns q (and, for full prefill over
fresh K/V, the rotated k and the v view) for the attention operators.
"""
from __future__ import annotations

import torch

from . import _lib
from .attention import (PER_TOKEN_HEAD_MODES, _DTYPES, _append, _block_table, _check_cache,
                        _check_token_scales, _ctx_lens, _decode, _dtype_code, _index_dtype, _require_gpu,
                        _stream, calibrate_fp8_per_tensor)


def qkv_norm_rope_append(qkv: torch.Tensor, positions: torch.Tensor, num_heads: int,
                         num_kv_heads: int, head_dim: int, cos_sin_cache: torch.Tensor,
                         k_cache: torch.Tensor | None, v_cache: torch.Tensor | None,
                         slot_mapping: torch.Tensor | None, block_size: int, *,
                         q_norm_weight: torch.Tensor | None = None,
                         k_norm_weight: torch.Tensor | None = None, eps: float = 1e-5,
                         kv_cache_dtype: str = "auto", k_scale: torch.Tensor | None = None,
                         v_scale: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                         return_k: bool = False):
    """One layer's producer step.

    qkv: (num_tokens, (num_heads + 2 * num_kv_heads) * head_dim) rows (a
    larger row stride is accepted); positions: (num_tokens,) int64;
    cos_sin_cache: (max_position, head_dim) = [cos | sin]
    (RotaryEmbedding.cos_sin_cache); q/k norm weights: (head_dim,) or None
    for models without q/k norms; eps: LayerNorm's eps (1e-5 for
    Qwen3's q_norm / k_norm, qwen3.py:50-51).  The cache arguments follow
    store_kvcache / store_kvcache_fp8 / store_kvcache_int8 for
    kv_cache_dtype 'auto' / 'fp8_per_tensor' / 'fp8_per_token_head' /
    'int8_per_token_head'; slot_mapping None appends nothing.

    Returns (q, k, v): q (num_tokens, num_heads, head_dim) normed and rotated
    in out_dtype (default: qkv's dtype); k the rotated k
    (num_tokens, num_kv_heads, head_dim) if return_k else None; v the view of
    qkv's v columns.
    """
    if qkv.dim() != 2:
        raise ValueError("qkv must be (num_tokens, (num_heads + 2 * num_kv_heads) * head_dim)")
    T = qkv.shape[0]
    width = (num_heads + 2 * num_kv_heads) * head_dim
    if qkv.shape[1] < width or qkv.stride(1) != 1:
        raise ValueError(f"qkv rows must hold {width} contiguous elements")
    dev = _require_gpu(qkv, positions, cos_sin_cache)
    out_dtype = out_dtype or qkv.dtype
    q = torch.empty(T, num_heads, head_dim, dtype=out_dtype, device=dev)
    k = torch.empty(T, num_kv_heads, head_dim, dtype=out_dtype, device=dev) if return_k else None
    v = qkv[:, (num_heads + num_kv_heads) * head_dim:width].view(T, num_kv_heads, head_dim)
    if T == 0:
        return q, k, v
    pos = positions.to(torch.int64).contiguous()
    if pos.numel() < T:
        raise ValueError(f"positions has {pos.numel()} entries for {T} tokens")
    cs = cos_sin_cache.contiguous()
    if cs.shape[-1] != head_dim:
        raise ValueError(f"cos_sin_cache must be (max_position, {head_dim})")
    wdt = None
    for w in (q_norm_weight, k_norm_weight):
        if w is not None:
            if w.numel() != head_dim or not w.is_contiguous():
                raise ValueError(f"norm weights must be contiguous ({head_dim},)")
            wdt = w.dtype
    if q_norm_weight is not None and k_norm_weight is not None and q_norm_weight.dtype != k_norm_weight.dtype:
        raise TypeError("q_norm_weight and k_norm_weight must share a dtype")

    append = slot_mapping is not None
    quant = append and kv_cache_dtype != "auto"
    mode = _lib.SCALE_PER_TENSOR
    flags = 0
    if append:
        _check_cache(k_cache, v_cache, num_kv_heads, head_dim)
        slots = slot_mapping.to(torch.int64).contiguous()
        if slots.numel() != T:
            raise ValueError(f"slot_mapping has {slots.numel()} entries for {T} tokens")
        if kv_cache_dtype in PER_TOKEN_HEAD_MODES:
            want = torch.int8 if kv_cache_dtype == "int8_per_token_head" else torch.float8_e4m3fn
            if k_cache.dtype != want:
                raise TypeError(f"{kv_cache_dtype} needs a {want} cache, got {k_cache.dtype}")
            _check_token_scales(k_scale, v_scale, k_cache)
            mode = _lib.SCALE_PER_TOKEN_HEAD
        elif kv_cache_dtype == "fp8_per_tensor":
            if k_cache.dtype != torch.float8_e4m3fn:
                raise TypeError(f"fp8 cache expected, got {k_cache.dtype}")
            if not (getattr(k_scale, "_mkv_calibrated", False) and getattr(v_scale, "_mkv_calibrated", False)):
                # first use of these scales: rotate without appending, run the
                # calibration kernel on the rotated k / v (store_kvcache_fp8's
                # calibrate-once rule, attention.py:308-323), then append
                q, k_full, v = qkv_norm_rope_append(
                    qkv, positions, num_heads, num_kv_heads, head_dim, cos_sin_cache, None, None,
                    None, block_size, q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight,
                    eps=eps, out_dtype=out_dtype, return_k=True)
                calibrate_fp8_per_tensor(k_full, v, k_scale, v_scale)
                k_scale._mkv_calibrated = True
                v_scale._mkv_calibrated = True
                _append(k_full, v, k_cache, v_cache, slots, k_scale, v_scale, calibrate_sentinel=True)
                return q, (k_full if return_k else None), v
            flags = _lib.APPEND_CALIBRATE_SENTINEL
        elif kv_cache_dtype == "auto":
            if k_cache.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                raise TypeError(f"kv_cache_dtype 'auto' needs a float cache, got {k_cache.dtype}")
        else:
            raise ValueError(f"unknown kv_cache_dtype {kv_cache_dtype!r}")
    _lib.call(
        "mkv_qkv_norm_rope_append", qkv.data_ptr(), qkv.stride(0), _dtype_code(qkv, "qkv"), T,
        num_heads, num_kv_heads, head_dim,
        q_norm_weight.data_ptr() if q_norm_weight is not None else None,
        k_norm_weight.data_ptr() if k_norm_weight is not None else None,
        _DTYPES.get(wdt, 0) if wdt is not None else 0, float(eps), cs.data_ptr(),
        _dtype_code(cs, "cos_sin_cache"), cs.shape[0], pos.data_ptr(), q.data_ptr(),
        k.data_ptr() if k is not None else None, _dtype_code(q, "out_dtype"),
        k_cache.data_ptr() if append else None, v_cache.data_ptr() if append else None,
        _dtype_code(k_cache, "k_cache") if append else 0, mode,
        k_scale.data_ptr() if quant else None, v_scale.data_ptr() if quant else None,
        slots.data_ptr() if append else None, block_size,
        k_cache.shape[0] if append else 0, flags, _stream(dev))
    return q, k, v


def qkv_norm_rope_append_decode(qkv: torch.Tensor, positions: torch.Tensor, num_heads: int,
                                num_kv_heads: int, head_dim: int, cos_sin_cache: torch.Tensor,
                                k_cache: torch.Tensor, v_cache: torch.Tensor,
                                slot_mapping: torch.Tensor, block_size: int,
                                block_tables: torch.Tensor, context_lens: torch.Tensor,
                                scale: float, *, q_norm_weight: torch.Tensor | None = None,
                                k_norm_weight: torch.Tensor | None = None, eps: float = 1e-5,
                                kv_cache_dtype: str = "auto", k_scale: torch.Tensor | None = None,
                                v_scale: torch.Tensor | None = None,
                                out_dtype: torch.dtype | None = None, split_tokens: int = 0,
                                out: torch.Tensor | None = None) -> torch.Tensor:
    """One layer's decode step from its qkv rows: the producer step of
    :func:`qkv_norm_rope_append` for the batch's one new token per sequence
    (row b of qkv is sequence b's token, appended at slot_mapping[b]), then
    the decode attention over the paged cache (mkv.attention's decode with
    split_tokens) on the produced q.  Returns the attention output
    (batch, num_heads, head_dim) in out_dtype (default: qkv's dtype).

    At head_dim 128 with at most 8 query heads per KV head, for a per-tensor
    FP8 cache whose scales are calibrated, an fp16 cache, or a bf16 or
    per-token-head FP8 / INT8 cache with a bf16 out_dtype, when the decode
    schedule is the workgroup route
    (the library's choice for the shape, or split_tokens = DECODE_WORKGROUP),
    both run in one launch (``mkv_qkv_norm_rope_append_decode``, the same
    bits as the two calls); otherwise as the two calls.  slot_mapping[b]
    must be the cache row of position context_lens[b] - 1 of sequence b (or
    -1), as a decode step's metadata has it."""
    T = qkv.shape[0] if qkv.dim() == 2 else -1
    out_dtype = out_dtype or qkv.dtype
    kdt = k_cache.dtype if k_cache is not None else None
    if kv_cache_dtype == "fp8_per_tensor":
        cache_ok = (kdt == torch.float8_e4m3fn and getattr(k_scale, "_mkv_calibrated", False)
                    and getattr(v_scale, "_mkv_calibrated", False))
    elif kv_cache_dtype in PER_TOKEN_HEAD_MODES:
        want = torch.int8 if kv_cache_dtype == "int8_per_token_head" else torch.float8_e4m3fn
        cache_ok = kdt == want and out_dtype == torch.bfloat16
    else:
        cache_ok = kv_cache_dtype == "auto" and (
            kdt == torch.float16 or (kdt == torch.bfloat16 and out_dtype == torch.bfloat16))
    fused = (cache_ok and head_dim == 128 and T > 0
             and num_heads % num_kv_heads == 0 and num_heads // num_kv_heads <= 8)
    if fused:
        kv_code = _DTYPES[kdt]
        per_token = kv_cache_dtype in PER_TOKEN_HEAD_MODES
        if per_token:
            _check_token_scales(k_scale, v_scale, k_cache)
        bt = _block_table(block_tables)
        cl = _ctx_lens(context_lens)
        route = split_tokens
        if split_tokens == 0:
            # 1-byte caches: where per-tensor FP8 would take the workgroup
            # route (the query's answer for that dtype); per-token-head
            # scales alone would take stream-K at up to 256 tokens a wave,
            # but the one launch saves the producer's (~6 us), more than the
            # workgroup route gives up there at the engine's decode shape
            # (27.5 against 24.8 us for 60 rows in 4-block tables)
            route_dt = _lib.DTYPE_FP8E4M3 if kv_code in (_lib.DTYPE_FP8E4M3, _lib.DTYPE_I8) else kv_code
            route = (_lib.DECODE_WORKGROUP
                     if _lib.query("mkv_paged_decode_route", T, num_heads, num_kv_heads, bt.shape[1],
                                   k_cache.shape[1], head_dim, route_dt, 0, 0)
                     == _lib.ROUTE_WORKGROUP else 0)
        fused = route == _lib.DECODE_WORKGROUP
    if not fused:
        q, _, _ = qkv_norm_rope_append(
            qkv, positions, num_heads, num_kv_heads, head_dim, cos_sin_cache, k_cache, v_cache,
            slot_mapping, block_size, q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight,
            eps=eps, kv_cache_dtype=kv_cache_dtype, k_scale=k_scale, v_scale=v_scale,
            out_dtype=out_dtype)
        quant = kv_cache_dtype != "auto"
        return _decode(q, k_cache, v_cache, block_tables, context_lens, scale, num_heads,
                       num_kv_heads, head_dim, k_scale if quant else None, v_scale if quant else None,
                       split_tokens=split_tokens, out=out,
                       per_token_head=kv_cache_dtype in PER_TOKEN_HEAD_MODES)

    width = (num_heads + 2 * num_kv_heads) * head_dim
    if qkv.shape[1] < width or qkv.stride(1) != 1:
        raise ValueError(f"qkv rows must hold {width} contiguous elements")
    dev = _require_gpu(qkv, positions, cos_sin_cache, k_cache, v_cache, block_tables, context_lens)
    _check_cache(k_cache, v_cache, num_kv_heads, head_dim)
    pos = positions.to(torch.int64).contiguous()
    slots = slot_mapping.to(torch.int64).contiguous()
    if pos.numel() < T or slots.numel() < T:
        raise ValueError(f"positions / slot_mapping cover fewer than the batch's {T} rows")
    if bt.dim() != 2 or bt.shape[0] < T or cl.numel() < T:
        raise ValueError(f"block_tables {tuple(bt.shape)} / context_lens {tuple(cl.shape)} cover fewer "
                         f"than the batch's {T} sequences")
    cs = cos_sin_cache.contiguous()
    if cs.shape[-1] != head_dim:
        raise ValueError(f"cos_sin_cache must be (max_position, {head_dim})")
    wdt = None
    for w in (q_norm_weight, k_norm_weight):
        if w is not None:
            if w.numel() != head_dim or not w.is_contiguous():
                raise ValueError(f"norm weights must be contiguous ({head_dim},)")
            wdt = w.dtype
    if q_norm_weight is not None and k_norm_weight is not None and q_norm_weight.dtype != k_norm_weight.dtype:
        raise TypeError("q_norm_weight and k_norm_weight must share a dtype")
    if out is None:
        out = torch.empty(T, num_heads, head_dim, dtype=out_dtype, device=dev)
    elif out.dtype != out_dtype or tuple(out.shape) != (T, num_heads, head_dim) or out.stride(2) != 1:
        raise ValueError(f"out must be ({T}, {num_heads}, {head_dim}) {out_dtype}")
    _lib.call(
        "mkv_qkv_norm_rope_append_decode", out.data_ptr(), out.stride(0), _dtype_code(out, "out"),
        qkv.data_ptr(), qkv.stride(0), _dtype_code(qkv, "qkv"),
        q_norm_weight.data_ptr() if q_norm_weight is not None else None,
        k_norm_weight.data_ptr() if k_norm_weight is not None else None,
        _DTYPES.get(wdt, 0) if wdt is not None else 0, float(eps), cs.data_ptr(),
        _dtype_code(cs, "cos_sin_cache"), cs.shape[0], pos.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), kv_code, k_cache.shape[0],
        k_scale.data_ptr() if kv_code in (_lib.DTYPE_FP8E4M3, _lib.DTYPE_I8) else None,
        v_scale.data_ptr() if kv_code in (_lib.DTYPE_FP8E4M3, _lib.DTYPE_I8) else None,
        _lib.SCALE_PER_TOKEN_HEAD if per_token else _lib.SCALE_PER_TENSOR, slots.data_ptr(),
        _lib.APPEND_CALIBRATE_SENTINEL if kv_code == _lib.DTYPE_FP8E4M3 and not per_token else 0,
        bt.data_ptr(), bt.stride(0), bt.shape[1], cl.data_ptr(), _index_dtype(cl), T, num_heads,
        num_kv_heads, head_dim, k_cache.shape[1], float(scale), _stream(dev))
    return out
