"""Drop-in KV-cache operators backed by the HIP kernels of libmkv.so.

Every public function keeps the name, argument order, argument meaning and
error behaviour of the reference engine's ``myvllm.layers.attention``
(src/myvllm/layers/attention.py), so the reference's runner, scheduler and
block manager can call these unchanged:

==============================  =========================================
this module                     reference
==============================  =========================================
store_kvcache                   attention.py:67-108
store_kvcache_fp8               attention.py:281-333 (per-tensor and
                                per-token-head modes)
store_kvcache_int8              attention.py:246-276
paged_attention_decode          attention.py:895-950
paged_attention_decode_quantized attention.py:1213-1268 (fp8_per_tensor,
                                fp8_per_token_head, int8_per_token_head)
paged_attention_prefill_triton  attention.py:852-891 (+ FP8 KV keywords)
flash_attention_prefill         attention.py:446-514
Attention                       attention.py:1617-1807
==============================  =========================================

All tensors must live on a ROCm GPU.  There is no CPU or eager fallback: a
missing libmkv.so, a CPU tensor or an unsupported combination raises.
Kernels are enqueued on the current torch stream; no function synchronises
with the host, so decode steps can be captured in a HIP graph once every
workspace has been allocated by a warm-up call.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .context import current_context

DECODE_WORKGROUP = _lib.DECODE_WORKGROUP
DECODE_STREAM = _lib.DECODE_STREAM

FP8_E4M3_MAX = 448.0
INT8_MAX = 127.0
INT8_MIN = -128.0

_DTYPES = {
    torch.float32: _lib.DTYPE_F32,
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.float16: _lib.DTYPE_F16,
    torch.float8_e4m3fn: _lib.DTYPE_FP8E4M3,
    torch.int8: _lib.DTYPE_I8,
}

# kv_cache_dtype strings of the reference's quantised modes and the scale
# granularity each uses (model_runner.py:222-229, :324-338).
PER_TOKEN_HEAD_MODES = ("fp8_per_token_head", "int8_per_token_head")

_workspaces: dict[tuple[int, str], torch.Tensor] = {}
# Workspaces replaced by larger ones.  A captured graph keeps the device
# address of the workspace it was captured with, so a replaced workspace is
# never handed back to the allocator (growth is geometric, so these hold at
# most as many bytes as the live ones).
_retired_workspaces: list[torch.Tensor] = []


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}") from None


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError("mkv kernels run on the GPU only; got a tensor on "
                             f"{t.device} (there is no CPU fallback)")
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


_side_streams: dict[int, torch.cuda.Stream] = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for work that can run
    beside the current stream's."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _side_streams.get(idx)
    if st is None:
        st = _side_streams[idx] = torch.cuda.Stream(device=dev)
    return st


def _workspace(dev: torch.device, name: str, nbytes: int, zeroed: bool = False) -> torch.Tensor:
    """Per-device scratch tensor, grown on demand (at least doubling) and then
    reused; a replaced one stays allocated for the life of the process."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), name)
    t = _workspaces.get(key)
    if t is None or t.numel() < nbytes:
        n = max(256, (nbytes + 255) // 256 * 256)
        if t is not None:
            n = max(n, 2 * t.numel())
            _retired_workspaces.append(t)
        t = (torch.zeros if zeroed else torch.empty)(n, dtype=torch.uint8, device=dev)
        _workspaces[key] = t
    return t


def _token_rows(x: torch.Tensor) -> torch.Tensor:
    """(tokens, kv_heads, head_dim) with contiguous rows; a row stride larger
    than the row (e.g. a k/v view into a fused qkv buffer) is kept as is."""
    T, H, D = x.shape
    if x.stride(2) == 1 and x.stride(1) == D and x.stride(0) >= H * D and \
            (x.stride(0) * x.element_size()) % 16 == 0 and x.data_ptr() % 16 == 0:
        return x
    return x.contiguous()


def _index_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.int64:
        return _lib.INDEX_I64
    if t.dtype == torch.int32:
        return _lib.INDEX_I32
    raise TypeError(f"context_lens must be int32 or int64, got {t.dtype}")


def _block_table(bt: torch.Tensor) -> torch.Tensor:
    if bt.dtype != torch.int32:
        bt = bt.to(torch.int32)
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    return bt


def _ctx_lens(cl: torch.Tensor) -> torch.Tensor:
    if cl.dtype not in (torch.int32, torch.int64):
        cl = cl.to(torch.int64)
    return cl.contiguous()


def _check_kv_rows(key: torch.Tensor, value: torch.Tensor) -> None:
    if key.dim() != 3 or key.shape != value.shape:
        raise ValueError("key and value must both be (num_tokens, num_kv_heads, head_dim); got "
                         f"{tuple(key.shape)} and {tuple(value.shape)}")


def _one_dtype(key: torch.Tensor, value: torch.Tensor):
    """The C ABI reads key and value with one element dtype.  A pair whose
    dtypes differ (e.g. a rotated k promoted to fp32 next to a bf16 v) is
    widened to fp32, which is exact; the reference's kernels load both as
    fp32 (attention.py:163-164, :225-226)."""
    if key.dtype != value.dtype:
        return key.float(), value.float()
    return key, value


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor, num_kv_heads: int, head_dim: int):
    if k_cache.dtype != v_cache.dtype:
        raise TypeError(f"k_cache and v_cache must share a dtype; got {k_cache.dtype} and {v_cache.dtype}")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache/v_cache must both be (num_blocks, block_size, num_kv_heads, "
                         f"head_dim); got {tuple(k_cache.shape)} and {tuple(v_cache.shape)}")
    if k_cache.shape[2] != num_kv_heads or k_cache.shape[3] != head_dim:
        raise ValueError(f"cache head layout {tuple(k_cache.shape[2:])} != ({num_kv_heads}, {head_dim})")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous per layer")


# ---------------------------------------------------------------------------
# K1: append
# ---------------------------------------------------------------------------
def _append(key, value, k_cache, v_cache, slot_mapping, k_scale=None, v_scale=None,
            calibrate_sentinel=False):
    _check_kv_rows(key, value)
    num_tokens, num_kv_heads, head_dim = key.shape
    dev = _require_gpu(key, value, k_cache, v_cache, slot_mapping)
    if k_cache.dtype != v_cache.dtype:
        raise TypeError("k_cache and v_cache must share a dtype")
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    if fp8 and (k_scale is None or v_scale is None):
        raise ValueError("an fp8 cache needs k_scale/v_scale (store_kvcache_fp8)")
    if slot_mapping.numel() != num_tokens:
        raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries for {num_tokens} tokens")
    if not fp8:
        # The reference's kernel casts on store; do the same cast on the GPU.
        if key.dtype != k_cache.dtype:
            key = key.to(k_cache.dtype)
        if value.dtype != v_cache.dtype:
            value = value.to(v_cache.dtype)
    elif key.dtype != value.dtype:
        key, value = _one_dtype(key, value)
        # the in-kernel calibration would round both amax values in fp32; the
        # callers calibrate such pairs per tensor beforehand
        calibrate_sentinel = False
    key = _token_rows(key)
    value = _token_rows(value)
    slots = slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.to(torch.int64)
    slots = slots.contiguous()
    _lib.call(
        "mkv_kv_append", key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr(), num_tokens, num_kv_heads,
        head_dim, k_cache.shape[1], k_cache.shape[0], _dtype_code(key, "key"),
        _dtype_code(k_cache, "k_cache"), k_scale.data_ptr() if fp8 else None,
        v_scale.data_ptr() if fp8 else None,
        _lib.APPEND_CALIBRATE_SENTINEL if (fp8 and calibrate_sentinel) else 0, _stream(dev))


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor, block_size: int) -> None:
    """Write key/value rows into their cache slots (slot -1 = skip).

    key, value: (num_tokens, num_kv_heads, head_dim); caches: (num_blocks,
    block_size, num_kv_heads, head_dim); slot_mapping: (num_tokens,).
    Reference: attention.py:67-108 (same asserts).
    """
    num_tokens, num_kv_heads, head_dim = key.shape
    assert k_cache.shape == v_cache.shape, "K and V cache shapes must match"
    assert slot_mapping.numel() == num_tokens, "Slot mapping size must match number of tokens"
    _check_cache(k_cache, v_cache, num_kv_heads, head_dim)
    _append(key, value, k_cache, v_cache, slot_mapping)


def _check_token_scales(k_scale, v_scale, k_cache):
    """Per-token-head scales: fp32 (num_blocks, block_size, num_kv_heads)
    tensors in slot order (model_runner.py:330-338)."""
    want = k_cache.shape[0] * k_cache.shape[1] * k_cache.shape[2]
    for name, sc in (("k_scale", k_scale), ("v_scale", v_scale)):
        if sc is None:
            raise ValueError(f"{name} is required for per-token-head scales")
        if sc.dtype != torch.float32 or not sc.is_contiguous() or sc.numel() < want:
            raise ValueError(f"{name} must be a contiguous float32 (num_blocks, block_size, "
                             f"num_kv_heads) tensor with >= {want} elements; got "
                             f"{sc.dtype} {tuple(sc.shape)}")


def _append_per_token_head(key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping):
    _check_kv_rows(key, value)
    num_tokens, num_kv_heads, head_dim = key.shape
    dev = _require_gpu(key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping)
    _check_token_scales(k_scale, v_scale, k_cache)
    if k_cache.dtype != v_cache.dtype:
        raise TypeError("k_cache and v_cache must share a dtype")
    if slot_mapping.numel() != num_tokens:
        raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries for {num_tokens} tokens")
    key, value = _one_dtype(key, value)
    key = _token_rows(key)
    value = _token_rows(value)
    slots = slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.to(torch.int64)
    slots = slots.contiguous()
    _lib.call(
        "mkv_kv_append_per_token_head", key.data_ptr(), key.stride(0), value.data_ptr(),
        value.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(),
        v_scale.data_ptr(), slots.data_ptr(), num_tokens, num_kv_heads, head_dim,
        k_cache.shape[1], k_cache.shape[0], _dtype_code(key, "key"),
        _dtype_code(k_cache, "k_cache"), _stream(dev))


def store_kvcache_int8(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, k_scale: torch.Tensor, v_scale: torch.Tensor,
                       slot_mapping: torch.Tensor, block_size: int) -> None:
    """Quantise key/value to INT8 with one scale per (token, kv head) and
    write codes and scales to their slots.  Reference: attention.py:246-276
    (kernel :194-243): scale = max(amax / 127, 1e-6), codes rounded half away
    from zero and clamped to [-128, 127]."""
    num_tokens, num_kv_heads, head_dim = key.shape
    _check_cache(k_cache, v_cache, num_kv_heads, head_dim)
    if k_cache.dtype != torch.int8:
        raise TypeError(f"int8 cache expected, got {k_cache.dtype}")
    _append_per_token_head(key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping)


def calibrate_fp8_per_tensor(key: torch.Tensor, value: torch.Tensor, k_scale: torch.Tensor,
                             v_scale: torch.Tensor) -> None:
    """Device-side form of the reference's calibrate-once rule
    (attention.py:308-323): a scale still equal to 1.0 becomes
    (x.abs().amax().clamp(min=1e-8) / 448) evaluated in x's dtype; any other
    value is left unchanged.  No host synchronisation."""
    dev = _require_gpu(key, value, k_scale, v_scale)
    if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
        raise TypeError("k_scale/v_scale must be float32 tensors")
    _check_kv_rows(key, value)
    if key.shape[0] == 0:
        raise RuntimeError("amax of an empty key/value tensor is undefined")
    if key.dtype != value.dtype:
        # the rule rounds in each tensor's own dtype: one launch per tensor,
        # the other scale pointing at a zero that is never the sentinel
        zero = _workspace(dev, "fp8_calibrate_zero", 4, zeroed=True)
        _calibrate_launch(dev, key, key, k_scale.data_ptr(), zero.data_ptr())
        _calibrate_launch(dev, value, value, zero.data_ptr(), v_scale.data_ptr())
        return
    _calibrate_launch(dev, key, value, k_scale.data_ptr(), v_scale.data_ptr())


def _calibrate_launch(dev, key, value, k_scale_ptr, v_scale_ptr) -> None:
    key = _token_rows(key)
    value = _token_rows(value)
    ws = _workspace(dev, "fp8_calibrate", _lib.query("mkv_fp8_calibrate_workspace_size"),
                    zeroed=True)
    _lib.call("mkv_fp8_calibrate_per_tensor", key.data_ptr(), key.stride(0), value.data_ptr(),
              value.stride(0), key.shape[0], key.shape[1] * key.shape[2],
              _dtype_code(key, "key"), k_scale_ptr, v_scale_ptr, ws.data_ptr(), _stream(dev))


def store_kvcache_fp8(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, k_scale: torch.Tensor, v_scale: torch.Tensor,
                      slot_mapping: torch.Tensor, block_size: int, kv_cache_dtype: str) -> None:
    """Quantise key/value to FP8 e4m3fn and write them to their cache slots.
    Reference: attention.py:281-333.

    'fp8_per_tensor': one scale per tensor, set by the reference's
    calibrate-once rule evaluated on the device: the first call on a scale
    tensor runs the calibration kernel; later calls pass the sentinel test to
    the append kernel itself, which calibrates in the rare case that the
    scale still holds 1.0, so the rule holds on every call with one launch
    instead of two.  'fp8_per_token_head': one
    scale per (token, kv head), amax / 448 (1 for an all-zero head), written
    to k_scale/v_scale of shape (num_blocks, block_size, num_kv_heads)
    (attention.py:166-181).
    """
    if kv_cache_dtype not in ("fp8_per_tensor", "fp8_per_token_head"):
        raise ValueError(f"store_kvcache_fp8: unknown kv_cache_dtype {kv_cache_dtype!r}")
    num_tokens, num_kv_heads, head_dim = key.shape
    _check_cache(k_cache, v_cache, num_kv_heads, head_dim)
    if k_cache.dtype != torch.float8_e4m3fn:
        raise TypeError(f"fp8 cache expected, got {k_cache.dtype}")
    if kv_cache_dtype == "fp8_per_token_head":
        _append_per_token_head(key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping)
        return
    mixed = key.dtype != value.dtype  # calibrated per tensor on every call (see _append)
    if mixed or not (getattr(k_scale, "_mkv_calibrated", False) and getattr(v_scale, "_mkv_calibrated", False)):
        calibrate_fp8_per_tensor(key, value, k_scale, v_scale)
        if not mixed:
            k_scale._mkv_calibrated = True
            v_scale._mkv_calibrated = True
    _append(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale, calibrate_sentinel=True)


# ---------------------------------------------------------------------------
# K2: decode
# ---------------------------------------------------------------------------
def _decode(query, k_cache, v_cache, block_tables, context_lens, scale, num_heads,
            num_kv_heads, head_dim, k_scale=None, v_scale=None, split_tokens=0,
            out=None, per_token_head=False) -> torch.Tensor:
    dev = _require_gpu(query, k_cache, v_cache, block_tables, context_lens)
    query = query.contiguous()
    batch = query.shape[0]
    if query.dim() != 3 or query.shape[1] != num_heads or query.shape[2] != head_dim:
        raise ValueError(f"query must be (batch, {num_heads}, {head_dim}); got {tuple(query.shape)}")
    _check_cache(k_cache, v_cache, num_kv_heads, head_dim)
    if out is None:
        out = torch.empty_like(query)
    if batch == 0:
        return out
    bt = _block_table(block_tables)
    cl = _ctx_lens(context_lens)
    if bt.dim() != 2 or bt.shape[0] < batch or cl.numel() < batch:
        raise ValueError(f"block_tables {tuple(bt.shape)} / context_lens {tuple(cl.shape)} cover fewer "
                         f"than the batch's {batch} sequences")
    max_blocks = bt.shape[1]
    bs = k_cache.shape[1]
    quant = k_cache.dtype in (torch.float8_e4m3fn, torch.int8)
    if quant and (k_scale is None or v_scale is None):
        raise ValueError("a quantised cache needs k_scale and v_scale")
    if per_token_head:
        _check_token_scales(k_scale, v_scale, k_cache)
    nbytes = _lib.query("mkv_paged_decode_workspace_size", batch, num_heads, num_kv_heads,
                        max_blocks, bs, head_dim, _dtype_code(k_cache, "k_cache"), split_tokens)
    ws = _workspace(dev, "decode", nbytes) if nbytes else None
    _lib.call(
        "mkv_paged_decode", out.data_ptr(), out.stride(0), query.data_ptr(), query.stride(0),
        _dtype_code(query, "query"), k_cache.data_ptr(), v_cache.data_ptr(),
        _dtype_code(k_cache, "k_cache"), k_cache.shape[0],
        k_scale.data_ptr() if quant else None, v_scale.data_ptr() if quant else None,
        _lib.SCALE_PER_TOKEN_HEAD if per_token_head else _lib.SCALE_PER_TENSOR,
        bt.data_ptr(), bt.stride(0), max_blocks, cl.data_ptr(), _index_dtype(cl), batch,
        num_heads, num_kv_heads, head_dim, bs, float(scale), split_tokens,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _stream(dev))
    return out


def paged_attention_decode(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                           num_heads: int, num_kv_heads: int, head_dim: int,
                           block_size: int, split_tokens: int = 0) -> torch.Tensor:
    """Decode attention over the paged cache: query (batch, num_heads,
    head_dim) -> output of the same shape and dtype.  Reference:
    attention.py:895-950.  Rows with context_lens == 0 yield zeros.
    head_dim 128, or 64 with an even num_kv_heads (the Llama-3.2-1B shape).
    split_tokens (an addition; 0 by default) selects the schedule:
    0 = the library's choice from the shape (the workgroup route when the
    (sequence, KV head) items fill the GPU's CUs with at least 4 waves each,
    else stream-K, else split-K); DECODE_STREAM (-2) = stream-K over the
    whole batch; n > 0 = split-K in n-token splits; DECODE_WORKGROUP (-1) =
    one workgroup per (sequence, KV head) whose waves split the sequence and
    merge in LDS (one launch, no workspace)."""
    return _decode(query, k_cache, v_cache, block_tables, context_lens, scale, num_heads,
                   num_kv_heads, head_dim, split_tokens=split_tokens)


def paged_attention_decode_quantized(query: torch.Tensor, k_cache: torch.Tensor,
                                     v_cache: torch.Tensor, k_scale: torch.Tensor,
                                     v_scale: torch.Tensor, block_tables: torch.Tensor,
                                     context_lens: torch.Tensor, scale: float, num_heads: int,
                                     num_kv_heads: int, head_dim: int, block_size: int,
                                     kv_cache_dtype: str, split_tokens: int = 0) -> torch.Tensor:
    """Decode attention over a quantised cache, dequantised as code * scale.
    Reference: attention.py:1213-1268.

    'fp8_per_tensor': FP8 cache, k_scale/v_scale of one element each.
    'fp8_per_token_head' / 'int8_per_token_head': FP8 / INT8 cache with
    float32 (num_blocks, block_size, num_kv_heads) scales; the K scale
    multiplies the score and the V scale the softmax weight of its token
    (the reference's tile kernel, attention.py:1124-1210).
    split_tokens as for paged_attention_decode.
    """
    if kv_cache_dtype == "fp8_per_tensor" or kv_cache_dtype == "fp8_per_token_head":
        if k_cache.dtype != torch.float8_e4m3fn:
            raise TypeError(f"{kv_cache_dtype} needs an fp8 cache, got {k_cache.dtype}")
    elif kv_cache_dtype == "int8_per_token_head":
        if k_cache.dtype != torch.int8:
            raise TypeError(f"{kv_cache_dtype} needs an int8 cache, got {k_cache.dtype}")
    else:
        raise ValueError(f"unknown quantized kv_cache_dtype {kv_cache_dtype!r}")
    return _decode(query, k_cache, v_cache, block_tables, context_lens, scale, num_heads,
                   num_kv_heads, head_dim, k_scale, v_scale, split_tokens=split_tokens,
                   per_token_head=kv_cache_dtype in PER_TOKEN_HEAD_MODES)


# ---------------------------------------------------------------------------
# K3: prefill
# ---------------------------------------------------------------------------
def paged_attention_prefill_triton(query: torch.Tensor, k_cache: torch.Tensor,
                                   v_cache: torch.Tensor, block_tables: torch.Tensor,
                                   context_lens: torch.Tensor, cu_seqlens_q: torch.Tensor,
                                   positions: torch.Tensor, scale: float, num_heads: int,
                                   num_kv_heads: int, head_dim: int, block_size: int, *,
                                   k_scale: torch.Tensor | None = None,
                                   v_scale: torch.Tensor | None = None,
                                   kv_cache_dtype: str = "auto") -> torch.Tensor:
    """Chunked-prefill / extend attention over the paged cache.

    Row i of sequence s attends to logical tokens [0, min(context_lens[s],
    positions[i] + 1)).  The name is kept for drop-in compatibility with
    attention.py:852-891; the work runs on the gfx950 MFMA kernel.  Quantised
    caches, which the reference's prefill does not implement
    (attention.py:1702-1708), take k_scale/v_scale: kv_cache_dtype
    'fp8_per_tensor' with (1,) scales, or 'fp8_per_token_head' /
    'int8_per_token_head' with (num_blocks, block_size, num_kv_heads) scales
    (the decode path's formats, attention.py:1124-1210).
    """
    dev = _require_gpu(query, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q,
                       positions)
    query = query.contiguous()
    out = torch.empty_like(query)
    total_q = query.shape[0]
    if total_q == 0:
        return out
    _check_cache(k_cache, v_cache, num_kv_heads, head_dim)
    quant = k_cache.dtype in (torch.float8_e4m3fn, torch.int8)
    per_token = kv_cache_dtype in PER_TOKEN_HEAD_MODES
    if per_token:
        want = torch.int8 if kv_cache_dtype == "int8_per_token_head" else torch.float8_e4m3fn
        if k_cache.dtype != want:
            raise TypeError(f"{kv_cache_dtype} needs a {want} cache, got {k_cache.dtype}")
        _check_token_scales(k_scale, v_scale, k_cache)
    elif k_cache.dtype == torch.int8:
        raise ValueError("an int8 cache needs kv_cache_dtype='int8_per_token_head' and its scales")
    elif quant:
        if kv_cache_dtype not in ("fp8_per_tensor", "auto") or k_scale is None or v_scale is None:
            raise ValueError("an fp8 cache needs kv_cache_dtype='fp8_per_tensor' and k_scale/v_scale")
    bt = _block_table(block_tables)
    cl = _ctx_lens(context_lens)
    cu = cu_seqlens_q.to(torch.int32).contiguous()
    pos = positions.to(torch.int64).contiguous()
    num_seqs = cl.shape[0]
    # (num_seqs comes from context_lens, as in attention.py:869; extra
    # cu_seqlens_q entries are ignored, missing ones would be read past its end)
    if cu.numel() < num_seqs + 1 or bt.dim() != 2 or bt.shape[0] < num_seqs or pos.numel() < total_q:
        raise ValueError(f"cu_seqlens_q {tuple(cu.shape)}, block_tables {tuple(bt.shape)} and positions "
                         f"{tuple(pos.shape)} must cover {num_seqs} sequences and {total_q} query rows")
    nbytes = _lib.query("mkv_paged_prefill_workspace_size", num_seqs, total_q, num_heads,
                        num_kv_heads)
    ws = _workspace(dev, "prefill", nbytes) if nbytes else None
    _lib.call(
        "mkv_paged_prefill", out.data_ptr(), query.data_ptr(), _dtype_code(query, "query"),
        k_cache.data_ptr(), v_cache.data_ptr(), _dtype_code(k_cache, "k_cache"), k_cache.shape[0],
        k_scale.data_ptr() if quant else None, v_scale.data_ptr() if quant else None,
        _lib.SCALE_PER_TOKEN_HEAD if per_token else _lib.SCALE_PER_TENSOR,
        bt.data_ptr(), bt.stride(0), bt.shape[1], cl.data_ptr(), _index_dtype(cl), cu.data_ptr(), pos.data_ptr(),
        num_seqs, total_q, num_heads, num_kv_heads, head_dim, k_cache.shape[1], float(scale),
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _stream(dev))
    return out


def flash_attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            cu_seqlens: torch.Tensor, scale: float, num_heads: int,
                            num_kv_heads: int, head_dim: int) -> torch.Tensor:
    """Causal varlen attention over fresh contiguous q/k/v (pure full
    prefill).  Reference: attention.py:446-514; unlike it, no host
    synchronisation is needed to size the launch."""
    dev = _require_gpu(q, k, v, cu_seqlens)
    q = q.contiguous()
    k = k.contiguous()
    v = v.contiguous()
    out = torch.empty_like(q)
    total = q.shape[0]
    if total == 0:
        return out
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k and v must share one dtype")
    if (q.dim() != 3 or tuple(q.shape[1:]) != (num_heads, head_dim) or k.shape != v.shape
            or tuple(k.shape) != (total, num_kv_heads, head_dim)):
        raise ValueError(f"q {tuple(q.shape)} and k/v {tuple(k.shape)} / {tuple(v.shape)} must be "
                         f"(total, {num_heads} / {num_kv_heads}, {head_dim}) with one total")
    cu = cu_seqlens.to(torch.int32).contiguous()
    num_seqs = cu.shape[0] - 1
    nbytes = _lib.query("mkv_flash_prefill_workspace_size", num_seqs, total, num_heads,
                        num_kv_heads)
    ws = _workspace(dev, "flash", nbytes) if nbytes else None
    _lib.call("mkv_flash_prefill", out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
              _dtype_code(q, "q"), cu.data_ptr(), num_seqs, total, num_heads, num_kv_heads,
              head_dim, float(scale), ws.data_ptr() if ws is not None else None,
              ws.numel() if ws is not None else 0, _stream(dev))
    return out


# ---------------------------------------------------------------------------
# K4: standalone gather
# ---------------------------------------------------------------------------
def gather_kv(cache: torch.Tensor, block_tables: torch.Tensor, context_lens: torch.Tensor,
              max_len: int | None = None) -> torch.Tensor:
    """Paged -> contiguous (batch, max_len, num_kv_heads, head_dim) copy of a
    cache through the block tables; rows past a sequence's context length or
    in an absent (-1) block are zero.  max_len defaults to the table's
    capacity (max_blocks * block_size), which needs no host synchronisation.
    The torch form of this gather is benchmark_decoding.py:166-178."""
    dev = _require_gpu(cache, block_tables, context_lens)
    bt = _block_table(block_tables)
    cl = _ctx_lens(context_lens)
    batch = bt.shape[0]
    num_blocks, bs, hkv, d = cache.shape
    if max_len is None:
        max_len = bt.shape[1] * bs
    out = torch.empty(batch, max_len, hkv, d, dtype=cache.dtype, device=dev)
    _lib.call("mkv_gather_kv", out.data_ptr(), cache.data_ptr(), _dtype_code(cache, "cache"),
              num_blocks, bt.data_ptr(), bt.stride(0), bt.shape[1], cl.data_ptr(),
              _index_dtype(cl), batch, max_len, hkv, d, bs, _stream(dev))
    return out


# ---------------------------------------------------------------------------
# Attention layer (the reference's only caller of the operators above)
# ---------------------------------------------------------------------------
class Attention(nn.Module):
    """Paged attention layer with the reference's constructor and
    ``forward(q, k, v)`` contract (attention.py:1617-1807).

    The runner injects ``k_cache``, ``v_cache``, ``k_scale``, ``v_scale`` and
    ``kv_cache_dtype`` ('auto', 'fp8_per_tensor', 'fp8_per_token_head' or
    'int8_per_token_head'), then sets the per-step
    :class:`~mkv.context.Context`.  Unlike the reference, which raises for
    any quantised cache there (attention.py:1702-1708), FP8 per-tensor and
    FP8 / INT8 per-token-head caches also work for chunked / mixed prefill.
    """

    def __init__(self, num_heads: int, head_dim: int, scale: float = 1.0,
                 num_kv_heads: int | None = None, block_size: int = 16):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads if num_kv_heads is not None else num_heads
        self.block_size = block_size
        self.k_cache = self.v_cache = torch.tensor([])
        self.kv_cache_dtype = "auto"
        self.k_scale = None
        self.v_scale = None
        # Mixed decode + prefill batches: "unified" runs every row through the
        # prefill kernel in one launch (a decode row is a chunk of one token:
        # visible = min(context_len, position + 1) = context_len); "split" is
        # the reference's route (attention.py:1711-1760): index_select the
        # decode and prefill rows, two kernels, index_copy_ back; "overlap"
        # is "split" with the decode rows on a second stream, concurrent with
        # the prefill kernel.  "unified" is the default: the prefill kernel
        # reads a decode row's K/V once per KV head, as the decode kernel
        # does, and its longest-first tile order runs the long decode rows
        # first and fills in around them, with no gathers and no second
        # launch.
        self.mixed_batch = "unified"
        # decode schedule: 0 = the library's choice (the default), or an
        # explicit one (DECODE_STREAM, n > 0 for n-token split-K,
        # DECODE_WORKGROUP), as for paged_attention_decode
        self.decode_split_tokens = 0

    def _mode(self) -> str:
        mode = self.kv_cache_dtype
        if mode in ("auto", "fp8_per_tensor") or mode in PER_TOKEN_HEAD_MODES:
            return mode
        if isinstance(mode, str) and mode.startswith("kivi"):
            raise NotImplementedError(f"kv_cache_dtype {mode!r} is not implemented by mkv")
        raise ValueError(f"unknown kv_cache_dtype {mode!r}")

    def _decode(self, q, block_tables, context_lens, scale):
        mode = self._mode()
        if mode != "auto":
            return paged_attention_decode_quantized(
                q, self.k_cache, self.v_cache, self.k_scale, self.v_scale, block_tables,
                context_lens, scale, self.num_heads, self.num_kv_heads, self.head_dim,
                self.block_size, mode, split_tokens=self.decode_split_tokens)
        return paged_attention_decode(q, self.k_cache, self.v_cache, block_tables, context_lens,
                                      scale, self.num_heads, self.num_kv_heads, self.head_dim,
                                      self.block_size, split_tokens=self.decode_split_tokens)

    def _prefill(self, q, block_tables, context_lens, cu_seqlens_q, positions, scale):
        quant = self._mode() != "auto"
        return paged_attention_prefill_triton(
            q, self.k_cache, self.v_cache, block_tables, context_lens, cu_seqlens_q, positions,
            scale, self.num_heads, self.num_kv_heads, self.head_dim, self.block_size,
            k_scale=self.k_scale if quant else None, v_scale=self.v_scale if quant else None,
            kv_cache_dtype=self.kv_cache_dtype)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                kv_appended: bool = False) -> torch.Tensor:
        """The reference's forward (store, then attend).  kv_appended=True:
        the step's K/V are already in the cache (mkv.producer's fused
        norm + rotary + append), so the store is skipped; k and v are still
        used by a full prefill."""
        context = current_context()
        mode = self._mode()
        if (not kv_appended and self.k_cache.numel() > 0 and self.v_cache.numel() > 0
                and context.slot_mapping is not None):
            if k.dim() == 4:
                k = k.reshape(-1, k.shape[-2], k.shape[-1])
                v = v.reshape(-1, v.shape[-2], v.shape[-1])
            if mode == "int8_per_token_head":
                store_kvcache_int8(k, v, self.k_cache, self.v_cache, self.k_scale, self.v_scale,
                                   context.slot_mapping, self.block_size)
            elif mode in ("fp8_per_tensor", "fp8_per_token_head"):
                store_kvcache_fp8(k, v, self.k_cache, self.v_cache, self.k_scale, self.v_scale,
                                  context.slot_mapping, self.block_size, mode)
            else:
                store_kvcache(k, v, self.k_cache, self.v_cache, context.slot_mapping,
                              self.block_size)

        scale = self.scale / (self.head_dim ** 0.5)
        if context.is_prefill:
            cu_seqlens = context.cu_seqlens_q
            if cu_seqlens is None:
                raise ValueError("cu_seqlens_q must be provided for varlen attention")
            if context.is_full_prefill:
                o = flash_attention_prefill(q, k, v, cu_seqlens, scale, self.num_heads,
                                            self.num_kv_heads, self.head_dim)
                return o.reshape(o.shape[0], self.num_heads * self.head_dim)
            if context.positions is None or context.context_lens is None or context.block_tables is None:
                raise ValueError("paged prefill requires positions, context_lens, and block_tables")
            split = context.mixed_attention_split
            if (self.mixed_batch in ("split", "overlap") and split is not None
                    and split.decode_token_indices and split.prefill_token_indices):
                if (split.decode_token_indices_tensor is None or split.decode_seq_indices_tensor is None
                        or split.prefill_token_indices_tensor is None
                        or split.prefill_seq_indices_tensor is None
                        or split.prefill_cu_seqlens_q_tensor is None):
                    raise ValueError("mixed attention split tensors must be prepared")
                o = torch.empty_like(q)
                dti = split.decode_token_indices_tensor
                dsi = split.decode_seq_indices_tensor
                pti = split.prefill_token_indices_tensor
                psi = split.prefill_seq_indices_tensor

                def decode_rows():
                    o.index_copy_(0, dti, self._decode(
                        q.index_select(0, dti), context.block_tables.index_select(0, dsi),
                        context.context_lens.index_select(0, dsi), scale))

                if self.mixed_batch == "overlap":
                    # the memory-bound decode rows run on a second stream while
                    # the MFMA-bound prefill rows run on this one
                    main = torch.cuda.current_stream(q.device)
                    side = _side_stream(q.device)
                    side.wait_stream(main)
                    with torch.cuda.stream(side):
                        decode_rows()
                else:
                    decode_rows()
                o.index_copy_(0, pti, self._prefill(
                    q.index_select(0, pti), context.block_tables.index_select(0, psi),
                    context.context_lens.index_select(0, psi), split.prefill_cu_seqlens_q_tensor,
                    context.positions.index_select(0, pti), scale))
                if self.mixed_batch == "overlap":
                    main.wait_stream(side)
                return o.reshape(o.shape[0], self.num_heads * self.head_dim)
            o = self._prefill(q, context.block_tables, context.context_lens, cu_seqlens,
                              context.positions, scale)
            return o.reshape(o.shape[0], self.num_heads * self.head_dim)
        o = self._decode(q, context.block_tables, context.context_lens, scale)
        return o.reshape(o.shape[0], self.num_heads * self.head_dim)
