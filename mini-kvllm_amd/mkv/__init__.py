"""mkv — MI355X-native (gfx950) KV-cache hot path of the mini-kvllm engine.

Hand-written HIP kernels behind a C ABI (include/mkv.h, libmkv.so), exposed
with the reference engine's Python call signatures:

* :func:`store_kvcache`, :func:`store_kvcache_fp8`, :func:`store_kvcache_int8`
  — slot-mapped append (plain copy, or fused FP8 e4m3fn / INT8 quantisation
  with per-tensor or per-token-head scales);
* :func:`paged_attention_decode`, :func:`paged_attention_decode_quantized` —
  paged decode attention with GQA sharing (stream-K, split-K or one
  workgroup per sequence and KV head);
* :func:`paged_attention_prefill_triton`, :func:`flash_attention_prefill` —
  causal prefill over the paged cache / over fresh contiguous K/V;
* :func:`gather_kv` — block-table gather;
* :class:`Attention` and :mod:`mkv.context` — the layer and per-step
  metadata the runner drives.
"""
from .attention import (DECODE_STREAM, DECODE_WORKGROUP, FP8_E4M3_MAX, Attention, calibrate_fp8_per_tensor,
                        flash_attention_prefill, gather_kv, paged_attention_decode,
                        paged_attention_decode_quantized, paged_attention_prefill_triton,
                        store_kvcache, store_kvcache_fp8, store_kvcache_int8)
from .context import (Context, MixedAttentionSplit, current_context, get_context, reset_context,
                      set_context, split_mixed_decode_prefill_metadata, use_context_provider)

__all__ = [
    "DECODE_STREAM", "DECODE_WORKGROUP", "FP8_E4M3_MAX", "Attention", "Context", "MixedAttentionSplit", "calibrate_fp8_per_tensor",
    "flash_attention_prefill", "gather_kv", "get_context", "paged_attention_decode",
    "paged_attention_decode_quantized", "paged_attention_prefill_triton", "reset_context",
    "set_context", "split_mixed_decode_prefill_metadata", "store_kvcache", "store_kvcache_fp8",
    "store_kvcache_int8",
    "current_context", "use_context_provider",
]
