"""Per-step attention metadata carried from the runner to the attention layers.

Same fields, defaults and helper functions as the reference engine's
``myvllm.utils.context`` (src/myvllm/utils/context.py:10-124), so a runner
written against the reference fills it unchanged:

* ``slot_mapping`` int64 (tokens,), -1 = do not store (model_runner.py:467);
* ``block_tables`` int32 (seqs, max_blocks) padded with -1 (:555-557);
* ``context_lens`` int64 (seqs,) = visible length after this step (:541);
* ``cu_seqlens_q`` int32 (seqs + 1,), ``positions`` int64 (tokens,).

The KIVI residual fields are kept for interface compatibility only; this
package implements no KIVI kernels.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch


@dataclass
class MixedAttentionSplit:
    """Row/sequence indices of the decode and prefill parts of a mixed batch
    (reference: context.py:10-21)."""

    decode_token_indices: list[int]
    decode_seq_indices: list[int]
    prefill_token_indices: list[int]
    prefill_seq_indices: list[int]
    prefill_cu_seqlens_q: list[int]
    decode_token_indices_tensor: torch.Tensor | None = None
    decode_seq_indices_tensor: torch.Tensor | None = None
    prefill_token_indices_tensor: torch.Tensor | None = None
    prefill_seq_indices_tensor: torch.Tensor | None = None
    prefill_cu_seqlens_q_tensor: torch.Tensor | None = None


@dataclass
class Context:
    """Reference: context.py:24-47."""

    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    positions: torch.Tensor | None = None
    query_lens: torch.Tensor | None = None
    is_decode: torch.Tensor | None = None
    mixed_attention_split: MixedAttentionSplit | None = None
    # True only when every sequence of the batch is a whole prompt starting at
    # position 0; only then may attention run on the fresh contiguous q/k/v.
    is_full_prefill: bool = False
    residual_slots: torch.Tensor | None = None
    residual_lens: torch.Tensor | None = None


def _as_list(values) -> list:
    return list(values.tolist()) if hasattr(values, "tolist") else list(values)


def split_mixed_decode_prefill_metadata(cu_seqlens_q: Sequence[int], query_lens: Sequence[int],
                                        is_decode: Sequence[bool]) -> MixedAttentionSplit:
    """Partition a mixed batch into decode rows and prefill rows, keeping the
    scheduler's order inside each part (reference: context.py:55-88)."""
    cu = _as_list(cu_seqlens_q)
    lens = _as_list(query_lens)
    flags = [bool(x) for x in _as_list(is_decode)]
    out = MixedAttentionSplit([], [], [], [], [0])
    for s, (qlen, dec) in enumerate(zip(lens, flags)):
        rows = range(cu[s], cu[s + 1])
        if dec:
            out.decode_token_indices.extend(rows)
            out.decode_seq_indices.append(s)
        else:
            out.prefill_token_indices.extend(rows)
            out.prefill_seq_indices.append(s)
            out.prefill_cu_seqlens_q.append(out.prefill_cu_seqlens_q[-1] + qlen)
    return out


_context = Context()
_provider = None


def get_context() -> Context:
    return _context


def use_context_provider(provider) -> None:
    """Make :class:`mkv.Attention` read its per-step metadata from
    ``provider()`` instead of this module's context, e.g. the engine's own
    ``myvllm.utils.context.get_context`` (its Context has the same field
    names).  ``None`` restores this module's context."""
    global _provider
    _provider = provider


def current_context():
    """The context :class:`mkv.Attention` uses for this step."""
    return _provider() if _provider is not None else _context


def reset_context() -> None:
    global _context
    _context = Context()


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, positions=None,
                query_lens=None, is_decode=None, mixed_attention_split=None,
                is_full_prefill=False, residual_slots=None, residual_lens=None) -> None:
    """Reference: context.py:103-124 (same keyword names and defaults)."""
    global _context
    _context = Context(
        is_prefill=is_prefill, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
        max_seqlen_q=max_seqlen_q, max_seqlen_k=max_seqlen_k, slot_mapping=slot_mapping,
        context_lens=context_lens, block_tables=block_tables, positions=positions,
        query_lens=query_lens, is_decode=is_decode, mixed_attention_split=mixed_attention_split,
        is_full_prefill=is_full_prefill, residual_slots=residual_slots,
        residual_lens=residual_lens)
