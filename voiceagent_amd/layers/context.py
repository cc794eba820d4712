"""Per-forward attention metadata (mirror of qwen_asr_vllm/layers/context.py:1-51).

The model runner assembles a batch and the attention layers, deep in the
stack, need its offsets; the two meet through a module-level value.  There is
no prefill/decode flag: a batch may mix both, and the attention layer picks
the decode kernel only when every sequence contributes exactly one query
(``max_seqlen_q == 1``).
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class AttentionContext:
    cu_seqlens_q: torch.Tensor | None = None
    """Cumulative query lengths (int32); a decode request contributes 1."""
    cu_seqlens_k: torch.Tensor | None = None
    """Cumulative context lengths (int32), including tokens already cached."""
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    """Physical KV slot of each query token (int32); ``-1`` skips the write."""
    block_tables: torch.Tensor | None = None
    """[num_seqs, width] int32 block ids; padding beyond a sequence is ignored."""
    max_seqlen_k_exact: bool = False
    """True when max_seqlen_k is the batch's exact longest context, as an eager
    step computes it (qwen_asr_vllm/engine/model_runner.py:213); decode then
    fixes its context partitions from it at any length (ops.SPLIT_EXACT).  Not
    a field of the reference's context: its runner leaves the default, and a
    graph's max_model_len bound must too."""


_CONTEXT = AttentionContext()


def get_attention_context() -> AttentionContext:
    return _CONTEXT


def set_attention_context(context: AttentionContext) -> None:
    global _CONTEXT
    _CONTEXT = context


@contextmanager
def attention_context(context: AttentionContext):
    previous = get_attention_context()
    set_attention_context(context)
    try:
        yield
    finally:
        set_attention_context(previous)
